// Row-tiled MFMA GEMV for MatMulNBits on gfx950 (int4 weights, block_size >= 32), in two
// arithmetic flavours, both optionally grouped by expert:
//
//   group_gemv_f16   fp16 activations; (q - zp) as exact fp16 on v_mfma_f32_16x16x32_f16, each
//                    32-k partial scaled by its block's scale in fp32 (the reference kernel's
//                    per-block fp32 partial, rust/shaders/glsl/templates/q_gemv.comp:571-579).
//   group_gemv_i8    accuracy_level = 4: activations quantised to int8 per (row, block) by
//                    quantize_a_int8 below; (q - zp) as int8 on v_mfma_i32_16x16x32_i8, exact
//                    int32 block dots, scaled by a_scale * b_scale in fp32.  ORT's CPU EP runs
//                    this level as SQNBIT_CompInt8 (third-party ONNX Runtime; the reference
//                    declines the level, rust/src/ops/quant.rs:191-200): the quantiser here is
//                    this build's declared definition (symmetric, amax / 127, round half even).
//
// Loads.  A wavefront owns 16 columns; lane (n = l%16, g = l/16) reads 16 contiguous bytes of
// column n per iteration -- 32-k chunk 4c+g -- so each load instruction covers 16 runs of 64
// bytes.  A 4 x 4 dword transpose across the four lane rows (v_permlane32_swap then
// v_permlane16_swap) turns that into MFMA operands: afterwards lane (n, g) holds dword g of
// chunks 4c..4c+3, i.e. for chunk t the eight k = 32t + 8g .. +8 that MFMA lane (n, g) supplies,
// so every MFMA covers one chunk of one block.
//
// Grouping.  For the expert-grouped (MoE) form, blockIdx.y is the expert: its rows are
// offsets[e] .. offsets[e+1] of Y, gathered from A through row_index, and its weights are the
// e-th of `experts` consecutive per-expert B / scales / zero_points tensors.  The dense form is
// one group with rows 0 .. M-1.  The W wavefronts of a workgroup split the K iterations and are
// summed in a fixed order through LDS, so results are run-to-run deterministic.
#include <type_traits>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

namespace {

// 4 x 4 transpose of dwords across the lane rows (16 lanes each) of a wavefront: on return,
// v[t] of a lane in row g is what v[g] of the same column lane in row t held.
__device__ __forceinline__ void transpose_rows(uint32_t& v0, uint32_t& v1, uint32_t& v2,
                                               uint32_t& v3) {
    auto a = __builtin_amdgcn_permlane32_swap(v0, v2, false, false);
    v0 = a[0];
    v2 = a[1];
    auto b = __builtin_amdgcn_permlane32_swap(v1, v3, false, false);
    v1 = b[0];
    v3 = b[1];
    auto c = __builtin_amdgcn_permlane16_swap(v0, v1, false, false);
    v0 = c[0];
    v1 = c[1];
    auto d = __builtin_amdgcn_permlane16_swap(v2, v3, false, false);
    v2 = d[0];
    v3 = d[1];
}

// Eight int4 weights (one dword, natural order e0..e7) as int8 (q - z) in the order
// [e0, e2, e4, e6, e1, e3, e5, e7] (the order quantize_a_int8 writes activations in).
__device__ __forceinline__ i32x2 qz_i8(uint32_t w, uint32_t zb) {
    // per byte: (q + 128 - z) has no carry for q, z in 0..15; XOR 0x80 gives (q - z) mod 256
    const uint32_t lo = ((w & 0x0F0F0F0Fu) + zb) ^ 0x80808080u;
    const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) + zb) ^ 0x80808080u;
    return i32x2{(int32_t)lo, (int32_t)hi};
}

}  // namespace

// T: activation / scale / output type (f16, or float for the int8 path's fp32 nodes).
// I8: false = fp16 activations (A is f16 [a_rows][K]); true = int8 activations (A is the
// quantiser's qa [a_rows][K] in permuted order, a_scale fp32 [a_rows][K/BS]).
template <typename T, bool I8, int BS, bool HAS_ZP, int MT>
__global__ void __launch_bounds__(512)
group_gemv(const void* __restrict__ Av, const float* __restrict__ a_scale,
           const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
           const uint8_t* __restrict__ B, const T* __restrict__ S, const uint8_t* __restrict__ Z,
           T* __restrict__ Y, int M, int N, int K) {
    extern __shared__ f32x4 red[];                       // [W][MT][64]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    const int nl = lane & 15;
    const int g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int col = min(n0 + nl, N - 1);
    const int bpc = K / BS;
    const int zpb = (bpc * 4 + 7) / 8;
    const int chunks = K / 32;                           // 32-k chunks per column
    const int iters = (chunks + 3) / 4;                  // 128-k iterations

    // Rows of this workgroup: group e, row tile blockIdx.z.
    int row_lo = 0, row_hi = M;
    int64_t wofs_b = 0, wofs_s = 0, wofs_z = 0;
    if (offsets) {
        const int e = blockIdx.y;
        row_lo = offsets[e];
        row_hi = offsets[e + 1];
        wofs_b = (int64_t)e * N * (K / 2);
        wofs_s = (int64_t)e * N * bpc;
        wofs_z = (int64_t)e * N * zpb;
    }
    const int r0 = row_lo + blockIdx.z * 16 * MT;
    if (r0 >= row_hi) return;                            // whole workgroup leaves: no barrier yet
    const uint8_t* __restrict__ bcol = B + wofs_b + (int64_t)col * (K / 2) + 16 * g;
    const T* __restrict__ scol = S + wofs_s + (int64_t)col * bpc;
    const uint8_t* __restrict__ zcol = HAS_ZP ? Z + wofs_z + (int64_t)col * zpb : nullptr;

    // A row of each 16-row tile this lane feeds (MFMA A operand: row l%16).
    int arow[MT];
    int srow[MT][4];                                     // rows of the lane's output values
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        int r = r0 + 16 * i + nl;
        r = r < row_hi ? r : row_hi - 1;
        arow[i] = row_index ? row_index[r] : r;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int rr = r0 + 16 * i + 4 * g + q;
            rr = rr < row_hi ? rr : row_hi - 1;
            srow[i][q] = row_index ? row_index[rr] : rr;
        }
    }

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Each wavefront takes runs of PF consecutive 128-k iterations: all weight, scale and
    // zero-point loads of a run are issued before any of it is computed.  Out-of-range chunks
    // load a clamped in-bounds address and are skipped (wave-uniformly) at compute time.
    constexpr int PF = group_pf(I8, BS, MT);
    constexpr int CPB = BS / 32;                         // 32-k chunks per block (1, 2 or 4)
    for (int c0 = wave * PF; c0 < iters; c0 += W * PF) {
        u32x4 raw[PF];
        T sr[PF][4];
        uint8_t zr[PF][4];
        float sa[I8 ? PF : 1][I8 ? 4 : 1][MT][4];        // int8 path: activation scales
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int c = c0 + p;
            int ch = 4 * c + g;
            const bool ok = ch < chunks;
            ch = ok ? ch : chunks - 1;
            raw[p] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(bcol - 16 * g + 16 * (int64_t)ch));
            if (!ok) raw[p] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int kc = 4 * c + t;
                kc = kc < chunks ? kc : chunks - 1;
                const int blk = (32 * kc) / BS;
                if (!I8 || (t + 1) % CPB == 0) sr[p][t] = scol[blk];
                if constexpr (HAS_ZP) zr[p][t] = zcol[blk >> 1];
                else zr[p][t] = 0;
                if constexpr (I8) {
                    if ((t + 1) % CPB == 0) {            // block ends: one scale per output row
#pragma unroll
                        for (int i = 0; i < MT; ++i)
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                sa[p][t][i][q] = a_scale[(int64_t)srow[i][q] * bpc + blk];
                    }
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int c = c0 + p;
            if (c >= iters) break;                       // wave-uniform
            const bool full = 4 * c + 3 < chunks;        // wave-uniform
            uint32_t v0 = raw[p].x, v1 = raw[p].y, v2 = raw[p].z, v3 = raw[p].w;
            transpose_rows(v0, v1, v2, v3);
            const uint32_t wt[4] = {v0, v1, v2, v3};
            if constexpr (!I8) {
                const f16* __restrict__ A = static_cast<const f16*>(Av);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int kc = 4 * c + t;
                    if (!full && kc >= chunks) break;    // wave-uniform
                    const int blk = (32 * kc) / BS;
                    const float s = (float)sr[p][t];
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((zr[p][t] >> ((blk & 1) * 4)) & 0xFu);
                    const f16x2 zo = zoff4(z);
                    f16x8 bop;
                    bop.s01 = nib_pair<0>(wt[t], zo);
                    bop.s23 = nib_pair<1>(wt[t], zo);
                    bop.s45 = nib_pair<2>(wt[t], zo);
                    bop.s67 = nib_pair<3>(wt[t], zo);
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        const f16x8 aop = *reinterpret_cast<const f16x8*>(A + (int64_t)arow[i] * K + 32 * kc + 8 * g);
                        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, d, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[i][q] = __builtin_fmaf(d[q], s, acc[i][q]);
                    }
                }
            } else {
                const int8_t* __restrict__ A = static_cast<const int8_t*>(Av);
                i32x4 dot[MT];
#pragma unroll
                for (int i = 0; i < MT; ++i) dot[i] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int kc = 4 * c + t;
                    if (!full && kc >= chunks) break;    // wave-uniform
                    const int blk = (32 * kc) / BS;
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((zr[p][t] >> ((blk & 1) * 4)) & 0xFu);
                    const uint32_t zb = (uint32_t)(128 - z) * 0x01010101u;
                    const i32x2 bop = qz_i8(wt[t], zb);
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        const i32x2 aop = *reinterpret_cast<const i32x2*>(A + (int64_t)arow[i] * K + 32 * kc + 8 * g);
                        dot[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            __builtin_bit_cast(long, aop), __builtin_bit_cast(long, bop), dot[i], 0, 0, 0);
                    }
                    // K % BS == 0, so a block always ends on a chunk with (t + 1) % CPB == 0.
                    if ((t + 1) % CPB == 0) {            // end of a block: scale it
                        const float sb = (float)sr[p][t];
#pragma unroll
                        for (int i = 0; i < MT; ++i) {
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                acc[i][q] = __builtin_fmaf((float)dot[i][q], sa[p][t][i][q] * sb, acc[i][q]);
                            dot[i] = i32x4{0, 0, 0, 0};
                        }
                    }
                }
            }
        }
    }

    // Fixed-order sum of the W wavefronts' partial tiles.
#pragma unroll
    for (int i = 0; i < MT; ++i) red[(wave * MT + i) * 64 + lane] = acc[i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 64 * MT; idx += blockDim.x) {
        f32x4 sum = red[idx];
        for (int w = 1; w < W; ++w) sum += red[w * MT * 64 + idx];
        const int i = idx >> 6;
        const int ll = idx & 63;
        const int cc = n0 + (ll & 15);
        if (cc >= N) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = r0 + 16 * i + 4 * (ll >> 4) + q;
            if (r < row_hi) Y[(int64_t)r * N + cc] = (T)sum[q];
        }
    }
}

// accuracy_level = 4 activation quantiser.  One thread per 8 consecutive activations; the
// BS/8 threads of a (row, block) reduce amax with shuffles.  scale = amax / 127,
// qa = clamp(rint(a * (127 / amax)), -127, 127) (0 when amax == 0), all in fp32 with
// round-half-even.  PERMUTED writes each group of eight as [0,2,4,6,1,3,5,7] (the order
// qz_i8 produces weights in); otherwise natural order plus the block sums of qa.
template <typename T, int BS, bool PERMUTED>
__global__ void __launch_bounds__(256)
quantize_a_int8(const T* __restrict__ A, int8_t* __restrict__ qa, float* __restrict__ scale,
                int32_t* __restrict__ qsum, int M, int K) {
    constexpr int G = BS / 8;                            // threads per block: 2..16
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t groups = (int64_t)M * (K / 8);
    const bool live = t < groups;
    const int64_t tt = live ? t : groups - 1;
    const int row = (int)(tt / (K / 8));
    const int k0 = (int)(tt % (K / 8)) * 8;
    float a[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (float)A[(int64_t)row * K + k0 + e];
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(a[e]));
    // G consecutive threads share a block (G divides 64 and blocks start at multiples of G).
#pragma unroll
    for (int off = G >> 1; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float inv = amax > 0.f ? 127.0f / amax : 0.f;
    int q[8];
    int s = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float v = rintf(a[e] * inv);
        v = fminf(fmaxf(v, -127.f), 127.f);
        q[e] = (int)v;
        s += q[e];
    }
    if (!live) return;
    const int blk = k0 / BS;
    const int bpc = K / BS;
    int8_t* out = qa + (int64_t)row * K + k0;
    if constexpr (PERMUTED) {
        const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (int8_t)q[order[e]];
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (int8_t)q[e];
    }
    if (k0 % BS == 0) scale[(int64_t)row * bpc + blk] = amax / 127.0f;
    if (qsum) {
        // block sum: the G partial sums meet in the block's first thread
        int bs_sum = s;
        for (int off = G >> 1; off > 0; off >>= 1) bs_sum += __shfl_xor(bs_sum, off, 64);
        if (k0 % BS == 0) qsum[(int64_t)row * bpc + blk] = bs_sum;
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

bool group_gemv_supported(int64_t k, int bits, int bs) {
    return bits == 4 && bs >= 32 && k > 0 && k % 32 == 0 && k % bs == 0;
}

GroupGeom group_geometry(int64_t rows, int64_t n, int64_t k, int64_t groups, bool i8, int bs) {
    GroupGeom g{};
    g.mt = rows <= 16 ? 1 : (rows <= 32 ? 2 : 4);
    const int64_t iters = (k / 32 + 3) / 4;
    const int pf = group_pf(i8, bs, g.mt);
    const int64_t runs = (iters + pf - 1) / pf;          // runs of pf iterations per wavefront
    // Enough wavefronts on each 16-column strip to fill the chip: about 8 per CU in total.
    const int64_t strips = ((n + 15) / 16) * groups;
    int64_t w = (8 * 256 + strips - 1) / strips;
    if (w < 1) w = 1;
    if (w > 8) w = 8;
    if (w > runs) w = runs;
    g.waves = (int)w;
    g.gx = (n + 15) / 16;
    g.gy = groups;
    g.gz = (rows + 16 * g.mt - 1) / (16 * g.mt);
    g.lds = (size_t)g.waves * g.mt * 64 * sizeof(f32x4);
    return g;
}

template <typename T, bool I8, int BS, bool HAS_ZP>
static hipError_t group_mt(const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, hipStream_t st) {
    const dim3 grid((unsigned)g.gx, (unsigned)g.gy, (unsigned)g.gz);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
    const T* S = static_cast<const T*>(s);
    T* Y = static_cast<T*>(y);
#define MNB_GROUP_GO(MT_)                                                                          \
    hipLaunchKernelGGL((group_gemv<T, I8, BS, HAS_ZP, MT_>), grid, block, g.lds, st, a, a_scale, \
                       row_index, offsets, b, S, z, Y, (int)m, (int)n, (int)k)
    switch (g.mt) {
        case 1: MNB_GROUP_GO(1); break;
        case 2: MNB_GROUP_GO(2); break;
        default: MNB_GROUP_GO(4); break;
    }
#undef MNB_GROUP_GO
    return hipGetLastError();
}

template <typename T, bool I8, int BS>
static hipError_t group_zp(const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, hipStream_t st) {
    if (z) return group_mt<T, I8, BS, true>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, st);
    return group_mt<T, I8, BS, false>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, st);
}

template <typename T, bool I8>
static hipError_t group_bs(int bs, const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, hipStream_t st) {
    switch (bs) {
        case 32: return group_zp<T, I8, 32>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, st);
        case 64: return group_zp<T, I8, 64>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, st);
        case 128: return group_zp<T, I8, 128>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_group_gemv_f16(const void* a, const int32_t* row_index, const int32_t* offsets,
                                 int64_t groups, int64_t max_rows, const uint8_t* b,
                                 const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                 int64_t k, int bits, int bs, hipStream_t st) {
    if (!group_gemv_supported(k, bits, bs)) return hipErrorInvalidValue;
    if (m == 0 || groups == 0) return hipSuccess;
    const GroupGeom g = group_geometry(offsets ? max_rows : m, n, k, offsets ? groups : 1, false, bs);
    return group_bs<f16, false>(bs, g, a, nullptr, row_index, offsets, b, s, z, y, m, n, k, st);
}

hipError_t launch_quantize_a_int8(const void* a, bool a_f16, int8_t* qa, float* scale,
                                  int32_t* qsum, bool permuted, int64_t m, int64_t k, int bs,
                                  hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (k % bs || (bs != 16 && bs != 32 && bs != 64 && bs != 128)) return hipErrorInvalidValue;
    const int64_t groups = m * (k / 8);
    const dim3 grid((unsigned)((groups + 255) / 256));
#define MNB_Q(T_, BS_)                                                                            \
    do {                                                                                          \
        if (permuted)                                                                             \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, true>), grid, dim3(256), 0, st,          \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k);      \
        else                                                                                      \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, false>), grid, dim3(256), 0, st,         \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k);      \
    } while (0)
#define MNB_QBS(T_)                                                                               \
    switch (bs) {                                                                                 \
        case 16: MNB_Q(T_, 16); break;                                                            \
        case 32: MNB_Q(T_, 32); break;                                                            \
        case 64: MNB_Q(T_, 64); break;                                                            \
        default: MNB_Q(T_, 128); break;                                                           \
    }
    if (a_f16) {
        MNB_QBS(f16);
    } else {
        MNB_QBS(float);
    }
#undef MNB_QBS
#undef MNB_Q
    return hipGetLastError();
}

size_t acc4_workspace_bytes(int64_t m, int64_t k, int bs) {
    const size_t qa = ((size_t)m * (size_t)k + 255) & ~(size_t)255;
    return qa + (size_t)m * (size_t)(k / bs) * sizeof(float);
}

hipError_t launch_acc4(const void* a, bool a_f16, const int32_t* row_index,
                       const int32_t* offsets, int64_t groups, int64_t max_rows,
                       const uint8_t* b, const void* s, const uint8_t* z, void* y, int64_t m,
                       int64_t n, int64_t k, int bits, int bs, void* workspace,
                       hipStream_t st) {
    if (!group_gemv_supported(k, bits, bs)) return hipErrorInvalidValue;
    if (m == 0 || groups == 0) return hipSuccess;
    int8_t* qa = static_cast<int8_t*>(workspace);
    float* sa = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                         (((size_t)m * (size_t)k + 255) & ~(size_t)255));
    hipError_t e = launch_quantize_a_int8(a, a_f16, qa, sa, nullptr, true, m, k, bs, st);
    if (e != hipSuccess) return e;
    const GroupGeom g = group_geometry(offsets ? max_rows : m, n, k, offsets ? groups : 1, true, bs);
    if (a_f16) return group_bs<f16, true>(bs, g, qa, sa, row_index, offsets, b, s, z, y, m, n, k, st);
    return group_bs<float, true>(bs, g, qa, sa, row_index, offsets, b, s, z, y, m, n, k, st);
}

}  // namespace mnb
