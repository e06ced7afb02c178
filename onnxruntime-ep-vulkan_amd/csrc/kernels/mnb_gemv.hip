// Decode-shaped MatMulNBits on gfx950: the streaming GEMV (M <= 64, fp16), the generic
// any-format kernel, and the bit-exact dequantiser.
//
// Reference behaviour reproduced (not its code): rust/shaders/glsl/templates/q_gemv.comp forms,
// per (column, quant block), the fp32 partial sum of a * (q - zp) over the block and scales it
// once in fp32 (q_gemv.comp:571-579), then reduces across the workgroup.  Here one workgroup owns
// 16 output columns and the whole K extent; its W wavefronts split the quant blocks between
// them, and every block of every column is one v_mfma_f32_16x16x32_f16 chain (16x16x16 for
// block 16) over exact integer (q - zp) fp16 operands, so the block partial is an fp32 MFMA
// result that is scaled by the block's scale in fp32 — the reference's arithmetic, with the
// block-local reduction done by the matrix core instead of a shared-memory tree.
//
// Lane mapping inside a block (lane l, column c = l % 16, lane group g = l / 16):
//     B operand = (q - zp) of B[n0 + c][blk*BS + g*BS/4 ... + BS/4)     one contiguous run of
//                                                                         BS*BITS/32 bytes
//     A operand = A[m][blk*BS + g*BS/4 + 8j ... + 8) for MFMA j           (row m = l % 16)
// The MFMA pairs A-lane (i, g) element e with B-lane (j, g) element e, so both sides name the
// same k and every MFMA stays inside one quant block.  Partial tiles of the W wavefronts are
// summed in a fixed order through LDS, so the result is run-to-run deterministic.
#include <type_traits>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// Bytes of one lane's share of a quant block: BS/4 weights.
template <int BITS, int BS>
struct LaneChunk {
    static constexpr int BYTES = (BS / 4) * BITS / 8;            // 2, 4, 8, 16 or 32
    static constexpr int WORDS = BYTES >= 4 ? BYTES / 4 : 1;
    uint32_t w[WORDS];

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < WORDS; ++i) w[i] = 0u;
    }
    __device__ __forceinline__ void load(const uint8_t* __restrict__ p) {
        if constexpr (BYTES == 2) {
            w[0] = *reinterpret_cast<const uint16_t*>(p);
        } else if constexpr (BYTES == 4) {
            w[0] = *reinterpret_cast<const uint32_t*>(p);
        } else if constexpr (BYTES == 8) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(p);
            w[0] = v.x;
            w[1] = v.y;
        } else {
#pragma unroll
            for (int h = 0; h < BYTES / 16; ++h) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(p + 16 * h);
                w[4 * h + 0] = v.x;
                w[4 * h + 1] = v.y;
                w[4 * h + 2] = v.z;
                w[4 * h + 3] = v.w;
            }
        }
    }
};

// Exact (q - z) operands.  x32: eight weights per MFMA; x16 (block 16): four.
__device__ __forceinline__ f16x8 qz8_4b(uint32_t w, f16x2 zo) {
    f16x8 r;
    r.s01 = nib_pair<0>(w, zo);
    r.s23 = nib_pair<1>(w, zo);
    r.s45 = nib_pair<2>(w, zo);
    r.s67 = nib_pair<3>(w, zo);
    return r;
}
__device__ __forceinline__ f16x8 qz8_8b(uint32_t w0, uint32_t w1, f16x2 zo) {
    f16x8 r;
    r.s01 = byte_pair_lo(w0, zo);
    r.s23 = byte_pair_hi(w0, zo);
    r.s45 = byte_pair_lo(w1, zo);
    r.s67 = byte_pair_hi(w1, zo);
    return r;
}
__device__ __forceinline__ f16x4 qz4_4b(uint32_t w, f16x2 zo) {
    f16x4 r;
    r.s01 = nib_pair<0>(w, zo);
    r.s23 = nib_pair<1>(w, zo);
    return r;
}
__device__ __forceinline__ f16x4 qz4_8b(uint32_t w, f16x2 zo) {
    f16x4 r;
    r.s01 = byte_pair_lo(w, zo);
    r.s23 = byte_pair_hi(w, zo);
    return r;
}

// Quant blocks whose loads one wavefront issues together (about 256 weights of K per column);
// fewer when several 16-row tiles multiply the prefetched A operands.
template <int BS, int MT>
constexpr int gemv_group_blocks() {
    constexpr int g = BS == 16 ? 8 : 256 / BS;
    return g / MT > 0 ? g / MT : 1;
}

template <int BITS, int BS, bool HAS_ZP, int MT>
__global__ void __launch_bounds__(kGemvMaxThreads)
gemv_f16_mfma(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
              const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K) {
    using Chunk = LaneChunk<BITS, BS>;
    constexpr bool X16 = BS == 16;                      // one 16x16x16 MFMA per block
    constexpr int EPB = BS / 4;                         // weights per lane per block
    constexpr int NMF = X16 ? 1 : BS / 32;              // MFMAs per block and M tile
    constexpr int BLOB = BS * BITS / 8;                 // packed bytes per (column, block)
    constexpr int GB = gemv_group_blocks<BS, MT>();
    using AOp = typename std::conditional<X16, f16x4, f16x8>::type;

    extern __shared__ f32x4 red[];                      // [W][MT][64]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    const int nl = lane & 15;
    const int g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int col = min(n0 + nl, N - 1);
    const int m0 = blockIdx.y * 16 * MT;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const uint8_t* __restrict__ bcol = B + (int64_t)col * ((int64_t)bpc * BLOB) + g * Chunk::BYTES;
    const f16* __restrict__ scol = S + (int64_t)col * bpc;

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int gb = wave * GB; gb < bpc; gb += W * GB) {
        Chunk bq[GB];
        f16 sv[GB];
        int zv[GB];
        AOp aop[GB][MT][NMF];
        // Issue every weight, scale, zero-point and activation load of the group first.
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            const int blk = gb + i;
            const bool ok = blk < bpc;                  // wave-uniform
            bq[i].zero();
            sv[i] = (f16)0.0f;
            zv[i] = 1 << (BITS - 1);
            if (ok) {
                bq[i].load(bcol + (int64_t)blk * BLOB);
                sv[i] = scol[blk];
                zv[i] = load_zp<BITS, HAS_ZP>(Z, col, blk, zpb);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int row = m0 + 16 * t + nl;
                const bool rok = ok && row < M;
                const f16* __restrict__ ap = A + (int64_t)row * K + blk * BS + g * EPB;
#pragma unroll
                for (int j = 0; j < NMF; ++j) {
                    if constexpr (X16) {
                        aop[i][t][j] = f16x4{0, 0, 0, 0};
                        if (rok) aop[i][t][j] = *reinterpret_cast<const f16x4*>(ap);
                    } else {
                        aop[i][t][j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
                        if (rok) aop[i][t][j] = *reinterpret_cast<const f16x8*>(ap + 8 * j);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            if (gb + i >= bpc) break;                   // wave-uniform
            const f16x2 zo = (BITS == 4) ? zoff4(zv[i]) : zoff8(zv[i]);
            const float s = (float)sv[i];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < NMF; ++j) {
                    if constexpr (X16) {
                        const f16x4 bop = (BITS == 4) ? qz4_4b(bq[i].w[0], zo) : qz4_8b(bq[i].w[0], zo);
                        d = __builtin_amdgcn_mfma_f32_16x16x16f16(aop[i][t][j], bop, d, 0, 0, 0);
                    } else {
                        const f16x8 bop = (BITS == 4) ? qz8_4b(bq[i].w[j], zo)
                                                      : qz8_8b(bq[i].w[2 * j], bq[i].w[2 * j + 1], zo);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i][t][j], bop, d, 0, 0, 0);
                    }
                }
                // rows 4g + r of the tile: skip r that no lane group can hold (wave-uniform)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (m0 + 16 * t + r < M) acc[t][r] = __builtin_fmaf(d[r], s, acc[t][r]);
            }
        }
    }

    // Output layout of the 16x16 MFMA tile: lane l holds D[4*(l/16) + r][l % 16], r = 0..3.
    if (W == 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int cc = n0 + nl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + 16 * t + 4 * g + r;
                if (row < M && cc < N) Y[(int64_t)row * N + cc] = (f16)acc[t][r];
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * MT; i += blockDim.x) {
        f32x4 sum = red[i];
        for (int w = 1; w < W; ++w) sum += red[w * MT * 64 + i];
        const int t = i >> 6;
        const int ll = i & 63;
        const int cc = n0 + (ll & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + 16 * t + 4 * (ll >> 4) + r;
            if (row < M && cc < N) Y[(int64_t)row * N + cc] = (f16)sum[r];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Generic kernel: any dtype (fp16/fp32), bits, block size, M.  One wavefront per (column,
// 4-row tile); lanes stride over quantisation blocks, form the per-block fp32 partial of
// a * (q - zp) and scale it once, the reference kernel's arithmetic (q_gemv.comp:571-579);
// the 64 lane partials are then summed by a fixed butterfly.
// ------------------------------------------------------------------------------------------
template <typename T, int BITS, int BS, bool HAS_ZP>
__global__ void __launch_bounds__(256)
matmul_generic(const T* __restrict__ A, const uint8_t* __restrict__ B, const T* __restrict__ S,
               const uint8_t* __restrict__ Z, T* __restrict__ Y, int M, int N, int K) {
    constexpr int BLOB = BS * BITS / 8;
    constexpr int PER_WORD = 32 / BITS;
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;                                   // whole wavefront leaves together
    const int m0 = blockIdx.y * 4;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int blk = lane; blk < bpc; blk += 64) {
        const float s = (float)S[(int64_t)n * bpc + blk];
        const float z = (float)load_zp<BITS, HAS_ZP>(Z, n, blk, zpb);
        const uint32_t* __restrict__ p =
            reinterpret_cast<const uint32_t*>(B + ((int64_t)n * bpc + blk) * BLOB);
        float bacc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int wd = 0; wd < BLOB / 4; ++wd) {
            const uint32_t w = p[wd];
#pragma unroll
            for (int i = 0; i < PER_WORD; ++i) {
                const float wq = (float)((w >> (i * BITS)) & ((1u << BITS) - 1u)) - z;
                const int k = blk * BS + wd * PER_WORD + i;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + r;
                    if (row < M) bacc[r] += (float)A[(int64_t)row * K + k] * wq;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += bacc[r] * s;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + r;
            if (row < M) Y[(int64_t)row * N + n] = (T)acc[r];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Dequantiser: W[n][k] = fp16_rne(fp32(q - zp) * fp32(s)), one dword of packed B per thread,
// through the same unpack helpers the MFMA kernels use.
// ------------------------------------------------------------------------------------------
template <int BITS, int BS, bool HAS_ZP>
__global__ void __launch_bounds__(256)
dequant_f16(const uint8_t* __restrict__ B, const f16* __restrict__ S,
            const uint8_t* __restrict__ Z, f16* __restrict__ W, int N, int K) {
    constexpr int PER_WORD = 32 / BITS;
    const int64_t words_per_col = (int64_t)K / PER_WORD;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * words_per_col) return;
    const int n = (int)(idx / words_per_col);
    const int e = (int)(idx % words_per_col) * PER_WORD;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const int blk = e / BS;
    const uint32_t w = reinterpret_cast<const uint32_t*>(B)[idx];
    const f16 sv = S[(int64_t)n * bpc + blk];
    const f16x2 s2 = {sv, sv};
    const int zv = load_zp<BITS, HAS_ZP>(Z, n, blk, zpb);
    f16* out = W + (int64_t)n * K + e;
    if constexpr (BITS == 4) {
        *reinterpret_cast<f16x8*>(out) = dequant8_4b(w, zoff4(zv), s2);
    } else {
        const f16x2 zo = zoff8(zv);
        f16x2* o2 = reinterpret_cast<f16x2*>(out);
        o2[0] = byte_pair_lo(w, zo) * s2;
        o2[1] = byte_pair_hi(w, zo) * s2;
    }
}

// ------------------------------------------------------------------------------------------
// Host launchers
// ------------------------------------------------------------------------------------------

bool gemv_supported(int64_t k, int bits, int block_size) {
    (void)bits;
    return k > 0 && block_size >= 16 && (k % block_size) == 0;
}

static int group_blocks(int bs, int mt) {
    const int g = bs == 16 ? 8 : 256 / bs;
    return g / mt > 0 ? g / mt : 1;
}

GemvGeom gemv_geometry(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    (void)bits;
    GemvGeom g{};
    g.mt = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int64_t bpc = k / bs;
    const int64_t groups = (bpc + group_blocks(bs, g.mt) - 1) / group_blocks(bs, g.mt);
    const int maxw = 16 / g.mt;
    int64_t w = groups;                            // one load group per wavefront when possible
    if (w < 1) w = 1;
    if (w > maxw) w = maxw;
    g.waves = (int)w;
    g.gx = (n + 15) / 16;
    g.gy = (m + 16 * g.mt - 1) / (16 * g.mt);
    g.lds = g.waves > 1 ? (size_t)g.waves * g.mt * 64 * sizeof(f32x4) : 0;
    return g;
}

template <int BITS, int BS, bool HAS_ZP>
static hipError_t gemv_dispatch_mt(const GemvGeom& g, const void* a, const uint8_t* b,
                                   const void* s, const uint8_t* z, void* y, int64_t m,
                                   int64_t n, int64_t k, hipStream_t stream) {
    if (g.waves < 1 || 64 * g.waves > kGemvMaxThreads) return hipErrorInvalidValue;
    const dim3 grid((unsigned)g.gx, (unsigned)g.gy, 1);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
    const f16* A = static_cast<const f16*>(a);
    const f16* S = static_cast<const f16*>(s);
    f16* Y = static_cast<f16*>(y);
    switch (g.mt) {
        case 1:
            hipLaunchKernelGGL((gemv_f16_mfma<BITS, BS, HAS_ZP, 1>), grid, block, g.lds, stream,
                               A, b, S, z, Y, (int)m, (int)n, (int)k);
            break;
        case 2:
            hipLaunchKernelGGL((gemv_f16_mfma<BITS, BS, HAS_ZP, 2>), grid, block, g.lds, stream,
                               A, b, S, z, Y, (int)m, (int)n, (int)k);
            break;
        default:
            hipLaunchKernelGGL((gemv_f16_mfma<BITS, BS, HAS_ZP, 4>), grid, block, g.lds, stream,
                               A, b, S, z, Y, (int)m, (int)n, (int)k);
            break;
    }
    return hipGetLastError();
}

template <int BITS, int BS>
static hipError_t gemv_dispatch_zp(const GemvGeom& g, const void* a, const uint8_t* b,
                                   const void* s, const uint8_t* z, void* y, int64_t m,
                                   int64_t n, int64_t k, hipStream_t stream) {
    if (z) return gemv_dispatch_mt<BITS, BS, true>(g, a, b, s, z, y, m, n, k, stream);
    return gemv_dispatch_mt<BITS, BS, false>(g, a, b, s, z, y, m, n, k, stream);
}

template <int BITS>
static hipError_t gemv_dispatch_bs(int bs, const GemvGeom& g, const void* a, const uint8_t* b,
                                   const void* s, const uint8_t* z, void* y, int64_t m,
                                   int64_t n, int64_t k, hipStream_t stream) {
    switch (bs) {
        case 16: return gemv_dispatch_zp<BITS, 16>(g, a, b, s, z, y, m, n, k, stream);
        case 32: return gemv_dispatch_zp<BITS, 32>(g, a, b, s, z, y, m, n, k, stream);
        case 64: return gemv_dispatch_zp<BITS, 64>(g, a, b, s, z, y, m, n, k, stream);
        case 128: return gemv_dispatch_zp<BITS, 128>(g, a, b, s, z, y, m, n, k, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_f16(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                           void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                           hipStream_t stream) {
    if (m == 0) return hipSuccess;
    const GemvGeom g = gemv_geometry(m, n, k, bits, bs);
    if (bits == 4) return gemv_dispatch_bs<4>(bs, g, a, b, s, z, y, m, n, k, stream);
    return gemv_dispatch_bs<8>(bs, g, a, b, s, z, y, m, n, k, stream);
}

template <typename T, int BITS, int BS>
static hipError_t generic_zp(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                             void* y, int64_t m, int64_t n, int64_t k, hipStream_t stream) {
    const dim3 grid((unsigned)((n + 3) / 4), (unsigned)((m + 3) / 4), 1);
    const dim3 block(256, 1, 1);
    const T* A = static_cast<const T*>(a);
    const T* S = static_cast<const T*>(s);
    T* Y = static_cast<T*>(y);
    if (z)
        hipLaunchKernelGGL((matmul_generic<T, BITS, BS, true>), grid, block, 0, stream, A, b, S,
                           z, Y, (int)m, (int)n, (int)k);
    else
        hipLaunchKernelGGL((matmul_generic<T, BITS, BS, false>), grid, block, 0, stream, A, b, S,
                           z, Y, (int)m, (int)n, (int)k);
    return hipGetLastError();
}

template <typename T, int BITS>
static hipError_t generic_bs(int bs, const void* a, const uint8_t* b, const void* s,
                             const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                             hipStream_t stream) {
    switch (bs) {
        case 16: return generic_zp<T, BITS, 16>(a, b, s, z, y, m, n, k, stream);
        case 32: return generic_zp<T, BITS, 32>(a, b, s, z, y, m, n, k, stream);
        case 64: return generic_zp<T, BITS, 64>(a, b, s, z, y, m, n, k, stream);
        case 128: return generic_zp<T, BITS, 128>(a, b, s, z, y, m, n, k, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_generic(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                          void* y, int64_t m, int64_t n, int64_t k, int bits, int bs, bool f16in,
                          hipStream_t stream) {
    if (m == 0) return hipSuccess;
    if (f16in) {
        if (bits == 4) return generic_bs<f16, 4>(bs, a, b, s, z, y, m, n, k, stream);
        return generic_bs<f16, 8>(bs, a, b, s, z, y, m, n, k, stream);
    }
    if (bits == 4) return generic_bs<float, 4>(bs, a, b, s, z, y, m, n, k, stream);
    return generic_bs<float, 8>(bs, a, b, s, z, y, m, n, k, stream);
}

template <int BITS, int BS>
static hipError_t dequant_zp(const uint8_t* b, const void* s, const uint8_t* z, void* w,
                             int64_t n, int64_t k, hipStream_t stream) {
    const int64_t words = n * k / (32 / BITS);
    const dim3 grid((unsigned)((words + 255) / 256), 1, 1);
    const f16* S = static_cast<const f16*>(s);
    f16* W = static_cast<f16*>(w);
    if (z)
        hipLaunchKernelGGL((dequant_f16<BITS, BS, true>), grid, dim3(256), 0, stream, b, S, z, W,
                           (int)n, (int)k);
    else
        hipLaunchKernelGGL((dequant_f16<BITS, BS, false>), grid, dim3(256), 0, stream, b, S, z,
                           W, (int)n, (int)k);
    return hipGetLastError();
}

template <int BITS>
static hipError_t dequant_bs(int bs, const uint8_t* b, const void* s, const uint8_t* z, void* w,
                             int64_t n, int64_t k, hipStream_t stream) {
    switch (bs) {
        case 16: return dequant_zp<BITS, 16>(b, s, z, w, n, k, stream);
        case 32: return dequant_zp<BITS, 32>(b, s, z, w, n, k, stream);
        case 64: return dequant_zp<BITS, 64>(b, s, z, w, n, k, stream);
        case 128: return dequant_zp<BITS, 128>(b, s, z, w, n, k, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dequant_f16(const uint8_t* b, const void* s, const uint8_t* z, void* w,
                              int64_t n, int64_t k, int bits, int bs, hipStream_t stream) {
    if (bits == 4) return dequant_bs<4>(bs, b, s, z, w, n, k, stream);
    return dequant_bs<8>(bs, b, s, z, w, n, k, stream);
}

}  // namespace mnb
