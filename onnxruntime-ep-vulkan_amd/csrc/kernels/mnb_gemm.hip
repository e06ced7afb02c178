// Prefill MatMulNBits on gfx950: dequantise-into-LDS fp16 MFMA GEMM (fp16 A, int4, block >= 32).
//
// Work split.  A workgroup of 4 wavefronts owns a BM x BN tile of Y; the wavefronts form a 2 x 2
// grid, each owning a (BM/2) x (BN/2) sub-tile made of 32 x 32 MFMA tiles.  K is walked in steps
// of KS = 64 (two quant blocks of 32, or part of one block of 64/128).
//
// Pipeline.  Global loads run two steps ahead of the MFMAs: step s+2 is requested into one of two
// register sets while step s is multiplied out of LDS, and step s+1 (requested a full step
// earlier) is written to the other LDS stage after it.  The B run of a column (16 bytes = 32
// int4 weights = one quant block of 32) is turned into exact (q - zp) fp16 values with the
// magic-number unpack (mnb_common.hpp) on its way to LDS, which stores A and B already in the
// v_mfma_f32_32x32x16_f16 operand order: every operand fetch is one conflict-free ds_read_b128
// of 64 consecutive 16-byte slots.
//
// Arithmetic.  Each 32 x 32 tile's partial over one quant block (32 k) is two MFMAs over the exact
// (q - zp) operands with fp32 accumulation -- the reference kernel's per-block fp32 partial
// (rust/shaders/glsl/templates/q_gemv.comp:571-579) -- added to the tile's accumulator scaled by
// the block's fp32 scale.  In the 32 x 32 output layout a lane's 16 values share one column, so
// one scale per lane per tile per block is applied.
#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kKS = 64;              // K per pipeline step
constexpr int kSub = 32;             // K per scaled partial (one block of 32)
constexpr int kSlot = 64 * 16;       // one operand slot set: 64 lanes x 16 bytes

template <int BM, int BN>
constexpr size_t gemm_lds_bytes() {
    // per stage: A + B operand slots for KS, plus fp32 scales of the step's sub-blocks
    return 2 * ((size_t)(BM / 32) * (kKS / 16) * kSlot + (size_t)(BN / 32) * (kKS / 16) * kSlot +
                (size_t)(kKS / kSub) * BN * 4);
}

}  // namespace

// Register staging of one step's B run for one thread (A is staged separately, one step ahead).
struct GemmStageB {
    u32x4 b;            // one column's 32 int4 weights (one sub-block)
    uint32_t s;         // the sub-block's fp16 scale bits
    uint32_t z;         // the packed zero-point byte holding the block's nibble
};

// LDS layout (per stage), operand slot sets of 64 lanes x 16 B:
//   A: [BM/32 m-tiles][KS/16 k-slices][64]  lane l: row l%32, k 16*slice + 8*(l/32) .. +8
//   B: [BN/32 n-tiles][KS/16 k-slices][64]  lane l: col l%32, same k
//   S: [KS/32 sub-blocks][BN] fp32
template <int BM, int BN, int BS, bool HAS_ZP>
__global__ void __launch_bounds__(256, 2)
gemm_f16_mfma(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
              const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K,
              int tiles_n) {
    static_assert(BN == 128 || BN == 256, "BN");
    static_assert(BM == 64 || BM == 128, "BM");
    static_assert(BS >= kSub, "block size below the sub-block");
    constexpr int MT = BM / 64;                      // 32-row tiles per wave
    constexpr int NT = BN / 64;                      // 32-col tiles per wave
    constexpr int SL = kKS / 16;                     // k-slices per step
    constexpr int A_BYTES = (BM / 32) * SL * kSlot;
    constexpr int B_BYTES = (BN / 32) * SL * kSlot;
    constexpr int STAGE = A_BYTES + B_BYTES + (kKS / kSub) * BN * 4;
    constexpr int A_PIECES = BM * kKS / 8;           // 16-byte pieces of A per step
    constexpr int A_PT = A_PIECES / 256;
    constexpr int SUBS = kKS / kSub;                 // sub-blocks per step
    static_assert(BN * SUBS <= 256 * 2, "B staging covers at most two runs per thread");
    static_assert(BN * SUBS == 256, "one B run per thread");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int tile_m = blockIdx.x / tiles_n;
    const int tile_n = blockIdx.x - tile_m * tiles_n;
    const int m0 = tile_m * BM;
    const int n0 = tile_n * BN;
    const int bpc = K / BS;
    const int zpb = (bpc * 4 + 7) / 8;
    const int64_t col_bytes = (int64_t)K / 2;
    const int steps = K / kKS;
    // B staging: thread -> (column of the tile, sub-block of the step)
    const int b_col = tid % BN;
    const int b_sub = tid / BN;
    int b_gcol = n0 + b_col;
    b_gcol = b_gcol < N ? b_gcol : N - 1;            // clamped columns are never stored
    const uint8_t* __restrict__ b_src = B + (int64_t)b_gcol * col_bytes;
    const uint16_t* __restrict__ s_src = reinterpret_cast<const uint16_t*>(S) + (int64_t)b_gcol * bpc;
    const uint8_t* __restrict__ z_src = HAS_ZP ? Z + (int64_t)b_gcol * zpb : nullptr;

    // A piece p (16 bytes = 8 k of one row) -> (row, k chunk).  Sixteen consecutive threads take
    // sixteen consecutive rows of one k chunk, so their LDS slots are 256 contiguous bytes (no
    // bank conflict on the ds_write_b128) while a wavefront still reads 64-byte runs of 16 rows.
    auto a_piece = [](int p, int& row, int& kc) {
        row = (p & 15) + 16 * (p / (16 * (kKS / 8)));
        kc = (p >> 4) & (kKS / 8 - 1);
    };

    auto fetch_a = [&](u32x4 (&ra)[A_PT], int step) {
        const int k0 = step * kKS;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            int row, kc;
            a_piece(tid + 256 * i, row, kc);
            int gm = m0 + row;
            gm = gm < M ? gm : M - 1;                // clamped rows are never stored
            ra[i] = *reinterpret_cast<const u32x4*>(A + (int64_t)gm * K + k0 + 8 * kc);
        }
    };

    auto fetch_b = [&](GemmStageB& r, int step) {
        const int kb = step * kKS + kSub * b_sub;    // first k of this thread's B run
        r.b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(b_src + kb / 2));
        const int blk = kb / BS;
        r.s = s_src[blk];
        if constexpr (HAS_ZP) r.z = z_src[blk >> 1];
        else r.z = 0u;
    };

    auto stash_a = [&](const u32x4 (&ra)[A_PT], int stage) {
        uint8_t* st = smem + stage * STAGE;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            int row, kc;                            // 8-wide k chunk: slice kc/2, lane half kc%2
            a_piece(tid + 256 * i, row, kc);
            const int slot = ((row >> 5) * SL + (kc >> 1)) * 64 + (row & 31) + 32 * (kc & 1);
            *reinterpret_cast<u32x4*>(st + slot * 16) = ra[i];
        }
    };

    auto stash_b = [&](const GemmStageB& r, int stage, int step) {
        uint8_t* st = smem + stage * STAGE;
        const int kb = step * kKS + kSub * b_sub;
        const int blk = kb / BS;
        int z = 8;
        if constexpr (HAS_ZP) z = (int)((r.z >> ((blk & 1) * 4)) & 0xFu);
        const f16x2 zo = zoff4(z);
        const uint32_t w[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        uint8_t* sb = st + A_BYTES;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // dword d = k 8d .. 8d+7 of the run: slice 2*b_sub + d/2, lane half d%2
            f16x8 v;
            v.s01 = nib_pair<0>(w[d], zo);
            v.s23 = nib_pair<1>(w[d], zo);
            v.s45 = nib_pair<2>(w[d], zo);
            v.s67 = nib_pair<3>(w[d], zo);
            const int slice = 2 * b_sub + (d >> 1);
            const int slot = ((b_col >> 5) * SL + slice) * 64 + (b_col & 31) + 32 * (d & 1);
            *reinterpret_cast<f16x8*>(sb + slot * 16) = v;
        }
        float* ss = reinterpret_cast<float*>(st + A_BYTES + B_BYTES);
        ss[b_sub * BN + b_col] = (float)__builtin_bit_cast(f16, (uint16_t)r.s);
    };

    f32x16 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto compute = [&](int stage) {
        const uint8_t* st = smem + stage * STAGE;
        const float* ss = reinterpret_cast<const float*>(st + A_BYTES + B_BYTES);
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
            f16x8 a[MT][2], b[NT][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int slice = 2 * sub + h;
#pragma unroll
                for (int i = 0; i < MT; ++i)
                    a[i][h] = *reinterpret_cast<const f16x8*>(
                        st + (((wm * MT + i) * SL + slice) * 64 + lane) * 16);
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    b[j][h] = *reinterpret_cast<const f16x8*>(
                        st + A_BYTES + (((wn * NT + j) * SL + slice) * 64 + lane) * 16);
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const float sc = ss[sub * BN + (wn * NT + j) * 32 + (lane & 31)];
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    f32x16 d = {};
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][0], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][1], b[j][1], d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(d[r], sc, acc[i][j][r]);
                }
                if constexpr (MT * NT > 2) __builtin_amdgcn_sched_barrier(0);
            }
            // Keep the scheduler from hoisting the next sub-block's MFMAs above this one's
            // epilogue: that would hold twice the partial tiles live and spill.
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // A is requested one step ahead (it is read by many workgroups and mostly hits in L2); B,
    // streamed from HBM, two steps ahead in two register sets.
    u32x4 ra[A_PT];
    GemmStageB r0, r1;
    fetch_a(ra, 0);
    fetch_b(r0, 0);
    if (steps > 1) fetch_b(r1, 1);
    stash_a(ra, 0);
    stash_b(r0, 0, 0);
    __syncthreads();

    // Two steps per trip so that the register sets are named at compile time.
    for (int s = 0; s < steps; s += 2) {
        // step s: stage 0 holds it, r1 holds B of step s+1, r0 is free
        if (s + 1 < steps) fetch_a(ra, s + 1);
        if (s + 2 < steps) fetch_b(r0, s + 2);
        compute(0);
        if (s + 1 < steps) {
            stash_a(ra, 1);
            stash_b(r1, 1, s + 1);
        }
        __syncthreads();
        if (s + 1 >= steps) break;
        // step s+1: stage 1 holds it, r0 holds B of step s+2, r1 is free
        if (s + 2 < steps) fetch_a(ra, s + 2);
        if (s + 3 < steps) fetch_b(r1, s + 3);
        compute(1);
        if (s + 2 < steps) {
            stash_a(ra, 0);
            stash_b(r0, 0, s + 2);
        }
        __syncthreads();
    }

    // ---- store: lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4 of each tile ----
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int col = n0 + (wn * NT + j) * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + (wm * MT + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M) Y[(int64_t)row * N + col] = (f16)acc[i][j][r];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

bool gemm_supported(int64_t m, int64_t k, int bits, int bs) {
    return m > 0 && bits == 4 && bs >= kSub && k > 0 && k % kKS == 0 && k % bs == 0;
}

GemmConfig gemm_config(int64_t m, int64_t n) {
    GemmConfig c{};
    // 128 x 128 while that still yields two workgroups per CU; otherwise 64-row tiles.
    const int64_t mid = ((m + 127) / 128) * ((n + 127) / 128);
    if (mid >= 512) {
        c.bm = 128;
        c.bn = 128;
    } else {
        c.bm = 64;
        c.bn = 128;
    }
    c.tiles_m = (m + c.bm - 1) / c.bm;
    c.tiles_n = (n + c.bn - 1) / c.bn;
    return c;
}

template <int BM, int BN, int BS, bool HAS_ZP>
static hipError_t gemm_go(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                          const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                          hipStream_t st) {
    constexpr size_t lds = gemm_lds_bytes<BM, BN>();
    auto kern = gemm_f16_mfma<BM, BN, BS, HAS_ZP>;
    // More than 64 KB of dynamic LDS must be allowed explicitly (for the current device).
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)(c.tiles_m * c.tiles_n), 1, 1);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, static_cast<const f16*>(a), b,
                       static_cast<const f16*>(s), z, static_cast<f16*>(y), (int)m, (int)n,
                       (int)k, (int)c.tiles_n);
    return hipGetLastError();
}

template <int BS, bool HAS_ZP>
static hipError_t gemm_tile(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                            const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    if (c.bm == 128 && c.bn == 128) return gemm_go<128, 128, BS, HAS_ZP>(c, a, b, s, z, y, m, n, k, st);
    if (c.bm == 64 && c.bn == 128) return gemm_go<64, 128, BS, HAS_ZP>(c, a, b, s, z, y, m, n, k, st);
    return hipErrorInvalidValue;
}

template <int BS>
static hipError_t gemm_zp(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                          const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                          hipStream_t st) {
    if (z) return gemm_tile<BS, true>(c, a, b, s, z, y, m, n, k, st);
    return gemm_tile<BS, false>(c, a, b, s, z, y, m, n, k, st);
}

hipError_t launch_gemm_cfg(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                           const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bits,
                           int bs, hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (!gemm_supported(m, k, bits, bs)) return hipErrorInvalidValue;
    switch (bs) {
        case 32: return gemm_zp<32>(c, a, b, s, z, y, m, n, k, st);
        case 64: return gemm_zp<64>(c, a, b, s, z, y, m, n, k, st);
        case 128: return gemm_zp<128>(c, a, b, s, z, y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const void* a, const uint8_t* b, const void* s, const uint8_t* z, void* y,
                       int64_t m, int64_t n, int64_t k, int bits, int bs, hipStream_t st) {
    return launch_gemm_cfg(gemm_config(m, n), a, b, s, z, y, m, n, k, bits, bs, st);
}

}  // namespace mnb
