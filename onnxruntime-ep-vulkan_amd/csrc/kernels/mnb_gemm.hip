// Prefill MatMulNBits on gfx950: dequantise-into-LDS fp16 MFMA GEMM (fp16 A, block_size >= 32).
//
// Work split.  A workgroup of 4 wavefronts owns a BM x BN tile of Y; the wavefronts form a 2 x 2
// grid, each owning a (BM/2) x (BN/2) sub-tile made of 32 x 32 MFMA tiles.  K is walked in steps
// of 32 (one quant block for block_size 32; a part of one for 64 and 128).
//
// Per step: every thread of the workgroup stages its share of the next step in registers while
// the current one is multiplied -- A as 16-byte pieces, and for B one 16-byte run of packed int4
// (one column's 32 weights) plus that column's scale and zero point.  The B run is turned into
// exact (q - zp) fp16 values with the magic-number unpack (mnb_common.hpp) and written to LDS
// already in the v_mfma_f32_32x32x16_f16 operand order, so every operand fetch is one
// conflict-free ds_read_b128 over 64 consecutive 16-byte slots.  Two LDS stages alternate.
//
// Arithmetic.  Each 32 x 32 tile's step partial is two MFMAs over the exact (q - zp) operands
// (fp32 accumulate), i.e. the per-block fp32 partial of the reference kernel
// (rust/shaders/glsl/templates/q_gemv.comp:571-579), then added to the tile's accumulator scaled
// by the block's fp32 scale.  With the 32 x 32 output layout every lane's 16 values share one
// column, so one scale per lane per tile is applied.
#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kStepK = 32;           // K per step: two 32x32x16 MFMAs

// Bytes of one LDS operand slot set: 64 lanes x 16 bytes.
constexpr int kSlot = 64 * 16;

}  // namespace

// LDS layout (per stage):
//   sA: [BM/32 m-tiles][2 k-halves][64 lanes] x 16 B   lane l: row l%32, k 8*(l/32) .. +8
//   sB: [BN/32 n-tiles][2 k-halves][64 lanes] x 16 B   lane l: col l%32, k 8*(l/32) .. +8
//   sS: [BN] fp32 scales of the step's block
template <int BM, int BN, int BITS, int BS, bool HAS_ZP>
__global__ void __launch_bounds__(256)
gemm_f16_mfma(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
              const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K,
              int tiles_n) {
    static_assert(BITS == 4, "the GEMM path is written for 4-bit weights");
    static_assert(BN == 256 || BN == 128, "BN");
    static_assert(BM == 128 || BM == 64, "BM");
    constexpr int MT = BM / 64;                     // 32-row tiles per wave (wave rows = BM/2)
    constexpr int NT = BN / 64;                     // 32-col tiles per wave (wave cols = BN/2)
    constexpr int A_SLOTS = BM / 32 * 2;            // 16-byte slot sets of A per stage
    constexpr int B_SLOTS = BN / 32 * 2;
    constexpr int A_PIECES = BM * kStepK / 8;       // 16-byte pieces of A per step
    constexpr int A_PER_THREAD = A_PIECES / 256;    // 2 (BM=128) or 1 (BM=64)
    constexpr int B_COLS_PER_THREAD = BN / 256 > 0 ? BN / 256 : 1;

    __shared__ __attribute__((aligned(16))) uint8_t sA[2][A_SLOTS * kSlot];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][B_SLOTS * kSlot];
    __shared__ float sS[2][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;                        // wave row in the 2x2 grid
    const int wn = wave & 1;
    const int tile_m = blockIdx.x / tiles_n;
    const int tile_n = blockIdx.x - tile_m * tiles_n;
    const int m0 = tile_m * BM;
    const int n0 = tile_n * BN;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const int64_t col_bytes = (int64_t)K * BITS / 8;
    const int steps = K / kStepK;

    // ---- global -> register staging -------------------------------------------------------
    u32x4 ra[A_PER_THREAD];
    u32x4 rb[B_COLS_PER_THREAD];
    uint16_t rs[B_COLS_PER_THREAD];
    uint32_t rz[B_COLS_PER_THREAD];
    // B threads: BN == 256 -> every thread loads one column; BN == 128 -> threads 0..127.
    const bool b_loader = tid < BN;

    auto fetch = [&](int step) {
        const int k0 = step * kStepK;
#pragma unroll
        for (int i = 0; i < A_PER_THREAD; ++i) {
            const int piece = tid + 256 * i;
            const int row = piece >> 2;              // 4 pieces of 8 halves per row
            const int kc = piece & 3;
            int gm = m0 + row;
            gm = gm < M ? gm : M - 1;                // clamped rows are never stored
            ra[i] = *reinterpret_cast<const u32x4*>(A + (int64_t)gm * K + k0 + 8 * kc);
        }
        if (b_loader) {
#pragma unroll
            for (int c = 0; c < B_COLS_PER_THREAD; ++c) {
                int col = n0 + tid + 256 * c;
                col = col < N ? col : N - 1;
                rb[c] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(B + (int64_t)col * col_bytes + k0 / 2));
                const int blk = k0 / BS;
                rs[c] = reinterpret_cast<const uint16_t*>(S)[(int64_t)col * bpc + blk];
                if constexpr (HAS_ZP) rz[c] = Z[(int64_t)col * zpb + (blk >> 1)];
                else rz[c] = 0u;
            }
        }
    };

    auto stash = [&](int stage, int step) {
#pragma unroll
        for (int i = 0; i < A_PER_THREAD; ++i) {
            const int piece = tid + 256 * i;
            const int row = piece >> 2;
            const int kc = piece & 3;
            const int slot = ((row >> 5) * 2 + (kc >> 1)) * 64 + (row & 31) + 32 * (kc & 1);
            *reinterpret_cast<u32x4*>(&sA[stage][slot * 16]) = ra[i];
        }
        if (b_loader) {
            const int blk = step * kStepK / BS;
#pragma unroll
            for (int c = 0; c < B_COLS_PER_THREAD; ++c) {
                const int colw = tid + 256 * c;      // column within the tile
                int z = 1 << (BITS - 1);
                if constexpr (HAS_ZP) z = (int)((rz[c] >> ((blk & 1) * 4)) & 0xFu);
                const f16x2 zo = zoff4(z);
                const uint32_t w[4] = {rb[c].x, rb[c].y, rb[c].z, rb[c].w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    // dword d = k 8d .. 8d+7 -> k-half d/2, lane half d%2
                    f16x8 v;
                    v.s01 = nib_pair<0>(w[d], zo);
                    v.s23 = nib_pair<1>(w[d], zo);
                    v.s45 = nib_pair<2>(w[d], zo);
                    v.s67 = nib_pair<3>(w[d], zo);
                    const int slot = ((colw >> 5) * 2 + (d >> 1)) * 64 + (colw & 31) + 32 * (d & 1);
                    *reinterpret_cast<f16x8*>(&sB[stage][slot * 16]) = v;
                }
                sS[stage][colw] = (float)__builtin_bit_cast(f16, rs[c]);
            }
        }
    };

    f32x16 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    fetch(0);
    stash(0, 0);
    __syncthreads();

    for (int step = 0; step < steps; ++step) {
        const int stage = step & 1;
        const bool more = step + 1 < steps;
        if (more) fetch(step + 1);

        // Operands of this wave for both k-halves.
        f16x8 a[MT][2], b[NT][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int slot = ((wm * MT + i) * 2 + h) * 64 + lane;
                a[i][h] = *reinterpret_cast<const f16x8*>(&sA[stage][slot * 16]);
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int slot = ((wn * NT + j) * 2 + h) * 64 + lane;
                b[j][h] = *reinterpret_cast<const f16x8*>(&sB[stage][slot * 16]);
            }
        }
        float sc[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) sc[j] = sS[stage][(wn * NT + j) * 32 + (lane & 31)];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                f32x16 d = {};
                d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][0], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][1], b[j][1], d, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(d[r], sc[j], acc[i][j][r]);
            }
        }
        if (more) stash(stage ^ 1, step + 1);
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
    return m > 0 && bits == 4 && bs >= 32 && k > 0 && k % kStepK == 0 && k % bs == 0;
}

GemmConfig gemm_config(int64_t m, int64_t n) {
    GemmConfig c{};
    // Fill the 256 CUs: the widest tile that still yields about one workgroup per CU.
    const int64_t big = ((m + 127) / 128) * ((n + 255) / 256);
    const int64_t mid = ((m + 127) / 128) * ((n + 127) / 128);
    if (big >= 256) {
        c.bm = 128;
        c.bn = 256;
    } else if (mid >= 256) {
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
    const dim3 grid((unsigned)(c.tiles_m * c.tiles_n), 1, 1);
    hipLaunchKernelGGL((gemm_f16_mfma<BM, BN, 4, BS, HAS_ZP>), grid, dim3(256), 0, st,
                       static_cast<const f16*>(a), b, static_cast<const f16*>(s), z,
                       static_cast<f16*>(y), (int)m, (int)n, (int)k, (int)c.tiles_n);
    return hipGetLastError();
}

template <int BS, bool HAS_ZP>
static hipError_t gemm_tile(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                            const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    if (c.bm == 128 && c.bn == 256) return gemm_go<128, 256, BS, HAS_ZP>(c, a, b, s, z, y, m, n, k, st);
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
