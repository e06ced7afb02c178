// Prefill MatMulNBits with fp32 activations, scales and output (M > 64 rows): an fp32 MFMA GEMM
// over weights dequantised into LDS.
//
// In fp32 the dequantised weight s * (q - zp) is exact (a 4- or 8-bit integer times an fp32 scale
// of 24 significant bits), so unlike the fp16 GEMM no per-block rescale is needed: each 32-k step
// turns the tile's packed weights into fp32 s * (q - zp) once per workgroup, and
// v_mfma_f32_32x32x2_f32 multiplies them with the fp32 activations into a partial per 32-k step
// that is then added to the tile's fp32 accumulator -- the reference's per-block fp32 partials
// summed over the blocks (rust/shaders/glsl/templates/q_gemv.comp:571-579), with the scale
// applied to each weight instead of to the partial.
//
// Work split.  One workgroup of 4 wavefronts owns a 128 x 128 tile of Y; the wavefronts form a
// 2 x 2 grid of 64 x 64 sub-tiles (four 32 x 32 MFMA tiles each).  K is walked in steps of 32,
// double-buffered in LDS: while step s is multiplied, step s + 1's activations (128 rows x 128
// bytes) and packed weights (128 columns x 16 or 32 bytes, with the step's block scale and zero
// point per column) are in flight in registers; they are stored -- the weights dequantised --
// into the other buffer after the step's MFMAs, and one barrier per step hands the buffers over.
// The fp32 matrix rate (16x below fp16) bounds the kernel: a step is 256 MFMA cycles per
// wavefront and tile against 2 loads and a few VALU per thread.
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kFBN = 128, kFKS = 32;
constexpr int kFAStride = kFKS + 4;                   // A rows in LDS: 36 floats (16-byte aligned)
constexpr int kFBStride = kFBN + 4;                   // B k-rows in LDS: 132 floats
constexpr int kFBFloats = kFKS * kFBStride;

// Tile rows BM (128, or 64 where 128-row tiles would leave CUs idle): the four wavefronts form a
// BM/64 x 4/(BM/64) grid of 64 x (128 / that) sub-tiles.
template <int BM>
struct F32Tile {
    static constexpr int kWM = BM / 64, kWN = 4 / kWM;
    static constexpr int kTN = kFBN / kWN / 32;       // 32-column MFMA tiles per wavefront: 2 or 1
    static constexpr int kAFloats = BM * kFAStride;
    static constexpr int kStage = kAFloats + kFBFloats;   // floats per buffer
    static constexpr size_t kLds = 2 * kStage * sizeof(float);   // 70,656 / 53,248 bytes
    static constexpr int kAV = BM / 32;               // 16-byte activation loads per thread and step
};

template <int BITS, bool HAS_ZP, int BM>
__global__ void __launch_bounds__(256)
gemm_f32_mfma(const float* __restrict__ A, const uint8_t* __restrict__ B,
              const float* __restrict__ S, const uint8_t* __restrict__ Z, float* __restrict__ Y,
              int M, int N, int K, int BS, int tiles_n) {
    using T = F32Tile<BM>;
    extern __shared__ __align__(16) float fsm[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / T::kWN, wn = wave % T::kWN;
    const int tile_m = (int)blockIdx.x / tiles_n;
    const int tile_n = (int)blockIdx.x - tile_m * tiles_n;
    const int m0 = tile_m * BM, n0 = tile_n * kFBN;
    const int steps = K / kFKS;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;

    // activations: thread t loads 4 kAV floats of row t / (256 / BM), part t % (256 / BM)
    constexpr int TPR = 256 / BM;                     // threads per activation row: 2 or 4
    const int a_row = tid / TPR, a_half = tid % TPR;
    const float* a_src = A + (int64_t)min(m0 + a_row, M - 1) * K + 4 * T::kAV * a_half;
    // weights: thread t dequantises 16 k (k quarter-pair t / 128) of column t % 128
    const int b_col = tid & 127, b_sub = tid >> 7;
    const int gcol = min(n0 + b_col, N - 1);
    constexpr int RAW = 16 * BITS / 8;                // packed bytes of 16 k: 8 or 16
    const uint8_t* b_src = B + (int64_t)gcol * ((int64_t)K * BITS / 8) + RAW * b_sub;

    f32x4 ra[T::kAV];
    uint32_t rb[RAW / 4];
    float rs = 0.f;
    int rz = 0;
    auto load = [&](int s) {
        const float* ap = a_src + (int64_t)s * kFKS;
#pragma unroll
        for (int i = 0; i < T::kAV; ++i) ra[i] = *reinterpret_cast<const f32x4*>(ap + 4 * i);
        const uint8_t* bp = b_src + (int64_t)s * (kFKS * BITS / 8);
        if constexpr (RAW == 8) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(bp);
            rb[0] = v.x;
            rb[1] = v.y;
        } else {
            const u32x4 v = *reinterpret_cast<const u32x4*>(bp);
            rb[0] = v.x;
            rb[1] = v.y;
            rb[2] = v.z;
            rb[3] = v.w;
        }
        const int blk = (s * kFKS + 16 * b_sub) / BS;
        rs = S[(int64_t)gcol * bpc + blk];
        if constexpr (HAS_ZP) {
            const uint32_t zb = Z[(int64_t)gcol * zpb + (BITS == 4 ? blk >> 1 : blk)];
            rz = BITS == 4 ? (int)((zb >> ((blk & 1) * 4)) & 0xFu) : (int)zb;
        } else {
            rz = 1 << (BITS - 1);
        }
    };
    auto store = [&](int buf) {
        float* sa = fsm + buf * T::kStage;
        float* sb = sa + T::kAFloats;
        float* arow = sa + a_row * kFAStride + 4 * T::kAV * a_half;
#pragma unroll
        for (int i = 0; i < T::kAV; ++i) *reinterpret_cast<f32x4*>(arow + 4 * i) = ra[i];
        // weight k = 16 b_sub + e of column b_col: int4 nibble e % 2 of byte e / 2, int8 byte e
        const float zf = (float)rz;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t q = BITS == 4 ? (rb[e >> 3] >> (4 * (e & 7))) & 0xFu
                                         : (rb[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            sb[(16 * b_sub + e) * kFBStride + b_col] = ((float)q - zf) * rs;
        }
    };

    constexpr int TN = T::kTN;
    f32x16 acc[2][TN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

    load(0);
    store(0);
    __syncthreads();
    // MFMA operands: lane l holds A[row l % 32][k l / 32] and B[k l / 32][column l % 32]
    const int orow = lane & 31, ok = lane >> 5;
    for (int s = 0; s < steps; ++s) {
        if (s + 1 < steps) load(s + 1);
        const float* sa = fsm + (s & 1) * T::kStage;
        const float* sb = sa + T::kAFloats;
        // the step's 32 k accumulate into fresh partial tiles, added to the accumulators once:
        // the reference's order (a 32-k partial, then a sum over the partials), which keeps the
        // fp32 rounding of one output well below that of a single 2-k-at-a-time chain over K
        f32x16 part[2][TN];
#pragma unroll
        for (int kk = 0; kk < kFKS / 2; ++kk) {
            const int k = 2 * kk + ok;
            float a[2], b[TN];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = sa[(64 * wm + 32 * i + orow) * kFAStride + k];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = sb[k * kFBStride + 32 * (TN * wn + j) + orow];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        a[i], b[j], kk == 0 ? f32x16{} : part[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
        if (s + 1 < steps) store((s + 1) & 1);
        __syncthreads();
    }

    // lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 of each 32 x 32 tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + 32 * (TN * wn + j) + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M) Y[(int64_t)row * N + col] = acc[i][j][r];
            }
        }
}

}  // namespace

// Tile rows: 128, or 64 where 128-row tiles number fewer than the 256 CUs (prefill at a few
// hundred rows: M = 256, N = 8192 has 128 of them).
int gemm_f32_tile_rows(int64_t m, int64_t n) {
    const int64_t tn = (n + kFBN - 1) / kFBN;
    return ((m + 127) / 128) * tn >= 256 ? 128 : 64;
}

bool gemm_f32_supported(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    if (bits != 4 && bits != 8) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    if (m < 1 || n < 1 || k < kFKS || k % kFKS || k % bs) return false;
    const int64_t tiles = ((m + 63) / 64) * ((n + kFBN - 1) / kFBN);
    return tiles <= 0x7fffffff && k < ((int64_t)1 << 31) / 4;
}

hipError_t launch_gemm_f32(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                           void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                           hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (!gemm_f32_supported(m, n, k, bits, bs)) return hipErrorInvalidValue;
    const int bm = gemm_f32_tile_rows(m, n);
    const int tiles_n = (int)((n + kFBN - 1) / kFBN);
    const int tiles = (int)((m + bm - 1) / bm) * tiles_n;
    const float* A = static_cast<const float*>(a);
    const float* S = static_cast<const float*>(s);
    float* Y = static_cast<float*>(y);
    auto go = [&](auto kern, size_t lds) {
        const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
        if (ea != hipSuccess) return ea;
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), lds, st, A, b, S, z, Y,
                           (int)m, (int)n, (int)k, bs, tiles_n);
        return hipGetLastError();
    };
    constexpr size_t L128 = F32Tile<128>::kLds, L64 = F32Tile<64>::kLds;
    if (bm == 128) {
        if (bits == 4) return z ? go(gemm_f32_mfma<4, true, 128>, L128) : go(gemm_f32_mfma<4, false, 128>, L128);
        return z ? go(gemm_f32_mfma<8, true, 128>, L128) : go(gemm_f32_mfma<8, false, 128>, L128);
    }
    if (bits == 4) return z ? go(gemm_f32_mfma<4, true, 64>, L64) : go(gemm_f32_mfma<4, false, 64>, L64);
    return z ? go(gemm_f32_mfma<8, true, 64>, L64) : go(gemm_f32_mfma<8, false, 64>, L64);
}

}  // namespace mnb
