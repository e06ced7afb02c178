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

constexpr int kFBM = 128, kFBN = 128, kFKS = 32;
constexpr int kFAStride = kFKS + 4;                   // A rows in LDS: 36 floats (16-byte aligned)
constexpr int kFBStride = kFBN + 4;                   // B k-rows in LDS: 132 floats
constexpr int kFAFloats = kFBM * kFAStride;
constexpr int kFBFloats = kFKS * kFBStride;
constexpr int kFStage = kFAFloats + kFBFloats;        // floats per buffer
constexpr size_t kFLds = 2 * kFStage * sizeof(float); // 70,656 bytes

template <int BITS, bool HAS_ZP>
__global__ void __launch_bounds__(256)
gemm_f32_mfma(const float* __restrict__ A, const uint8_t* __restrict__ B,
              const float* __restrict__ S, const uint8_t* __restrict__ Z, float* __restrict__ Y,
              int M, int N, int K, int BS, int tiles_n) {
    extern __shared__ __align__(16) float fsm[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int tile_m = (int)blockIdx.x / tiles_n;
    const int tile_n = (int)blockIdx.x - tile_m * tiles_n;
    const int m0 = tile_m * kFBM, n0 = tile_n * kFBN;
    const int steps = K / kFKS;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;

    // activations: thread t loads 16 floats (64 bytes) of row t / 2, k half t % 2 of the step
    const int a_row = tid >> 1, a_half = tid & 1;
    const float* a_src = A + (int64_t)min(m0 + a_row, M - 1) * K + 16 * a_half;
    // weights: thread t dequantises 16 k (k quarter-pair t / 128) of column t % 128
    const int b_col = tid & 127, b_sub = tid >> 7;
    const int gcol = min(n0 + b_col, N - 1);
    constexpr int RAW = 16 * BITS / 8;                // packed bytes of 16 k: 8 or 16
    const uint8_t* b_src = B + (int64_t)gcol * ((int64_t)K * BITS / 8) + RAW * b_sub;

    f32x4 ra[4];
    uint32_t rb[RAW / 4];
    float rs = 0.f;
    int rz = 0;
    auto load = [&](int s) {
        const float* ap = a_src + (int64_t)s * kFKS;
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = *reinterpret_cast<const f32x4*>(ap + 4 * i);
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
        float* sa = fsm + buf * kFStage;
        float* sb = sa + kFAFloats;
        float* arow = sa + a_row * kFAStride + 16 * a_half;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<f32x4*>(arow + 4 * i) = ra[i];
        // weight k = 16 b_sub + e of column b_col: int4 nibble e % 2 of byte e / 2, int8 byte e
        const float zf = (float)rz;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t q = BITS == 4 ? (rb[e >> 3] >> (4 * (e & 7))) & 0xFu
                                         : (rb[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            sb[(16 * b_sub + e) * kFBStride + b_col] = ((float)q - zf) * rs;
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    load(0);
    store(0);
    __syncthreads();
    // MFMA operands: lane l holds A[row l % 32][k l / 32] and B[k l / 32][column l % 32]
    const int orow = lane & 31, ok = lane >> 5;
    for (int s = 0; s < steps; ++s) {
        if (s + 1 < steps) load(s + 1);
        const float* sa = fsm + (s & 1) * kFStage;
        const float* sb = sa + kFAFloats;
        // the step's 32 k accumulate into fresh partial tiles, added to the accumulators once:
        // the reference's order (a 32-k partial, then a sum over the partials), which keeps the
        // fp32 rounding of one output well below that of a single 2-k-at-a-time chain over K
        f32x16 part[2][2];
#pragma unroll
        for (int kk = 0; kk < kFKS / 2; ++kk) {
            const int k = 2 * kk + ok;
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = sa[(64 * wm + 32 * i + orow) * kFAStride + k];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = sb[k * kFBStride + 64 * wn + 32 * j + orow];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        a[i], b[j], kk == 0 ? f32x16{} : part[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] += part[i][j];
        if (s + 1 < steps) store((s + 1) & 1);
        __syncthreads();
    }

    // lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 of each 32 x 32 tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + 64 * wn + 32 * j + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M) Y[(int64_t)row * N + col] = acc[i][j][r];
            }
        }
}

}  // namespace

bool gemm_f32_supported(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    if (bits != 4 && bits != 8) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    if (m < 1 || n < 1 || k < kFKS || k % kFKS || k % bs) return false;
    const int64_t tiles = ((m + kFBM - 1) / kFBM) * ((n + kFBN - 1) / kFBN);
    return tiles <= 0x7fffffff && k < ((int64_t)1 << 31) / 4;
}

size_t gemm_f32_lds() { return kFLds; }

hipError_t launch_gemm_f32(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                           void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                           hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (!gemm_f32_supported(m, n, k, bits, bs)) return hipErrorInvalidValue;
    const int tiles_n = (int)((n + kFBN - 1) / kFBN);
    const int tiles = (int)((m + kFBM - 1) / kFBM) * tiles_n;
    const float* A = static_cast<const float*>(a);
    const float* S = static_cast<const float*>(s);
    float* Y = static_cast<float*>(y);
    auto go = [&](auto kern) {
        const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), kFLds);
        if (ea != hipSuccess) return ea;
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), kFLds, st, A, b, S, z, Y,
                           (int)m, (int)n, (int)k, bs, tiles_n);
        return hipGetLastError();
    };
    if (bits == 4) return z ? go(gemm_f32_mfma<4, true>) : go(gemm_f32_mfma<4, false>);
    return z ? go(gemm_f32_mfma<8, true>) : go(gemm_f32_mfma<8, false>);
}

}  // namespace mnb
