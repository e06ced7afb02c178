// RMSNorm with the residual add fused (com.microsoft::SkipSimplifiedLayerNormalization) and
// without it (SimplifiedLayerNormalization), fp16 or fp32, over the last axis.
//
// Semantics follow the reference kernel (rust/shaders/glsl/skip_simplified_layer_norm_f16.comp,
// bound by rust/src/ops/common/templates.rs:426-528): r = x + skip (+ bias) in fp32 from the
// stored values; out3 = r stored in the tensor type (the residual sum, output slot 3);
// inv = 1 / sqrt(sum(r^2) / H + epsilon); out0 = r * inv * gamma, stored in the tensor type.
//
// One wavefront per row: lane l holds the 16-byte chunks l, l + 64, ... of the row in registers
// (NJ chunks), so the row is read once; the sum of squares is a wave-wide shuffle reduction with
// no LDS and no barrier.  Four rows per workgroup.
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

template <typename T>
struct Chunk;
template <>
struct Chunk<f16> {
    static constexpr int kN = 8;
    typedef f16x8 V;
};
template <>
struct Chunk<float> {
    static constexpr int kN = 4;
    typedef f32x4 V;
};

}  // namespace

template <typename T, int NJ>
__global__ void __launch_bounds__(256)
skip_rmsnorm(const T* __restrict__ x, const T* __restrict__ skip, const T* __restrict__ gamma,
             const T* __restrict__ bias, T* __restrict__ y, T* __restrict__ sum_out,
             int64_t rows, int hidden, float eps) {
    using V = typename Chunk<T>::V;
    constexpr int CN = Chunk<T>::kN;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;                             // whole wavefront
    const int chunks = hidden / CN;
    const T* xr = x + row * hidden;
    const T* sr = skip ? skip + row * hidden : nullptr;
    float r[NJ][CN];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
            const V xv = *reinterpret_cast<const V*>(xr + (int64_t)c * CN);
            V sv = {}, bv = {};
            if (sr) sv = *reinterpret_cast<const V*>(sr + (int64_t)c * CN);
            if (bias) bv = *reinterpret_cast<const V*>(bias + (int64_t)c * CN);
#pragma unroll
            for (int e = 0; e < CN; ++e) {
                r[j][e] = (float)xv[e] + (float)sv[e] + (float)bv[e];
                ss = __builtin_fmaf(r[j][e], r[j][e], ss);
            }
        } else {
#pragma unroll
            for (int e = 0; e < CN; ++e) r[j][e] = 0.f;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float inv = 1.f / sqrtf(ss / (float)hidden + eps);
    T* yr = y + row * hidden;
    T* qr = sum_out ? sum_out + row * hidden : nullptr;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = lane + 64 * j;
        if (c >= chunks) continue;
        const V g = *reinterpret_cast<const V*>(gamma + (int64_t)c * CN);
        V o, q;
#pragma unroll
        for (int e = 0; e < CN; ++e) {
            o[e] = (T)(r[j][e] * inv * (float)g[e]);
            q[e] = (T)r[j][e];
        }
        *reinterpret_cast<V*>(yr + (int64_t)c * CN) = o;
        if (qr) *reinterpret_cast<V*>(qr + (int64_t)c * CN) = q;
    }
}

bool rmsnorm_supported(int64_t hidden, bool is_f16) {
    const int cn = is_f16 ? 8 : 4;
    return hidden > 0 && hidden % cn == 0 && hidden / cn <= 64 * 16;
}

template <typename T>
static hipError_t rms_go(const void* x, const void* skip, const void* gamma, const void* bias,
                         void* y, void* sum_out, int64_t rows, int64_t hidden, float eps,
                         hipStream_t st) {
    const int chunks = (int)(hidden / Chunk<T>::kN);
    const int nj = (chunks + 63) / 64;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const T* xs = static_cast<const T*>(x);
    const T* ks = static_cast<const T*>(skip);
    const T* gs = static_cast<const T*>(gamma);
    const T* bs = static_cast<const T*>(bias);
    T* ys = static_cast<T*>(y);
    T* qs = static_cast<T*>(sum_out);
#define MNB_RMS(NJ_)                                                                              \
    hipLaunchKernelGGL((skip_rmsnorm<T, NJ_>), grid, dim3(256), 0, st, xs, ks, gs, bs, ys, qs,  \
                       rows, (int)hidden, eps)
    if (nj <= 1) MNB_RMS(1);
    else if (nj <= 2) MNB_RMS(2);
    else if (nj <= 4) MNB_RMS(4);
    else if (nj <= 8) MNB_RMS(8);
    else MNB_RMS(16);
#undef MNB_RMS
    return hipGetLastError();
}

hipError_t launch_skip_rmsnorm(const void* x, const void* skip, const void* gamma,
                               const void* bias, void* y, void* sum_out, int64_t rows,
                               int64_t hidden, float eps, bool is_f16, hipStream_t st) {
    if (!rmsnorm_supported(hidden, is_f16)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    return is_f16 ? rms_go<f16>(x, skip, gamma, bias, y, sum_out, rows, hidden, eps, st)
                  : rms_go<float>(x, skip, gamma, bias, y, sum_out, rows, hidden, eps, st);
}

}  // namespace mnb
