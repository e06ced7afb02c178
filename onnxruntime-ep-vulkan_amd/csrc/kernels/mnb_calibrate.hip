// Roofline calibration: the fp16 MFMA rate this device sustains on a given operand stream.
//
// The nominal dense fp16 peak assumes the top engine clock.  Under a full-chip MFMA load the
// clock is set by the power the matrix cores draw, which depends on how many operand bits toggle:
// the same instruction stream runs markedly slower on random fp16 data than on constant data.
// This kernel measures that ceiling directly so that a GEMM's achieved rate can be read against
// what the chip can do on data of the same kind.  No counterpart in the reference (which has no
// MFMA path); it is a measurement utility used by bench.py.
//
// Each wavefront keeps sixteen independent 32 x 32 accumulators (in AGPRs: this file is built
// without the VGPR MFMA form) and cycles through four A and four B operands loaded once from
// `operands` (or constants when it is null).  One launch performs
// workgroups * 4 * iters * 16 v_mfma_f32_32x32x16_f16.
#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256)
mfma_calibrate(const f16x8* __restrict__ operands, float* __restrict__ out, int iters) {
    const int gid = blockIdx.x * 256 + threadIdx.x;
    f16x8 a[4], b[4];
    if (operands) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = operands[(int64_t)gid * 8 + i];
            b[i] = operands[(int64_t)gid * 8 + 4 + i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a[i][e] = (f16)1.0f;
                b[i][e] = (f16)0.0f;
            }
    }
    f32x16 c[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) c[t] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 16; ++t)
            c[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[t & 3], b[t >> 2], c[t], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += c[t][r];
    out[gid] = s;                                    // keeps the MFMAs live
}

hipError_t launch_mfma_calibrate(const void* operands, float* out, int workgroups, int iters,
                                 hipStream_t st) {
    hipLaunchKernelGGL(mfma_calibrate, dim3((unsigned)workgroups), dim3(256), 0, st,
                       static_cast<const f16x8*>(operands), out, iters);
    return hipGetLastError();
}

}  // namespace mnb
