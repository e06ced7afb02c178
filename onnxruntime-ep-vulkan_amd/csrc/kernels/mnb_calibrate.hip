// Roofline calibration: the fp16 MFMA rate this device sustains on a given operand stream, and
// the shortest time one launch needs to read a given number of bytes from HBM.
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

// HBM read floor of one launch: the time a kernel needs just to read `n16` 16-byte units once,
// the lower bound for any kernel that streams that many bytes in one launch.  Every wavefront
// issues all of its L loads (16 bytes per lane, non-temporal, 1 KB per instruction) before it
// uses any result, so the whole launch's requests are in flight as early as the hardware takes
// them.  Wavefront w reads 1 KB runs w*L .. w*L+L-1 (CONTIG) or w, w+W, .. w+(L-1)*W (grid
// stride over the W wavefronts launched).  The XOR of the data is written only when it equals a
// constant no input produces in practice, which keeps the loads live without a store stream.
template <int L, bool CONTIG>
__global__ void __launch_bounds__(1024)
read_floor(const u32x4* __restrict__ src, int64_t n16, uint32_t* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    u32x4 v[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
        const int64_t run = CONTIG ? wave * L + j : wave + (int64_t)j * waves;
        const int64_t i = run * 64 + lane;
        v[j] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
    u32x4 acc = v[0];
#pragma unroll
    for (int j = 1; j < L; ++j) acc ^= v[j];
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) out[threadIdx.x] = 1u;
}

template <int L>
static hipError_t read_floor_go(const void* src, int64_t n16, int wpg, bool contig,
                                uint32_t* out, hipStream_t st) {
    const int64_t runs = (n16 + 63) / 64;
    const int64_t waves = (runs + L - 1) / L;
    const int64_t groups = (waves + wpg - 1) / wpg;
    if (groups > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)groups), block((unsigned)(64 * wpg));
    const u32x4* s = static_cast<const u32x4*>(src);
    if (contig)
        hipLaunchKernelGGL((read_floor<L, true>), grid, block, 0, st, s, n16, out);
    else
        hipLaunchKernelGGL((read_floor<L, false>), grid, block, 0, st, s, n16, out);
    return hipGetLastError();
}

hipError_t launch_read_floor(const void* src, int64_t n16, int loads_per_lane, int wpg,
                             bool contig, uint32_t* out, hipStream_t st) {
    // read_floor is compiled for at most 1024 threads per workgroup
    if (wpg < 1 || wpg > 16 || n16 <= 0) return hipErrorInvalidValue;
    switch (loads_per_lane) {
        case 1: return read_floor_go<1>(src, n16, wpg, contig, out, st);
        case 2: return read_floor_go<2>(src, n16, wpg, contig, out, st);
        case 4: return read_floor_go<4>(src, n16, wpg, contig, out, st);
        case 8: return read_floor_go<8>(src, n16, wpg, contig, out, st);
        case 16: return read_floor_go<16>(src, n16, wpg, contig, out, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mnb
