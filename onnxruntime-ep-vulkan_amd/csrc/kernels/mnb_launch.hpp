// Host-side launchers for the MatMulNBits kernels (internal to libmnb_hip.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnb {

// Geometry shared by the planner (host) and the launchers.
struct GemvGeom {
    int mt;        // 16-row M tiles per workgroup (1, 2 or 4)
    int waves;     // wavefronts per workgroup
    int64_t gx;    // ceil(N / 16)
    int64_t gy;    // ceil(M / (16 * mt))
    size_t lds;    // dynamic LDS bytes
};

GemvGeom gemv_geometry(int64_t m, int64_t n, int64_t k, int bits, int bs);
bool gemv_supported(int64_t k, int bits, int block_size);

hipError_t launch_gemv_f16(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                           void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                           hipStream_t stream);

hipError_t launch_generic(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                          void* y, int64_t m, int64_t n, int64_t k, int bits, int bs, bool f16,
                          hipStream_t stream);

hipError_t launch_dequant_f16(const uint8_t* b, const void* s, const uint8_t* z, void* w,
                              int64_t n, int64_t k, int bits, int bs, hipStream_t stream);

}  // namespace mnb
