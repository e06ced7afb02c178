// Host-tensor staging of a session call: byte copies between the session's pinned host buffer
// (mapped into the device's address space) and device memory, several segments in one launch.
//
// A small transfer through the runtime's copy engine costs a DMA submission and completion of
// its own per tensor (5-7 us each above about 16 KB, measured on MI355X); a kernel whose lanes
// read or write the pinned buffer over PCIe costs one launch in the stream for all of a call's
// inputs and one for all of its outputs.  Each segment is one row of the grid (blockIdx.y);
// 16-byte loads and stores where both ends are 16-byte aligned, bytes otherwise, and the tail
// of a 16-byte body in bytes.
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

__global__ void __launch_bounds__(256) stage_copy(StageList l) {
    const StageSeg sg = l.seg[blockIdx.y];
    const uint8_t* __restrict__ src = static_cast<const uint8_t*>(sg.src);
    uint8_t* __restrict__ dst = static_cast<uint8_t*>(sg.dst);
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t body = 0;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
        const uint64_t n16 = sg.bytes >> 4;
        const uint4* s16 = reinterpret_cast<const uint4*>(src);
        uint4* d16 = reinterpret_cast<uint4*>(dst);
        for (uint64_t i = tid; i < n16; i += stride) d16[i] = s16[i];
        body = n16 << 4;
    }
    for (uint64_t i = body + tid; i < sg.bytes; i += stride) dst[i] = src[i];
}

hipError_t launch_stage_copy(const StageList& l, hipStream_t stream) {
    if (l.n <= 0) return hipSuccess;
    if (l.n > kMaxStageSegs) return hipErrorInvalidValue;
    uint64_t most = 0;
    for (int i = 0; i < l.n; ++i) {
        if (l.seg[i].bytes && (!l.seg[i].src || !l.seg[i].dst)) return hipErrorInvalidValue;
        most = std::max<uint64_t>(most, l.seg[i].bytes);
    }
    if (most == 0) return hipSuccess;
    // one 16-byte unit per lane and round, up to 1024 workgroups of 256 lanes per segment
    const uint64_t blocks = std::min<uint64_t>(1024, (most / 16 + 255) / 256 + 1);
    stage_copy<<<dim3((unsigned)blocks, (unsigned)l.n), 256, 0, stream>>>(l);
    return hipGetLastError();
}

}  // namespace mnb
