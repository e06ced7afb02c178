// Instantiates the streaming decode GEMV for 4-bit weights (kernel in mnb_gemv_stream.hpp).
#include "mnb_gemv_stream.hpp"

namespace mnb {

template hipError_t stream_bits<4>(const StreamConfig&, const void*, const uint8_t*, const void*,
                                   const uint8_t*, void*, int64_t, int64_t, int64_t, int,
                                   hipStream_t);

}  // namespace mnb
