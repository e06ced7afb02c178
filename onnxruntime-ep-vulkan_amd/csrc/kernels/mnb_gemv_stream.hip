// Launch configuration of the streaming decode GEMV (kernel in mnb_gemv_stream.hpp, instantiated
// per bit width in mnb_gemv_stream_b4.hip / mnb_gemv_stream_b8.hip).
#include "mnb_launch.hpp"

namespace mnb {

template <int BITS>
hipError_t stream_bits(const StreamConfig& c, const void* a, const uint8_t* b, const void* s,
                       const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bs,
                       hipStream_t st);
extern template hipError_t stream_bits<4>(const StreamConfig&, const void*, const uint8_t*,
                                          const void*, const uint8_t*, void*, int64_t, int64_t,
                                          int64_t, int, hipStream_t);
extern template hipError_t stream_bits<8>(const StreamConfig&, const void*, const uint8_t*,
                                          const void*, const uint8_t*, void*, int64_t, int64_t,
                                          int64_t, int, hipStream_t);

namespace {

constexpr int kNumCUs = 256;

// Chunks-per-lane capacity for MR rows held in registers.
int cpl_cap(int mr) { return mr == 1 ? 8 : (mr == 2 ? 4 : 2); }

int rows_tile(int64_t m) { return m <= 1 ? 1 : (m == 2 ? 2 : (m == 3 ? 3 : 4)); }

}  // namespace

bool gemv_stream_supported(int64_t m, int64_t k, int bits, int bs) {
    if (bits != 4 && bits != 8) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    const int wpc = 128 / bits;
    if (k <= 0 || k % wpc || k % bs) return false;
    const int mr = rows_tile(m);
    if (m < 1 || m > 4) return false;
    const int64_t cpc = k / wpc;
    return cpc <= (int64_t)64 * cpl_cap(mr);
}

StreamConfig gemv_stream_config(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    (void)bs;
    StreamConfig c{};
    c.mr = rows_tile(m);
    const int64_t cpc = k / (128 / bits);
    const int cap = cpl_cap(c.mr);
    // Lane-group width: weigh the fraction of lane slots that hold a chunk against having enough
    // wavefronts in flight (about 16 per CU) to cover HBM latency.  Measured on MI355X for the
    // Phi-3.5 shapes: 96 chunks per column -> G = 32 when N >= 9216, G = 64 for N = 3072;
    // 256 chunks -> G = 64.
    double best = -1.0;
    int g = 64;
    for (int cand : {64, 32, 16}) {                 // ties go to the wider group
        const int64_t cpl = (cpc + cand - 1) / cand;
        if (cpl > cap) continue;
        const double fill = (double)cpc / (double)(cand * cpl);
        const double waves = (double)n * cand / 64.0;
        const double par = waves >= 16.0 * kNumCUs ? 1.0 : waves / (16.0 * kNumCUs);
        const double score = fill * __builtin_sqrt(par);
        if (score > best + 1e-9) { best = score; g = cand; }
    }
    c.g = g;
    c.cpl = (int)((cpc + g - 1) / g);
    c.u = 1;
    c.waves_per_group = 4;
    c.nontemporal = 1;
    const int ng = 64 / g;
    const int64_t tasks = (n + (int64_t)ng * c.u - 1) / ((int64_t)ng * c.u);
    c.tasks = tasks;
    // Up to 8 wavefronts per CU; the rest of the columns are covered by looping, which keeps
    // the next pass's loads in flight while the current one is reduced.
    c.total_waves = tasks < 8 * kNumCUs ? tasks : 8 * kNumCUs;
    return c;
}

hipError_t launch_gemv_stream_cfg(const StreamConfig& c, const void* a, const uint8_t* b,
                                  const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                  int64_t k, int bits, int bs, hipStream_t st) {
    if (m == 0) return hipSuccess;
    // the kernel is compiled for kStreamMaxThreads threads per workgroup
    if (c.waves_per_group < 1 || 64 * c.waves_per_group > kStreamMaxThreads)
        return hipErrorInvalidValue;
    if (c.mr < 1 || c.mr > 4 || (c.u != 1 && c.u != 2) || c.tasks < 1 || c.total_waves < 1)
        return hipErrorInvalidValue;
    if (c.g != 16 && c.g != 32 && c.g != 64) return hipErrorInvalidValue;
    if ((int64_t)c.g * c.cpl * (128 / bits) < k) return hipErrorInvalidValue;
    if (bits == 4) return stream_bits<4>(c, a, b, s, z, y, m, n, k, bs, st);
    if (bits == 8) return stream_bits<8>(c, a, b, s, z, y, m, n, k, bs, st);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_stream(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                              void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                              hipStream_t st) {
    const StreamConfig c = gemv_stream_config(m, n, k, bits, bs);
    return launch_gemv_stream_cfg(c, a, b, s, z, y, m, n, k, bits, bs, st);
}

}  // namespace mnb
