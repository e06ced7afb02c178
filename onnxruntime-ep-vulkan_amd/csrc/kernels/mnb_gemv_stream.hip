// Launch configuration of the streaming decode GEMV (kernel in mnb_gemv_stream.hpp, instantiated
// per bit width in mnb_gemv_stream_b4.hip / mnb_gemv_stream_b8.hip).
#include <algorithm>
#include <cmath>

#include "mnb_gemv_stream.hpp"

namespace mnb {

extern template hipError_t stream_bits<4>(const StreamConfig&, const void*, const uint8_t*,
                                          const void*, const uint8_t*, void*, int64_t, int64_t,
                                          int64_t, int, hipStream_t);
extern template hipError_t stream_bits<8>(const StreamConfig&, const void*, const uint8_t*,
                                          const void*, const uint8_t*, void*, int64_t, int64_t,
                                          int64_t, int, hipStream_t);

namespace {

constexpr int kNumCUs = 256;
// Largest dynamic LDS a decode workgroup may take: with more the decode shapes would fit one
// workgroup per CU and the launch is left to the row-tiled kernels.
constexpr int64_t kStreamMaxLds = 96 * 1024;

// Chunks per lane the kernel is instantiated for (one column per lane group).
constexpr int kStreamMaxCpl = 8;

// Fills the derived fields (workgroups along N, LDS bytes) of a shape; false when the shape is
// malformed or exceeds what the kernel is compiled for.
bool derive(StreamConfig& c, int64_t n, int64_t k, int bits, int bs) {
    if (c.mr < 1 || c.mr > 4 || c.u != 1) return false;
    if (c.waves_per_group < 1 || 64 * c.waves_per_group > kStreamMaxThreads) return false;
    if (c.g != 16 && c.g != 32 && c.g != 64) return false;
    if (bits != 4 && bits != 8) return false;
    const int64_t wpc = 128 / bits;
    if (k <= 0 || k % wpc || k % bs || n <= 0) return false;
    const int64_t cpc = k / wpc;
    if (c.cpl < 1 || c.cpl > kStreamMaxCpl || (int64_t)c.g * c.cpl < cpc) return false;
    const int64_t cols = (int64_t)c.waves_per_group * (64 / c.g) * c.u;
    const int64_t bpc = k / bs;
    const int64_t zpb = (bpc * bits + 7) / 8;
    c.groups = (n + cols - 1) / cols;
    // the activations, and unless each lane loads its own, the columns' scale and zero-point bytes
    // (c.cpl and the instantiated chunk count agree on that: both are at most 4 where it holds)
    const int segs = (128 / bits) > bs ? (128 / bits) / bs : 1;
    c.lds = c.mr * cpc * (bits == 4 ? stream_chunk_stride<4>() : stream_chunk_stride<8>()) +
            (stream_lane_scales(c.cpl, c.u, segs)
                 ? 0
                 : ((cols * bpc * 2 + 15) & ~15) + ((cols * zpb + 15) & ~15));
    return c.groups <= 0x7fffffff && c.lds <= kStreamMaxLds;
}

}  // namespace

static StreamConfig stream_config_search(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    StreamConfig c{};
    const int64_t cpc = k / (128 / bits);
    auto lane_group = [&](int cand) { return (cpc + cand - 1) / cand <= kStreamMaxCpl; };
    // One row-tile of all M rows (up to 4): the weights are streamed once.
    c.mr = m <= 1 ? 1 : (int)(m < 4 ? m : 4);
    // Lane-group width: the best-filled group (G * CPL chunk slots for cpc chunks); among equally
    // filled ones, at one row the one whose lanes load their own scales (at most four chunks per
    // lane), then the one that puts closest to 16 wavefronts on each CU (one per 64/G columns),
    // 10 with four rows (each wavefront then reads four rows of activations per chunk, so fewer,
    // longer wavefronts win).  Measured on MI355X: one row, G=32 for gate_up (6.46 us against
    // 6.71 with G=16), N=32064 (10.4 against 11.4), K=4096 N=14336 (7.3 against 8.3); two to four
    // rows, gate_up G=16 (at four rows 11.3 against 12.8 with G=32), qkv G=32 up to three rows
    // and G=16 at four, o G=32 and down G=64 throughout.
    auto waves_per_cu = [&](int cand) {
        return (double)((n + 64 / cand - 1) / (64 / cand)) / kNumCUs;
    };
    const int segs = (128 / bits) > bs ? (128 / bits) / bs : 1;
    const double target = c.mr <= 3 ? 16.0 : 10.0;
    double best_fill = -1.0, best_dist = 0.0;
    bool best_lane = false;
    int g = 64;
    for (int cand : {64, 32, 16}) {
        if (!lane_group(cand)) continue;
        const int64_t cpl = (cpc + cand - 1) / cand;
        const double fill = (double)cpc / (double)(cand * cpl);
        const bool lane = c.mr == 1 && stream_lane_scales((int)cpl, 1, segs);
        const double dist = __builtin_fabs(waves_per_cu(cand) - target);
        const bool better =
            fill > best_fill + 1e-9 ||
            (fill > best_fill - 1e-9 && (lane > best_lane || (lane == best_lane && dist < best_dist)));
        if (better) {
            best_fill = fill;
            best_lane = lane;
            best_dist = dist;
            g = cand;
        }
    }
    c.g = g;
    c.cpl = (int)((cpc + g - 1) / g);
    // One column per lane group (two measured slower once lanes load their own scales: gate_up
    // 6.89 against 6.46 us, N=32064 11.5 against 10.4).
    c.u = 1;
    const double wpc = waves_per_cu(g);
    // Workgroups: each stages the whole activation vector (2*K bytes per row) before it streams
    // weights, so more workgroups mean more of that traffic ahead of the weights.  Measured over
    // every shape of 4..16 wavefronts (MI355X, K=3072: N = 3072, 8192, 9216, 16384, 32064; K=2048,
    // 2880, 4096, 8192, 14336): the wavefront count that fills the CUs most evenly (the busiest
    // CU's workgroups against the mean), then the one closest to about eight wavefronts per
    // workgroup (wavefronts per CU / 8 workgroups per CU, 1 to 4), then the larger (gate_up
    // 1024 x 8 6.46 us; qkv 512 x 9 4.89 us against 922 x 5 4.98; o 256 x 6 3.30 against 384 x 4
    // 3.34; K=2880 N=5120 256 x 10 3.71 against 640 x 4 3.74; K=4096 N=4096 512 x 8 3.71 against
    // 1024 x 4 3.90; down 256 x 12 4.43 against 512 x 6 4.83).  At least K / 1024 wavefronts, so
    // that the first staging batch (2 * MR 16-byte units per thread) covers all of A.
    const int64_t wmin = std::max<int64_t>(4, (k + 1023) / 1024);
    const int64_t wmax = kStreamMaxThreads / 64;
    const double waves_total = wpc * kNumCUs;
    int64_t w = wmin;
    if (wpc <= 32.0) {
        // (with several rows, four workgroups per CU: qkv at two rows 768 x 6 6.2 us against
        // 512 x 9 6.5 us)
        const double want = c.mr == 1 ? std::min(4.0, std::max(1.0, wpc / 8.0)) : 4.0;
        double best_imb = 0.0, best_d = 0.0;
        for (int64_t cand = wmin; cand <= wmax; ++cand) {
            const double groups = std::ceil(waves_total / (double)cand);
            const double imb = std::ceil(groups / kNumCUs) * kNumCUs / groups;
            const double d = __builtin_fabs(groups / kNumCUs - want);
            if (best_imb == 0.0 || imb < best_imb - 1e-9 ||
                (imb < best_imb + 1e-9 && d < best_d + 1e-9)) {
                best_imb = imb;
                best_d = d;
                w = cand;
            }
        }
    }
    // (above 32 wavefronts per CU, more than a CU holds at once: the smallest workgroups, which
    // the CUs take up as they finish others; N=32064: 4008 x 4 10.4 us against 1002 x 16 11.6 us)
    c.waves_per_group = (int)w;
    derive(c, n, k, bits, bs);
    return c;
}

// The search above runs for the planner's support check, its plan and the launch of every call;
// a shape repeats from one token to the next, so each thread keeps its last eight answers.
StreamConfig gemv_stream_config(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    struct Memo {
        int64_t m, n, k;
        int bits, bs;
        StreamConfig c;
        bool used;
    };
    thread_local Memo memo[8];
    thread_local unsigned next = 0;
    for (const Memo& e : memo)
        if (e.used && e.m == m && e.n == n && e.k == k && e.bits == bits && e.bs == bs) return e.c;
    const StreamConfig c = stream_config_search(m, n, k, bits, bs);
    memo[next++ & 7] = Memo{m, n, k, bits, bs, c, true};
    return c;
}

bool gemv_stream_supported(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    if (bits != 4 && bits != 8) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    if (m < 1 || m > 4 || n < 1) return false;
    const int wpc = 128 / bits;
    if (k <= 0 || k % wpc || k % bs) return false;
    StreamConfig c = gemv_stream_config(m, n, k, bits, bs);
    return derive(c, n, k, bits, bs);
}

hipError_t launch_gemv_stream_cfg(const StreamConfig& cfg, const void* a, const uint8_t* b,
                                  const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                  int64_t k, int bits, int bs, hipStream_t st) {
    if (m == 0) return hipSuccess;
    StreamConfig c = cfg;
    // the shape is checked (the kernel is compiled for kStreamMaxThreads threads per workgroup,
    // U == 1, CPL <= 8) and its derived fields recomputed before anything is launched; row-tiles
    // of MR rows cover M (grid y)
    if (m < 0 || !derive(c, n, k, bits, bs)) return hipErrorInvalidValue;
    const int64_t cols = (int64_t)c.waves_per_group * (64 / c.g) * c.u;
    const int64_t bpc = k / bs;
    const int64_t zpb = (bpc * bits + 7) / 8;
    c.vec_s = (reinterpret_cast<uintptr_t>(s) % 16 == 0) && (cols * bpc * 2) % 16 == 0;
    c.vec_z = z && (reinterpret_cast<uintptr_t>(z) % 16 == 0) && (cols * zpb) % 16 == 0;
    if (bits == 4) return stream_bits<4>(c, a, b, s, z, y, m, n, k, bs, st);
    return stream_bits<8>(c, a, b, s, z, y, m, n, k, bs, st);
}

hipError_t launch_gemv_stream(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                              void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                              hipStream_t st) {
    const StreamConfig c = gemv_stream_config(m, n, k, bits, bs);
    return launch_gemv_stream_cfg(c, a, b, s, z, y, m, n, k, bits, bs, st);
}

}  // namespace mnb
