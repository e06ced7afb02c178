// Host-side launchers for the MatMulNBits kernels (internal to libmnb_hip.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <utility>

namespace mnb {

// Dynamic LDS above 64 KiB must be allowed per kernel (hipFuncAttributeMaxDynamicSharedMemorySize).
// The attribute is set once per kernel and device, to the largest size that kernel has been
// launched with there, so repeated launches (an EP's decode loop, a graph capture) make no
// further runtime call beyond a table lookup.
inline hipError_t allow_dynamic_lds(const void* kern, size_t bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, size_t> allowed;
    std::lock_guard<std::mutex> lock(mu);
    size_t& have = allowed[{kern, dev}];
    if (have >= bytes) return hipSuccess;
    const hipError_t e =
        hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) have = bytes;
    return e;
}

// Threads per workgroup each kernel family is compiled for (its __launch_bounds__).  A launcher
// refuses a launch shape above its kernel's limit before anything reaches the device: a
// workgroup larger than the compiled bound fails as an unspecified launch failure.
constexpr int kStreamMaxThreads = 1024;  // gemv_stream
constexpr int kGroupMaxThreads = 512;    // group_gemv
constexpr int kGemvMaxThreads = 1024;    // gemv_f16_mfma

// Geometry shared by the planner (host) and the launchers.
struct GemvGeom {
    int mt;        // 16-row M tiles per workgroup (1, 2 or 4)
    int waves;     // wavefronts per workgroup
    int64_t gx;    // ceil(N / 16)
    int64_t gy;    // ceil(M / (16 * mt))
    size_t lds;    // dynamic LDS bytes
};

// Launch shape of the streaming decode GEMV (mnb_gemv_stream.hip).  Each wavefront makes one
// pass over u columns per lane group; a workgroup covers waves_per_group * (64/g) * u columns
// (about one workgroup per CU).
struct StreamConfig {
    int mr;              // rows of A per workgroup row-tile (1..4)
    int g;               // lanes per column (16, 32, 64)
    int cpl;             // 16-byte chunks per lane (ceil(chunks per column / g))
    int u;               // columns per lane group (1; the launcher refuses others)
    int waves_per_group; // wavefronts per workgroup (1..16)
    int vec_s, vec_z;    // scale / zero-point bytes staged with 16-byte loads (set at launch)
    int64_t groups;      // workgroups along N (derived)
    int64_t lds;         // dynamic LDS bytes (derived)
};

bool gemv_stream_supported(int64_t m, int64_t n, int64_t k, int bits, int bs);
StreamConfig gemv_stream_config(int64_t m, int64_t n, int64_t k, int bits, int bs);
hipError_t launch_gemv_stream(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                              void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                              hipStream_t stream);
// fp32 prefill (mnb_gemm_f32.hip): fp32 MFMA GEMM, 128 (or 64) x 128 tiles of 4 wavefronts,
// K % 32 == 0.
bool gemm_f32_supported(int64_t m, int64_t n, int64_t k, int bits, int bs);
int gemm_f32_tile_rows(int64_t m, int64_t n);       // 128, or 64 when 128-row tiles under-fill
hipError_t launch_gemm_f32(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                           void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                           hipStream_t stream);
// fp32 activations, scales and output (mnb_gemv_f32.hip): the fp16 launch shape with fp32 staging;
// false when the shape is outside what the kernel is compiled for.
bool gemv_stream_f32_config(int64_t m, int64_t n, int64_t k, int bits, int bs, StreamConfig* out);
hipError_t launch_gemv_stream_f32(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                                  void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                                  hipStream_t stream);
hipError_t launch_gemv_stream_cfg(const StreamConfig& c, const void* a, const uint8_t* b,
                                  const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                  int64_t k, int bits, int bs, hipStream_t stream);

// Tile shape of the prefill GEMM (mnb_gemm.hip).
struct GemmConfig {
    int bm, bn;          // workgroup tile
    int64_t tiles_m, tiles_n;
    int ksplit;          // workgroups per tile along K (fp32 partials summed by a second launch)
};

bool gemm_supported(int64_t m, int64_t n, int64_t k, int bits, int bs, bool has_zp);
GemmConfig gemm_config(int64_t m, int64_t n, int64_t k);
// fp32 partials of a K split (0 when the config does not split)
size_t gemm_workspace_bytes(const GemmConfig& c, int64_t m, int64_t n);
// With less workspace than gemm_workspace_bytes (or none) the launch runs without the K split.
hipError_t launch_gemm(const void* a, const uint8_t* b, const void* s, const uint8_t* z, void* y,
                       int64_t m, int64_t n, int64_t k, int bits, int bs, hipStream_t stream,
                       void* workspace = nullptr, size_t workspace_bytes = 0);
hipError_t launch_gemm_cfg(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                           const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bits,
                           int bs, hipStream_t stream, void* workspace = nullptr,
                           size_t workspace_bytes = 0);
// Y = the sum of `ksplit` fp32 partial planes of m*n elements, in split order.
hipError_t launch_splitk_sum(const float* part, void* y, int64_t mn, int ksplit,
                             hipStream_t stream);

// Launch shape of the row-tiled MFMA GEMV (mnb_group_gemv.hip).
struct GroupGeom {
    int mt;              // 16-row tiles per workgroup (1, 2 or 4)
    int waves;           // wavefronts per workgroup (split K within the workgroup)
    int ksplit;          // workgroups per strip (split K across workgroups; int8 path only)
    int runs_per_split;  // prefetched runs of iterations per split
    int64_t gx, gy, gz;  // column strips, groups, row tiles
    size_t lds;
};

// 128-k iterations whose loads one wavefront issues together.  The int8 path also holds one
// activation scale per output value and block end, so its runs shrink to keep those within
// 32 registers per run where one iteration allows it (64 at most: block 32, 64 rows).
constexpr int group_pf(bool i8, int bs, int mt) {
    if (!i8) return 4;
    const int per_iter = (128 / bs) * mt * 4;            // activation scales per iteration
    const int pf = 32 / per_iter;
    return pf < 1 ? 1 : (pf > 4 ? 4 : pf);
}

bool group_gemv_supported(int64_t k, int bits, int bs);
GroupGeom group_geometry(int64_t rows, int64_t n, int64_t k, int64_t groups, bool i8, int bs,
                         bool allow_split);
hipError_t launch_group_gemv_f16(const void* a, const int32_t* row_index, const int32_t* offsets,
                                 int64_t groups, int64_t max_rows, const uint8_t* b,
                                 const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                 int64_t k, int bits, int bs, hipStream_t stream);
// The same with rows per group known only on the device: `rows_bound` bounds every group (the
// grid covers it), `rows_hint` (the expected rows per group) sets the tile height.
hipError_t launch_group_gemv_f16_bounded(const void* a, const int32_t* row_index,
                                         const int32_t* offsets, int64_t groups,
                                         int64_t rows_bound, int64_t rows_hint, const uint8_t* b,
                                         const void* s, const uint8_t* z, void* y, int64_t m,
                                         int64_t n, int64_t k, int bits, int bs,
                                         hipStream_t stream, const uint8_t* b_strips = nullptr);
// Launch shape of the strip GEMV (mnb_strip_gemv.hip): at most 16 rows per group, the
// activations of a wavefront's K share held in registers across a run of column strips.
struct StripGeom {
    int waves;           // wavefronts per workgroup (split K)
    int qw;              // 128-k quads per wavefront (register arrays of the instantiation)
    int strips;          // 16-column strips per workgroup
    int64_t gx, gy, gz;  // runs of strips, groups, 16-row tiles
    size_t lds;
};
bool strip_geometry(int64_t n, int64_t k, int64_t groups, int64_t rows_bound, bool i8, int bs,
                    bool has_zp, StripGeom* out);
// The pointer alignment the strip GEMV needs (A and B 16 bytes).
bool strip_gemv_aligned(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                        bool i8);
// True when MNB_FORCE_KERNEL=group asks for the row-tiled GEMV instead.
bool strip_gemv_forced_off();
// SwiGLU applied by the strip GEMV as it stores interleaved (gate, linear) column pairs
// (QMoE fc1 with swiglu_fusion = 1): y[r][c / 2] = act(h[r][c] + b[c], h[r][c + 1] + b[c + 1])
// for even c, h rounded to fp16 before the bias, y row stride N / 2 (N even).
// With expert_of set (QMoE decode batches: R = T * k <= 1024 assignments, groups <= 64) the
// kernel also finds each expert's rows itself: expert e's rows are the assignments a with
// expert_of[a] == e in order (token a / k), at grouped positions from #{a : expert_of[a] < e};
// the first workgroup of each expert publishes offsets[e] (and offsets[E] = R) and pos_of[a]
// of its assignments for the launches that follow.  row_index is then unused.
struct StripSwiglu {
    const void* bias;    // fp16 [groups][N] or null
    float alpha, beta, limit;
    int has_limit;
    const int32_t* expert_of;   // [R] or null
    int32_t* offsets;           // [groups + 1], written
    int32_t* pos_of;            // [R], written
    int R, k;
};
// fp16 scales and Y; A is fp16, or for i8 (accuracy_level = 4) the int8 codes of
// quantize_a_int8 in its quad-interleaved layout (quads = true) with their fp32 scales
// block-major over 16 rows, a_scale [K / bs][16].
// swiglu (fp16 A, no zero points) stores the activation instead of Y.
hipError_t launch_strip_gemv(const StripGeom& g, bool i8, const void* a, const float* a_scale,
                             const int32_t* row_index,
                             const int32_t* offsets, const uint8_t* b, const void* s,
                             const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bs,
                             hipStream_t stream, const StripSwiglu* swiglu = nullptr,
                             const uint8_t* b_strips = nullptr);

// cnt / ncnt: split-K counters of a following int8 GEMV, cleared by the quantiser (may be null).
// scale_rows > 0 writes the scales block-major, [k/bs][scale_rows] (rows >= m untouched).
// quads: the strip GEMV's layout -- permuted, and within every whole 128-k quad the 8-byte group
// of chunk t, lane row g stored at (t / 2) * 64 + 16 g + (t % 2) * 8.
hipError_t launch_quantize_a_int8(const void* a, bool a_f16, int8_t* qa, float* scale,
                                  int32_t* qsum, bool permuted, int64_t m, int64_t k, int bs,
                                  hipStream_t stream, int* cnt = nullptr, int64_t ncnt = 0,
                                  int64_t scale_rows = 0, bool quads = false);
size_t acc4_workspace_bytes(int64_t m, int64_t n, int64_t k, int bs, bool a_f16);
// accuracy_level = 4 at up to 16 fp16 rows (mnb_acc4_stream.hip): one 16-column strip per
// workgroup over all of K, `waves` wavefronts of r quads each (waves * r == K / 128), the
// workgroup's partial tiles added in LDS.  K % 128 == 0, (K / bs) % 4 == 0, K up to 8192.
struct Acc4StreamGeom {
    int r;               // 128-k quads per wavefront: 1, 2, 4 or 8
    int waves;           // wavefronts per workgroup, K / (128 r), 1..16
    int64_t gx;          // workgroups: 16-column strips
    size_t lds;          // bytes: staged codes and activation scales, partial tiles
};
bool acc4_stream_geometry(int64_t m, int64_t n, int64_t k, int bs, Acc4StreamGeom* out);
// The geometry when the accuracy_level = 4 planner takes this kernel (fp16 A, and no
// MNB_FORCE_KERNEL=strip or =group asking for the other int8 GEMVs).
bool acc4_stream_planned(bool a_f16, int64_t m, int64_t n, int64_t k, int bs,
                         Acc4StreamGeom* out);
// Codes and B 16-byte, scales 8-byte, zero points 2-byte aligned.
bool acc4_stream_aligned(const void* qa, const uint8_t* b, const void* s, const uint8_t* z);
// b_strips: the strip-major copy of B (launch_strip_pack), read in place of b when not null.
hipError_t launch_acc4_stream(const Acc4StreamGeom& g, const int8_t* qa, const float* a_scale,
                              const uint8_t* b, const void* s, const uint8_t* z, void* y,
                              int64_t m, int64_t n, int64_t k, int bs, hipStream_t stream,
                              const uint8_t* b_strips = nullptr);
// Batched decode at up to 16 fp16 rows, int4 weights (mnb_batch_stream.hip): s 16-column
// strips per workgroup over all of K, `waves` wavefronts of r quads each (waves * r == K / 128),
// activations loaded straight into MFMA registers.  K % 128 == 0, (K / bs) % 4 == 0, bs >= 32.
struct BatchStreamGeom {
    int r;               // 128-k quads per wavefront: 1..4
    int s;               // 16-column strips per workgroup: 1 to 4
    int waves;           // wavefronts per workgroup, K / (128 r), 1..16
    int64_t gx;          // workgroups: ceil(strips / s)
};
bool batch_stream_geometry(int64_t m, int64_t n, int64_t k, int bs, BatchStreamGeom* out);
// A and B 16-byte, scales 8-byte, zero points 2-byte aligned.
bool batch_stream_aligned(const void* a, const uint8_t* b, const void* s, const uint8_t* z);
// b_strips: the MFMA-native strip-major copy of B (launch_strip_pack with native set), read in
// place of b when not null.
hipError_t launch_batch_stream(const BatchStreamGeom& g, const void* a, const uint8_t* b,
                               const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                               int64_t k, int bs, hipStream_t stream,
                               const uint8_t* b_strips = nullptr);
// The strip-major copy of an int4 B [groups][N][K / 2] (K % 32 == 0):
// [groups][ceil(N / 16)][ceil(K / 128)][16 columns][4 chunks] x 16 bytes, strip_pack_bytes
// bytes, 16-byte aligned; columns past N and chunks past K zero.  In the MFMA orders each
// 16-byte piece (lane (n, g)) instead holds dword g of the quad's four chunks -- the operand
// dwords the kernels otherwise form with a 4 x 4 transpose across lanes -- and for the fp16
// kernels (the level-0 copies read by launch_batch_stream, the QMoE expert copies read by the
// fp16 strip GEMV) each dword's nibbles reordered to k0 k2 k4 k6 k1 k3 k5 k7; the int8 kernel
// (the level-4 copies, launch_acc4) unpacks the natural nibble order.
enum StripOrder : int { kStripPlain = 0, kStripMfmaF16 = 1, kStripMfmaI8 = 2 };
int64_t strip_pack_bytes(int64_t n, int64_t k, int64_t groups = 1);
hipError_t launch_strip_pack(const uint8_t* b, uint8_t* dst, int64_t n, int64_t k,
                             hipStream_t stream, int64_t groups = 1, int order = kStripPlain);
hipError_t launch_acc4(const void* a, bool a_f16, const uint8_t* b, const void* s,
                       const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bits,
                       int bs, void* workspace, hipStream_t stream,
                       const uint8_t* b_strips = nullptr);

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

// Fused QMoE (mnb_qmoe.hip).
struct QmoeArgs {
    int64_t rows, hidden, inter, experts;
    int k, block_size, fusion, normalize, has_limit, router_f32;
    float alpha, beta, limit;
};
size_t qmoe_workspace_bytes(const QmoeArgs& q);
// fc1_strips / fc2_strips: strip-major copies of the expert weights (launch_strip_pack over the
// experts), read by the strip GEMV in place of fc1 / fc2 when not null.
hipError_t launch_qmoe(const QmoeArgs& q, const void* x, const void* logits, const uint8_t* fc1,
                       const void* fc1_s, const void* fc1_b, const uint8_t* fc2, const void* fc2_s,
                       const void* fc2_b, void* y, void* workspace, hipStream_t stream,
                       const uint8_t* fc1_strips = nullptr, const uint8_t* fc2_strips = nullptr);

// RMSNorm with optional fused residual add (mnb_rmsnorm.hip).
bool rmsnorm_supported(int64_t hidden, bool f16);
hipError_t launch_skip_rmsnorm(const void* x, const void* skip, const void* gamma,
                               const void* bias, void* y, void* sum_out, int64_t rows,
                               int64_t hidden, float eps, bool f16, hipStream_t stream);

// GroupQueryAttention with packed QKV and fused RoPE (mnb_gqa.hip).
struct GqaArgs {
    int64_t batch, seq, past_stride, present_len, max_seq;
    int nq, nkv, d, rot;
    float scale;
    bool copy_past;      // present is its own buffer: the past tokens are copied into it
};
struct GqaPlan {
    int waves;           // wavefronts per workgroup (16 query rows each)
    int splits;          // workgroups along the keys of one row block
    int64_t row_blocks;  // row blocks per (batch, KV head)
    int64_t chunk;       // keys per split (a multiple of 64)
};
bool gqa_supported(int head_dim);
GqaPlan gqa_plan(const GqaArgs& a);
size_t gqa_workspace_bytes(const GqaArgs& a);
hipError_t launch_gqa(const GqaArgs& a, const void* qkv, const void* past_k, const void* past_v,
                      const int32_t* seqlens, const void* cos_cache, const void* sin_cache,
                      void* out, void* pres_k, void* pres_v, void* workspace, hipStream_t stream);

// Byte copies between pinned host memory and device memory, up to kMaxStageSegs segments in
// one launch (mnb_stage.hip).  Host pointers must be device-accessible (hipHostMalloc).
constexpr int kMaxStageSegs = 8;
struct StageSeg {
    const void* src;
    void* dst;
    uint64_t bytes;
};
struct StageList {
    StageSeg seg[kMaxStageSegs];
    int n;
};
hipError_t launch_stage_copy(const StageList& l, hipStream_t stream);

// Roofline calibration (mnb_calibrate.hip): workgroups x 4 wavefronts x iters x 16 MFMAs.
hipError_t launch_mfma_calibrate(const void* operands, float* out, int workgroups, int iters,
                                 hipStream_t stream);
// Read floor (mnb_calibrate.hip): n16 16-byte units, loads_per_lane in {1,2,4,8,16} 1 KB runs
// per wavefront, wpg wavefronts per workgroup (1..16), contiguous or grid-stride runs.
hipError_t launch_read_floor(const void* src, int64_t n16, int loads_per_lane, int wpg,
                             bool contig, uint32_t* out, hipStream_t stream);

}  // namespace mnb
