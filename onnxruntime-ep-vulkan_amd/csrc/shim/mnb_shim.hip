// C ABI of the MatMulNBits HIP shim (declared in include/mnb_hip.h).
//
// Replaces, for this one op, the reference's Vulkan session: the dispatch translation of
// rust/src/ops/quant.rs:521-651 becomes mnb_plan + one kernel launch; the constant-input weight
// cache of rust/src/vk/session.rs:1633-1700 becomes mnb_weights_upload (hipMalloc + copy once);
// the submit/fence/readback of rust/src/vk/session.rs:2635-2736,2791 becomes
// mnb_session_run_host on one hipStream_t per session.  Errors never abort: every entry point
// returns a code and leaves a message for mnb_last_error().
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <cmath>
#include <string>
#include <vector>

#include "../../../include/mnb_hip.h"
#include "../kernels/mnb_launch.hpp"

namespace {

thread_local std::string g_last_error;
std::atomic<uint64_t> g_launches{0};
std::atomic<uint64_t> g_device_allocs{0};

// Every device allocation the library makes on its own behalf (weights and caches at upload,
// session staging and workspace as they grow) goes through here and is counted, so a test can
// show that steady-state calls allocate nothing.  mnb_device_malloc, the caller's allocator,
// is not counted.
template <class T>
hipError_t counted_malloc(T** p, size_t bytes) {
    const hipError_t e = hipMalloc(reinterpret_cast<void**>(p), bytes);
    if (e == hipSuccess) g_device_allocs.fetch_add(1);
    return e;
}

// The pinned host staging of a session's host-I/O calls, counted with the device allocations.
hipError_t counted_host_malloc(void** p, size_t bytes) {
    const hipError_t e = hipHostMalloc(p, bytes, hipHostMallocDefault);
    if (e == hipSuccess) g_device_allocs.fetch_add(1);
    return e;
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(MNB_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Rows above which the prefill GEMM replaces the 16-row MFMA GEMV.
constexpr int64_t kGemmMinRows = 64;
// Rows from which the batched decode kernel is planned (below: the streaming GEMV).  Measured on
// the Phi-3.5 decode shapes at four rows on ORT's layout (cold weights, the batched kernel at its
// planned geometry): qkv 7.83 against 9.51-9.65 us on the streaming GEMV, o 4.26 against 5.32,
// gate_up 9.10-9.16 against 11.88-11.95, down 8.00 against 8.22-8.32; at 2-3 rows the streaming
// GEMV on every node (a node with the MFMA-native copy moves to the batched kernel at 3 rows,
// in matmul_impl).
constexpr int64_t kBatchMinRows = 4;

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t bpc_of(const mnb_problem* p) { return p->k / p->block_size; }
int64_t b_bytes_of(const mnb_problem* p) { return p->n * (p->k * p->bits / 8); }
int64_t zp_bytes_per_col(const mnb_problem* p) { return (bpc_of(p) * p->bits + 7) / 8; }
int64_t elem_bytes(int32_t dtype) { return dtype == MNB_DTYPE_F16 ? 2 : 4; }

// Environment override of the planner, the counterpart of the reference's A/B controls
// (ONNXRUNTIME_EP_VULKAN_GEMV_PACKED / _GEMV_MAX_ROWS, rust/src/ops/quant.rs:373-449).
// Read on every plan (tests flip it at run time); getenv is a short scan of the environment.
int forced_kernel() {
    const char* v = std::getenv("MNB_FORCE_KERNEL");
    if (!v || !*v) return 0;
    if (!std::strcmp(v, "gemv")) return MNB_KERNEL_GEMV_MFMA;
    if (!std::strcmp(v, "gemm")) return MNB_KERNEL_GEMM_MFMA;
    if (!std::strcmp(v, "generic")) return MNB_KERNEL_GENERIC;
    if (!std::strcmp(v, "stream")) return MNB_KERNEL_GEMV_STREAM;
    if (!std::strcmp(v, "group")) return MNB_KERNEL_GROUP_MFMA;
    if (!std::strcmp(v, "strip")) return MNB_KERNEL_STRIP_MFMA;
    if (!std::strcmp(v, "batch")) return MNB_KERNEL_BATCH_STREAM;
    return 0;
}

}  // namespace

extern "C" {

const char* mnb_last_error(void) { return g_last_error.c_str(); }

int mnb_version(void) { return 1; }

uint64_t mnb_launch_count(void) { return g_launches.load(); }

uint64_t mnb_device_alloc_count(void) { return g_device_allocs.load(); }

int mnb_calibrate_mfma(int32_t workgroups, int32_t iters, const void* operands_f16, float* out,
                       void* stream) {
    if (workgroups < 1 || workgroups > 65536 || iters < 1 || iters > 1000000)
        return fail(MNB_ERR_INVALID, "workgroups = %d, iters = %d", workgroups, iters);
    if (!out) return fail(MNB_ERR_INVALID, "out is NULL");
    if (operands_f16 && !aligned(operands_f16, 16))
        return fail(MNB_ERR_INVALID, "operands must be 16-byte aligned");
    hipError_t e = mnb::launch_mfma_calibrate(operands_f16, out, workgroups, iters,
                                              static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "calibration launch");
    return MNB_OK;
}

int mnb_calibrate_read(const void* src, size_t bytes, int32_t loads_per_lane,
                       int32_t waves_per_group, int32_t contiguous, uint32_t* out, void* stream) {
    if (!src || !out) return fail(MNB_ERR_INVALID, "src and out must not be NULL");
    if (!aligned(src, 16) || bytes == 0 || bytes % 16)
        return fail(MNB_ERR_INVALID, "src must be 16-byte aligned and bytes a positive multiple "
                                     "of 16 (got %zu)", bytes);
    if (loads_per_lane != 1 && loads_per_lane != 2 && loads_per_lane != 4 &&
        loads_per_lane != 8 && loads_per_lane != 16)
        return fail(MNB_ERR_INVALID, "loads_per_lane = %d; 1, 2, 4, 8 or 16", loads_per_lane);
    if (waves_per_group < 1 || waves_per_group > 16)
        return fail(MNB_ERR_INVALID, "waves_per_group = %d; 1..16 (the kernel is compiled for "
                                     "1024 threads)", waves_per_group);
    hipError_t e = mnb::launch_read_floor(src, (int64_t)(bytes / 16), loads_per_lane,
                                          waves_per_group, contiguous != 0, out,
                                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "read-floor launch");
    return MNB_OK;
}

int mnb_check_problem(const mnb_problem* p) {
    if (!p) return fail(MNB_ERR_INVALID, "problem is NULL");
    if (p->bits != 4 && p->bits != 8)
        return fail(MNB_ERR_UNSUPPORTED, "bits = %d; this library implements 4 and 8", p->bits);
    if (p->block_size != 16 && p->block_size != 32 && p->block_size != 64 && p->block_size != 128)
        return fail(MNB_ERR_UNSUPPORTED, "block_size = %d; this library implements 16/32/64/128",
                    p->block_size);
    if (p->k <= 0 || p->n <= 0)
        return fail(MNB_ERR_INVALID, "K = %lld, N = %lld; both must be positive",
                    (long long)p->k, (long long)p->n);
    if (p->m < 0) return fail(MNB_ERR_INVALID, "M = %lld is negative", (long long)p->m);
    if (p->k % p->block_size)
        return fail(MNB_ERR_UNSUPPORTED, "K = %lld is not a multiple of block_size = %d",
                    (long long)p->k, p->block_size);
    if (p->dtype != MNB_DTYPE_F16 && p->dtype != MNB_DTYPE_F32)
        return fail(MNB_ERR_UNSUPPORTED, "dtype %d; A/scales/Y must be fp16 or fp32", p->dtype);
    if (p->accuracy_level < 0 || p->accuracy_level > 4)
        return fail(MNB_ERR_INVALID, "accuracy_level = %d is outside 0..4", p->accuracy_level);
    const int64_t lim = (int64_t)1 << 31;
    if (p->k >= lim || p->n >= lim || p->m >= lim || p->m * p->k >= ((int64_t)1 << 40))
        return fail(MNB_ERR_UNSUPPORTED, "extent too large (M=%lld N=%lld K=%lld)",
                    (long long)p->m, (long long)p->n, (long long)p->k);
    return MNB_OK;
}

static int plan_search(const mnb_problem* p, mnb_plan_info* out) {
    int rc = mnb_check_problem(p);
    if (rc) return rc;
    if (!out) return fail(MNB_ERR_INVALID, "plan output is NULL");
    std::memset(out, 0, sizeof(*out));
    if (p->accuracy_level == 4) {
        // int8 activations (ORT's SQNBIT_CompInt8 level): quantiser + int8 MFMA GEMV.
        if (!mnb::group_gemv_supported(p->k, p->bits, p->block_size))
            return fail(MNB_ERR_UNSUPPORTED,
                        "accuracy_level 4 is implemented for bits = 4, block_size >= 32 and "
                        "K %% 32 == 0 (got bits = %d, block_size = %d, K = %lld)",
                        p->bits, p->block_size, (long long)p->k);
        const bool f16 = p->dtype == MNB_DTYPE_F16;
        out->kernel = MNB_KERNEL_ACC4_I8;
        out->tile_n = 16;
        mnb::Acc4StreamGeom ag{};
        if (mnb::acc4_stream_planned(f16, p->m, p->n, p->k, p->block_size, &ag)) {
            // up to 16 rows: one 16-column strip per workgroup over all of K
            out->kernel = MNB_KERNEL_ACC4_STREAM;
            out->waves_per_group = ag.waves;
            out->tile_m = 16;
            out->grid_x = ag.gx;
            out->grid_y = 1;
        } else {
            const mnb::GroupGeom g =
                mnb::group_geometry(p->m, p->n, p->k, 1, true, p->block_size, true);
            out->waves_per_group = g.waves;
            out->tile_m = 16 * g.mt;
            out->grid_x = g.gx * g.ksplit;
            out->grid_y = g.gz;
        }
        out->workspace_bytes =
            (int64_t)mnb::acc4_workspace_bytes(p->m, p->n, p->k, p->block_size, f16);
        return MNB_OK;
    }
    const bool f16 = p->dtype == MNB_DTYPE_F16;
    const bool fast = f16 && mnb::gemv_supported(p->k, p->bits, p->block_size);
    const bool stream = f16 && mnb::gemv_stream_supported(p->m, p->n, p->k, p->bits, p->block_size);
    const bool group = f16 && mnb::group_gemv_supported(p->k, p->bits, p->block_size);
    const bool gemm = f16 && mnb::gemm_supported(p->m, p->n, p->k, p->bits, p->block_size,
                                                  p->has_zero_points != 0);
    int kern = MNB_KERNEL_GENERIC;
    if (fast) kern = MNB_KERNEL_GEMV_MFMA;               // bits 8, block 16: 16-row MFMA GEMV
    if (group) kern = MNB_KERNEL_GROUP_MFMA;             // int4, block >= 32: any row count
    if (gemm && p->m > kGemmMinRows) kern = MNB_KERNEL_GEMM_MFMA;
    mnb::StripGeom sg{};
    const bool strip = group && p->m <= 16 &&
                       mnb::strip_geometry(p->n, p->k, 1, p->m, false, p->block_size,
                                           p->has_zero_points != 0, &sg);
    if (strip) kern = MNB_KERNEL_STRIP_MFMA;             // 5..16 rows
    mnb::BatchStreamGeom bg{};
    const bool batch = f16 && p->bits == 4 &&
                       mnb::batch_stream_geometry(p->m, p->n, p->k, p->block_size, &bg);
    const bool batch_rows = p->m >= kBatchMinRows || !stream;
    if (batch && p->m >= 4 && batch_rows) kern = MNB_KERNEL_BATCH_STREAM;
    if (stream && !(batch && batch_rows)) kern = MNB_KERNEL_GEMV_STREAM;
    // fp32 activations, M <= 4: the fp32 streaming GEMV (same launch shape as the fp16 one)
    mnb::StreamConfig c32{};
    const bool stream32 = !f16 && mnb::gemv_stream_f32_config(p->m, p->n, p->k, p->bits,
                                                              p->block_size, &c32);
    // fp32 activations above that: the fp32 MFMA GEMM over weights dequantised into LDS
    const bool gemm32 = !f16 && mnb::gemm_f32_supported(p->m, p->n, p->k, p->bits, p->block_size);
    if (stream32) kern = MNB_KERNEL_GEMV_STREAM;
    else if (gemm32) kern = MNB_KERNEL_GEMM_MFMA;
    const int forced = forced_kernel();
    if (forced == MNB_KERNEL_GENERIC) kern = MNB_KERNEL_GENERIC;
    if (forced == MNB_KERNEL_GEMV_MFMA && fast) kern = MNB_KERNEL_GEMV_MFMA;
    if (forced == MNB_KERNEL_GEMV_STREAM && (stream || stream32)) kern = MNB_KERNEL_GEMV_STREAM;
    if (forced == MNB_KERNEL_GEMM_MFMA && (gemm || gemm32)) kern = MNB_KERNEL_GEMM_MFMA;
    if (forced == MNB_KERNEL_GROUP_MFMA && group) kern = MNB_KERNEL_GROUP_MFMA;
    if (forced == MNB_KERNEL_STRIP_MFMA && strip) kern = MNB_KERNEL_STRIP_MFMA;
    if (forced == MNB_KERNEL_BATCH_STREAM && batch) kern = MNB_KERNEL_BATCH_STREAM;
    out->kernel = kern;
    if (kern == MNB_KERNEL_GEMM_MFMA && !f16) {
        const int bm = mnb::gemm_f32_tile_rows(p->m, p->n);
        out->waves_per_group = 4;                        // bm x 128 tiles, no K split
        out->tile_n = 128;
        out->tile_m = bm;
        out->grid_x = ((p->m + bm - 1) / bm) * ((p->n + 127) / 128);
        out->grid_y = 1;
        out->workspace_bytes = 0;
        return MNB_OK;
    }
    if (kern == MNB_KERNEL_GEMM_MFMA) {
        const mnb::GemmConfig c = mnb::gemm_config(p->m, p->n, p->k);
        out->waves_per_group = 8;
        out->tile_n = c.bn;
        out->tile_m = c.bm;
        out->grid_x = c.tiles_m * c.tiles_n * c.ksplit;
        out->grid_y = 1;
        out->workspace_bytes = (int64_t)mnb::gemm_workspace_bytes(c, p->m, p->n);
        return MNB_OK;
    } else if (kern == MNB_KERNEL_GEMV_STREAM) {
        const mnb::StreamConfig c =
            f16 ? mnb::gemv_stream_config(p->m, p->n, p->k, p->bits, p->block_size) : c32;
        out->waves_per_group = c.waves_per_group;
        out->tile_n = c.waves_per_group * (64 / c.g) * c.u;
        out->tile_m = c.mr;
        out->grid_x = c.groups;
        out->grid_y = (p->m + c.mr - 1) / c.mr;
    } else if (kern == MNB_KERNEL_BATCH_STREAM) {
        out->waves_per_group = bg.waves;
        out->tile_n = 16 * bg.s;
        out->tile_m = 16;
        out->grid_x = bg.gx;
        out->grid_y = 1;
    } else if (kern == MNB_KERNEL_STRIP_MFMA) {
        out->waves_per_group = sg.waves;
        out->tile_n = 16 * sg.strips;
        out->tile_m = 16;
        out->grid_x = sg.gx;
        out->grid_y = sg.gz;
    } else if (kern == MNB_KERNEL_GROUP_MFMA) {
        const mnb::GroupGeom g =
            mnb::group_geometry(p->m, p->n, p->k, 1, false, p->block_size, false);
        out->waves_per_group = g.waves;
        out->tile_n = 16;
        out->tile_m = 16 * g.mt;
        out->grid_x = g.gx;
        out->grid_y = g.gz;
    } else if (kern == MNB_KERNEL_GEMV_MFMA) {
        const mnb::GemvGeom g = mnb::gemv_geometry(p->m, p->n, p->k, p->bits, p->block_size);
        out->waves_per_group = g.waves;
        out->tile_n = 16;
        out->tile_m = 16 * g.mt;
        out->grid_x = g.gx;
        out->grid_y = g.gy;
    } else {
        out->waves_per_group = 4;
        out->tile_n = 4;
        out->tile_m = 4;
        out->grid_x = (p->n + 3) / 4;
        out->grid_y = (p->m + 3) / 4;
    }
    out->workspace_bytes = 0;
    return MNB_OK;
}

// The plan depends only on the problem and on MNB_FORCE_KERNEL, and a session asks for the same
// few shapes on every token -- twice per call (the workspace size, then the launch) -- so each
// thread keeps its last eight answers (the one-row search alone took 0.64 us per call on the
// host).  Only successful plans are kept: a failing problem is searched, and reported, anew.
int mnb_plan(const mnb_problem* p, mnb_plan_info* out) {
    if (!p || !out) return plan_search(p, out);
    struct Memo {
        mnb_problem p;
        int forced;
        mnb_plan_info info;
        bool used;
    };
    thread_local Memo memo[8];
    thread_local unsigned next = 0;
    const int forced = forced_kernel();
    for (const Memo& e : memo)
        if (e.used && e.forced == forced && std::memcmp(&e.p, p, sizeof(*p)) == 0) {
            *out = e.info;
            return MNB_OK;
        }
    const int rc = plan_search(p, out);
    if (rc == MNB_OK) memo[next++ & 7] = Memo{*p, forced, *out, true};
    return rc;
}

int mnb_workspace_bytes(const mnb_problem* p, size_t* bytes) {
    mnb_plan_info info;
    int rc = mnb_plan(p, &info);
    if (rc) return rc;
    if (!bytes) return fail(MNB_ERR_INVALID, "bytes is NULL");
    *bytes = (size_t)info.workspace_bytes;
    return MNB_OK;
}

}  // extern "C"

// mnb_matmul_nbits with, from the session layer, the node's strip-major copy of B
// (mnb_weights_prepack), which the batched decode kernel reads in place of B when it runs.
static int matmul_impl(const mnb_problem* p, const void* a, const uint8_t* b,
                       const uint8_t* b_strips, const void* scales, const uint8_t* zero_points,
                       void* y, void* workspace, size_t workspace_bytes, void* stream) {
    mnb_plan_info info;
    int rc = mnb_plan(p, &info);
    if (rc) return rc;
    if (p->m == 0) return MNB_OK;
    if (!a || !b || !scales || !y) return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    if (p->has_zero_points && !zero_points)
        return fail(MNB_ERR_INVALID, "has_zero_points is set but zero_points is NULL");
    if (!p->has_zero_points) zero_points = nullptr;
    // The prefill GEMM's workspace is optional: with less, it runs without splitting K.
    if (info.kernel != MNB_KERNEL_GEMM_MFMA &&
        ((size_t)info.workspace_bytes > workspace_bytes ||
         (info.workspace_bytes > 0 && !workspace)))
        return fail(MNB_ERR_INVALID, "workspace of %zu bytes is smaller than the %lld needed",
                    workspace_bytes, (long long)info.workspace_bytes);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e;
    int kern = info.kernel;
    // The MFMA path loads A in 16-byte and B in 16-byte units; fall back when a caller hands
    // over a sub-aligned view.
    if ((kern == MNB_KERNEL_GEMV_MFMA || kern == MNB_KERNEL_GEMV_STREAM ||
         kern == MNB_KERNEL_GEMM_MFMA || kern == MNB_KERNEL_GROUP_MFMA ||
         kern == MNB_KERNEL_STRIP_MFMA || kern == MNB_KERNEL_BATCH_STREAM) &&
        (!aligned(a, 16) || !aligned(b, 16)))
        kern = MNB_KERNEL_GENERIC;
    // A node with the MFMA-native strip copy: from 3 rows on the batched kernel reading it beats
    // the streaming GEMV on ORT's layout (Phi-3.5 set, same box, session calls: 3 rows qkv / o /
    // gate_up / down 6.82 / 4.44 / 9.00 / 6.41 us against 7.67 / 4.84 / 9.76 / 6.71; at 2 rows
    // the streaming GEMV stays ahead, 6.18 / 4.12 / 8.15 / 5.80 against 6.87 / 4.36 / 8.98 / 6.47).
    if (b_strips && kern == MNB_KERNEL_GEMV_STREAM && p->m >= 3 && forced_kernel() == 0) {
        mnb::BatchStreamGeom bg{};
        if (mnb::batch_stream_geometry(p->m, p->n, p->k, p->block_size, &bg))
            kern = MNB_KERNEL_BATCH_STREAM;
    }
    // The batched decode loads scales as 8-byte and zero points as 2-byte runs.
    if (kern == MNB_KERNEL_BATCH_STREAM &&
        !mnb::batch_stream_aligned(a, b, scales, zero_points)) {
        mnb::StripGeom sg{};
        kern = mnb::strip_geometry(p->n, p->k, 1, p->m, false, p->block_size,
                                   zero_points != nullptr, &sg)
                   ? MNB_KERNEL_STRIP_MFMA
                   : MNB_KERNEL_GROUP_MFMA;
    }
    // The GEMM's LDS DMA also fetches scales and zero points as aligned dwords; the row-tiled
    // GEMV (int4, block >= 32), else the 16-row MFMA GEMV or the generic kernel, takes any other
    // case of the same form.
    if (kern == MNB_KERNEL_STRIP_MFMA && !mnb::strip_gemv_aligned(a, b, scales, zero_points, false))
        kern = MNB_KERNEL_GROUP_MFMA;
    if (kern == MNB_KERNEL_GEMM_MFMA && p->dtype == MNB_DTYPE_F16 &&
        (!aligned(scales, 4) || !aligned(zero_points, 4) ||
         !mnb::gemm_supported(p->m, p->n, p->k, p->bits, p->block_size, zero_points != nullptr))) {
        if (mnb::group_gemv_supported(p->k, p->bits, p->block_size))
            kern = MNB_KERNEL_GROUP_MFMA;
        else if (mnb::gemv_supported(p->k, p->bits, p->block_size))
            kern = MNB_KERNEL_GEMV_MFMA;
        else
            kern = MNB_KERNEL_GENERIC;
    }
    if (kern == MNB_KERNEL_ACC4_I8 || kern == MNB_KERNEL_ACC4_STREAM) {
        // the int8 path reads B in 16-byte units and stages its own aligned copy of A
        if (!aligned(b, 16) || !aligned(workspace, 256))
            return fail(MNB_ERR_INVALID, "accuracy_level 4 needs B 16-byte and the workspace "
                                         "256-byte aligned");
        e = mnb::launch_acc4(a, p->dtype == MNB_DTYPE_F16, b, scales, zero_points, y, p->m,
                             p->n, p->k, p->bits, p->block_size, workspace, st, b_strips);
    } else if (kern == MNB_KERNEL_BATCH_STREAM) {
        mnb::BatchStreamGeom bg{};
        if (!mnb::batch_stream_geometry(p->m, p->n, p->k, p->block_size, &bg))
            return fail(MNB_ERR_UNSUPPORTED, "batched decode geometry");
        e = mnb::launch_batch_stream(bg, a, b, scales, zero_points, y, p->m, p->n, p->k,
                                     p->block_size, st, b_strips);
    } else if (kern == MNB_KERNEL_STRIP_MFMA) {
        mnb::StripGeom sg{};
        if (!mnb::strip_geometry(p->n, p->k, 1, p->m, false, p->block_size,
                                 zero_points != nullptr, &sg))
            return fail(MNB_ERR_UNSUPPORTED, "strip GEMV geometry");
        e = mnb::launch_strip_gemv(sg, false, a, nullptr, nullptr, nullptr, b, scales, zero_points, y,
                                   p->m, p->n, p->k, p->block_size, st);
    } else if (kern == MNB_KERNEL_GROUP_MFMA) {
        e = mnb::launch_group_gemv_f16(a, nullptr, nullptr, 1, p->m, b, scales, zero_points, y,
                                       p->m, p->n, p->k, p->bits, p->block_size, st);
    } else if (kern == MNB_KERNEL_GEMM_MFMA) {
        e = p->dtype == MNB_DTYPE_F16
                ? mnb::launch_gemm(a, b, scales, zero_points, y, p->m, p->n, p->k, p->bits,
                                   p->block_size, st, workspace, workspace_bytes)
                : mnb::launch_gemm_f32(a, b, scales, zero_points, y, p->m, p->n, p->k, p->bits,
                                       p->block_size, st);
    } else if (kern == MNB_KERNEL_GEMV_STREAM) {
        e = p->dtype == MNB_DTYPE_F16
                ? mnb::launch_gemv_stream(a, b, scales, zero_points, y, p->m, p->n, p->k, p->bits,
                                          p->block_size, st)
                : mnb::launch_gemv_stream_f32(a, b, scales, zero_points, y, p->m, p->n, p->k,
                                              p->bits, p->block_size, st);
    } else if (kern == MNB_KERNEL_GEMV_MFMA) {
        e = mnb::launch_gemv_f16(a, b, scales, zero_points, y, p->m, p->n, p->k, p->bits,
                                 p->block_size, st);
    } else {
        if (!aligned(b, 4)) return fail(MNB_ERR_INVALID, "B must be 4-byte aligned");
        e = mnb::launch_generic(a, b, scales, zero_points, y, p->m, p->n, p->k, p->bits,
                                p->block_size, p->dtype == MNB_DTYPE_F16, st);
    }
    if (e != hipSuccess) return hip_fail(e, "MatMulNBits kernel launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

extern "C" {

int mnb_matmul_nbits(const mnb_problem* p, const void* a, const uint8_t* b, const void* scales,
                     const uint8_t* zero_points, void* y, void* workspace,
                     size_t workspace_bytes, void* stream) {
    return matmul_impl(p, a, b, nullptr, scales, zero_points, y, workspace, workspace_bytes,
                       stream);
}

}  // extern "C"

// ---- allocation-free MatMulNBits ------------------------------------------------------------
//
// Scratch for mnb_matmul_nbits_noalloc: a file-scope device array, one copy per GPU the library
// runs on (held until the process ends).  Host code never passes `scratch` itself to a kernel or
// a copy -- in host code the name is a stand-in, not a device address -- but the address
// hipGetSymbolAddress returns for it on that device, looked up once per device.
namespace {
constexpr size_t kScratchBytes = (size_t)48 << 20;
constexpr int kScratchDevices = 64;
struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kScratchDevices];
}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
// The scratch array's address on `device` (made current for the lookup, then restored).
int scratch_on(int device, void** out) {
    if (device < 0 || device >= kScratchDevices)
        return fail(MNB_ERR_UNSUPPORTED, "device %d is beyond the %d devices the scratch table "
                                         "covers", device, kScratchDevices);
    ScratchSlot& slot = g_scratch[device];
    std::call_once(slot.once, [&] {
        int prev = -1;
        hipError_t e = hipGetDevice(&prev);
        if (e == hipSuccess && prev != device) e = hipSetDevice(device);
        if (e == hipSuccess) e = hipGetSymbolAddress(&slot.ptr, HIP_SYMBOL(scratch));
        if (prev >= 0 && prev != device) {
            const hipError_t r = hipSetDevice(prev);
            if (e == hipSuccess) e = r;
        }
        if (e == hipSuccess && !slot.ptr) e = hipErrorInvalidSymbol;
        slot.err = e;
    });
    if (slot.err != hipSuccess) return hip_fail(slot.err, "scratch address (hipGetSymbolAddress)");
    *out = slot.ptr;
    return MNB_OK;
}
}  // namespace

extern "C" {

size_t mnb_noalloc_scratch_bytes(void) { return kScratchBytes; }

int mnb_matmul_nbits_noalloc(const mnb_problem* p, const void* a, const uint8_t* b,
                             const void* scales, const uint8_t* zero_points, void* y,
                             void* stream) {
    mnb_plan_info info;
    int rc = mnb_plan(p, &info);
    if (rc) return rc;
    const size_t need = (size_t)info.workspace_bytes;
    // accuracy_level 4 needs its workspace; the prefill GEMM's is optional (without it the GEMM
    // runs unsplit along K)
    if ((info.kernel == MNB_KERNEL_ACC4_I8 || info.kernel == MNB_KERNEL_ACC4_STREAM) &&
        need > kScratchBytes)
        return fail(MNB_ERR_UNSUPPORTED, "accuracy_level 4 at M = %lld, N = %lld, K = %lld needs "
                    "%zu bytes of scratch; the allocation-free entry point holds %zu (call "
                    "mnb_matmul_nbits with a workspace instead)", (long long)p->m,
                    (long long)p->n, (long long)p->k, need, kScratchBytes);
    if (p->m == 0) return MNB_OK;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    if (need > 0 && need <= kScratchBytes) {
        int device = -1;
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const hipError_t e = st ? hipStreamGetDevice(st, &device) : hipGetDevice(&device);
        if (e != hipSuccess) return hip_fail(e, "device of the stream");
        rc = scratch_on(device, &ws);
        if (rc) return rc;
        ws_bytes = need;
    }
    return mnb_matmul_nbits(p, a, b, scales, zero_points, y, ws, ws_bytes, stream);
}

int mnb_dequantize_f16(int64_t n, int64_t k, int32_t bits, int32_t block_size,
                       const uint8_t* b, const void* scales_f16, const uint8_t* zero_points,
                       void* w_out_f16, void* stream) {
    mnb_problem p{};
    p.m = 1;
    p.n = n;
    p.k = k;
    p.bits = bits;
    p.block_size = block_size;
    p.dtype = MNB_DTYPE_F16;
    int rc = mnb_check_problem(&p);
    if (rc) return rc;
    if (!b || !scales_f16 || !w_out_f16) return fail(MNB_ERR_INVALID, "a NULL pointer was passed");
    if (!aligned(b, 4) || !aligned(w_out_f16, 16))
        return fail(MNB_ERR_INVALID, "B must be 4-byte and W 16-byte aligned");
    hipError_t e = mnb::launch_dequant_f16(b, scales_f16, zero_points, w_out_f16, n, k, bits,
                                           block_size, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

int mnb_quantize_a_int8(int64_t m, int64_t k, int32_t block_size, int32_t dtype, const void* a,
                        int8_t* qa, float* a_scale, int32_t* qsum, void* stream) {
    if (m < 0 || k <= 0) return fail(MNB_ERR_INVALID, "M = %lld, K = %lld", (long long)m, (long long)k);
    if (block_size != 16 && block_size != 32 && block_size != 64 && block_size != 128)
        return fail(MNB_ERR_UNSUPPORTED, "block_size = %d", block_size);
    if (k % block_size) return fail(MNB_ERR_INVALID, "K is not a multiple of block_size");
    if (dtype != MNB_DTYPE_F16 && dtype != MNB_DTYPE_F32)
        return fail(MNB_ERR_UNSUPPORTED, "dtype %d", dtype);
    if (m == 0) return MNB_OK;
    if (!a || !qa || !a_scale) return fail(MNB_ERR_INVALID, "a NULL pointer was passed");
    hipError_t e = mnb::launch_quantize_a_int8(a, dtype == MNB_DTYPE_F16, qa, a_scale, qsum,
                                               false, m, k, block_size,
                                               static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

int mnb_moe_grouped(const mnb_moe_problem* p, const void* a, const int32_t* row_index,
                    const int32_t* offsets, const uint8_t* b, const void* scales,
                    const uint8_t* zero_points, void* y, void* stream) {
    if (!p) return fail(MNB_ERR_INVALID, "problem is NULL");
    mnb_problem q{};
    q.m = p->total_rows;
    q.n = p->n;
    q.k = p->k;
    q.bits = p->bits;
    q.block_size = p->block_size;
    q.has_zero_points = p->has_zero_points;
    q.dtype = p->dtype;
    int rc = mnb_check_problem(&q);
    if (rc) return rc;
    if (p->dtype != MNB_DTYPE_F16 || !mnb::group_gemv_supported(p->k, p->bits, p->block_size))
        return fail(MNB_ERR_UNSUPPORTED, "the grouped kernel is fp16, bits = 4, block_size >= 32, "
                                         "K %% 32 == 0");
    if (p->num_experts < 0 || p->num_experts > 65535 || p->max_rows_per_expert < 0 ||
        p->a_rows < 0 || p->total_rows < 0)
        return fail(MNB_ERR_INVALID, "negative or oversized expert/row counts");
    if (p->total_rows == 0 || p->num_experts == 0) return MNB_OK;
    if (!a || !row_index || !offsets || !b || !scales || !y)
        return fail(MNB_ERR_INVALID, "a NULL pointer was passed");
    if (p->has_zero_points && !zero_points)
        return fail(MNB_ERR_INVALID, "has_zero_points is set but zero_points is NULL");
    if (!aligned(a, 16) || !aligned(b, 16))
        return fail(MNB_ERR_INVALID, "A and B must be 16-byte aligned");
    hipError_t e = mnb::launch_group_gemv_f16(a, row_index, offsets, p->num_experts,
                                              p->max_rows_per_expert, b, scales,
                                              p->has_zero_points ? zero_points : nullptr, y,
                                              p->total_rows, p->n, p->k, p->bits, p->block_size,
                                              static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "grouped MatMulNBits launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

// ---- fused QMoE ---------------------------------------------------------------------------

static mnb::QmoeArgs qmoe_args(const mnb_qmoe_problem* p) {
    mnb::QmoeArgs q{};
    q.rows = p->rows;
    q.hidden = p->hidden;
    q.inter = p->inter;
    q.experts = p->num_experts;
    q.k = p->k;
    q.block_size = p->block_size;
    q.fusion = p->swiglu_fusion;
    q.normalize = p->normalize_routing ? 1 : 0;
    q.has_limit = p->has_swiglu_limit ? 1 : 0;
    q.router_f32 = p->router_dtype == MNB_DTYPE_F32 ? 1 : 0;
    q.alpha = p->activation_alpha;
    q.beta = p->activation_beta;
    q.limit = p->swiglu_limit;
    return q;
}

int mnb_qmoe_check(const mnb_qmoe_problem* p) {
    if (!p) return fail(MNB_ERR_INVALID, "problem is NULL");
    if (p->rows < 0) return fail(MNB_ERR_INVALID, "rows = %lld is negative", (long long)p->rows);
    if (p->num_experts < 1 || p->num_experts > 1024)
        return fail(MNB_ERR_UNSUPPORTED, "num_experts = %lld; this library routes 1..1024",
                    (long long)p->num_experts);
    if (p->k < 1 || p->k > 8 || p->k > p->num_experts)
        return fail(MNB_ERR_UNSUPPORTED, "k = %d; this library routes 1..min(8, E)", p->k);
    if (p->rows * p->k > 16384)
        return fail(MNB_ERR_UNSUPPORTED, "rows * k = %lld exceeds 16384",
                    (long long)(p->rows * p->k));
    if (p->block_size != 32 && p->block_size != 64 && p->block_size != 128)
        return fail(MNB_ERR_UNSUPPORTED, "block_size = %d; the expert kernels take 32/64/128",
                    p->block_size);
    if (p->hidden <= 0 || p->inter <= 0 || p->hidden % 32 || p->inter % 32 ||
        p->hidden % p->block_size || p->inter % p->block_size)
        return fail(MNB_ERR_UNSUPPORTED, "hidden = %lld and inter = %lld must be positive "
                    "multiples of 32 and of block_size", (long long)p->hidden, (long long)p->inter);
    if (p->hidden >= (1ll << 31) || 2 * p->inter >= (1ll << 31))
        return fail(MNB_ERR_UNSUPPORTED, "extents do not fit 32 bits");
    if (p->swiglu_fusion != 1 && p->swiglu_fusion != 2)
        return fail(MNB_ERR_UNSUPPORTED, "swiglu_fusion = %d; this library implements 1 "
                    "(interleaved) and 2 (concatenated)", p->swiglu_fusion);
    if (p->dtype != MNB_DTYPE_F16) return fail(MNB_ERR_UNSUPPORTED, "QMoE runs fp16 tensors");
    if (p->router_dtype != MNB_DTYPE_F16 && p->router_dtype != MNB_DTYPE_F32)
        return fail(MNB_ERR_INVALID, "router dtype %d", p->router_dtype);
    if (!std::isfinite(p->activation_alpha) || !std::isfinite(p->activation_beta) ||
        (p->has_swiglu_limit && !std::isfinite(p->swiglu_limit)))
        return fail(MNB_ERR_INVALID, "activation_alpha, activation_beta and swiglu_limit must be "
                                     "finite");
    return MNB_OK;
}

int mnb_qmoe_workspace_bytes(const mnb_qmoe_problem* p, size_t* bytes) {
    if (!bytes) return fail(MNB_ERR_INVALID, "bytes is NULL");
    *bytes = 0;
    const int rc = mnb_qmoe_check(p);
    if (rc) return rc;
    *bytes = mnb::qmoe_workspace_bytes(qmoe_args(p));
    return MNB_OK;
}

}  // extern "C"

// mnb_qmoe with, from the session layer, strip-major copies of the expert weights
// (mnb_qmoe_weights_prepack), which the strip GEMV reads in place of fc1 / fc2 when it runs.
static int qmoe_impl(const mnb_qmoe_problem* p, const void* x, const void* router_logits,
                     const uint8_t* fc1_weights, const void* fc1_scales, const void* fc1_bias,
                     const uint8_t* fc2_weights, const void* fc2_scales, const void* fc2_bias,
                     void* y, void* workspace, size_t workspace_bytes, void* stream,
                     const uint8_t* fc1_strips, const uint8_t* fc2_strips) {
    int rc = mnb_qmoe_check(p);
    if (rc) return rc;
    if (p->rows == 0) return MNB_OK;
    if (!x || !router_logits || !fc1_weights || !fc1_scales || !fc2_weights || !fc2_scales || !y)
        return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    const mnb::QmoeArgs q = qmoe_args(p);
    const size_t need = mnb::qmoe_workspace_bytes(q);
    if (!workspace || workspace_bytes < need)
        return fail(MNB_ERR_INVALID, "workspace holds %zu bytes, QMoE needs %zu", workspace_bytes,
                    need);
    if (!aligned(workspace, 256)) return fail(MNB_ERR_INVALID, "workspace must be 256-byte aligned");
    if (!aligned(x, 16) || !aligned(fc1_weights, 16) || !aligned(fc2_weights, 16) ||
        !aligned(y, 16) || (fc1_bias && !aligned(fc1_bias, 16)) ||
        (fc2_bias && !aligned(fc2_bias, 16)))
        return fail(MNB_ERR_INVALID, "x, y, the weights and the biases must be 16-byte aligned");
    hipError_t e = mnb::launch_qmoe(q, x, router_logits, fc1_weights, fc1_scales, fc1_bias,
                                    fc2_weights, fc2_scales, fc2_bias, y, workspace,
                                    static_cast<hipStream_t>(stream), fc1_strips, fc2_strips);
    if (e != hipSuccess) return hip_fail(e, "QMoE launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

extern "C" {

int mnb_qmoe(const mnb_qmoe_problem* p, const void* x, const void* router_logits,
             const uint8_t* fc1_weights, const void* fc1_scales, const void* fc1_bias,
             const uint8_t* fc2_weights, const void* fc2_scales, const void* fc2_bias, void* y,
             void* workspace, size_t workspace_bytes, void* stream) {
    return qmoe_impl(p, x, router_logits, fc1_weights, fc1_scales, fc1_bias, fc2_weights,
                     fc2_scales, fc2_bias, y, workspace, workspace_bytes, stream, nullptr,
                     nullptr);
}

// ---- RMSNorm --------------------------------------------------------------------------------

int mnb_rmsnorm_check(const mnb_rmsnorm_problem* p) {
    if (!p) return fail(MNB_ERR_INVALID, "problem is NULL");
    if (p->rows < 0) return fail(MNB_ERR_INVALID, "rows = %lld is negative", (long long)p->rows);
    if (p->dtype != MNB_DTYPE_F16 && p->dtype != MNB_DTYPE_F32)
        return fail(MNB_ERR_INVALID, "dtype %d", p->dtype);
    if (!mnb::rmsnorm_supported(p->hidden, p->dtype == MNB_DTYPE_F16))
        return fail(MNB_ERR_UNSUPPORTED, "hidden = %lld: a positive multiple of %d up to %d",
                    (long long)p->hidden, p->dtype == MNB_DTYPE_F16 ? 8 : 4,
                    p->dtype == MNB_DTYPE_F16 ? 8192 : 4096);
    if (!std::isfinite(p->epsilon) || p->epsilon < 0.f)
        return fail(MNB_ERR_INVALID, "epsilon must be finite and non-negative");
    if (p->has_bias && !p->has_skip)
        return fail(MNB_ERR_INVALID, "a bias comes with the skip input");
    return MNB_OK;
}

int mnb_skip_rmsnorm(const mnb_rmsnorm_problem* p, const void* x, const void* skip,
                     const void* gamma, const void* bias, void* y, void* sum_out, void* stream) {
    int rc = mnb_rmsnorm_check(p);
    if (rc) return rc;
    if (p->rows == 0) return MNB_OK;
    if (!x || !gamma || !y || (p->has_skip && !skip) || (p->has_bias && !bias) ||
        (p->want_sum && !sum_out))
        return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    for (const void* q : {x, skip, gamma, bias, static_cast<const void*>(y),
                          static_cast<const void*>(sum_out)})
        if (q && !aligned(q, 16)) return fail(MNB_ERR_INVALID, "tensors must be 16-byte aligned");
    hipError_t e = mnb::launch_skip_rmsnorm(x, p->has_skip ? skip : nullptr, gamma,
                                            p->has_bias ? bias : nullptr, y,
                                            p->want_sum ? sum_out : nullptr, p->rows, p->hidden,
                                            p->epsilon, p->dtype == MNB_DTYPE_F16,
                                            static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "RMSNorm launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

// ---- GroupQueryAttention ----------------------------------------------------------------------

static mnb::GqaArgs gqa_args(const mnb_gqa_problem* p, bool copy_past) {
    mnb::GqaArgs a{};
    a.batch = p->batch;
    a.seq = p->seq_len;
    a.past_stride = p->past_len_max;
    a.present_len = p->present_len;
    a.max_seq = p->max_seq;
    a.nq = p->num_heads;
    a.nkv = p->kv_num_heads;
    a.d = p->head_dim;
    a.rot = p->rotary_dim;
    a.scale = p->scale;
    a.copy_past = copy_past;
    return a;
}

int mnb_gqa_check(const mnb_gqa_problem* p) {
    if (!p) return fail(MNB_ERR_INVALID, "problem is NULL");
    if (p->batch < 0 || p->seq_len < 0 || p->past_len_max < 0 || p->present_len < 0)
        return fail(MNB_ERR_INVALID, "batch, seq_len, past_len_max and present_len must be >= 0");
    if (p->dtype != MNB_DTYPE_F16)
        return fail(MNB_ERR_UNSUPPORTED, "GroupQueryAttention runs fp16 tensors");
    if (p->num_heads < 1 || p->kv_num_heads < 1 || p->num_heads % p->kv_num_heads)
        return fail(MNB_ERR_UNSUPPORTED, "num_heads = %d and kv_num_heads = %d; num_heads must "
                    "be a positive multiple of kv_num_heads", p->num_heads, p->kv_num_heads);
    if (!mnb::gqa_supported(p->head_dim))
        return fail(MNB_ERR_UNSUPPORTED, "head_dim = %d; this library takes multiples of 16 up "
                    "to 256", p->head_dim);
    if (p->rotary_dim < 2 || p->rotary_dim % 2 || p->rotary_dim > p->head_dim)
        return fail(MNB_ERR_INVALID, "rotary_dim = %d is not an even value in 2..head_dim = %d",
                    p->rotary_dim, p->head_dim);
    if (p->max_seq < 1) return fail(MNB_ERR_INVALID, "max_seq = %lld", (long long)p->max_seq);
    if (p->present_len < p->past_len_max + p->seq_len && p->present_len != p->past_len_max)
        return fail(MNB_ERR_INVALID, "present length %lld is neither the shared-buffer extent "
                    "(%lld) nor the growing-cache extent (%lld + %lld or more)",
                    (long long)p->present_len, (long long)p->past_len_max,
                    (long long)p->past_len_max, (long long)p->seq_len);
    if (!std::isfinite(p->scale)) return fail(MNB_ERR_INVALID, "scale is not finite");
    const double heads = (double)p->num_heads + 2.0 * p->kv_num_heads;
    if ((double)p->batch * p->seq_len * heads * p->head_dim >= (double)(1ll << 40) ||
        (double)p->batch * p->kv_num_heads * (p->present_len + p->past_len_max) * p->head_dim >=
            (double)(1ll << 40) ||
        (double)p->batch * p->num_heads * p->seq_len >= (double)(1ll << 31))
        return fail(MNB_ERR_UNSUPPORTED, "extents too large");
    return MNB_OK;
}

int mnb_gqa_workspace_bytes(const mnb_gqa_problem* p, size_t* bytes) {
    if (!bytes) return fail(MNB_ERR_INVALID, "bytes is NULL");
    *bytes = 0;
    const int rc = mnb_gqa_check(p);
    if (rc) return rc;
    if (p->batch && p->seq_len) *bytes = mnb::gqa_workspace_bytes(gqa_args(p, false));
    return MNB_OK;
}

int mnb_gqa(const mnb_gqa_problem* p, const void* packed_qkv, const void* past_key,
            const void* past_value, const int32_t* seqlens_k, const void* cos_cache,
            const void* sin_cache, void* attn_out, void* present_key, void* present_value,
            void* workspace, size_t workspace_bytes, void* stream) {
    int rc = mnb_gqa_check(p);
    if (rc) return rc;
    if (p->batch == 0 || p->seq_len == 0) return MNB_OK;
    if (!packed_qkv || !seqlens_k || !cos_cache || !sin_cache || !attn_out ||
        (p->past_len_max && (!past_key || !past_value)) ||
        (p->present_len && (!present_key || !present_value)))
        return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    const bool alias_k = p->past_len_max && present_key == past_key;
    const bool alias_v = p->past_len_max && present_value == past_value;
    if (alias_k != alias_v)
        return fail(MNB_ERR_INVALID, "present_key and present_value must both alias their past "
                                     "tensors or neither");
    if (alias_k && p->present_len != p->past_len_max)
        return fail(MNB_ERR_INVALID, "present aliases past but present length %lld differs from "
                    "the past buffer's %lld", (long long)p->present_len,
                    (long long)p->past_len_max);
    for (const void* q : {packed_qkv, past_key, past_value, static_cast<const void*>(attn_out),
                          static_cast<const void*>(present_key),
                          static_cast<const void*>(present_value)})
        if (q && !aligned(q, 16)) return fail(MNB_ERR_INVALID, "tensors must be 16-byte aligned");
    const mnb::GqaArgs a = gqa_args(p, !alias_k);
    const size_t need = mnb::gqa_workspace_bytes(a);
    if (!workspace || workspace_bytes < need)
        return fail(MNB_ERR_INVALID, "workspace holds %zu bytes, GroupQueryAttention needs %zu",
                    workspace_bytes, need);
    if (!aligned(workspace, 256)) return fail(MNB_ERR_INVALID, "workspace must be 256-byte aligned");
    hipError_t e = mnb::launch_gqa(a, packed_qkv, past_key, past_value, seqlens_k, cos_cache,
                                   sin_cache, attn_out, present_key, present_value, workspace,
                                   static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "GroupQueryAttention launch");
    g_launches.fetch_add(1);
    return MNB_OK;
}

// ---- session layer ------------------------------------------------------------------------

struct mnb_session {
    int device = 0;
    hipStream_t stream = nullptr;
    bool async = false;             // device-only calls return once enqueued
    std::mutex mu;
    void* a_dev = nullptr;
    size_t a_cap = 0;
    void* y_dev = nullptr;
    size_t y_cap = 0;
    void* ws = nullptr;
    size_t ws_cap = 0;
    // Pinned host staging of host tensors (HostIo), and its device-side address
    void* pin = nullptr;
    void* pin_dev = nullptr;
    size_t pin_cap = 0;
};

struct mnb_weights {
    mnb_session* s = nullptr;
    mnb_problem node{};
    uint8_t* b = nullptr;
    void* scales = nullptr;
    uint8_t* zp = nullptr;
    uint8_t* strips = nullptr;   // strip-major copy of B (mnb_weights_prepack), or null
};

int mnb_device_count(int* count) {
    if (!count) return fail(MNB_ERR_INVALID, "count is NULL");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) {
        *count = 0;
        return hip_fail(e, "hipGetDeviceCount");
    }
    *count = c;
    return MNB_OK;
}

int mnb_device_arch(int device_index, char* buf, size_t len) {
    if (!buf || len == 0) return fail(MNB_ERR_INVALID, "buffer is NULL or empty");
    buf[0] = '\0';
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device_index);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    std::snprintf(buf, len, "%s", prop.gcnArchName);
    return MNB_OK;
}

int mnb_device_malloc(int device_index, size_t bytes, void** out) {
    if (!out) return fail(MNB_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (bytes == 0) return MNB_OK;
    hipError_t e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        *out = nullptr;
        return fail(MNB_ERR_NOMEM, "hipMalloc(%zu) on device %d: %s", bytes, device_index,
                    hipGetErrorString(e));
    }
    return MNB_OK;
}

int mnb_device_free(int device_index, void* p) {
    if (!p) return MNB_OK;
    hipError_t e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    e = hipFree(p);
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipFree");
}

int mnb_memcpy(int device_index, void* dst, const void* src, size_t bytes, int kind) {
    if (bytes == 0) return MNB_OK;
    if (!dst || !src) return fail(MNB_ERR_INVALID, "a NULL copy pointer was passed");
    hipMemcpyKind k;
    switch (kind) {
        case MNB_COPY_HOST_TO_DEVICE: k = hipMemcpyHostToDevice; break;
        case MNB_COPY_DEVICE_TO_HOST: k = hipMemcpyDeviceToHost; break;
        case MNB_COPY_DEVICE_TO_DEVICE: k = hipMemcpyDeviceToDevice; break;
        default: return fail(MNB_ERR_INVALID, "copy kind %d", kind);
    }
    hipError_t e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    e = hipMemcpy(dst, src, bytes, k);
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipMemcpy");
}

int mnb_session_create(int device_index, mnb_session** out) {
    if (!out) return fail(MNB_ERR_INVALID, "out is NULL");
    *out = nullptr;
    int c = 0;
    int rc = mnb_device_count(&c);
    if (rc) return rc;
    if (device_index < 0 || device_index >= c)
        return fail(MNB_ERR_INVALID, "device index %d outside [0, %d)", device_index, c);
    hipError_t e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    mnb_session* s = new (std::nothrow) mnb_session();
    if (!s) return fail(MNB_ERR_NOMEM, "session allocation failed");
    s->device = device_index;
    e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipStreamCreateWithFlags");
    }
    *out = s;
    return MNB_OK;
}

int mnb_session_destroy(mnb_session* s) {
    if (!s) return MNB_OK;
    (void)hipSetDevice(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->a_dev) (void)hipFree(s->a_dev);
    if (s->y_dev) (void)hipFree(s->y_dev);
    if (s->ws) (void)hipFree(s->ws);
    if (s->pin) (void)hipHostFree(s->pin);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return MNB_OK;
}

void* mnb_session_stream(mnb_session* s) { return s ? static_cast<void*>(s->stream) : nullptr; }

int mnb_session_synchronize(mnb_session* s) {
    if (!s) return fail(MNB_ERR_INVALID, "session is NULL");
    (void)hipSetDevice(s->device);
    hipError_t e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipStreamSynchronize");
}

int mnb_session_set_async(mnb_session* s, int enabled) {
    if (!s) return fail(MNB_ERR_INVALID, "session is NULL");
    std::lock_guard<std::mutex> lk(s->mu);
    s->async = enabled != 0;
    return MNB_OK;
}

int mnb_memcpy_on_stream(int device_index, void* dst, const void* src, size_t bytes, int kind,
                         void* stream) {
    if (bytes == 0) return MNB_OK;
    if (!dst || !src) return fail(MNB_ERR_INVALID, "a NULL copy pointer was passed");
    hipMemcpyKind k;
    switch (kind) {
        case MNB_COPY_HOST_TO_DEVICE: k = hipMemcpyHostToDevice; break;
        case MNB_COPY_DEVICE_TO_HOST: k = hipMemcpyDeviceToHost; break;
        case MNB_COPY_DEVICE_TO_DEVICE: k = hipMemcpyDeviceToDevice; break;
        default: return fail(MNB_ERR_INVALID, "copy kind %d", kind);
    }
    hipError_t e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    e = hipMemcpyAsync(dst, src, bytes, k, st);
    // host memory involved: complete before returning (the caller may reuse or read it)
    if (e == hipSuccess && kind != MNB_COPY_DEVICE_TO_DEVICE) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipMemcpyAsync");
}

int mnb_stream_synchronize(int device_index, void* stream) {
    hipError_t e = hipSetDevice(device_index);
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipStreamSynchronize");
}

int mnb_device_synchronize(int device_index) {
    hipError_t e = hipSetDevice(device_index);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipDeviceSynchronize");
}

int mnb_event_create(int device_index, void** event) {
    if (!event) return fail(MNB_ERR_INVALID, "event is NULL");
    *event = nullptr;
    hipError_t e = hipSetDevice(device_index);
    hipEvent_t ev = nullptr;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags");
    *event = ev;
    return MNB_OK;
}

int mnb_event_destroy(void* event) {
    if (!event) return MNB_OK;
    const hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipEventDestroy");
}

int mnb_event_record(void* event, void* stream) {
    if (!event) return fail(MNB_ERR_INVALID, "event is NULL");
    const hipError_t e =
        hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipEventRecord");
}

int mnb_stream_wait_event(void* stream, void* event) {
    if (!event) return fail(MNB_ERR_INVALID, "event is NULL");
    const hipError_t e =
        hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0);
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipStreamWaitEvent");
}

int mnb_event_synchronize(void* event) {
    if (!event) return fail(MNB_ERR_INVALID, "event is NULL");
    const hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(event));
    return e == hipSuccess ? MNB_OK : hip_fail(e, "hipEventSynchronize");
}

static int grow(void** p, size_t* cap, size_t need) {
    if (need <= *cap) return MNB_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    hipError_t e = counted_malloc(p, need);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(MNB_ERR_NOMEM, "hipMalloc(%zu): %s", need, hipGetErrorString(e));
    }
    *cap = need;
    return MNB_OK;
}

// A session buffer of at least `need` bytes.  In async mode, work already enqueued on the
// session's stream may still use the old buffer: the stream is drained before it is freed.
static int sgrow(mnb_session* s, void** p, size_t* cap, size_t need) {
    if (need <= *cap) return MNB_OK;
    if (s->async && *p) {
        const hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    }
    return grow(p, cap, need);
}

// The session's pinned staging buffer, at least `need` bytes.  The stream is drained before an
// old buffer is freed: a copy enqueued from it may still run.
static int pin_grow(mnb_session* s, size_t need) {
    if (need <= s->pin_cap) return MNB_OK;
    if (s->pin) {
        const hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void)hipHostFree(s->pin);
    }
    s->pin = s->pin_dev = nullptr;
    s->pin_cap = 0;
    hipError_t e = counted_host_malloc(&s->pin, need);
    if (e != hipSuccess) {
        s->pin = nullptr;
        return fail(MNB_ERR_NOMEM, "hipHostMalloc(%zu): %s", need, hipGetErrorString(e));
    }
    e = hipHostGetDevicePointer(&s->pin_dev, s->pin, 0);
    if (e != hipSuccess) {
        (void)hipHostFree(s->pin);
        s->pin = s->pin_dev = nullptr;
        return hip_fail(e, "hipHostGetDevicePointer");
    }
    s->pin_cap = need;
    return MNB_OK;
}

// The host tensors of one session call.  Inputs are copied on the CPU into the session's pinned
// buffer and moved to their device staging by one copy launch; outputs are moved into the pinned
// buffer by one launch after the node's kernels and copied out on the CPU once the stream has
// drained.  So a call is upload launch -> kernels -> download launch -> one synchronisation,
// instead of a runtime copy per tensor.  Use: in() / out() for every host tensor, upload(), the
// kernels, download(), end().
struct HostIo {
    mnb_session* s;
    mnb::StageList up{}, down{};
    const void* in_host[mnb::kMaxStageSegs] = {};
    void* out_host[mnb::kMaxStageSegs] = {};
    size_t in_off[mnb::kMaxStageSegs] = {}, out_off[mnb::kMaxStageSegs] = {};
    size_t total = 0;
    bool enqueued = false;

    explicit HostIo(mnb_session* sess) : s(sess) {}
    bool any() const { return up.n + down.n > 0; }
    static size_t slot(size_t b) { return (b + 255) & ~(size_t)255; }
    void in(const void* host, void* dev, size_t bytes) {
        in_off[up.n] = total;
        in_host[up.n] = host;
        up.seg[up.n++] = {nullptr, dev, bytes};
        total += slot(bytes);
    }
    void out(void* host, const void* dev, size_t bytes) {
        out_off[down.n] = total;
        out_host[down.n] = host;
        down.seg[down.n++] = {dev, nullptr, bytes};
        total += slot(bytes);
    }
    int upload() {
        if (!any()) return MNB_OK;
        int rc = pin_grow(s, total);
        if (rc) return rc;
        uint8_t* ph = static_cast<uint8_t*>(s->pin);
        uint8_t* pd = static_cast<uint8_t*>(s->pin_dev);
        for (int i = 0; i < up.n; ++i) {
            std::memcpy(ph + in_off[i], in_host[i], up.seg[i].bytes);
            up.seg[i].src = pd + in_off[i];
        }
        for (int i = 0; i < down.n; ++i) down.seg[i].dst = pd + out_off[i];
        enqueued = true;
        const hipError_t e = mnb::launch_stage_copy(up, s->stream);
        return e == hipSuccess ? MNB_OK : hip_fail(e, "host input upload");
    }
    int download() {
        const hipError_t e = mnb::launch_stage_copy(down, s->stream);
        return e == hipSuccess ? MNB_OK : hip_fail(e, "host output download");
    }
    // The call's end: `rc` is its status so far.  Host tensors are complete when this returns;
    // after a failure the stream is still drained, so no copy reads the pinned buffer later.
    int end(int rc) {
        if (rc) {
            if (enqueued) (void)hipStreamSynchronize(s->stream);
            return rc;
        }
        if (!any()) {
            if (s->async) return MNB_OK;
            const hipError_t e = hipStreamSynchronize(s->stream);
            return e == hipSuccess ? MNB_OK : hip_fail(e, "hipStreamSynchronize");
        }
        const hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        const uint8_t* ph = static_cast<const uint8_t*>(s->pin);
        for (int i = 0; i < down.n; ++i) std::memcpy(out_host[i], ph + out_off[i], down.seg[i].bytes);
        return MNB_OK;
    }
};

int mnb_weights_upload(mnb_session* s, const mnb_problem* node, const void* b_host,
                       size_t b_bytes, const void* scales_host, size_t scales_bytes,
                       const void* zp_host, size_t zp_bytes, mnb_weights** out) {
    if (!s || !node || !out) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    *out = nullptr;
    mnb_problem p = *node;
    p.m = 0;
    int rc = mnb_check_problem(&p);
    if (rc) return rc;
    const size_t want_b = (size_t)b_bytes_of(&p);
    const size_t want_s = (size_t)(p.n * bpc_of(&p) * elem_bytes(p.dtype));
    const size_t want_z = (size_t)(p.n * zp_bytes_per_col(&p));
    if (!b_host || b_bytes != want_b)
        return fail(MNB_ERR_INVALID, "B holds %zu bytes, the layout needs %zu", b_bytes, want_b);
    if (!scales_host || scales_bytes != want_s)
        return fail(MNB_ERR_INVALID, "scales hold %zu bytes, the layout needs %zu", scales_bytes,
                    want_s);
    if (p.has_zero_points && (!zp_host || zp_bytes != want_z))
        return fail(MNB_ERR_INVALID, "zero_points hold %zu bytes, the layout needs %zu", zp_bytes,
                    want_z);
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    mnb_weights* w = new (std::nothrow) mnb_weights();
    if (!w) return fail(MNB_ERR_NOMEM, "weights allocation failed");
    w->s = s;
    w->node = p;
    hipError_t e = counted_malloc(&w->b, want_b);
    if (e == hipSuccess) e = counted_malloc(&w->scales, want_s);
    if (e == hipSuccess && p.has_zero_points) e = counted_malloc(&w->zp, want_z);
    if (e == hipSuccess) e = hipMemcpyAsync(w->b, b_host, want_b, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(w->scales, scales_host, want_s, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess && p.has_zero_points)
        e = hipMemcpyAsync(w->zp, zp_host, want_z, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        if (w->b) (void)hipFree(w->b);
        if (w->scales) (void)hipFree(w->scales);
        if (w->zp) (void)hipFree(w->zp);
        delete w;
        return hip_fail(e, "weight upload");
    }
    *out = w;
    return MNB_OK;
}

int mnb_weights_release(mnb_weights* w) {
    if (!w) return MNB_OK;
    (void)hipSetDevice(w->s->device);
    (void)hipStreamSynchronize(w->s->stream);
    if (w->b) (void)hipFree(w->b);
    if (w->scales) (void)hipFree(w->scales);
    if (w->zp) (void)hipFree(w->zp);
    if (w->strips) (void)hipFree(w->strips);
    delete w;
    return MNB_OK;
}

int mnb_weights_prepack(mnb_weights* w, int64_t* bytes) {
    if (bytes) *bytes = 0;
    if (!w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    const mnb_problem& p = w->node;
    // the kernels that read the copy: the batched decode kernel, and at accuracy_level 4 the
    // strip-per-workgroup int8 GEMV
    mnb::BatchStreamGeom bg{};
    mnb::Acc4StreamGeom ag{};
    const bool reader =
        p.dtype == MNB_DTYPE_F16 && p.bits == 4 &&
        (p.accuracy_level == 4 ? mnb::acc4_stream_geometry(16, p.n, p.k, p.block_size, &ag)
                               : mnb::batch_stream_geometry(16, p.n, p.k, p.block_size, &bg));
    if (!reader)
        return fail(MNB_ERR_UNSUPPORTED,
                    "no strip-major layout for this node: the kernels that read it take fp16 "
                    "A, 4-bit B, K %% 128 == 0 and blocks of 32, 64 or 128 with whole groups of "
                    "four (and K <= 8192 at accuracy_level 4) (N=%lld K=%lld bits=%d "
                    "block_size=%d level=%d)",
                    (long long)p.n, (long long)p.k, p.bits, p.block_size, p.accuracy_level);
    const int64_t nb = mnb::strip_pack_bytes(p.n, p.k);
    std::lock_guard<std::mutex> lk(w->s->mu);
    (void)hipSetDevice(w->s->device);
    if (!w->strips) {
        uint8_t* d = nullptr;
        hipError_t e = counted_malloc(&d, (size_t)nb);
        if (e != hipSuccess)
            return fail(MNB_ERR_NOMEM, "hipMalloc(%lld) for the strip-major copy: %s",
                        (long long)nb, hipGetErrorString(e));
        // the MFMA order of the kernel that reads the copy: the batched fp16 kernel (level 0)
        // or the int8 kernel (level 4)
        e = mnb::launch_strip_pack(w->b, d, p.n, p.k, w->s->stream, 1,
                                   p.accuracy_level == 4 ? mnb::kStripMfmaI8 : mnb::kStripMfmaF16);
        if (e == hipSuccess) e = hipStreamSynchronize(w->s->stream);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(e, "strip-major copy");
        }
        w->strips = d;
    }
    if (bytes) *bytes = nb;
    return MNB_OK;
}

static int run_locked(mnb_session* s, const mnb_weights* w, int64_t m, const void* a_dev,
                      void* y_dev) {
    mnb_problem p = w->node;
    p.m = m;
    size_t ws = 0;
    int rc = mnb_workspace_bytes(&p, &ws);
    if (rc) return rc;
    if (ws) {
        rc = sgrow(s, &s->ws, &s->ws_cap, ws);
        if (rc) return rc;
    }
    return matmul_impl(&p, a_dev, w->b, w->strips, w->scales, w->zp, y_dev, s->ws, s->ws_cap,
                       s->stream);
}

int mnb_session_run_device(mnb_session* s, const mnb_weights* w, int64_t m, const void* a_dev,
                           void* y_dev) {
    if (!s || !w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    return run_locked(s, w, m, a_dev, y_dev);
}

int mnb_session_run(mnb_session* s, const mnb_weights* w, int64_t m, const void* a,
                    int a_on_device, void* y, int y_on_device) {
    if (!s || !w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    if (m < 0) return fail(MNB_ERR_INVALID, "M = %lld is negative", (long long)m);
    if (m == 0) return MNB_OK;
    if (!a || !y) return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    const size_t eb = (size_t)elem_bytes(w->node.dtype);
    const size_t a_bytes = (size_t)m * (size_t)w->node.k * eb;
    const size_t y_bytes = (size_t)m * (size_t)w->node.n * eb;
    const void* a_dev = a;
    void* y_dev = y;
    int rc;
    HostIo io(s);
    if (!a_on_device) {
        rc = sgrow(s, &s->a_dev, &s->a_cap, a_bytes);
        if (rc) return rc;
        io.in(a, s->a_dev, a_bytes);
        a_dev = s->a_dev;
    }
    if (!y_on_device) {
        rc = sgrow(s, &s->y_dev, &s->y_cap, y_bytes);
        if (rc) return rc;
        io.out(y, s->y_dev, y_bytes);
        y_dev = s->y_dev;
    }
    rc = io.upload();
    if (!rc) rc = run_locked(s, w, m, a_dev, y_dev);
    if (!rc) rc = io.download();
    return io.end(rc);
}

struct mnb_qmoe_weights {
    mnb_session* s = nullptr;
    mnb_qmoe_problem node{};
    void* buf[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};  // w1 s1 b1 w2 s2 b2
    uint8_t* strips[2] = {nullptr, nullptr};   // strip-major fc1 / fc2 (mnb_qmoe_weights_prepack)
};

int mnb_qmoe_weights_release(mnb_qmoe_weights* w) {
    if (!w) return MNB_OK;
    (void)hipSetDevice(w->s->device);
    (void)hipStreamSynchronize(w->s->stream);
    for (void* b : w->buf)
        if (b) (void)hipFree(b);
    for (uint8_t* b : w->strips)
        if (b) (void)hipFree(b);
    delete w;
    return MNB_OK;
}

int mnb_qmoe_weights_prepack(mnb_qmoe_weights* w, int64_t* bytes) {
    if (bytes) *bytes = 0;
    if (!w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    const mnb_qmoe_problem& p = w->node;
    // fc1 is [E][2 I][H / 2], fc2 [E][H][I / 2]: N and K of each expert GEMV
    const int64_t n[2] = {2 * p.inter, p.hidden}, kk[2] = {p.hidden, p.inter};
    int64_t total = 0;
    std::lock_guard<std::mutex> lk(w->s->mu);
    (void)hipSetDevice(w->s->device);
    for (int f = 0; f < 2; ++f) {
        const int64_t nb = mnb::strip_pack_bytes(n[f], kk[f], p.num_experts);
        total += nb;
        if (w->strips[f]) continue;
        uint8_t* d = nullptr;
        hipError_t e = counted_malloc(&d, (size_t)nb);
        if (e != hipSuccess)
            return fail(MNB_ERR_NOMEM, "hipMalloc(%lld) for the strip-major fc%d: %s",
                        (long long)nb, f + 1, hipGetErrorString(e));
        // the MFMA-native order the fused QMoE's fp16 strip GEMV reads
        e = mnb::launch_strip_pack(static_cast<const uint8_t*>(w->buf[3 * f]), d, n[f], kk[f],
                                   w->s->stream, p.num_experts, mnb::kStripMfmaF16);
        if (e == hipSuccess) e = hipStreamSynchronize(w->s->stream);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(e, "strip-major copy of the QMoE weights");
        }
        w->strips[f] = d;
    }
    if (bytes) *bytes = total;
    return MNB_OK;
}

int mnb_qmoe_weights_upload(mnb_session* s, const mnb_qmoe_problem* node,
                            int32_t scales_per_channel, const void* fc1_weights,
                            size_t fc1_weights_bytes, const void* fc1_scales,
                            size_t fc1_scales_bytes, const void* fc1_bias, size_t fc1_bias_bytes,
                            const void* fc2_weights, size_t fc2_weights_bytes,
                            const void* fc2_scales, size_t fc2_scales_bytes, const void* fc2_bias,
                            size_t fc2_bias_bytes, mnb_qmoe_weights** out) {
    if (!s || !node || !out) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    *out = nullptr;
    mnb_qmoe_problem p = *node;
    p.rows = 0;
    int rc = mnb_qmoe_check(&p);
    if (rc) return rc;
    const size_t E = (size_t)p.num_experts, H = (size_t)p.hidden, I = (size_t)p.inter;
    const size_t bs = (size_t)p.block_size;
    const size_t n[2] = {2 * I, H}, kk[2] = {H, I};
    const void* src_w[2] = {fc1_weights, fc2_weights};
    const size_t got_w[2] = {fc1_weights_bytes, fc2_weights_bytes};
    const void* src_s[2] = {fc1_scales, fc2_scales};
    const size_t got_s[2] = {fc1_scales_bytes, fc2_scales_bytes};
    const void* src_b[2] = {fc1_bias, fc2_bias};
    const size_t got_b[2] = {fc1_bias_bytes, fc2_bias_bytes};
    std::vector<uint16_t> expanded[2];
    const void* host[6];
    size_t size[6];
    for (int f = 0; f < 2; ++f) {
        const size_t want_w = E * n[f] * kk[f] / 2;
        const size_t blocks = kk[f] / bs;
        const size_t want_s = E * n[f] * (scales_per_channel ? 1 : blocks) * 2;
        const size_t want_b = E * n[f] * 2;
        if (!src_w[f] || got_w[f] != want_w)
            return fail(MNB_ERR_INVALID, "fc%d weights hold %zu bytes, the layout needs %zu", f + 1,
                        got_w[f], want_w);
        if (!src_s[f] || got_s[f] != want_s)
            return fail(MNB_ERR_INVALID, "fc%d scales hold %zu bytes, the layout needs %zu", f + 1,
                        got_s[f], want_s);
        if (src_b[f] && got_b[f] != want_b)
            return fail(MNB_ERR_INVALID, "fc%d bias holds %zu bytes, the layout needs %zu", f + 1,
                        got_b[f], want_b);
        host[3 * f] = src_w[f];
        size[3 * f] = want_w;
        if (scales_per_channel) {
            // one scale per output channel: the same scale for every block of the channel
            const uint16_t* sc = static_cast<const uint16_t*>(src_s[f]);
            expanded[f].resize(E * n[f] * blocks);
            for (size_t c = 0; c < E * n[f]; ++c)
                for (size_t b = 0; b < blocks; ++b) expanded[f][c * blocks + b] = sc[c];
            host[3 * f + 1] = expanded[f].data();
            size[3 * f + 1] = expanded[f].size() * 2;
        } else {
            host[3 * f + 1] = src_s[f];
            size[3 * f + 1] = want_s;
        }
        host[3 * f + 2] = src_b[f];
        size[3 * f + 2] = src_b[f] ? want_b : 0;
    }
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    mnb_qmoe_weights* w = new (std::nothrow) mnb_qmoe_weights();
    if (!w) return fail(MNB_ERR_NOMEM, "weights allocation failed");
    w->s = s;
    w->node = p;
    hipError_t e = hipSuccess;
    for (int i = 0; i < 6 && e == hipSuccess; ++i) {
        if (!host[i]) continue;
        e = counted_malloc(&w->buf[i], size[i]);
        if (e == hipSuccess)
            e = hipMemcpyAsync(w->buf[i], host[i], size[i], hipMemcpyHostToDevice, s->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        for (void* b : w->buf)
            if (b) (void)hipFree(b);
        delete w;
        return hip_fail(e, "QMoE weight upload");
    }
    *out = w;
    return MNB_OK;
}

int mnb_session_run_qmoe(mnb_session* s, const mnb_qmoe_weights* w, int64_t rows, const void* x,
                         int x_on_device, const void* router_logits, int logits_on_device,
                         void* y, int y_on_device) {
    if (!s || !w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    mnb_qmoe_problem p = w->node;
    p.rows = rows;
    int rc = mnb_qmoe_check(&p);
    if (rc) return rc;
    if (rows == 0) return MNB_OK;
    if (!x || !router_logits || !y) return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    const size_t x_bytes = (size_t)rows * (size_t)p.hidden * 2;
    const size_t l_bytes = (size_t)rows * (size_t)p.num_experts *
                           (p.router_dtype == MNB_DTYPE_F32 ? 4 : 2);
    const size_t ws = mnb::qmoe_workspace_bytes(qmoe_args(&p));
    // one staging buffer for x and the logits, one for y; the workspace after them
    const size_t x_off = 0, l_off = (x_bytes + 255) & ~(size_t)255;
    const size_t stage = l_off + l_bytes;
    rc = sgrow(s, &s->a_dev, &s->a_cap, stage);
    if (rc) return rc;
    rc = sgrow(s, &s->y_dev, &s->y_cap, x_bytes);
    if (rc) return rc;
    rc = sgrow(s, &s->ws, &s->ws_cap, ws);
    if (rc) return rc;
    uint8_t* st = static_cast<uint8_t*>(s->a_dev);
    const void* xd = x;
    const void* ld = router_logits;
    void* yd = y_on_device ? y : s->y_dev;
    HostIo io(s);
    if (!x_on_device) {
        io.in(x, st + x_off, x_bytes);
        xd = st + x_off;
    }
    if (!logits_on_device) {
        io.in(router_logits, st + l_off, l_bytes);
        ld = st + l_off;
    }
    if (!y_on_device) io.out(y, s->y_dev, x_bytes);
    rc = io.upload();
    if (!rc)
        rc = qmoe_impl(&p, xd, ld, static_cast<const uint8_t*>(w->buf[0]), w->buf[1], w->buf[2],
                       static_cast<const uint8_t*>(w->buf[3]), w->buf[4], w->buf[5], yd, s->ws,
                       s->ws_cap, s->stream, w->strips[0], w->strips[1]);
    if (!rc) rc = io.download();
    return io.end(rc);
}

struct mnb_rmsnorm_weights {
    mnb_session* s = nullptr;
    mnb_rmsnorm_problem node{};
    void* gamma = nullptr;
    void* bias = nullptr;
};

int mnb_rmsnorm_weights_release(mnb_rmsnorm_weights* w) {
    if (!w) return MNB_OK;
    (void)hipSetDevice(w->s->device);
    (void)hipStreamSynchronize(w->s->stream);
    if (w->gamma) (void)hipFree(w->gamma);
    if (w->bias) (void)hipFree(w->bias);
    delete w;
    return MNB_OK;
}

int mnb_rmsnorm_weights_upload(mnb_session* s, const mnb_rmsnorm_problem* node,
                               const void* gamma, size_t gamma_bytes, const void* bias,
                               size_t bias_bytes, mnb_rmsnorm_weights** out) {
    if (!s || !node || !out) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    *out = nullptr;
    mnb_rmsnorm_problem p = *node;
    p.rows = 0;
    int rc = mnb_rmsnorm_check(&p);
    if (rc) return rc;
    const size_t want = (size_t)p.hidden * (size_t)elem_bytes(p.dtype);
    if (!gamma || gamma_bytes != want)
        return fail(MNB_ERR_INVALID, "gamma holds %zu bytes, the node needs %zu", gamma_bytes, want);
    if (p.has_bias && (!bias || bias_bytes != want))
        return fail(MNB_ERR_INVALID, "bias holds %zu bytes, the node needs %zu", bias_bytes, want);
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    mnb_rmsnorm_weights* w = new (std::nothrow) mnb_rmsnorm_weights();
    if (!w) return fail(MNB_ERR_NOMEM, "weights allocation failed");
    w->s = s;
    w->node = p;
    hipError_t e = counted_malloc(&w->gamma, want);
    if (e == hipSuccess) e = hipMemcpyAsync(w->gamma, gamma, want, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess && p.has_bias) {
        e = counted_malloc(&w->bias, want);
        if (e == hipSuccess) e = hipMemcpyAsync(w->bias, bias, want, hipMemcpyHostToDevice, s->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        if (w->gamma) (void)hipFree(w->gamma);
        if (w->bias) (void)hipFree(w->bias);
        delete w;
        return hip_fail(e, "RMSNorm constant upload");
    }
    *out = w;
    return MNB_OK;
}

int mnb_session_run_rmsnorm(mnb_session* s, const mnb_rmsnorm_weights* w, int64_t rows,
                            const void* x, int x_on_device, const void* skip,
                            int skip_on_device, void* y, int y_on_device, void* sum_out,
                            int sum_on_device) {
    if (!s || !w) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    mnb_rmsnorm_problem p = w->node;
    p.rows = rows;
    p.want_sum = sum_out != nullptr;
    int rc = mnb_rmsnorm_check(&p);
    if (rc) return rc;
    if (rows == 0) return MNB_OK;
    if (!x || !y || (p.has_skip && !skip))
        return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    const size_t bytes = (size_t)rows * (size_t)p.hidden * (size_t)elem_bytes(p.dtype);
    const size_t slot = (bytes + 255) & ~(size_t)255;
    // inputs staged one after the other in the A buffer, outputs in the Y buffer
    rc = sgrow(s, &s->a_dev, &s->a_cap, 2 * slot);
    if (rc) return rc;
    rc = sgrow(s, &s->y_dev, &s->y_cap, 2 * slot);
    if (rc) return rc;
    uint8_t* in = static_cast<uint8_t*>(s->a_dev);
    uint8_t* outb = static_cast<uint8_t*>(s->y_dev);
    const void* xd = x;
    const void* kd = p.has_skip ? skip : nullptr;
    void* yd = y_on_device ? y : outb;
    void* qd = sum_out ? (sum_on_device ? sum_out : outb + slot) : nullptr;
    HostIo io(s);
    if (!x_on_device) {
        io.in(x, in, bytes);
        xd = in;
    }
    if (p.has_skip && !skip_on_device) {
        io.in(skip, in + slot, bytes);
        kd = in + slot;
    }
    if (!y_on_device) io.out(y, yd, bytes);
    if (sum_out && !sum_on_device) io.out(sum_out, qd, bytes);
    rc = io.upload();
    if (!rc) rc = mnb_skip_rmsnorm(&p, xd, kd, w->gamma, w->bias, yd, qd, s->stream);
    if (!rc) rc = io.download();
    return io.end(rc);
}

struct mnb_gqa_caches {
    mnb_session* s = nullptr;
    mnb_gqa_problem node{};
    void* cos = nullptr;
    void* sin = nullptr;
};

int mnb_gqa_caches_release(mnb_gqa_caches* c) {
    if (!c) return MNB_OK;
    (void)hipSetDevice(c->s->device);
    (void)hipStreamSynchronize(c->s->stream);
    if (c->cos) (void)hipFree(c->cos);
    if (c->sin) (void)hipFree(c->sin);
    delete c;
    return MNB_OK;
}

int mnb_gqa_caches_upload(mnb_session* s, const mnb_gqa_problem* node, const void* cos_cache,
                          size_t cos_bytes, const void* sin_cache, size_t sin_bytes,
                          mnb_gqa_caches** out) {
    if (!s || !node || !out) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    *out = nullptr;
    mnb_gqa_problem p = *node;
    p.batch = 0;
    p.seq_len = 0;
    p.past_len_max = 0;
    p.present_len = 0;
    int rc = mnb_gqa_check(&p);
    if (rc) return rc;
    const size_t want = (size_t)p.max_seq * (size_t)(p.rotary_dim / 2) * 2;
    const bool resident = cos_cache || sin_cache;
    if (resident && (!cos_cache || cos_bytes != want || !sin_cache || sin_bytes != want))
        return fail(MNB_ERR_INVALID, "cos/sin caches hold %zu and %zu bytes, the node needs %zu "
                    "each", cos_bytes, sin_bytes, want);
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    mnb_gqa_caches* c = new (std::nothrow) mnb_gqa_caches();
    if (!c) return fail(MNB_ERR_NOMEM, "cache allocation failed");
    c->s = s;
    c->node = p;
    if (!resident) {
        *out = c;
        return MNB_OK;
    }
    hipError_t e = counted_malloc(&c->cos, want);
    if (e == hipSuccess) e = counted_malloc(&c->sin, want);
    if (e == hipSuccess) e = hipMemcpyAsync(c->cos, cos_cache, want, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->sin, sin_cache, want, hipMemcpyHostToDevice, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        if (c->cos) (void)hipFree(c->cos);
        if (c->sin) (void)hipFree(c->sin);
        delete c;
        return hip_fail(e, "GroupQueryAttention cache upload");
    }
    *out = c;
    return MNB_OK;
}

int mnb_session_run_gqa(mnb_session* s, const mnb_gqa_caches* c, const mnb_gqa_problem* shape,
                        const void* packed_qkv, const void* past_key, const void* past_value,
                        const int32_t* seqlens_k, const void* cos_cache,
                        const void* sin_cache, void* attn_out, void* present_key,
                        void* present_value, uint32_t on_device) {
    if (!s || !c || !shape) return fail(MNB_ERR_INVALID, "a NULL argument was passed");
    const mnb_gqa_problem& n = c->node;
    const bool own_caches = cos_cache || sin_cache;
    if (own_caches && (!cos_cache || !sin_cache))
        return fail(MNB_ERR_INVALID, "pass both cos_cache and sin_cache or neither");
    if (!own_caches && !c->cos)
        return fail(MNB_ERR_INVALID, "the node has no resident cos/sin caches; pass them");
    if (shape->num_heads != n.num_heads || shape->kv_num_heads != n.kv_num_heads ||
        shape->head_dim != n.head_dim || shape->rotary_dim != n.rotary_dim ||
        (!own_caches && shape->max_seq != n.max_seq) || shape->scale != n.scale ||
        shape->dtype != n.dtype)
        return fail(MNB_ERR_INVALID, "the call's head counts, head_dim, rotary_dim, max_seq, scale "
                                     "or dtype differ from the node's");
    const mnb_gqa_problem p = *shape;
    int rc = mnb_gqa_check(&p);
    if (rc) return rc;
    if (p.batch == 0 || p.seq_len == 0) return MNB_OK;
    if (!packed_qkv || !seqlens_k || !attn_out ||
        (p.past_len_max && (!past_key || !past_value)) ||
        (p.present_len && (!present_key || !present_value)))
        return fail(MNB_ERR_INVALID, "a NULL tensor pointer was passed");
    const bool qkv_dev = on_device & MNB_GQA_ON_DEVICE_QKV;
    const bool past_dev = on_device & MNB_GQA_ON_DEVICE_PAST;
    const bool seq_dev = on_device & MNB_GQA_ON_DEVICE_SEQLENS;
    const bool out_dev = on_device & MNB_GQA_ON_DEVICE_OUT;
    const bool pres_dev = on_device & MNB_GQA_ON_DEVICE_PRESENT;
    const bool cache_dev = on_device & MNB_GQA_ON_DEVICE_CACHES;
    // a present tensor given as its past tensor (same memory) is updated in place
    const bool in_place = p.past_len_max && present_key == past_key && past_dev == pres_dev;
    if (in_place != (p.past_len_max && present_value == past_value && past_dev == pres_dev))
        return fail(MNB_ERR_INVALID, "present_key and present_value must both alias their past "
                                     "tensors or neither");
    std::lock_guard<std::mutex> lk(s->mu);
    (void)hipSetDevice(s->device);
    const size_t heads = (size_t)p.num_heads + 2 * (size_t)p.kv_num_heads;
    const size_t qkv_b = (size_t)p.batch * p.seq_len * heads * p.head_dim * 2;
    const size_t past_b = (size_t)p.batch * p.kv_num_heads * p.past_len_max * p.head_dim * 2;
    const size_t seq_b = (size_t)p.batch * 4;
    const size_t out_b = (size_t)p.batch * p.seq_len * p.num_heads * p.head_dim * 2;
    const size_t pres_b = (size_t)p.batch * p.kv_num_heads * p.present_len * p.head_dim * 2;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    // inputs staged in the A buffer, outputs in the Y buffer
    const size_t cache_b = own_caches && !cache_dev
                               ? (size_t)p.max_seq * (size_t)(p.rotary_dim / 2) * 2 : 0;
    const size_t o_qkv = 0, o_pk = al(qkv_b), o_pv = o_pk + al(past_b), o_seq = o_pv + al(past_b);
    const size_t o_cos = o_seq + al(seq_b), o_sin = o_cos + al(cache_b);
    const size_t in_total = o_sin + al(cache_b);
    const size_t o_out = 0, o_rk = al(out_b), o_rv = o_rk + al(pres_b);
    const size_t out_total = o_rv + al(pres_b);
    rc = sgrow(s, &s->a_dev, &s->a_cap, in_total);
    if (!rc) rc = sgrow(s, &s->y_dev, &s->y_cap, out_total);
    size_t ws = 0;
    if (!rc) rc = mnb_gqa_workspace_bytes(&p, &ws);
    if (!rc) rc = sgrow(s, &s->ws, &s->ws_cap, ws);
    if (rc) return rc;
    uint8_t* in = static_cast<uint8_t*>(s->a_dev);
    uint8_t* ob = static_cast<uint8_t*>(s->y_dev);
    const void* qd = packed_qkv;
    const void* pkd = past_key;
    const void* pvd = past_value;
    const int32_t* sd = seqlens_k;
    void* od = out_dev ? attn_out : ob + o_out;
    void* rkd = present_key;
    void* rvd = present_value;
    HostIo io(s);
    auto up = [&](const void* src, size_t off, size_t bytes) -> const void* {
        if (bytes) io.in(src, in + off, bytes);
        return in + off;
    };
    if (!qkv_dev) qd = up(packed_qkv, o_qkv, qkv_b);
    if (!past_dev && p.past_len_max) {
        pkd = up(past_key, o_pk, past_b);
        pvd = up(past_value, o_pv, past_b);
    }
    if (!seq_dev) sd = static_cast<const int32_t*>(up(seqlens_k, o_seq, seq_b));
    const void* cd = own_caches ? cos_cache : c->cos;
    const void* snd = own_caches ? sin_cache : c->sin;
    if (own_caches && !cache_dev) {
        cd = up(cos_cache, o_cos, cache_b);
        snd = up(sin_cache, o_sin, cache_b);
    }
    if (in_place) {
        rkd = const_cast<void*>(pkd);
        rvd = const_cast<void*>(pvd);
    } else if (!pres_dev && p.present_len) {
        rkd = ob + o_rk;
        rvd = ob + o_rv;
    }
    if (!out_dev) io.out(attn_out, od, out_b);
    if (!pres_dev && p.present_len) {
        io.out(present_key, rkd, pres_b);
        io.out(present_value, rvd, pres_b);
    }
    rc = io.upload();
    if (!rc) rc = mnb_gqa(&p, qd, pkd, pvd, sd, cd, snd, od, rkd, rvd, s->ws, s->ws_cap, s->stream);
    if (!rc) rc = io.download();
    return io.end(rc);
}

int mnb_session_run_host(mnb_session* s, const mnb_weights* w, int64_t m, const void* a_host,
                         void* y_host) {
    return mnb_session_run(s, w, m, a_host, 0, y_host, 0);
}

}  // extern "C"
