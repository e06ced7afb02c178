/*
 * mnb_hip.h — C ABI of the MI355X (gfx950) MatMulNBits HIP shim.
 *
 * This is the device layer that the ORT plugin EP (include/onnxruntime_mi355x_ep.h) calls from
 * its Compute, and that any other host (ctypes, cgo, a C++ engine) can bind directly.  It
 * replaces the reference's Vulkan session and dispatch plumbing for this op:
 *
 *   mnb_matmul_nbits        replaces the q_gemv dispatch recorded by matmul_nbits_gemv
 *                           (rust/src/ops/quant.rs:521-651) and executed by
 *                           VulkanSession::dispatch_ort (rust/src/vk/session.rs:1036, :2540)
 *   mnb_session_* /         replace the per-session device, queue and the constant-input
 *   mnb_weights_*           weight cache keyed by (host ptr, bytes) that uploads B / scales /
 *                           zero_points once (rust/src/vk/session.rs:1633-1700)
 *   mnb_session_run_host    the host-I/O Compute path: stage A in, one launch, Y out, fence
 *                           (rust/src/vk/session.rs:1077-1134, :2635-2736, :2791)
 *   mnb_dequantize_f16      the Regime-1 dequant the reference checks bit-exact
 *                           (docs/OP_COVERAGE.md:5648-5651; tests/ops/test_matmulnbits.py:94-175)
 *   mnb_moe_grouped         expert-grouped MatMulNBits (no reference kernel: rust/src/ops/moe.rs:92-94,118)
 *   mnb_quantize_a_int8     the accuracy_level=4 activation quantiser (no reference kernel:
 *                           rust/src/ops/quant.rs:191-200 declines the level)
 *
 * Conventions
 *   - Every function returns MNB_OK (0) or an MNB_ERR_* code; mnb_last_error() returns the
 *     calling thread's last message.  No function aborts the process.
 *   - Device pointers are plain addresses from hipMalloc (or any allocator of the same device).
 *   - `stream` is a hipStream_t passed as void*; NULL means the legacy default stream.
 *     Device-pointer entry points are stream-ordered and do not synchronise.
 *   - Layouts are ORT's MatMulNBits layouts: A [M, K] row-major; B [N][K/bs][bs*bits/8] bytes;
 *     scales [N * K/bs]; zero_points [N][ceil((K/bs)*bits/8)] bytes (4-bit: two blocks per byte,
 *     low nibble first); Y [M, N] row-major.  A, scales and Y share one dtype (fp16 or fp32).
 */
#ifndef MNB_HIP_H_
#define MNB_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MNB_OK 0
#define MNB_ERR_INVALID 1     /* bad argument or shape */
#define MNB_ERR_UNSUPPORTED 2 /* well-formed, but a form this library does not implement */
#define MNB_ERR_HIP 3         /* a HIP runtime call failed */
#define MNB_ERR_NOMEM 4       /* device or host allocation failed */

#define MNB_DTYPE_F16 1
#define MNB_DTYPE_F32 2

/* Kernel families the planner can select (reported by mnb_plan, forced by MNB_FORCE_KERNEL). */
#define MNB_KERNEL_GEMV_MFMA 1   /* fp16, M <= 64: streaming GEMV on 16x16x32 f16 MFMA */
#define MNB_KERNEL_GEMM_MFMA 2   /* M > 64: dequantise-into-LDS MFMA GEMM (fp16, or fp32 M > 64) */
#define MNB_KERNEL_GENERIC 3     /* any dtype/bits/block: per-block fp32 partial, scaled once */
#define MNB_KERNEL_ACC4_I8 4     /* accuracy_level 4: int8 A, int8 MFMA, int32 block dots */
#define MNB_KERNEL_GEMV_STREAM 5 /* M <= 4: coalesced 16-byte-chunk streaming GEMV (fp16 or fp32) */
#define MNB_KERNEL_GROUP_MFMA 6  /* fp16, int4, block >= 32: row-tiled 16x16x32 MFMA GEMV */
#define MNB_KERNEL_STRIP_MFMA 7  /* fp16, int4, block >= 32, 5..16 rows: activations held in
                                    registers across a run of 16-column strips */
#define MNB_KERNEL_ACC4_STREAM 8 /* accuracy_level 4, fp16, <= 16 rows, K % 128 == 0 up to 8192:
                                    int8 MFMA, one 16-column strip per workgroup over all of K */
#define MNB_KERNEL_BATCH_STREAM 9 /* fp16, int4, block >= 32, 4..16 rows, K % 128 == 0: f16 MFMA,
                                     1 or 4 16-column strips per workgroup over all of K */

/* One MatMulNBits node: the attributes plus the row count of this call. */
typedef struct mnb_problem {
    int64_t m;              /* rows: product of A's leading dimensions (may be 0) */
    int64_t n;              /* attribute N */
    int64_t k;              /* attribute K */
    int32_t bits;           /* attribute bits: 4 or 8 */
    int32_t block_size;     /* attribute block_size: 16, 32, 64 or 128 */
    int32_t has_zero_points;/* 1 when input 3 (uint8 zero_points) is present */
    int32_t dtype;          /* MNB_DTYPE_F16 or MNB_DTYPE_F32 for A, scales and Y */
    int32_t accuracy_level; /* attribute accuracy_level (0 when absent) */
    int32_t reserved;
} mnb_problem;

/* The launch the planner chose for a problem (host-only; no device work). */
typedef struct mnb_plan_info {
    int32_t kernel;         /* MNB_KERNEL_* */
    int32_t waves_per_group;/* wavefronts per workgroup */
    int32_t tile_n;         /* output columns per workgroup */
    int32_t tile_m;         /* output rows per workgroup */
    int64_t grid_x;
    int64_t grid_y;
    int64_t workspace_bytes;/* device scratch: accuracy_level 4 (needed), or the fp32 partials
                             * of a prefill GEMM split along K (optional; 0 elsewhere) */
} mnb_plan_info;

const char* mnb_last_error(void);
int mnb_version(void);

/* Validates a problem against the claim domain (bits, block_size, K % block_size, dtype). */
int mnb_check_problem(const mnb_problem* p);
/* Fills `out` with the launch the planner would make for `p`. */
int mnb_plan(const mnb_problem* p, mnb_plan_info* out);
/* Device scratch in bytes for `p`: required for accuracy_level 4; for a prefill GEMM whose row
 * tiles alone would leave CUs idle (e.g. M = 256) it holds the fp32 partials of a split along K,
 * and a smaller workspace (or none) runs the GEMM unsplit; 0 otherwise. */
int mnb_workspace_bytes(const mnb_problem* p, size_t* bytes);

/* Y = A @ dequant(B)^T on device pointers.  `workspace` (16-byte aligned) may be NULL when
 * mnb_workspace_bytes() reports 0 or the plan's kernel is MNB_KERNEL_GEMM_MFMA; otherwise it must
 * hold at least that many bytes. */
int mnb_matmul_nbits(const mnb_problem* p, const void* a, const uint8_t* b, const void* scales,
                     const uint8_t* zero_points, void* y, void* workspace,
                     size_t workspace_bytes, void* stream);

/* mnb_matmul_nbits with no allocation and no workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory at call time (code under HIP
 * graph capture, tight serving loops, hosts that forbid hipMalloc).  The scratch the kernels need
 * (the accuracy_level 4 int8 activations and split-K partials, the prefill GEMM's K-split
 * partials) comes from a device array of mnb_noalloc_scratch_bytes() bytes (48 MiB) inside the
 * library, one per GPU, held until the process ends; nothing is allocated and no library routine
 * that allocates is called.  accuracy_level 4 problems whose workspace exceeds it are rejected
 * with MNB_ERR_UNSUPPORTED; a prefill GEMM whose K-split partials exceed it runs unsplit.  Every
 * call on one GPU uses that GPU's array, so calls that overlap in time on one GPU (other streams
 * or host threads) race; what must start at zero is cleared by the call itself.  The GPU is the
 * stream's (the current device for the NULL stream).  Stream-ordered, like mnb_matmul_nbits. */
int mnb_matmul_nbits_noalloc(const mnb_problem* p, const void* a, const uint8_t* b,
                             const void* scales, const uint8_t* zero_points, void* y,
                             void* stream);
size_t mnb_noalloc_scratch_bytes(void);

/* W[n][k] = fp16_rne(fp32(q - zp) * fp32(scale)), written as fp16 [N][K]. */
int mnb_dequantize_f16(int64_t n, int64_t k, int32_t bits, int32_t block_size,
                       const uint8_t* b, const void* scales_f16, const uint8_t* zero_points,
                       void* w_out_f16, void* stream);

/* accuracy_level=4 activation quantiser: per (row, block) amax, scale = amax/127,
 * qa = clamp(rint(a * (127/amax)), -127, 127) (0 when amax is 0), fp32 arithmetic, round half
 * to even.  a is fp16 [m][k] (dtype MNB_DTYPE_F16) or fp32; writes qa int8 [m][k] in natural
 * order, scale fp32 [m][k/bs] and, when qsum is not NULL, qsum int32 [m][k/bs] = sum of qa over
 * the block.  Stream-ordered. */
int mnb_quantize_a_int8(int64_t m, int64_t k, int32_t block_size, int32_t dtype, const void* a,
                        int8_t* qa, float* a_scale, int32_t* qsum, void* stream);

/* Expert-grouped MatMulNBits (gpt-oss style routed experts; no counterpart in the reference,
 * whose QMoE rows are staged without a kernel: rust/src/ops/moe.rs:92-94,118).
 * For expert e, rows i in [offsets[e], offsets[e+1]):
 *   Y[i, :] = A[row_index[i], :] @ dequant(B_e)^T
 * B/scales/zero_points hold `num_experts` consecutive per-expert tensors of one node's layout.
 * offsets is int32 [num_experts+1] and row_index int32 [offsets[num_experts]] on the device
 * (values in [0, a_rows)); `total_rows` must equal offsets[num_experts] and
 * `max_rows_per_expert` bound every group (the launch covers that many rows per expert).
 * fp16, bits = 4, block_size >= 32, K % 32 == 0.  Stream-ordered. */
typedef struct mnb_moe_problem {
    int64_t num_experts;
    int64_t total_rows;         /* rows of Y (= assignments) */
    int64_t max_rows_per_expert;
    int64_t a_rows;             /* rows of A (tokens) */
    int64_t n;
    int64_t k;
    int32_t bits;
    int32_t block_size;
    int32_t has_zero_points;
    int32_t dtype;              /* MNB_DTYPE_F16 only */
} mnb_moe_problem;

int mnb_moe_grouped(const mnb_moe_problem* p, const void* a, const int32_t* row_index,
                    const int32_t* offsets, const uint8_t* b, const void* scales,
                    const uint8_t* zero_points, void* y, void* stream);

/* Fused QMoE: com.microsoft::QMoE with int4 experts and SwiGLU (gpt-oss style).  No kernel
 * counterpart in the reference, which registers the op staged and declines top-k > 2
 * (rust/src/ops/moe.rs:40-118; gpt-oss attribute values docs/OP_COVERAGE.md:831-835); the
 * arithmetic is the build's declared reading of ONNX Runtime's QMoE (third-party):
 *   softmax over the E router logits of each token, the k largest (ties to the lower expert
 *   id), renormalised to sum to one when normalize_routing is set;
 *   h = x W1_e^T + b1_e (W1_e: 2I x H int4, symmetric, implied zero point 8);
 *   act = gate * sigmoid(alpha * gate) * (linear + beta), gate = min(gate, limit) and
 *   linear = clamp(linear, -limit, limit) when has_swiglu_limit, gate/linear = columns
 *   (2i, 2i+1) when swiglu_fusion = 1 or (i, I+i) when 2;
 *   y[t] = sum over the token's experts of w * (act W2_e^T + b2_e) (W2_e: H x I).
 * Weights: fc1 [E][2I][H/2] and fc2 [E][H][I/2] uint8, low nibble first (per expert the
 * MatMulNBits B layout); scales fp16 [E][N][K/block_size]; biases fp16 [E][2I] and [E][H] or
 * NULL.  x and y fp16 [rows][H]; router logits fp16 or fp32 [rows][E].  Limits: E <= 1024,
 * k <= min(8, E), rows * k <= 16384, H and I multiples of 32 and of block_size.  Intermediates
 * (h before the bias, act, act W2^T before the bias) are stored as fp16; accumulation is fp32.
 * Stream-ordered; the workspace (mnb_qmoe_workspace_bytes, 256-byte aligned) holds the routing
 * tables and the intermediates. */
typedef struct mnb_qmoe_problem {
    int64_t rows;               /* tokens (leading dims of x folded) */
    int64_t hidden;             /* H: K of fc1, N of fc2 */
    int64_t inter;              /* I: fc1 has 2I output channels (gate and linear) */
    int64_t num_experts;        /* E */
    int32_t k;                  /* experts per token */
    int32_t block_size;         /* quantisation block along K of fc1 and fc2: 32, 64 or 128 */
    int32_t swiglu_fusion;      /* 1 interleaved, 2 concatenated */
    int32_t normalize_routing;
    float activation_alpha;
    float activation_beta;
    float swiglu_limit;
    int32_t has_swiglu_limit;
    int32_t router_dtype;       /* MNB_DTYPE_F16 or MNB_DTYPE_F32 */
    int32_t dtype;              /* MNB_DTYPE_F16 */
} mnb_qmoe_problem;

int mnb_qmoe_check(const mnb_qmoe_problem* p);
int mnb_qmoe_workspace_bytes(const mnb_qmoe_problem* p, size_t* bytes);
int mnb_qmoe(const mnb_qmoe_problem* p, const void* x, const void* router_logits,
             const uint8_t* fc1_weights, const void* fc1_scales, const void* fc1_bias,
             const uint8_t* fc2_weights, const void* fc2_scales, const void* fc2_bias, void* y,
             void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm over the last axis, with the residual add fused:
 * com.microsoft::SkipSimplifiedLayerNormalization (has_skip) and SimplifiedLayerNormalization.
 * Replaces the reference's skip_simplified_layer_norm / simplified_layer_norm kernels
 * (rust/src/ops/norm.rs:68-140, bound in rust/src/ops/common/templates.rs:426-660):
 *   r = x + skip + bias (fp32 from the stored values; skip and bias optional);
 *   y = r / sqrt(mean(r^2) + epsilon) * gamma, stored in the tensor type;
 *   sum_out (optional, the node's output slot 3) = r stored in the tensor type.
 * x, skip, y, sum_out [rows][hidden]; gamma, bias [hidden]; fp16 or fp32, 16-byte aligned;
 * hidden a multiple of 8 (fp16) or 4 (fp32), at most 8192 (fp16) or 4096 (fp32).
 * Stream-ordered. */
typedef struct mnb_rmsnorm_problem {
    int64_t rows;
    int64_t hidden;
    float epsilon;
    int32_t has_skip;
    int32_t has_bias;
    int32_t want_sum;
    int32_t dtype;              /* MNB_DTYPE_F16 or MNB_DTYPE_F32 */
} mnb_rmsnorm_problem;

int mnb_rmsnorm_check(const mnb_rmsnorm_problem* p);
int mnb_skip_rmsnorm(const mnb_rmsnorm_problem* p, const void* x, const void* skip,
                     const void* gamma, const void* bias, void* y, void* sum_out, void* stream);

/* com.microsoft::GroupQueryAttention, the form the reference claims
 * (rust/src/ops/attention.rs:172-269) and computes (translate_gqa, attention.rs:388-735, kernel
 * rust/shaders/glsl/gqa_f16.comp): packed QKV, do_rotary=1 with half-rotation (neox) RoPE,
 * causal softmax, KV cache with seqlens_k.  fp16 tensors:
 *   packed_qkv [B, S, (Nq + 2 Nkv) D]; past_key/past_value [B, Nkv, past_len_max, D];
 *   seqlens_k [B] int32 (device memory); cos_cache/sin_cache [max_seq, rotary_dim / 2];
 *   attn_out [B, S, Nq D]; present_key/present_value [B, Nkv, present_len, D].
 * Per batch past_len = clamp(seqlens_k[b] + 1 - S, 0, past_len_max); query s sits at
 * tok_pos = past_len + s (cos/sin row min(tok_pos, max_seq - 1)) and attends to keys
 * [0, tok_pos].  The new rotated K and V are written to present at tok_pos when
 * tok_pos < present_len.  present_len is past_len_max + S or more (growing cache: the past
 * tokens [0, past_len) are copied into present) or equal to past_len_max (shared buffer:
 * present_key may be past_key itself, updated in place; if it is another buffer the past tokens
 * are copied too).  Present positions past past_len + S are left as they were.  Tensors 16-byte
 * aligned; head_dim a multiple of 16 up to 256.  Stream-ordered. */
typedef struct mnb_gqa_problem {
    int64_t batch;              /* B */
    int64_t seq_len;            /* S, new tokens per batch row */
    int64_t past_len_max;       /* past_key.shape[2] */
    int64_t present_len;        /* present_key.shape[2] */
    int64_t max_seq;            /* cos_cache.shape[0] */
    int32_t num_heads;          /* Nq, a positive multiple of kv_num_heads */
    int32_t kv_num_heads;       /* Nkv */
    int32_t head_dim;           /* D */
    int32_t rotary_dim;         /* even, 2 .. D */
    float scale;                /* applied to q . k before the softmax */
    int32_t dtype;              /* MNB_DTYPE_F16 */
} mnb_gqa_problem;

int mnb_gqa_check(const mnb_gqa_problem* p);
int mnb_gqa_workspace_bytes(const mnb_gqa_problem* p, size_t* bytes);
int mnb_gqa(const mnb_gqa_problem* p, const void* packed_qkv, const void* past_key,
            const void* past_value, const int32_t* seqlens_k, const void* cos_cache,
            const void* sin_cache, void* attn_out, void* present_key, void* present_value,
            void* workspace, size_t workspace_bytes, void* stream);

/* ---- session layer: one device, one stream, weights uploaded once ---------------------- */

typedef struct mnb_session mnb_session;
typedef struct mnb_weights mnb_weights;

int mnb_device_count(int* count);
/* The device's architecture name (hipDeviceProp_t::gcnArchName, e.g. "gfx950:sramecc+:xnack-"). */
int mnb_device_arch(int device_index, char* buf, size_t len);
int mnb_session_create(int device_index, mnb_session** out);
int mnb_session_destroy(mnb_session* s);
/* The session's hipStream_t (as void*). */
void* mnb_session_stream(mnb_session* s);
int mnb_session_synchronize(mnb_session* s);
/* Async mode (off by default): a session call whose tensors all live in the session device's
 * memory returns once its work is enqueued on the session's stream, without waiting for it;
 * calls with a host tensor still return after the stream has finished.  Stream-ordered work
 * that follows sees the results; the host sees them after mnb_session_synchronize or an event.
 * Backs the EP's OrtSyncStreamImpl: ORT's stream-aware EPs enqueue Compute on the stream ORT
 * hands them (onnxruntime_ep_c_api.h OrtSyncStreamImpl, OrtEpFactory::IsStreamAware /
 * CreateSyncStreamForDevice); the reference declines streams (rust/src/factory.rs:1268-1280). */
int mnb_session_set_async(mnb_session* s, int enabled);

/* Streams and events for the EP's OrtSyncStreamImpl / OrtSyncNotificationImpl (hipStream_t and
 * hipEvent_t as void*; events are created without timing).  No counterpart in the reference,
 * which has no streams. */
int mnb_stream_synchronize(int device_index, void* stream);
int mnb_device_synchronize(int device_index);
int mnb_event_create(int device_index, void** event);
int mnb_event_destroy(void* event);
int mnb_event_record(void* event, void* stream);        /* event completes after prior work */
int mnb_stream_wait_event(void* stream, void* event);   /* later work on stream waits for it */
int mnb_event_synchronize(void* event);                 /* host waits for it */

/* Uploads one node's constant inputs to HBM (hipMalloc + copy), once.  Byte sizes are checked
 * against the problem's layout.  zero_points may be NULL (implied zero point). */
int mnb_weights_upload(mnb_session* s, const mnb_problem* node, const void* b_host,
                       size_t b_bytes, const void* scales_host, size_t scales_bytes,
                       const void* zp_host, size_t zp_bytes, mnb_weights** out);
int mnb_weights_release(mnb_weights* w);

/* Upload-time weight layout for the batched decode kernels (4 to 16 fp16 rows, and the int8
 * GEMV of accuracy_level 4 at up to 16 rows): adds a copy of B in which each 16-column strip's
 * weights for each 128-k quad are one contiguous 1 KB run in the kernels' lane order (ORT's
 * layout spreads the same bytes over 16 columns x 64 bytes), made on the device from the
 * uploaded B.  Session calls whose plan is one of those kernels then read the copy; every other
 * kernel (the streaming GEMV at 1 to 3 rows, the prefill GEMM, ...) keeps reading B in ORT's
 * layout, which stays resident, so the node holds its weights twice.  Once per node (a second
 * call does nothing); *bytes (may be NULL) receives the copy's size.  MNB_ERR_UNSUPPORTED for
 * nodes those kernels never run (not fp16 x int4, K % 128 != 0, blocks other than 32/64/128,
 * K > 8192 at accuracy_level 4).  Replaces the reference's prepack seam, where
 * a kernel may re-lay a node's weights once at upload (rust/src/engine.rs:372-468; its
 * MatMulNBits prepack is the identity, rust/src/ops/quant.rs:676-682). */
int mnb_weights_prepack(mnb_weights* w, int64_t* bytes);

/* Device memory behind the EP's ORT allocator and data transfer (replace the reference's
 * Vulkan allocator and transfer: rust/src/allocator.rs, rust/src/transfer.rs, wired in
 * rust/src/factory.rs:1043-1285).  Allocations are plain hipMalloc memory of the given device;
 * copies are synchronous. */
#define MNB_COPY_HOST_TO_DEVICE 1
#define MNB_COPY_DEVICE_TO_HOST 2
#define MNB_COPY_DEVICE_TO_DEVICE 3
int mnb_device_malloc(int device_index, size_t bytes, void** out);
int mnb_device_free(int device_index, void* p);
int mnb_memcpy(int device_index, void* dst, const void* src, size_t bytes, int kind);
/* The same copy ordered on `stream` (a hipStream_t): device-to-device copies return once
 * enqueued, copies that touch host memory once complete. */
int mnb_memcpy_on_stream(int device_index, void* dst, const void* src, size_t bytes, int kind,
                         void* stream);

/* Compute with device-resident A and Y (stream-ordered on the session stream, no sync). */
int mnb_session_run_device(mnb_session* s, const mnb_weights* w, int64_t m, const void* a_dev,
                           void* y_dev);
/* Compute with A and Y each in host memory or in the session device's memory (flags): host
 * tensors are staged through HBM; returns after the stream has finished (ORT's synchronous
 * Compute of a non-stream-aware EP, rust/src/ep.rs:2538-2716). */
int mnb_session_run(mnb_session* s, const mnb_weights* w, int64_t m, const void* a,
                    int a_on_device, void* y, int y_on_device);
/* Compute with host A and Y: stage A in, launch, copy Y out, synchronise (ORT host I/O). */
int mnb_session_run_host(mnb_session* s, const mnb_weights* w, int64_t m, const void* a_host,
                         void* y_host);

/* QMoE weights of one node uploaded once (the constant-initializer upload of
 * rust/src/vk/session.rs:1633-1700, applied to the expert tensors).  Byte sizes are checked
 * against the problem.  scales_per_channel: fc1 scales [E][2I] and fc2 scales [E][H] (one
 * scale per output channel, QMoE without a block_size attribute), expanded here to blocks of
 * node->block_size; otherwise [E][N][K/block_size].  Biases may be NULL. */
typedef struct mnb_qmoe_weights mnb_qmoe_weights;
int mnb_qmoe_weights_upload(mnb_session* s, const mnb_qmoe_problem* node,
                            int32_t scales_per_channel, const void* fc1_weights,
                            size_t fc1_weights_bytes, const void* fc1_scales,
                            size_t fc1_scales_bytes, const void* fc1_bias, size_t fc1_bias_bytes,
                            const void* fc2_weights, size_t fc2_weights_bytes,
                            const void* fc2_scales, size_t fc2_scales_bytes, const void* fc2_bias,
                            size_t fc2_bias_bytes, mnb_qmoe_weights** out);
int mnb_qmoe_weights_release(mnb_qmoe_weights* w);
/* mnb_weights_prepack for a QMoE node: strip-major copies of the fc1 and fc2 expert weights
 * ([E][ceil(N/16)][ceil(K/128)] 1 KB runs, chunks past K zero), read by the expert-grouped strip
 * GEMV (up to 16 expected rows per expert) in place of ORT's layout, which stays resident for
 * the row-tiled GEMV of larger batches; the node then holds its expert weights twice.  Once per
 * node; *bytes (may be NULL) receives the copies' size.  Same seam as mnb_weights_prepack
 * (rust/src/engine.rs:372-468); the reference has no QMoE kernel (rust/src/ops/moe.rs:92-94). */
int mnb_qmoe_weights_prepack(mnb_qmoe_weights* w, int64_t* bytes);
/* One QMoE Compute with x, the router logits and y each in host memory or in the session
 * device's memory; host tensors are staged through HBM; returns after the stream finished. */
int mnb_session_run_qmoe(mnb_session* s, const mnb_qmoe_weights* w, int64_t rows, const void* x,
                         int x_on_device, const void* router_logits, int logits_on_device,
                         void* y, int y_on_device);

/* RMSNorm node constants (gamma, optional bias) uploaded once, and one Compute with x, skip,
 * y and the residual sum each in host memory or the session device's memory (the last two
 * may be NULL when the problem has no skip / no sum output).  Returns after the stream. */
typedef struct mnb_rmsnorm_weights mnb_rmsnorm_weights;
int mnb_rmsnorm_weights_upload(mnb_session* s, const mnb_rmsnorm_problem* node,
                               const void* gamma, size_t gamma_bytes, const void* bias,
                               size_t bias_bytes, mnb_rmsnorm_weights** out);
int mnb_rmsnorm_weights_release(mnb_rmsnorm_weights* w);
int mnb_session_run_rmsnorm(mnb_session* s, const mnb_rmsnorm_weights* w, int64_t rows,
                            const void* x, int x_on_device, const void* skip,
                            int skip_on_device, void* y, int y_on_device, void* sum_out,
                            int sum_on_device);

/* GroupQueryAttention node record: the cos/sin caches uploaded once when they are constant
 * initializers (as in the graphs the reference targets), or NULL when every call passes them.
 * One Compute takes its shapes from `shape` (head counts, head_dim, rotary_dim, scale and dtype
 * must match the node's; max_seq too when the caches are resident).  cos_cache/sin_cache NULL
 * use the resident caches.  Each tensor is in host memory or the session device's memory per
 * bit of `on_device` (MNB_GQA_ON_DEVICE_*); host tensors are staged through HBM, and a present
 * tensor passed as the same memory as its past tensor is updated in place.  Returns after the
 * stream has finished. */
#define MNB_GQA_ON_DEVICE_QKV 1u
#define MNB_GQA_ON_DEVICE_PAST 2u          /* past_key and past_value */
#define MNB_GQA_ON_DEVICE_SEQLENS 4u
#define MNB_GQA_ON_DEVICE_OUT 8u
#define MNB_GQA_ON_DEVICE_PRESENT 16u      /* present_key and present_value */
#define MNB_GQA_ON_DEVICE_CACHES 32u       /* per-call cos_cache and sin_cache */
typedef struct mnb_gqa_caches mnb_gqa_caches;
int mnb_gqa_caches_upload(mnb_session* s, const mnb_gqa_problem* node, const void* cos_cache,
                          size_t cos_bytes, const void* sin_cache, size_t sin_bytes,
                          mnb_gqa_caches** out);
int mnb_gqa_caches_release(mnb_gqa_caches* c);
int mnb_session_run_gqa(mnb_session* s, const mnb_gqa_caches* c, const mnb_gqa_problem* shape,
                        const void* packed_qkv, const void* past_key, const void* past_value,
                        const int32_t* seqlens_k, const void* cos_cache, const void* sin_cache,
                        void* attn_out, void* present_key, void* present_value,
                        uint32_t on_device);

/* Number of MatMulNBits-family kernel launches made by this process (proves the GPU ran). */
uint64_t mnb_launch_count(void);
/* Number of device allocations the library has made on its own behalf in this process: weights
 * and caches at upload, session staging and workspace when a call needs more than the session
 * holds (mnb_device_malloc, the caller's allocator, is not counted).  Counterpart of the
 * reference's AllocRecorder (rust/src/ops/quant.rs:1400-1547): a steady-state decode call leaves
 * it unchanged, which shows that no dequantised weight or per-call buffer is ever created. */
uint64_t mnb_device_alloc_count(void);

/* Roofline calibration; no counterpart in the reference (a measurement utility for bench.py).
 * Runs `workgroups` x 4 wavefronts x `iters` x 16 v_mfma_f32_32x32x16_f16 (32768 flops each) on
 * operands read once from `operands_f16` (workgroups * 256 * 8 fp16x8 values, 16-byte aligned;
 * NULL = constant operands) and writes one float per thread to `out` (workgroups * 256).  The
 * rate it sustains on random operands is the chip's power-limited fp16 MFMA ceiling. */
int mnb_calibrate_mfma(int32_t workgroups, int32_t iters, const void* operands_f16, float* out,
                       void* stream);

/* Read floor; no counterpart in the reference (a measurement utility for bench.py).  Reads
 * `bytes` (a positive multiple of 16) at `src` (16-byte aligned) once: every wavefront issues
 * `loads_per_lane` (1, 2, 4, 8 or 16) non-temporal 16-byte loads per lane, 1 KB per instruction,
 * all before using any, over contiguous runs (contiguous != 0) or runs strided by the number of
 * wavefronts; `waves_per_group` 1..16.  `out` holds 1024 uint32 and is written only in a case
 * no real data produces.  The shortest time over launch shapes is the least time any kernel
 * needs to stream that many bytes in one launch. */
int mnb_calibrate_read(const void* src, size_t bytes, int32_t loads_per_lane,
                       int32_t waves_per_group, int32_t contiguous, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MNB_HIP_H_ */
