// MatMulNBits claim predicate of the MI355X plugin EP, over plain facts read from an OrtNode.
//
// Mirrors the reference predicate `matmul_nbits` (rust/src/ops/quant.rs:110-203) and its schema
// fingerprint `MATMUL_NBITS` (quant.rs:52-69): A float-typed; bits in {4, 8}; block_size in
// {16, 32, 64, 128}; K, N > 0; K % block_size == 0; no act-order `g_idx` (input 4); no fused
// `bias` (input 5).  Two deliberate differences, both widening the claim:
//   * the reference declines an fp16 output with an odd element count because its shader stores
//     pairs of halves through shared 32-bit words (quant.rs:149-162); the HIP kernels here store
//     each half on its own, so odd counts are claimed;
//   * the reference declines accuracy_level = 4 because it has no int8-activation kernel
//     (quant.rs:174-200); this EP claims it when `int8_path` is set (the level-4 kernel).
// The predicate is host code with no ORT or HIP dependency, so the mock host and the unit tests
// exercise it directly.
#pragma once

#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

namespace mi355x_ep {

// ONNX TensorProto element types used here (onnx.proto numbering, as ORT's
// ONNXTensorElementDataType).
enum ElemType : int32_t {
    kElemUndefined = 0,
    kElemFloat = 1,
    kElemUint8 = 2,
    kElemFloat16 = 10,
    kElemInt32 = 6,
};

struct InputFacts {
    bool present = false;        // a non-null value info in this input slot
    int32_t elem_type = 0;       // kElem* or another ONNX type
    bool has_shape = false;
    std::vector<int64_t> dims;   // -1 (or any negative) for a symbolic extent
    bool constant = false;       // constant initializer
};

struct NodeFacts {
    std::string op_type;
    std::string domain;
    std::vector<InputFacts> inputs;
    size_t num_outputs = 0;
    // Integer attributes; `has_*` false when the attribute is absent.
    bool has_k = false, has_n = false, has_bits = false, has_block_size = false;
    bool has_accuracy_level = false;
    int64_t k = 0, n = 0, bits = 0, block_size = 0, accuracy_level = 0;
};

struct ClaimDecision {
    bool claim = false;
    std::string reason;          // why it was declined (empty when claimed)
};

inline bool is_matmul_nbits(const NodeFacts& f) {
    return f.op_type == "MatMulNBits" && f.domain == "com.microsoft";
}

inline ClaimDecision decline(std::string why) { return ClaimDecision{false, std::move(why)}; }

// The claim predicate.  `int8_path` says whether the accuracy_level = 4 kernel is available.
inline ClaimDecision claim_matmul_nbits(const NodeFacts& f, bool int8_path) {
    if (!is_matmul_nbits(f)) return decline("not com.microsoft::MatMulNBits");
    // Arity of the contrib schema: 3..6 inputs, exactly one output (quant.rs:58-61).
    if (f.inputs.size() < 3 || f.inputs.size() > 6)
        return decline("MatMulNBits arity outside 3..6 inputs");
    if (f.num_outputs != 1) return decline("MatMulNBits must have exactly one output");
    const InputFacts& a = f.inputs[0];
    if (!a.present) return decline("input A is absent");
    if (a.elem_type != kElemFloat && a.elem_type != kElemFloat16)
        return decline("input A is neither float nor float16");
    if (!f.has_bits || !f.has_block_size || !f.has_k || !f.has_n)
        return decline("a required attribute (K, N, bits, block_size) is missing");
    if (f.bits != 4 && f.bits != 8)
        return decline("bits = " + std::to_string(f.bits) + "; this EP implements 4 and 8");
    if (f.block_size != 16 && f.block_size != 32 && f.block_size != 64 && f.block_size != 128)
        return decline("block_size = " + std::to_string(f.block_size) +
                       "; this EP implements 16/32/64/128");
    if (f.k <= 0 || f.n <= 0) return decline("K and N must be positive");
    if (f.k % f.block_size)
        return decline("K = " + std::to_string(f.k) + " is not a multiple of block_size = " +
                       std::to_string(f.block_size));
    if (f.k >= (int64_t(1) << 31) || f.n >= (int64_t(1) << 31))
        return decline("K or N does not fit the kernels' 32-bit extents");
    if (f.inputs.size() > 4 && f.inputs[4].present)
        return decline("supplies the act-order permutation g_idx (input 4)");
    if (f.inputs.size() > 5 && f.inputs[5].present)
        return decline("supplies the fused bias (input 5)");
    // Weights: packed uint8 B, scales in A's dtype, optional packed uint8 zero points.
    const InputFacts& b = f.inputs[1];
    const InputFacts& s = f.inputs[2];
    if (!b.present || b.elem_type != kElemUint8) return decline("input B must be uint8");
    if (!s.present || s.elem_type != a.elem_type)
        return decline("scales must be present and share A's element type");
    if (f.inputs.size() > 3 && f.inputs[3].present && f.inputs[3].elem_type != kElemUint8)
        return decline("only packed uint8 zero_points are implemented");
    // A's reduction extent, when known, must equal K.
    if (a.has_shape) {
        if (a.dims.empty()) return decline("input A is a scalar");
        const int64_t last = a.dims.back();
        if (last >= 0 && last != f.k) return decline("A's last dimension differs from K");
    }
    // accuracy_level: 0..3 resolve to ORT's fp32 compute path (quant.rs:164-190); 4 quantizes A
    // to int8 per block.
    if (f.has_accuracy_level) {
        if (f.accuracy_level < 0 || f.accuracy_level > 4)
            return decline("accuracy_level outside 0..4");
        if (f.accuracy_level == 4 && !int8_path)
            return decline("accuracy_level = 4 needs the int8 activation kernel");
    }
    return ClaimDecision{true, {}};
}

// ---- com.microsoft::QMoE ---------------------------------------------------------------------
//
// The reference registers QMoE with a fingerprint and no kernel (rust/src/ops/moe.rs:40-118:
// 8..21 inputs, one output, `k` required, top-1/2 only, activations silu/swiglu/relu/gelu,
// use_sparse_mixer 0, int weights).  This EP has the kernel (the HIP library's fused QMoE) and
// claims what it implements, which is the gpt-oss form the reference records
// (docs/OP_COVERAGE.md:831-835) widened in top-k and narrowed in activation:
//   * k in 1..8 (the reference: 1..2), k <= E;
//   * activation_type "swiglu" only, with swiglu_fusion 1 (interleaved) or 2 (concatenated),
//     or 0 with no fc3 inputs: the form gpt-oss-20b ships (docs/OP_COVERAGE.md:831-835: 8 of 11
//     inputs occupied, fc1 [E, 2I, H/2]).  Its fc1 channels are gpt-oss's gate/linear pairs,
//     interleaved, and the reference's census asks only for the attribute to read 1 for ORT's
//     CPU kernel to accept the same weights (tests/ops/test_phi35.py:1445-1453; ORT's CPU
//     kernel refuses fusion 0, docs/OP_COVERAGE.md:2199-2204), so it runs as fusion 1.
//     Fusion 0 with separate fc3 weights is declined by the rule on inputs 8 and above;
//   * use_sparse_mixer 0; expert_weight_bits 4; quant_type absent or "int"; block_size absent
//     or 0 (one scale per output channel) or 32/64/128;
//   * x float16 [.., H]; router logits float16 or float [rows, E];
//   * fc1 [E, 2I, H/2] and fc2 [E, H, I/2] uint8, scales float16 [E, N] or [E, N, K/bs],
//     optional float16 biases [E, 2I] and [E, H], all constant initializers with static shapes;
//     inputs 8 and above (fc3, zero points, FP4/FP8 scales) absent;
//   * H and I multiples of 32 and of block_size, E <= 1024.

struct QmoeFacts {
    std::string op_type;
    std::string domain;
    std::vector<InputFacts> inputs;
    size_t num_outputs = 0;
    bool has_k = false;
    int64_t k = 0;
    std::string activation_type = "relu";        // ORT's default
    int64_t normalize_routing_weights = 0;
    int64_t use_sparse_mixer = 0;
    int64_t swiglu_fusion = 0;
    int64_t expert_weight_bits = 4;
    int64_t block_size = 0;
    int64_t weights_prepacked = 0;
    bool has_quant_type = false;
    std::string quant_type;
    float activation_alpha = 1.0f;
    float activation_beta = 0.0f;
    bool has_swiglu_limit = false;
    float swiglu_limit = 0.0f;
    // Session option ep.qmoe_unfused_as_interleaved: claim swiglu_fusion = 0 without fc3 (the
    // gpt-oss export as recorded) and run it as the interleaved layout.  That reading is inferred
    // from the reference's census, not pinned by any fixture, so it is off unless asked for.
    bool unfused_as_interleaved = false;
};

// Extents read off the weight shapes when the claim succeeds.
struct QmoeShape {
    int64_t experts = 0, hidden = 0, inter = 0;
    bool per_channel = false;
    int32_t swiglu_fusion = 1;   // the layout the kernel runs: 1 interleaved, 2 concatenated
};

inline bool is_qmoe(const std::string& op_type, const std::string& domain) {
    return op_type == "QMoE" && domain == "com.microsoft";
}

inline bool static_dims(const InputFacts& f, size_t rank) {
    if (!f.has_shape || f.dims.size() != rank) return false;
    for (int64_t d : f.dims)
        if (d <= 0) return false;
    return true;
}

inline ClaimDecision claim_qmoe(const QmoeFacts& f, QmoeShape* shape = nullptr) {
    if (!is_qmoe(f.op_type, f.domain)) return decline("not com.microsoft::QMoE");
    if (f.inputs.size() < 8 || f.inputs.size() > 21)
        return decline("QMoE arity outside 8..21 inputs");
    if (f.num_outputs != 1) return decline("QMoE must have exactly one output");
    if (!f.has_k) return decline("the required attribute k is missing");
    if (f.activation_type != "swiglu")
        return decline("activation_type = " + f.activation_type + "; this EP implements swiglu");
    if (f.swiglu_fusion < 0 || f.swiglu_fusion > 2)
        return decline("swiglu_fusion = " + std::to_string(f.swiglu_fusion) +
                       "; this EP implements 0 (gpt-oss, no fc3), 1 (interleaved) and 2 "
                       "(concatenated)");
    if (f.use_sparse_mixer != 0) return decline("use_sparse_mixer changes the routing");
    if (f.expert_weight_bits != 4)
        return decline("expert_weight_bits = " + std::to_string(f.expert_weight_bits) +
                       "; this EP implements 4");
    if (f.has_quant_type && f.quant_type != "int")
        return decline("quant_type = " + f.quant_type + "; this EP implements int");
    if (f.weights_prepacked != 0) return decline("weights_prepacked is set");
    if (f.block_size != 0 && f.block_size != 32 && f.block_size != 64 && f.block_size != 128)
        return decline("block_size = " + std::to_string(f.block_size) +
                       "; this EP implements per-channel (0) and 32/64/128");
    for (size_t i = 8; i < f.inputs.size(); ++i)
        if (f.inputs[i].present)
            return decline("input " + std::to_string(i) +
                           " (fc3 / zero points / FP4-FP8 scales) is not implemented");
    if (f.swiglu_fusion == 0 && !f.unfused_as_interleaved)
        return decline("swiglu_fusion = 0 without fc3: its layout is not specified by ORT; set "
                       "ep.qmoe_unfused_as_interleaved=1 to run it as the interleaved layout");
    const InputFacts& x = f.inputs[0];
    const InputFacts& r = f.inputs[1];
    if (!x.present || x.elem_type != kElemFloat16) return decline("input is not float16");
    if (!r.present || (r.elem_type != kElemFloat16 && r.elem_type != kElemFloat))
        return decline("router_probs is neither float16 nor float");
    for (int i : {2, 3, 5, 6})
        if (!f.inputs[(size_t)i].present)
            return decline("expert weight input " + std::to_string(i) + " is absent");
    for (size_t i = 2; i < 8; ++i)
        if (f.inputs[i].present && !f.inputs[i].constant)
            return decline("expert tensors must be constant initializers");
    const InputFacts& w1 = f.inputs[2];
    const InputFacts& s1 = f.inputs[3];
    const InputFacts& b1 = f.inputs[4];
    const InputFacts& w2 = f.inputs[5];
    const InputFacts& s2 = f.inputs[6];
    const InputFacts& b2 = f.inputs[7];
    if (w1.elem_type != kElemUint8 || w2.elem_type != kElemUint8)
        return decline("expert weights must be packed uint8");
    if (s1.elem_type != kElemFloat16 || s2.elem_type != kElemFloat16)
        return decline("expert scales must be float16");
    if ((b1.present && b1.elem_type != kElemFloat16) || (b2.present && b2.elem_type != kElemFloat16))
        return decline("expert biases must be float16");
    if (!static_dims(w1, 3) || !static_dims(w2, 3))
        return decline("expert weights need static [E, N, K/2] shapes");
    const int64_t E = w1.dims[0], N1 = w1.dims[1], H = 2 * w1.dims[2];
    if (N1 % 2) return decline("fc1 has an odd number of output channels");
    const int64_t I = N1 / 2;
    if (w2.dims[0] != E || w2.dims[1] != H || 2 * w2.dims[2] != I)
        return decline("fc2's shape does not match fc1's (expected [E, H, I/2])");
    if (E > 1024) return decline("more than 1024 experts");
    if (f.k < 1 || f.k > 8 || f.k > E)
        return decline("k = " + std::to_string(f.k) + "; this EP routes 1..min(8, E)");
    const int64_t bs = f.block_size == 0 ? 32 : f.block_size;
    if (H % 32 || I % 32 || H % bs || I % bs)
        return decline("hidden and inter sizes must be multiples of 32 and of block_size");
    const bool per_channel = f.block_size == 0;
    auto scales_ok = [&](const InputFacts& s, int64_t n, int64_t kk) {
        if (per_channel) return static_dims(s, 2) && s.dims[0] == E && s.dims[1] == n;
        return static_dims(s, 3) && s.dims[0] == E && s.dims[1] == n && s.dims[2] == kk / bs;
    };
    if (!scales_ok(s1, N1, H) || !scales_ok(s2, H, I))
        return decline(per_channel ? "scales must be [E, N] (per channel)"
                                   : "scales must be [E, N, K/block_size]");
    if ((b1.present && !(static_dims(b1, 2) && b1.dims[0] == E && b1.dims[1] == N1)) ||
        (b2.present && !(static_dims(b2, 2) && b2.dims[0] == E && b2.dims[1] == H)))
        return decline("biases must be [E, 2I] and [E, H]");
    if (x.has_shape) {
        if (x.dims.empty()) return decline("input is a scalar");
        if (x.dims.back() >= 0 && x.dims.back() != H) return decline("input's last dim is not H");
    }
    if (r.has_shape) {
        if (r.dims.size() != 2) return decline("router_probs must be 2-D");
        if (r.dims[1] >= 0 && r.dims[1] != E) return decline("router_probs' last dim is not E");
    }
    if (shape) {
        shape->experts = E;
        shape->hidden = H;
        shape->inter = I;
        shape->per_channel = per_channel;
        shape->swiglu_fusion = f.swiglu_fusion == 2 ? 2 : 1;
    }
    return ClaimDecision{true, {}};
}

// ---- RMSNorm: SkipSimplifiedLayerNormalization / SimplifiedLayerNormalization ----------------
//
// Mirrors the reference rows (rust/src/ops/norm.rs:53-140): the skip form (com.microsoft, 3..5
// inputs, up to 4 outputs) and the plain form (com.microsoft and the default domain, in which
// the ORT GenAI builder emits it, norm.rs:118-133; 2 inputs, 1 output, the last axis).  Like the
// reference, output slots that the kernel does not write are declined: the plain form's
// inv_std_var (norm.rs:97-108) and the skip form's mean and inv_std_var (slots 1 and 2); the
// skip form's residual sum (slot 3) is written.  Narrower than the reference where this EP
// needs constants: gamma and the optional bias must be constant initializers of static length
// H, uploaded at Compile.  Widened: the skip form's optional bias (input 3) is applied.

struct NormFacts {
    std::string op_type;
    std::string domain;
    std::vector<InputFacts> inputs;
    std::vector<bool> outputs;                   // per declared slot: present
    bool has_axis = false;
    int64_t axis = -1;
    bool has_stash_type = false;
    int64_t stash_type = 1;
    float epsilon = 1e-5f;                       // the reference's default (templates.rs:399)
};

inline bool is_skip_norm(const std::string& op, const std::string& domain) {
    return op == "SkipSimplifiedLayerNormalization" && domain == "com.microsoft";
}
inline bool is_plain_norm(const std::string& op, const std::string& domain) {
    return op == "SimplifiedLayerNormalization" &&
           (domain == "com.microsoft" || domain.empty() || domain == "ai.onnx");
}

// The element budget of the HIP kernel: H a multiple of 8 (fp16) or 4 (fp32) elements, at
// most 8192 (fp16) or 4096 (fp32).
inline bool norm_hidden_ok(int64_t h, bool f16) {
    const int64_t cn = f16 ? 8 : 4;
    return h > 0 && h % cn == 0 && h / cn <= 1024;
}

inline ClaimDecision claim_norm(const NormFacts& f, int64_t* hidden = nullptr) {
    const bool skip = is_skip_norm(f.op_type, f.domain);
    if (!skip && !is_plain_norm(f.op_type, f.domain))
        return decline("not a (Skip)SimplifiedLayerNormalization");
    const size_t nin = f.inputs.size();
    if (skip ? (nin < 3 || nin > 5) : nin != 2)
        return decline(skip ? "arity outside 3..5 inputs" : "arity is not 2 inputs");
    if (f.outputs.empty() || !f.outputs[0]) return decline("output 0 is absent");
    if (skip) {
        if (f.outputs.size() > 4) return decline("more than 4 outputs");
        if ((f.outputs.size() > 1 && f.outputs[1]) || (f.outputs.size() > 2 && f.outputs[2]))
            return decline("asks for mean or inv_std_var (outputs 1 and 2), which are not written");
    } else if (f.outputs.size() > 1 && f.outputs[1]) {
        return decline("asks for inv_std_var (output 1), which is not written");
    }
    if (nin > 4 && f.inputs[4].present) return decline("input 4 is not implemented");
    const InputFacts& x = f.inputs[0];
    if (!x.present || (x.elem_type != kElemFloat16 && x.elem_type != kElemFloat))
        return decline("input is neither float16 nor float");
    if (!x.has_shape || x.dims.empty() || x.dims.back() <= 0)
        return decline("the normalised extent (last dim) must be static");
    const int64_t H = x.dims.back();
    if (f.has_axis) {
        const int64_t rank = (int64_t)x.dims.size();
        if (f.axis != -1 && f.axis != rank - 1) return decline("normalises over another axis than the last");
    }
    if (f.has_stash_type && f.stash_type != 1) return decline("stash_type other than float");
    const bool f16 = x.elem_type == kElemFloat16;
    if (!norm_hidden_ok(H, f16))
        return decline("hidden size " + std::to_string(H) + " is outside the kernel's range");
    const size_t gi = skip ? 2 : 1;
    auto const_vec = [&](size_t i) {
        const InputFacts& v = f.inputs[i];
        return v.present && v.constant && v.elem_type == x.elem_type && v.has_shape &&
               v.dims.size() == 1 && v.dims[0] == H;
    };
    if (!const_vec(gi)) return decline("gamma must be a constant [H] of the input's type");
    if (skip) {
        const InputFacts& k = f.inputs[1];
        if (!k.present || k.elem_type != x.elem_type) return decline("skip must share the input's type");
        if (k.has_shape) {
            if (k.dims.size() != x.dims.size()) return decline("skip's rank differs from the input's");
            for (size_t i = 0; i < k.dims.size(); ++i)
                if (k.dims[i] >= 0 && x.dims[i] >= 0 && k.dims[i] != x.dims[i])
                    return decline("skip's shape differs from the input's (broadcast skip)");
        }
        if (nin > 3 && f.inputs[3].present && !const_vec(3))
            return decline("bias must be a constant [H] of the input's type");
    }
    if (hidden) *hidden = H;
    return ClaimDecision{true, {}};
}

// ---- com.microsoft::GroupQueryAttention ------------------------------------------------------
//
// The claimed form is the reference's (rust/src/ops/attention.rs:172-269 claim, :388-560
// translate): packed QKV in input 0 with inputs 1 and 2 absent, past_key/past_value and
// seqlens_k present, do_rotary = 1 with half-rotation RoPE (rotary_interleaved = 0) from the
// cos/sin caches in inputs 7 and 8, fp16, and every numerics-changing option off
// (local_window_size -1, softcap 0, smooth_softmax <= 0, qk_output 0, no KV quantisation, inputs
// 10..15 absent).  The reference reads only input 0's shape, so it would compute a separate-QKV
// node with a wrong head_dim; that form is declined here.

struct GqaFacts {
    std::string op_type;
    std::string domain;
    std::vector<InputFacts> inputs;
    std::vector<InputFacts> outputs;             // declared outputs (present false when absent)
    bool has_num_heads = false, has_kv_num_heads = false, has_scale = false;
    int64_t num_heads = 0, kv_num_heads = 0;
    int64_t local_window_size = -1, do_rotary = 0, rotary_interleaved = 0;
    int64_t smooth_softmax = 0, qk_output = 0, kv_cache_bit_width = 0;
    int64_t rotary_embedding_dim = 0;
    float softcap = 0.f, scale = 0.f;
    std::string k_quant_type = "NONE", v_quant_type = "NONE";
};

struct GqaShape {
    int64_t head_dim = 0, rotary_dim = 0, packed = 0;
    int64_t declared_present_len = -1;           // present_key.shape[2] when static, else -1
    float scale = 0.f;                           // the effective softmax scale
};

inline bool is_gqa(const std::string& op, const std::string& domain) {
    return op == "GroupQueryAttention" && domain == "com.microsoft";
}

// The kernel's head_dim range: a multiple of 16 up to 256.
inline bool gqa_head_dim_ok(int64_t d) { return d >= 16 && d <= 256 && d % 16 == 0; }

inline ClaimDecision claim_gqa(const GqaFacts& f, GqaShape* shape = nullptr) {
    if (!is_gqa(f.op_type, f.domain)) return decline("not a com.microsoft GroupQueryAttention");
    const size_t nin = f.inputs.size();
    auto has = [&](size_t i) { return i < nin && f.inputs[i].present; };
    auto typed = [&](size_t i, int32_t t) { return has(i) && f.inputs[i].elem_type == t; };
    if (!typed(0, kElemFloat16)) return decline("packed_qkv (input 0) must be float16");
    if (has(1) || has(2))
        return decline("separate key/value inputs: only the packed-QKV form is implemented");
    if (!typed(3, kElemFloat16) || !typed(4, kElemFloat16))
        return decline("past_key and past_value (inputs 3 and 4) must be present float16 tensors");
    if (!has(5)) return decline("seqlens_k (input 5) is required for the per-batch past length");
    if (f.inputs[5].elem_type != kElemInt32) return decline("seqlens_k must be int32");
    if (!f.has_num_heads || !f.has_kv_num_heads) return decline("num_heads and kv_num_heads are required");
    if (f.num_heads <= 0 || f.kv_num_heads <= 0 || f.num_heads % f.kv_num_heads)
        return decline("num_heads must be a positive multiple of kv_num_heads");
    if (f.local_window_size != -1) return decline("local_window_size other than -1 (sliding window)");
    if (f.softcap != 0.f) return decline("softcap other than 0");
    if (f.smooth_softmax > 0) return decline("smooth_softmax (attention sink) is not implemented");
    if (f.qk_output != 0) return decline("qk_output other than 0");
    if (f.kv_cache_bit_width != 0 || f.k_quant_type != "NONE" || f.v_quant_type != "NONE")
        return decline("a quantised KV cache is not implemented");
    if (f.do_rotary != 1) return decline("do_rotary other than 1: RoPE is fused, the kernel needs it");
    if (f.rotary_interleaved != 0) return decline("rotary_interleaved = 1 (alternating pairs)");
    if (!typed(7, kElemFloat16) || !typed(8, kElemFloat16))
        return decline("cos_cache and sin_cache (inputs 7 and 8) must be present float16 tensors");
    static const char* const kOptional[] = {"attention_bias", "head_sink", "k_scale", "v_scale",
                                            "q_norm_weight", "k_norm_weight"};
    for (size_t i = 10; i < nin && i < 16; ++i)
        if (f.inputs[i].present) return decline(std::string(kOptional[i - 10]) + " is not implemented");
    if (nin > 16) return decline("more than 16 inputs");
    const InputFacts& x = f.inputs[0];
    if (!x.has_shape || x.dims.size() != 3 || x.dims[2] <= 0)
        return decline("packed_qkv must be rank 3 with a static last dimension");
    const int64_t heads = f.num_heads + 2 * f.kv_num_heads;
    if (x.dims[2] % heads) return decline("packed width is not (num_heads + 2 kv_num_heads) x head_dim");
    const int64_t D = x.dims[2] / heads;
    if (!gqa_head_dim_ok(D)) return decline("head_dim " + std::to_string(D) + " is outside the kernel's range");
    for (size_t i : {size_t(3), size_t(4)}) {
        const InputFacts& p = f.inputs[i];
        if (!p.has_shape) continue;
        if (p.dims.size() != 4) return decline("past_key/past_value must be rank 4");
        if ((p.dims[1] >= 0 && p.dims[1] != f.kv_num_heads) || (p.dims[3] >= 0 && p.dims[3] != D))
            return decline("past_key/past_value are not [B, kv_num_heads, S, head_dim]");
    }
    int64_t rd = f.rotary_embedding_dim;
    const InputFacts& c = f.inputs[7];
    if (rd <= 0) {
        if (!c.has_shape || c.dims.size() != 2 || c.dims[1] <= 0)
            return decline("no rotary_embedding_dim and cos_cache has no static second dimension: "
                           "the rotary width is not recoverable");
        rd = 2 * c.dims[1];
    }
    if (rd > D || rd % 2) return decline("rotary_dim is not an even value at most head_dim");
    for (size_t i : {size_t(7), size_t(8)}) {
        const InputFacts& t = f.inputs[i];
        if (t.has_shape && (t.dims.size() != 2 || (t.dims[1] >= 0 && t.dims[1] != rd / 2)))
            return decline("cos/sin caches are not [max_seq, rotary_dim / 2]");
    }
    if (f.outputs.size() < 3 || !f.outputs[0].present || !f.outputs[1].present || !f.outputs[2].present)
        return decline("output, present_key and present_value are required outputs");
    if (f.outputs.size() > 3 && f.outputs[3].present) return decline("output_qk is not written");
    if (shape) {
        shape->head_dim = D;
        shape->rotary_dim = rd;
        shape->packed = x.dims[2];
        const InputFacts& pk = f.outputs[1];
        shape->declared_present_len =
            pk.has_shape && pk.dims.size() == 4 && pk.dims[2] > 0 ? pk.dims[2] : -1;
        // ORT's schema: a scale of 0 (the attribute's default) means 1 / sqrt(head_dim)
        shape->scale = f.has_scale && f.scale != 0.f ? f.scale : 1.f / std::sqrt((float)D);
    }
    return ClaimDecision{true, {}};
}

}  // namespace mi355x_ep
