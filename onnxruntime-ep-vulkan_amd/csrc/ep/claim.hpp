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

}  // namespace mi355x_ep
