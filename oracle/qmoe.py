"""CPU restatement of ``com.microsoft::QMoE`` with int4 experts and SwiGLU — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU leg may import this module,
and only as the checker; the product path never calls it.

What the reference holds for this op: a claim row without a kernel (``rust/src/ops/moe.rs:40-67,
92-118``: the schema fingerprint with the gpt-oss attribute vocabulary, top-1/2 only, int
weights only) and the attribute values of the only real graph it has seen, gpt-oss-20b
(``docs/OP_COVERAGE.md:831-835``: ``k = 4``, ``activation_type = "swiglu"``,
``activation_alpha = 1.702``, ``activation_beta = 1.0``, ``swiglu_limit = 7.0``,
``normalize_routing_weights = 1``, ``expert_weight_bits = 4``).  The arithmetic lives in
third-party ONNX Runtime v1.28.0 (``contrib_ops/cpu/moe``; not under ``/root/reference``), whose
CPU kernel refuses that graph anyway (``docs/OP_COVERAGE.md:2199-2204``).  This module is
therefore this build's declared reading of the op:

* ``router_probs`` ``[T, E]`` are logits: softmax over the experts, the ``k`` largest
  probabilities chosen (ties toward the lower expert id), renormalised to sum to one when
  ``normalize_routing_weights`` is set;
* expert weights are int4, two per byte, low nibble first, symmetric (implied zero point 8),
  ``fc1`` ``[E, 2I, H/2]`` and ``fc2`` ``[E, H, I/2]`` — per expert the MatMulNBits ``B`` layout;
  scales per output channel ``[E, N]`` or per block of ``block_size`` along K ``[E, N, K/bs]``;
  optional biases ``[E, 2I]`` and ``[E, H]``;
* SwiGLU over ``h = x W1^T + b1``: gate/linear interleaved (``swiglu_fusion = 1``: columns
  ``2i``, ``2i+1``) or concatenated (``swiglu_fusion = 2``: columns ``i``, ``I + i``);
  ``gate = min(gate, limit)``, ``linear = clamp(linear, -limit, limit)`` when a limit is given;
  ``act = gate * sigmoid(alpha * gate) * (linear + beta)``;
* ``y[t] = sum_s w[t, s] * (act W2^T + b2)`` over the token's chosen experts.

Parity against ORT is unpinned (ORT is absent here and refuses the one real graph).  The
restatement is pinned instead by closed forms and structure in ``tests/test_qmoe_oracle.py``:
SwiGLU special values, a pure-Python brute force on a tiny case, the reduction of one expert to
two chained MatMulNBits (the pinned ``matmul_nbits`` oracle), expert-relabelling invariance,
interleaved vs concatenated layouts of the same weights, per-channel vs replicated block scales,
and bias linearity.
"""

from __future__ import annotations

import numpy as np

from . import matmul_nbits as mnb


def route(logits, k: int, normalize: bool = True):
    """Softmax over experts, top-``k`` (ties to the lower id).  ``(experts [T,k], weights [T,k])``."""
    lg = np.asarray(logits, dtype=np.float64)
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, order, axis=1)
    if normalize:
        w = w / w.sum(axis=1, keepdims=True)
    return order.astype(np.int32), w


def swiglu(gate, linear, alpha: float, beta: float, limit: float | None):
    g = np.asarray(gate, dtype=np.float64)
    lin = np.asarray(linear, dtype=np.float64)
    if limit is not None:
        g = np.minimum(g, limit)
        lin = np.clip(lin, -limit, limit)
    return g / (1.0 + np.exp(-alpha * g)) * (lin + beta)


def split_gate_linear(h, fusion: int):
    h = np.asarray(h)
    inter = h.shape[-1] // 2
    if fusion == 1:
        return h[..., 0::2], h[..., 1::2]
    if fusion == 2:
        return h[..., :inter], h[..., inter:]
    raise ValueError(f"swiglu_fusion {fusion}")


def block_scales(scales, n: int, k: int, block_size: int):
    """Per-channel scales ``[E, N]`` or block scales ``[E, N, K/bs]`` as ``[E, N * K/bs]``."""
    s = np.asarray(scales)
    E = s.shape[0]
    if s.ndim == 2:                                   # per channel: one block spanning K
        s = np.repeat(s[:, :, None], k // block_size, axis=2)
    return s.reshape(E, n * (k // block_size))


def expert_weight(B, scales, n: int, k: int, block_size: int) -> np.ndarray:
    """Dequantised ``[N, K]`` float64 weight of one expert (B ``[N, K/2]`` or ``[N, K/bs, bs/2]``)."""
    b = np.asarray(B, dtype=np.uint8).reshape(n, k // block_size, block_size // 2)
    return mnb.dequantize_f32(b, np.asarray(scales).reshape(-1), None, n, k, 4,
                              block_size).astype(np.float64)


def qmoe(x, logits, fc1, fc1_scales, fc2, fc2_scales, *, k: int, inter: int, block_size: int,
         fc1_bias=None, fc2_bias=None, fusion: int = 1, alpha: float = 1.702, beta: float = 1.0,
         limit: float | None = 7.0, normalize: bool = True, f16_points: bool = False):
    """``y [T, H]`` float64.  ``block_size`` is the K block the scales use (for per-channel scales
    ``[E, N]`` pass any divisor of K, e.g. 32: the channel scale is then repeated per block).

    ``f16_points`` rounds to fp16 where the HIP path stores intermediates: ``x W1^T`` before the
    bias, the SwiGLU output, and ``act W2^T`` before the bias.
    """
    x = np.asarray(x)
    T, H = x.shape
    E = np.asarray(fc1).shape[0]
    n1 = 2 * inter
    s1 = block_scales(fc1_scales, n1, H, block_size)
    s2 = block_scales(fc2_scales, H, inter, block_size)
    experts, w = route(logits, k, normalize)
    xf = x.astype(np.float64)
    y = np.zeros((T, H), dtype=np.float64)
    r16 = (lambda v: v.astype(np.float16).astype(np.float64)) if f16_points else (lambda v: v)
    for e in range(E):
        tok, slot = np.nonzero(experts == e)
        if tok.size == 0:
            continue
        W1 = expert_weight(fc1[e], s1[e], n1, H, block_size)
        W2 = expert_weight(fc2[e], s2[e], H, inter, block_size)
        h = r16(xf[tok] @ W1.T)
        if fc1_bias is not None:
            h = h + np.asarray(fc1_bias[e], dtype=np.float64)
        g, lin = split_gate_linear(h, fusion)
        act = r16(swiglu(g, lin, alpha, beta, limit))
        o = r16(act @ W2.T)
        if fc2_bias is not None:
            o = o + np.asarray(fc2_bias[e], dtype=np.float64)
        y[tok] += w[tok, slot][:, None] * o
    return y


def make_qmoe_inputs(T: int, H: int, inter: int, E: int, *, block_size: int = 32,
                     per_channel: bool = False, bias: bool = True, seed: int = 20260801,
                     scale: float = 0.02):
    """Seeded synthetic QMoE inputs (gpt-oss conventions): x, logits ~ N(0,1) fp16; uniform
    nibbles; scales |N(0,1)| * scale; biases N(0,1) * 0.1 fp16."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    logits = rng.standard_normal((T, E), dtype=np.float32).astype(np.float16)

    def weights(n, kk):
        q = rng.integers(0, 16, size=(E, n, kk), dtype=np.uint8)
        return (q[:, :, 0::2] | (q[:, :, 1::2] << 4)).astype(np.uint8)

    def scales(n, kk):
        shape = (E, n) if per_channel else (E, n, kk // block_size)
        return (np.abs(rng.standard_normal(shape, dtype=np.float32)) * scale).astype(np.float16)

    fc1 = weights(2 * inter, H)
    fc1_s = scales(2 * inter, H)
    fc2 = weights(H, inter)
    fc2_s = scales(H, inter)
    b1 = (rng.standard_normal((E, 2 * inter), dtype=np.float32) * 0.1).astype(np.float16) if bias else None
    b2 = (rng.standard_normal((E, H), dtype=np.float32) * 0.1).astype(np.float16) if bias else None
    return {"x": x, "logits": logits, "fc1": fc1, "fc1_scales": fc1_s, "fc2": fc2,
            "fc2_scales": fc2_s, "fc1_bias": b1, "fc2_bias": b2}
