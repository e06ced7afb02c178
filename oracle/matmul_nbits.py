"""CPU restatement of ``com.microsoft::MatMulNBits`` — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker.  The product path (the HIP kernels behind the C ABI) never
calls into it and fails loudly when its HIP library is missing.

Semantics restated here, with the reference file each one follows (paths are relative to the
reference checkout):

* ``B`` is ``[N][blocks_per_col][blob]`` with ``blob = block_size * bits / 8``; row ``n`` of ``B``
  is output column ``n``:  ``Y[m][n] = sum_k A[m][k] * W[n][k]``
  (``docs/OP_COVERAGE.md:4210-4230``; ``rust/shaders/glsl/templates/q_gemv.comp:71-84``).
* 4-bit nibbles are low-first: element ``2i`` is ``byte[i] & 0xF``, element ``2i+1`` is
  ``byte[i] >> 4`` (``q_gemv.comp:315-329``).  8-bit weights are one byte per element
  (``q_gemv.comp:332-338``).
* ``W[n][k] = (q[n][k] - zp[n][k / bs]) * scale[n * bpc + k / bs]`` — the zero point is
  subtracted (``docs/OP_COVERAGE.md:4225-4230``; ``bench/test_weight_reread.py:99-107``).
* Absent ``zero_points`` means the implied zero point ``1 << (bits - 1)``
  (``rust/src/ops/quant.rs:684-705``; ``q_gemv.comp:290-294``).
* ``zero_points`` is packed like ``B``: two blocks per byte (low nibble first) at 4 bits, one
  byte per block at 8 bits, each column's run padded to a whole byte, i.e.
  ``zp_bytes_per_col = ceil(bpc * bits / 8)`` (``q_gemv.comp:284-306``).  Both the 2-D
  ``[N, zpb]`` form (``tests/ops/_models.py:2549-2553``) and the flat ``[N * zpb]`` form
  (``rust/tools/ledger_case_models.py:73-77``) are accepted; they are the same bytes.
* Accumulation is fp32-or-better over exact products; the reference's kernel forms a per-block
  fp32 partial over unscaled terms and scales it once (``q_gemv.comp:571-579``), ORT's CPU EP
  (``SQNBIT_CompFp32``, third-party ONNX Runtime v1.28.0, not present in the reference tree)
  dequantises to fp32 and accumulates in fp32.  ``matmul_nbits`` below accumulates in fp64 (the
  strictest reference); ``matmul_nbits_blockwise_f32`` restates the reference kernel's order.

``accuracy_level = 4`` and the expert-grouped MoE variant have no reference kernel
(``rust/src/ops/quant.rs:191-200``; ``rust/src/ops/moe.rs:92-94,118``): the functions for them
restate this build's own declared definitions, pinned by exact integer closed forms in
``tests/test_oracle.py``.  The int8 activation quantiser of ORT's ``SQNBIT_CompInt8`` is not
available here, so its agreement with ORT is *parity unpinned*; only the declared definition is
pinned.
"""

from __future__ import annotations

import numpy as np

SUPPORTED_BITS = (4, 8)                  # rust/src/ops/quant.rs:97-99
SUPPORTED_BLOCK_SIZES = (16, 32, 64, 128)  # rust/src/ops/quant.rs:105-107


# ---------------------------------------------------------------------------------------------
# Geometry
# ---------------------------------------------------------------------------------------------

def blocks_per_col(K: int, block_size: int) -> int:
    """``ceil(K / block_size)`` (``tests/ops/_models.py:2540``)."""
    return -(-K // block_size)


def blob_bytes(bits: int, block_size: int) -> int:
    """Packed bytes per (column, block) (``q_gemv.comp:284``)."""
    return block_size * bits // 8


def zp_bytes_per_col(bpc: int, bits: int) -> int:
    """Packed zero-point bytes per column, padded to a whole byte (``q_gemv.comp:287``)."""
    return (bpc * bits + 7) // 8


def implied_zero_point(bits: int) -> int:
    """``1 << (bits - 1)`` (``rust/src/ops/quant.rs:684-705``)."""
    return 1 << (bits - 1)


# ---------------------------------------------------------------------------------------------
# Unpacking
# ---------------------------------------------------------------------------------------------

def unpack_weights(B: np.ndarray, N: int, K: int, bits: int, block_size: int) -> np.ndarray:
    """Quantised values ``q[n][k]`` as uint8 ``[N, K]`` from packed ``B``."""
    bpc = blocks_per_col(K, block_size)
    blob = blob_bytes(bits, block_size)
    b = np.ascontiguousarray(B, dtype=np.uint8).reshape(N, bpc, blob)
    if bits == 4:
        q = np.empty((N, bpc, block_size), dtype=np.uint8)
        q[:, :, 0::2] = b & 0x0F
        q[:, :, 1::2] = b >> 4
    elif bits == 8:
        q = b.copy()
    else:
        raise ValueError(f"bits={bits} is not supported")
    return q.reshape(N, bpc * block_size)[:, :K]


def unpack_zero_points(zp: np.ndarray | None, N: int, bpc: int, bits: int) -> np.ndarray:
    """Per-(column, block) zero points as int32 ``[N, bpc]``; implied when ``zp`` is None."""
    if zp is None:
        return np.full((N, bpc), implied_zero_point(bits), dtype=np.int32)
    zpb = zp_bytes_per_col(bpc, bits)
    z = np.ascontiguousarray(zp, dtype=np.uint8).reshape(N, zpb)
    if bits == 4:
        out = np.empty((N, zpb * 2), dtype=np.int32)
        out[:, 0::2] = z & 0x0F
        out[:, 1::2] = z >> 4
        return out[:, :bpc]
    return z[:, :bpc].astype(np.int32)


# ---------------------------------------------------------------------------------------------
# Dequantisation (Regime 1: bit-exact)
# ---------------------------------------------------------------------------------------------

def dequantize_f32(B, scales, zp, N: int, K: int, bits: int, block_size: int) -> np.ndarray:
    """``fp32((q - zp) * scale)`` as float32 ``[N, K]``.

    With fp16 scales the product is exact in fp32 (at most 9 significant bits times 11), so this
    is also the exact real-number dequant.  With fp32 scales it is the fp32 product, rounded
    to nearest even once.
    """
    bpc = blocks_per_col(K, block_size)
    q = unpack_weights(B, N, K, bits, block_size).astype(np.int32)
    z = unpack_zero_points(zp, N, bpc, bits)
    s = np.asarray(scales).reshape(N, bpc).astype(np.float32)
    kb = np.arange(K) // block_size
    diff = (q - z[:, kb]).astype(np.float32)
    return diff * s[:, kb]


def dequantize_f16(B, scales, zp, N: int, K: int, bits: int, block_size: int) -> np.ndarray:
    """``fp16_rne(fp32(q - zp) * fp32(scale))`` as float16 ``[N, K]`` — the bit-exact target."""
    return dequantize_f32(B, scales, zp, N, K, bits, block_size).astype(np.float16)


# ---------------------------------------------------------------------------------------------
# MatMulNBits
# ---------------------------------------------------------------------------------------------

def matmul_nbits(A, B, scales, zp, N: int, K: int, bits: int, block_size: int,
                 acc: str = "f64") -> np.ndarray:
    """``Y[.., n] = sum_k A[.., k] * W[n][k]``, returned as float32 ``A.shape[:-1] + (N,)``.

    ``acc="f64"`` accumulates the exact products in float64 (the strictest reference);
    ``acc="f32"`` is a plain fp32 GEMM over the fp32 dequantised weight, the shape of ORT's
    ``SQNBIT_CompFp32`` (summation order is BLAS's, not MLAS's).
    """
    A = np.asarray(A)
    lead = A.shape[:-1]
    if A.shape[-1] != K:
        raise ValueError(f"A has last dim {A.shape[-1]}, expected K={K}")
    a2 = A.reshape(-1, K)
    W = dequantize_f32(B, scales, zp, N, K, bits, block_size)
    if acc == "f64":
        y = a2.astype(np.float64) @ W.astype(np.float64).T
    elif acc == "f32":
        y = a2.astype(np.float32) @ W.T
    else:
        raise ValueError(acc)
    return y.astype(np.float32).reshape(*lead, N)


def matmul_nbits_blockwise_f32(A, B, scales, zp, N: int, K: int, bits: int,
                               block_size: int) -> np.ndarray:
    """The reference kernel's order: per-block fp32 partial of ``a * (q - zp)``, scaled once.

    ``bacc = sum_{k in blk} a * (q - zp)`` in fp32, then ``acc += bacc * s``
    (``q_gemv.comp:571-579``).  Sequential over k and over blocks; pure numpy fp32 ops.
    """
    A = np.asarray(A)
    lead = A.shape[:-1]
    a2 = A.reshape(-1, K).astype(np.float32)
    bpc = blocks_per_col(K, block_size)
    q = unpack_weights(B, N, K, bits, block_size).astype(np.int32)
    z = unpack_zero_points(zp, N, bpc, bits)
    s = np.asarray(scales).reshape(N, bpc).astype(np.float32)
    acc = np.zeros((a2.shape[0], N), dtype=np.float32)
    for blk in range(bpc):
        k0, k1 = blk * block_size, min(K, (blk + 1) * block_size)
        w = (q[:, k0:k1] - z[:, blk:blk + 1]).astype(np.float32)       # [N, bs]
        bacc = np.zeros((a2.shape[0], N), dtype=np.float32)
        for k in range(k1 - k0):
            bacc = (bacc + a2[:, k0 + k:k0 + k + 1] * w[None, :, k]).astype(np.float32)
        acc = (acc + bacc * s[None, :, blk]).astype(np.float32)
    return acc.reshape(*lead, N)


# ---------------------------------------------------------------------------------------------
# accuracy_level = 4 (this build's declared definition; no reference kernel exists)
# ---------------------------------------------------------------------------------------------

def quantize_a_int8(A, block_size: int):
    """Per-(row, block) symmetric int8 quantisation of the activation.

    Declared definition, evaluated in fp32 exactly as the GPU does it:
    ``amax = max |a|`` over the block; ``scale = amax / 127``; ``inv = 127 / amax`` (0 when
    ``amax == 0``); ``qa = clamp(rint(fp32(a * inv)), -127, 127)`` with round-half-even.
    Returns ``(qa int8 [M, K], scale float32 [M, bpc], qsum int32 [M, bpc])``; ``qsum`` is
    ``sum qa`` over the block (what the zero-point correction multiplies).
    """
    a = np.asarray(A).astype(np.float32)
    M, K = a.reshape(-1, a.shape[-1]).shape
    a = a.reshape(M, K)
    bpc = blocks_per_col(K, block_size)
    qa = np.zeros((M, K), dtype=np.int8)
    sc = np.zeros((M, bpc), dtype=np.float32)
    qs = np.zeros((M, bpc), dtype=np.int32)
    for blk in range(bpc):
        k0, k1 = blk * block_size, min(K, (blk + 1) * block_size)
        amax = np.max(np.abs(a[:, k0:k1]), axis=1).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
        sc[:, blk] = (amax / np.float32(127.0)).astype(np.float32)
        prod = (a[:, k0:k1] * inv[:, None]).astype(np.float32)
        q = np.clip(np.rint(prod), -127, 127).astype(np.int8)
        qa[:, k0:k1] = q
        qs[:, blk] = q.astype(np.int32).sum(axis=1)
    return qa, sc, qs


def matmul_nbits_acc4(A, B, scales, zp, N: int, K: int, bits: int, block_size: int):
    """``accuracy_level = 4``: int8 activations, integer block dots, scaled in float.

    ``Y[m][n] = sum_blk (sA[m][blk] * sB[n][blk]) * sum_{k in blk} qa[m][k] * (q[n][k] - zp)``.
    The integer dots are exact (int64 here, int32 on the GPU — at most 127 * 255 * 128 per
    block); the float combination is done in float64.  Returns float32 ``[.., N]``.
    """
    A = np.asarray(A)
    lead = A.shape[:-1]
    a2 = A.reshape(-1, K)
    M = a2.shape[0]
    bpc = blocks_per_col(K, block_size)
    qa, sa, _ = quantize_a_int8(a2, block_size)
    q = unpack_weights(B, N, K, bits, block_size).astype(np.int64)
    z = unpack_zero_points(zp, N, bpc, bits).astype(np.int64)
    s = np.asarray(scales).reshape(N, bpc).astype(np.float64)
    y = np.zeros((M, N), dtype=np.float64)
    for blk in range(bpc):
        k0, k1 = blk * block_size, min(K, (blk + 1) * block_size)
        w = q[:, k0:k1] - z[:, blk:blk + 1]                              # [N, bs]
        dot = qa[:, k0:k1].astype(np.int64) @ w.T                        # [M, N] exact
        y += sa[:, blk:blk + 1].astype(np.float64) * s[None, :, blk] * dot
    return y.astype(np.float32).reshape(*lead, N)


# ---------------------------------------------------------------------------------------------
# Expert-grouped MatMulNBits (MoE; this build's declared definition, no reference kernel)
# ---------------------------------------------------------------------------------------------

def route_topk(logits, k: int):
    """Softmax over experts, then the ``k`` largest probabilities per token.

    Returns ``(experts int32 [T, k], weights float32 [T, k])``; ties break toward the lower
    expert id (stable sort).  The weights are the softmax probabilities of the chosen experts,
    renormalised to sum to one (gpt-oss style).
    """
    lg = np.asarray(logits, dtype=np.float64)
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, order, axis=1)
    w /= w.sum(axis=1, keepdims=True)
    return order.astype(np.int32), w.astype(np.float32)


def group_by_expert(experts, num_experts: int):
    """Sort (token, slot) assignments by expert.

    Returns ``(offsets int32 [E+1], rows int32 [T*k])`` where ``rows[offsets[e]:offsets[e+1]]``
    are the token indices routed to expert ``e`` in ascending (token, slot) order.
    """
    ex = np.asarray(experts, dtype=np.int64)
    T, k = ex.shape
    flat = ex.reshape(-1)
    order = np.argsort(flat, kind="stable")
    rows = (order // k).astype(np.int32)
    counts = np.bincount(flat, minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return offsets, rows


def moe_grouped_matmul_nbits(A, rows, offsets, B, scales, zp, N: int, K: int, bits: int,
                             block_size: int) -> np.ndarray:
    """For expert ``e``: ``Y[i] = A[rows[i]] @ W_e^T`` for ``i`` in ``[offsets[e], offsets[e+1])``.

    ``B``/``scales``/``zp`` carry a leading expert axis ``[E, ...]`` of per-expert MatMulNBits
    tensors.  Returns float32 ``[len(rows), N]`` in grouped order.
    """
    A = np.asarray(A)
    rows = np.asarray(rows)
    E = len(offsets) - 1
    out = np.zeros((len(rows), N), dtype=np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        ze = None if zp is None else zp[e]
        out[lo:hi] = matmul_nbits(A[rows[lo:hi]], B[e], scales[e], ze, N, K, bits, block_size)
    return out


# ---------------------------------------------------------------------------------------------
# Input construction (seeded synthetic data of the benchmark's shape)
# ---------------------------------------------------------------------------------------------

def pack_weights(q: np.ndarray, bits: int, block_size: int) -> np.ndarray:
    """Inverse of :func:`unpack_weights`: uint8 ``[N, K]`` values to ``[N, bpc, blob]`` bytes."""
    N, K = q.shape
    bpc = blocks_per_col(K, block_size)
    qq = np.zeros((N, bpc * block_size), dtype=np.uint8)
    qq[:, :K] = q
    qq = qq.reshape(N, bpc, block_size)
    if bits == 4:
        return (qq[:, :, 0::2] & 0xF) | ((qq[:, :, 1::2] & 0xF) << 4)
    return qq.copy()


def pack_zero_points(z: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of :func:`unpack_zero_points`: int ``[N, bpc]`` to uint8 ``[N, zpb]``."""
    N, bpc = z.shape
    zpb = zp_bytes_per_col(bpc, bits)
    if bits == 4:
        zz = np.zeros((N, zpb * 2), dtype=np.uint8)
        zz[:, :bpc] = z
        return (zz[:, 0::2] & 0xF) | ((zz[:, 1::2] & 0xF) << 4)
    return z.astype(np.uint8).copy()


def make_inputs(M: int, N: int, K: int, bits: int = 4, block_size: int = 32,
                with_zp: bool = False, seed: int = 20260801, a_dtype=np.float16,
                scale_mode: str = "abs_normal"):
    """Seeded synthetic MatMulNBits inputs in the BASELINE shape conventions.

    ``A ~ N(0,1)``; weights uniform over ``0 .. 2^bits - 1``; zero points uniform over the
    same range; scales ``|N(0,1)| * 0.02`` (``scale_mode="abs_normal"``) or
    ``U(0.001, 0.1)`` (``"uniform"``, the reference test's choice, ``tests/ops/_models.py:2549``).
    Returns a dict with ``A, B, scales, zp`` (``zp`` is None when ``with_zp`` is False).
    """
    rng = np.random.default_rng(seed)
    bpc = blocks_per_col(K, block_size)
    A = rng.standard_normal((M, K), dtype=np.float32).astype(a_dtype)
    q = rng.integers(0, 1 << bits, size=(N, bpc * block_size), dtype=np.uint8)[:, :K]
    B = pack_weights(q, bits, block_size)
    if scale_mode == "abs_normal":
        s = (np.abs(rng.standard_normal(N * bpc, dtype=np.float32)) * np.float32(0.02))
    else:
        s = rng.uniform(0.001, 0.1, size=N * bpc).astype(np.float32)
    scales = s.astype(a_dtype)
    zp = None
    if with_zp:
        z = rng.integers(0, 1 << bits, size=(N, bpc))
        zp = pack_zero_points(z, bits)
    return {"A": A, "B": B, "scales": scales, "zp": zp}


# ---------------------------------------------------------------------------------------------
# Error metric (the tolerance definition)
# ---------------------------------------------------------------------------------------------

def max_rel_err_significant(y, y_ref, frac: float = 0.1) -> float:
    """max ``|y - y_ref| / |y_ref|`` over elements with ``|y_ref| >= frac * RMS(y_ref)``.

    The denominator the reference itself uses for real-weights checks
    (``docs/PERF.md:4350-4372``): a max relative error over *all* elements is unbounded under
    cancellation, so elements below a tenth of the RMS are excluded.
    """
    y = np.asarray(y, dtype=np.float64).ravel()
    r = np.asarray(y_ref, dtype=np.float64).ravel()
    if r.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(r * r)))
    if rms == 0.0:
        return float(np.max(np.abs(y - r))) if y.size else 0.0
    sig = np.abs(r) >= frac * rms
    if not np.any(sig):
        return 0.0
    return float(np.max(np.abs(y[sig] - r[sig]) / np.abs(r[sig])))


def max_err_rms_normalised(y, y_ref) -> float:
    """max ``|y - y_ref| / max(|y_ref|, RMS(y_ref))`` over every element."""
    y = np.asarray(y, dtype=np.float64).ravel()
    r = np.asarray(y_ref, dtype=np.float64).ravel()
    if r.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(r * r)))
    den = np.maximum(np.abs(r), rms if rms > 0 else 1.0)
    return float(np.max(np.abs(y - r) / den))
