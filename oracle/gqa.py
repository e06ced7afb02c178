"""CPU restatement of ``com.microsoft::GroupQueryAttention`` (packed QKV, fused RoPE) — TEST
INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU leg may import this module,
and only as the checker; the product path never calls it.

Follows the reference kernel ``rust/shaders/glsl/gqa_f16.comp`` (dispatched by
``rust/src/ops/attention.rs:388-650``; claim ``attention.rs:172-269``):

* ``packed_qkv`` ``[B, S, (Nq + 2 Nkv) D]``: Q heads, then K heads, then V heads;
* per batch ``past_len = max(seqlens_k[b] + 1 - S, 0)``; query ``s`` sits at absolute position
  ``tok_pos = past_len + s`` (``gqa_f16.comp`` step 0);
* RoPE, half-rotation (neox): for ``i < rotary_dim / 2`` the pair ``(x[i], x[i + rd/2])`` is
  rotated by ``cos_cache[tok_pos, i]``, ``sin_cache[tok_pos, i]``; dims at or past
  ``rotary_dim`` are not rotated (step 2);
* the new K (rotated) and V are written to ``present`` at ``tok_pos``; under the growing
  convention ``present`` also holds the past (step 3a);
* causal attention of every query over keys ``[0, tok_pos]`` of KV head ``h // (Nq / Nkv)``,
  ``softmax(scale * q . k) v`` with ``scale`` default ``1 / sqrt(D)`` (step 4);
* ``present`` length: ``max(total_sequence_length, past_S)`` (the past buffer itself when it
  is already that long: the shared-buffer convention).

``f16_points`` stores present K/V as fp16 and reads every key from there, as the HIP path does
(the reference keeps the new tokens' keys in fp32 for their own dot products; ORT's CPU kernel
reads them from its fp16 present buffer).

Pinned in ``tests/test_gqa_oracle.py`` against ``torch.nn.functional.scaled_dot_product_attention``
(a library routine, on the rotated tensors), closed forms (a single key returns its value, a
zero rotation is the identity, a rotation preserves norms) and a pure-Python brute force.
"""

from __future__ import annotations

import numpy as np


def rope_neox(x, cos, sin, rotary_dim: int):
    """Rotate the first ``rotary_dim`` dims of ``x [..., D]`` (neox halves); cos/sin
    ``[..., rotary_dim/2]`` broadcast against ``x``'s leading dims."""
    x = np.asarray(x, dtype=np.float64).copy()
    rh = rotary_dim // 2
    c = np.asarray(cos, dtype=np.float64)
    s = np.asarray(sin, dtype=np.float64)
    x1 = x[..., :rh].copy()
    x2 = x[..., rh:2 * rh].copy()
    x[..., :rh] = x1 * c - x2 * s
    x[..., rh:2 * rh] = x2 * c + x1 * s
    return x


def gqa(packed_qkv, past_k, past_v, seqlens_k, total_seq_len: int, cos_cache, sin_cache,
        num_heads: int, kv_num_heads: int, scale: float | None = None,
        rotary_dim: int | None = None, f16_points: bool = False):
    """``(attn [B, S, Nq D], present_k, present_v)`` in float64."""
    qkv = np.asarray(packed_qkv, dtype=np.float64)
    B, S, P = qkv.shape
    Nq, Nkv = num_heads, kv_num_heads
    D = P // (Nq + 2 * Nkv)
    G = Nq // Nkv
    rd = rotary_dim if rotary_dim is not None else 2 * np.asarray(cos_cache).shape[1]
    sc = scale if scale is not None else 1.0 / np.sqrt(D)
    past_S = np.asarray(past_k).shape[2]
    plen = max(int(total_seq_len), past_S)
    pk = np.zeros((B, Nkv, plen, D))
    pv = np.zeros((B, Nkv, plen, D))
    q = qkv[..., :Nq * D].reshape(B, S, Nq, D)
    k = qkv[..., Nq * D:(Nq + Nkv) * D].reshape(B, S, Nkv, D)
    v = qkv[..., (Nq + Nkv) * D:].reshape(B, S, Nkv, D)
    r16 = (lambda a: a.astype(np.float16).astype(np.float64)) if f16_points else (lambda a: a)
    out = np.zeros((B, S, Nq, D))
    for b in range(B):
        past_len = max(int(seqlens_k[b]) + 1 - S, 0)
        pk[b, :, :past_len] = np.asarray(past_k, dtype=np.float64)[b, :, :past_len]
        pv[b, :, :past_len] = np.asarray(past_v, dtype=np.float64)[b, :, :past_len]
        pos = past_len + np.arange(S)
        c = np.asarray(cos_cache, dtype=np.float64)[pos][:, None, :]
        s_ = np.asarray(sin_cache, dtype=np.float64)[pos][:, None, :]
        qr = rope_neox(q[b], c, s_, rd)                       # [S, Nq, D]
        kr = rope_neox(k[b], c, s_, rd)                       # [S, Nkv, D]
        for si in range(S):
            pk[b, :, pos[si]] = r16(kr[si])
            pv[b, :, pos[si]] = r16(v[b, si])
        kq = np.repeat(pk[b], G, axis=0)                      # [Nq, plen, D], head h -> h // G
        vq = np.repeat(pv[b], G, axis=0)
        for si in range(S):
            tp = pos[si]
            scores = sc * np.einsum("htd,hd->ht", kq[:, :tp + 1], qr[si])
            scores = scores - scores.max(axis=1, keepdims=True)
            p = np.exp(scores)
            p /= p.sum(axis=1, keepdims=True)
            out[b, si] = np.einsum("ht,htd->hd", p, vq[:, :tp + 1])
    return out.reshape(B, S, Nq * D), pk, pv


def rope_caches(max_seq: int, rotary_dim: int, base: float = 10000.0, dtype=np.float16):
    """Standard RoPE angle tables ``[max_seq, rotary_dim/2]`` (fp16 as the graphs ship them)."""
    inv = 1.0 / base ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(dtype), np.sin(ang).astype(dtype)


def make_inputs(B: int, S: int, past: int, Nq: int, Nkv: int, D: int, *, max_seq: int = 256,
                rotary_dim: int | None = None, seed: int = 20260801, past_buffer: int | None = None):
    """Seeded GQA inputs: packed QKV, a past cache of ``past`` valid tokens in a buffer of
    ``past_buffer`` (default ``past``) positions, seqlens_k = past + S - 1 for every batch."""
    rng = np.random.default_rng(seed)
    pb = past if past_buffer is None else past_buffer
    qkv = rng.standard_normal((B, S, (Nq + 2 * Nkv) * D), dtype=np.float32).astype(np.float16)
    pk = rng.standard_normal((B, Nkv, pb, D), dtype=np.float32).astype(np.float16)
    pv = rng.standard_normal((B, Nkv, pb, D), dtype=np.float32).astype(np.float16)
    seqlens = np.full(B, past + S - 1, dtype=np.int32)
    rd = rotary_dim if rotary_dim is not None else D
    cos, sin = rope_caches(max_seq, rd)
    return {"qkv": qkv, "past_k": pk, "past_v": pv, "seqlens_k": seqlens,
            "total": np.int32(past + S), "cos": cos, "sin": sin}
