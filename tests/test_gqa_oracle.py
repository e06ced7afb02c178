"""Pin the GroupQueryAttention restatement (oracle/gqa.py) before it checks the GPU.

Against a library routine (torch.nn.functional.scaled_dot_product_attention in float64 on the
rotated tensors, causal, grouped heads), closed forms (one key returns its value; a zero angle
is the identity; a rotation keeps pair norms; rotation by a and then -a is the identity), and a
pure-Python brute force on a tiny case.  Each catches a plausible mistake: the wrong RoPE pairing
(interleaved vs halves), the KV head map, the causal bound, the past length from seqlens_k, the
scale.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import gqa as og


def test_single_key_returns_its_value():
    inp = og.make_inputs(1, 1, 0, 2, 1, 8, seed=1)
    attn, pk, pv = og.gqa(inp["qkv"], inp["past_k"], inp["past_v"], inp["seqlens_k"],
                          int(inp["total"]), inp["cos"], inp["sin"], 2, 1)
    v = inp["qkv"][0, 0, (2 + 1) * 8:].astype(np.float64)
    assert np.allclose(attn[0, 0, :8], v) and np.allclose(attn[0, 0, 8:], v)
    assert np.array_equal(pv[0, 0, 0], v)


def test_rotation_closed_forms():
    x = np.random.default_rng(0).standard_normal((3, 8))
    assert np.array_equal(og.rope_neox(x, np.ones(4), np.zeros(4), 8), x)
    a = 0.7
    r = og.rope_neox(x, np.full(4, math.cos(a)), np.full(4, math.sin(a)), 8)
    assert np.allclose(r[:, :4] ** 2 + r[:, 4:] ** 2, x[:, :4] ** 2 + x[:, 4:] ** 2)
    back = og.rope_neox(r, np.full(4, math.cos(a)), np.full(4, -math.sin(a)), 8)
    assert np.allclose(back, x)
    # partial rotary: dims past rotary_dim untouched
    p = og.rope_neox(x, np.full(2, math.cos(a)), np.full(2, math.sin(a)), 4)
    assert np.array_equal(p[:, 4:], x[:, 4:])


@pytest.mark.parametrize("B,S,past,Nq,Nkv,D", [(2, 3, 5, 4, 2, 16), (1, 1, 9, 4, 4, 8),
                                              (1, 4, 0, 6, 2, 8)])
def test_matches_torch_sdpa(B, S, past, Nq, Nkv, D):
    import torch

    inp = og.make_inputs(B, S, past, Nq, Nkv, D, seed=B + S + past)
    attn, pk, pv = og.gqa(inp["qkv"], inp["past_k"], inp["past_v"], inp["seqlens_k"],
                          int(inp["total"]), inp["cos"], inp["sin"], Nq, Nkv)
    qkv = inp["qkv"].astype(np.float64)
    q = qkv[..., :Nq * D].reshape(B, S, Nq, D)
    pos = past + np.arange(S)
    qr = og.rope_neox(q, inp["cos"][pos][None, :, None, :], inp["sin"][pos][None, :, None, :], D)
    T = past + S
    qt = torch.from_numpy(qr).permute(0, 2, 1, 3)                       # [B, Nq, S, D]
    kt = torch.from_numpy(pk[:, :, :T])
    vt = torch.from_numpy(pv[:, :, :T])
    mask = torch.from_numpy(np.arange(T)[None, :] <= pos[:, None])      # causal with an offset
    want = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask,
                                                            enable_gqa=True)
    want = want.permute(0, 2, 1, 3).reshape(B, S, Nq * D).numpy()
    assert np.max(np.abs(attn - want)) < 1e-12
    # the new keys land at past .. past + S - 1, rotated
    k = qkv[..., Nq * D:(Nq + Nkv) * D].reshape(B, S, Nkv, D)
    kr = og.rope_neox(k, inp["cos"][pos][None, :, None, :], inp["sin"][pos][None, :, None, :], D)
    assert np.allclose(pk[:, :, past:T], kr.transpose(0, 2, 1, 3))
    assert np.array_equal(pk[:, :, :past], inp["past_k"][:, :, :past].astype(np.float64))


def test_brute_force_tiny():
    B, S, past, Nq, Nkv, D = 1, 2, 2, 2, 1, 4
    inp = og.make_inputs(B, S, past, Nq, Nkv, D, seed=9)
    attn, _, _ = og.gqa(inp["qkv"], inp["past_k"], inp["past_v"], inp["seqlens_k"],
                        int(inp["total"]), inp["cos"], inp["sin"], Nq, Nkv)
    qkv = inp["qkv"].astype(float)
    cos = inp["cos"].astype(float)
    sin = inp["sin"].astype(float)

    def rot(vec, p):
        h = D // 2
        return ([vec[i] * cos[p][i] - vec[i + h] * sin[p][i] for i in range(h)]
                + [vec[i + h] * cos[p][i] + vec[i] * sin[p][i] for i in range(h)])

    keys = [list(inp["past_k"][0, 0, t].astype(float)) for t in range(past)]
    vals = [list(inp["past_v"][0, 0, t].astype(float)) for t in range(past)]
    for s in range(S):
        keys.append(rot(list(qkv[0, s, Nq * D:Nq * D + D]), past + s))
        vals.append(list(qkv[0, s, (Nq + 1) * D:(Nq + 2) * D]))
    for s in range(S):
        for h in range(Nq):
            qv = rot(list(qkv[0, s, h * D:(h + 1) * D]), past + s)
            sc = [sum(a * b for a, b in zip(qv, keys[t])) / math.sqrt(D) for t in range(past + s + 1)]
            m = max(sc)
            e = [math.exp(x - m) for x in sc]
            tot = sum(e)
            o = [sum(e[t] / tot * vals[t][d] for t in range(len(e))) for d in range(D)]
            assert np.max(np.abs(attn[0, s, h * D:(h + 1) * D] - np.array(o))) < 1e-12


def test_shared_buffer_convention_keeps_the_buffer_length():
    inp = og.make_inputs(1, 1, 3, 2, 2, 8, past_buffer=16, seed=4)
    _, pk, _ = og.gqa(inp["qkv"], inp["past_k"], inp["past_v"], inp["seqlens_k"],
                      int(inp["total"]), inp["cos"], inp["sin"], 2, 2)
    assert pk.shape[2] == 16
