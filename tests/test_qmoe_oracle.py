"""Pin the QMoE restatement (oracle/qmoe.py) before it checks the GPU.

ORT's QMoE is not available here (and refuses the one real graph the reference has seen), so
nothing pins this op's values against ORT: parity is unpinned and the restatement is the build's
declared definition.  What these checks pin is that the restatement computes that definition:
each is chosen so a plausible mistake fails one of them — gate and linear swapped, the wrong
interleave, a dropped bias, the clamp on the wrong operand, softmax before vs after top-k,
renormalisation missing, weights applied to the wrong expert, per-channel scales indexed as
blocks.  Expected values come from closed forms, a pure-Python brute force, or the pinned
MatMulNBits oracle — not from re-running the vectorised formula.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import matmul_nbits as orc
from oracle import qmoe as q


def test_swiglu_closed_forms():
    # gate = 0 -> 0 whatever the linear half
    assert q.swiglu(0.0, 5.0, 1.702, 1.0, 7.0) == 0.0
    # linear = -beta -> 0
    assert q.swiglu(2.0, -1.0, 1.702, 1.0, 7.0) == 0.0
    # gate 1, linear 0, alpha 1, beta 1: 1 * sigmoid(1) * 1
    assert abs(q.swiglu(1.0, 0.0, 1.0, 1.0, None) - 1.0 / (1.0 + math.exp(-1.0))) < 1e-15
    # the clamp caps the gate from above only and the linear half on both sides
    got = q.swiglu(100.0, -50.0, 1.702, 1.0, 7.0)
    want = 7.0 / (1.0 + math.exp(-1.702 * 7.0)) * (-7.0 + 1.0)
    assert abs(got - want) < 1e-12
    got = q.swiglu(-100.0, 3.0, 1.0, 0.0, 7.0)      # a large negative gate is not clamped
    assert abs(got - (-100.0 / (1.0 + math.exp(100.0)) * 3.0)) < 1e-40
    # no limit: nothing is clamped
    assert abs(q.swiglu(9.0, 9.0, 1.0, 0.0, None) - 9.0 / (1.0 + math.exp(-9.0)) * 9.0) < 1e-12


def test_routing_topk_softmax_and_ties():
    logits = np.array([[0.0, 2.0, 1.0, 2.0],         # tie between experts 1 and 3
                       [3.0, -1.0, 0.5, 0.25]])
    ex, w = q.route(logits, 2, normalize=True)
    assert ex.tolist() == [[1, 3], [0, 2]]
    assert np.allclose(w.sum(axis=1), 1.0)
    assert np.allclose(w[0], [0.5, 0.5])
    # renormalised top-k == softmax over the chosen logits
    want = np.exp([3.0, 0.5]) / np.exp([3.0, 0.5]).sum()
    assert np.allclose(w[1], want, rtol=0, atol=1e-15)
    # without renormalisation the weights are the full softmax probabilities
    _, w0 = q.route(logits, 2, normalize=False)
    p = np.exp(logits[1]) / np.exp(logits[1]).sum()
    assert np.allclose(w0[1], [p[0], p[2]], rtol=0, atol=1e-15)


def _nibble(b, idx):
    byte = int(b[idx // 2])
    return (byte & 0xF) if idx % 2 == 0 else (byte >> 4)


def test_brute_force_tiny_case():
    """Pure-Python loops over bytes, no vectorised helper, on 3 tokens x 4 experts, top-2."""
    T, H, I, E, k, bs = 3, 32, 32, 4, 2, 32
    inp = q.make_qmoe_inputs(T, H, I, E, block_size=bs, seed=7)
    alpha, beta, limit = 1.702, 1.0, 7.0
    x = inp["x"].astype(float)
    lg = inp["logits"].astype(float)
    y = [[0.0] * H for _ in range(T)]
    for t in range(T):
        mx = max(lg[t])
        ex = [math.exp(v - mx) for v in lg[t]]
        sm = sum(ex)
        p = [v / sm for v in ex]
        chosen = sorted(range(E), key=lambda e: (-p[e], e))[:k]
        tot = sum(p[e] for e in chosen)
        for e in chosen:
            wgt = p[e] / tot
            h = []
            for n in range(2 * I):
                acc = 0.0
                for kk in range(H):
                    qv = _nibble(inp["fc1"][e, n], kk)
                    s = float(inp["fc1_scales"][e, n, kk // bs])
                    acc += x[t][kk] * (qv - 8) * s
                h.append(acc + float(inp["fc1_bias"][e, n]))
            act = []
            for i in range(I):
                g, lin = min(h[2 * i], limit), min(max(h[2 * i + 1], -limit), limit)
                act.append(g / (1.0 + math.exp(-alpha * g)) * (lin + beta))
            for c in range(H):
                acc = 0.0
                for i in range(I):
                    qv = _nibble(inp["fc2"][e, c], i)
                    s = float(inp["fc2_scales"][e, c, i // bs])
                    acc += act[i] * (qv - 8) * s
                y[t][c] += wgt * (acc + float(inp["fc2_bias"][e, c]))
    got = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                 inp["fc2_scales"], k=k, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"],
                 fc2_bias=inp["fc2_bias"], fusion=1, alpha=alpha, beta=beta, limit=limit)
    assert np.max(np.abs(got - np.array(y))) < 1e-12


def test_one_expert_is_two_chained_matmul_nbits():
    T, H, I, bs = 5, 64, 32, 32
    inp = q.make_qmoe_inputs(T, H, I, 1, block_size=bs, seed=11)
    got = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                 inp["fc2_scales"], k=1, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"],
                 fc2_bias=inp["fc2_bias"], fusion=2, alpha=1.0, beta=0.0, limit=None)
    B1 = inp["fc1"][0].reshape(2 * I, H // bs, bs // 2)
    h = orc.matmul_nbits(inp["x"], B1, inp["fc1_scales"][0].reshape(-1), None, 2 * I, H, 4, bs)
    h = h.astype(np.float64) + inp["fc1_bias"][0]
    g, lin = h[:, :I], h[:, I:]
    act = g / (1.0 + np.exp(-g)) * lin                           # SiLU(gate) * linear
    B2 = inp["fc2"][0].reshape(H, I // bs, bs // 2)
    o = orc.matmul_nbits(act, B2, inp["fc2_scales"][0].reshape(-1), None, H, I, 4, bs)
    want = o.astype(np.float64) + inp["fc2_bias"][0]
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


def test_expert_relabelling_invariance():
    T, H, I, E, bs = 6, 64, 32, 5, 32
    inp = q.make_qmoe_inputs(T, H, I, E, block_size=bs, seed=3)
    kw = dict(k=3, inter=I, block_size=bs, fusion=1)
    y = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
               inp["fc2_scales"], fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"], **kw)
    perm = np.array([3, 0, 4, 1, 2])
    y2 = q.qmoe(inp["x"], inp["logits"][:, perm], inp["fc1"][perm], inp["fc1_scales"][perm],
                inp["fc2"][perm], inp["fc2_scales"][perm], fc1_bias=inp["fc1_bias"][perm],
                fc2_bias=inp["fc2_bias"][perm], **kw)
    assert np.max(np.abs(y - y2)) < 1e-12


def test_interleaved_and_concatenated_layouts_agree():
    T, H, I, E, bs = 4, 64, 32, 3, 32
    inp = q.make_qmoe_inputs(T, H, I, E, block_size=bs, seed=5)
    kw = dict(k=2, inter=I, block_size=bs)
    y1 = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                inp["fc2_scales"], fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"],
                fusion=1, **kw)
    # rows 0,2,4,.. are gates and 1,3,5,.. linears in the interleaved form
    order = np.concatenate([np.arange(0, 2 * I, 2), np.arange(1, 2 * I, 2)])
    y2 = q.qmoe(inp["x"], inp["logits"], inp["fc1"][:, order], inp["fc1_scales"][:, order],
                inp["fc2"], inp["fc2_scales"], fc1_bias=inp["fc1_bias"][:, order],
                fc2_bias=inp["fc2_bias"], fusion=2, **kw)
    assert np.max(np.abs(y1 - y2)) < 1e-12
    # and a swapped split is not the same function
    y3 = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                inp["fc2_scales"], fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"],
                fusion=2, **kw)
    assert np.max(np.abs(y1 - y3)) > 1e-3


def test_per_channel_scales_equal_replicated_block_scales():
    T, H, I, E, bs = 3, 64, 32, 2, 32
    inp = q.make_qmoe_inputs(T, H, I, E, per_channel=True, seed=9)
    kw = dict(k=1, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"])
    y = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
               inp["fc2_scales"], **kw)
    s1 = np.repeat(inp["fc1_scales"][:, :, None], H // bs, axis=2)
    s2 = np.repeat(inp["fc2_scales"][:, :, None], I // bs, axis=2)
    y2 = q.qmoe(inp["x"], inp["logits"], inp["fc1"], s1, inp["fc2"], s2, **kw)
    assert np.max(np.abs(y - y2)) == 0.0


def test_output_bias_is_linear_under_normalised_routing():
    T, H, I, E, bs = 4, 64, 32, 4, 32
    inp = q.make_qmoe_inputs(T, H, I, E, block_size=bs, seed=13)
    kw = dict(k=2, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"], normalize=True)
    y = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
               inp["fc2_scales"], fc2_bias=inp["fc2_bias"], **kw)
    c = np.linspace(-1.0, 1.0, H)
    y2 = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                inp["fc2_scales"], fc2_bias=inp["fc2_bias"].astype(np.float64) + c, **kw)
    assert np.max(np.abs((y2 - y) - c)) < 1e-12


@pytest.mark.parametrize("fusion", [1, 2])
def test_f16_points_stay_close_to_the_exact_form(fusion):
    T, H, I, E, bs = 8, 128, 64, 4, 32
    inp = q.make_qmoe_inputs(T, H, I, E, block_size=bs, seed=17)
    kw = dict(k=2, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"],
              fusion=fusion)
    y = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
               inp["fc2_scales"], **kw)
    y16 = q.qmoe(inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"],
                 inp["fc2_scales"], f16_points=True, **kw)
    assert 0 < orc.max_err_rms_normalised(y16, y) < 5e-3
