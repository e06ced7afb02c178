"""GPU parity of GroupQueryAttention (mnb_gqa, mnb_session_run_gqa) against oracle/gqa.py.

Bars:
* attn_output: max relative error 2e-3 over significant elements (|ref| >= 0.1 RMS) and
  RMS-normalised error 2e-3 against the float64 oracle, with present K/V rounded to fp16 as
  stored (f16_points).  The fp16 output rounding alone is up to 4.9e-4.
* present_value and the copied past: bit-exact (they are copies).
* present_key at the new positions: the fp32 rotation rounded once to fp16, so within one fp16
  ulp of the float64 rotation (|diff| <= 2^-10 |ref| + 2^-24).
Positions of present past past_len + S are not compared (the kernel leaves them unwritten).

Cases follow the reference's tests (tests/ops/test_gqa.py: 8 query / 2 KV heads, head_dim 32,
partial rotary 16, past 0/4/16, decode; tests/ops/test_gqa_grouping.py: 32 / 8 heads, head_dim
128, prefill and the shared-buffer arena) and the Phi-3.5 shape (32 / 32 heads, head_dim 96).
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import gqa as og
from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu


def _inputs(B, S, seqlens, Nq, Nkv, D, *, past_buffer, rotary_dim=None, max_seq=None, seed=0):
    rng = np.random.default_rng(seed)
    rd = rotary_dim if rotary_dim is not None else D
    ms = max_seq if max_seq is not None else max(64, past_buffer + S)
    qkv = rng.standard_normal((B, S, (Nq + 2 * Nkv) * D), dtype=np.float32).astype(np.float16)
    pk = rng.standard_normal((B, Nkv, past_buffer, D), dtype=np.float32).astype(np.float16)
    pv = rng.standard_normal((B, Nkv, past_buffer, D), dtype=np.float32).astype(np.float16)
    cos, sin = og.rope_caches(ms, rd)
    return {"qkv": qkv, "past_k": pk, "past_v": pv, "seqlens_k": np.asarray(seqlens, np.int32),
            "cos": cos, "sin": sin, "rd": rd}


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check(inp, attn, prk, prv, Nq, Nkv, scale=None):
    B, S, _ = inp["qkv"].shape
    total = int(inp["past_k"].shape[2]) + S
    want, wk, wv = og.gqa(inp["qkv"], inp["past_k"], inp["past_v"], inp["seqlens_k"], total,
                          inp["cos"], inp["sin"], Nq, Nkv, scale=scale, rotary_dim=inp["rd"],
                          f16_points=True)
    attn = np.asarray(attn, dtype=np.float64)
    assert np.all(np.isfinite(attn))
    assert orc.max_rel_err_significant(attn, want) <= 2e-3
    assert orc.max_err_rms_normalised(attn, want) <= 2e-3
    for b in range(B):
        past_len = max(int(inp["seqlens_k"][b]) + 1 - S, 0)
        hi = past_len + S
        assert np.array_equal(prv[b, :, :past_len], inp["past_v"][b, :, :past_len])
        assert np.array_equal(prk[b, :, :past_len], inp["past_k"][b, :, :past_len])
        assert np.array_equal(prv[b, :, past_len:hi].astype(np.float64), wv[b, :, past_len:hi])
        ref = wk[b, :, past_len:hi]
        got = prk[b, :, past_len:hi].astype(np.float64)
        assert np.all(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 2.0 ** -24)


def _run(cuda, inp, Nq, Nkv, *, present_len=None, in_place=False, scale=None):
    import mnb
    import torch

    d = {k: _t(inp[k], cuda) for k in ("qkv", "past_k", "past_v", "seqlens_k", "cos", "sin")}
    kw = {}
    if in_place:
        kw = {"present_k": d["past_k"], "present_v": d["past_v"]}
    attn, prk, prv = mnb.gqa(d["qkv"], d["past_k"], d["past_v"], d["seqlens_k"], d["cos"],
                             d["sin"], num_heads=Nq, kv_num_heads=Nkv, rotary_dim=inp["rd"],
                             present_len=present_len, scale=scale, **kw)
    torch.cuda.synchronize()
    return attn.cpu().numpy(), prk.cpu().numpy(), prv.cpu().numpy()


@pytest.mark.parametrize("past", [0, 4, 16])
def test_reference_decode_shape(cuda, past):
    """tests/ops/test_gqa.py: 8 / 2 heads, head_dim 32, rotary 16, max_seq 64, growing cache."""
    inp = _inputs(1, 1, [past], 8, 2, 32, past_buffer=past, rotary_dim=16, max_seq=64, seed=past)
    _check(inp, *_run(cuda, inp, 8, 2), 8, 2)


@pytest.mark.parametrize("B,S,past,Nq,Nkv,D", [
    (1, 64, 0, 32, 8, 128),      # Llama-3 prefill
    (1, 17, 33, 32, 8, 128),     # prefill on a past
    (1, 1, 200, 32, 8, 128),     # decode, split keys
    (1, 1, 1000, 32, 32, 96),    # Phi-3.5 decode, split keys
    (1, 300, 0, 32, 32, 96),     # Phi-3.5 prefill, several row blocks
    (2, 5, 70, 4, 1, 64),        # multi-query
    (1, 32, 900, 16, 4, 128),    # prefill rows with split keys
    (1, 3, 9, 2, 2, 80),         # head_dim with a 16-deep tail
    (1, 2, 5, 2, 1, 16),
    (1, 9, 40, 4, 2, 256),
    (1, 130, 7, 2, 2, 48),
])
def test_matches_oracle(cuda, B, S, past, Nq, Nkv, D):
    inp = _inputs(B, S, [past + S - 1] * B, Nq, Nkv, D, past_buffer=past, seed=B * 7 + S + past)
    _check(inp, *_run(cuda, inp, Nq, Nkv), Nq, Nkv)


def test_ragged_batch_and_partial_rotary(cuda):
    """Per-batch past lengths inside a larger past buffer (seqlens_k differ), rotary 32 of 64."""
    seqlens = [2, 40, 17]                                # S = 3: past 0, 38, 15
    inp = _inputs(3, 3, seqlens, 8, 2, 64, past_buffer=48, rotary_dim=32, seed=5)
    _check(inp, *_run(cuda, inp, 8, 2), 8, 2)


def test_custom_scale(cuda):
    inp = _inputs(1, 4, [11], 4, 2, 64, past_buffer=8, seed=6)
    _check(inp, *_run(cuda, inp, 4, 2, scale=0.3), 4, 2, scale=0.3)


@pytest.mark.parametrize("S", [1, 5])
def test_shared_buffer_in_place(cuda, S):
    """Shared-buffer convention: present is the past tensor, updated at tok_pos in place; the
    buffer's tail past the valid tokens keeps its contents."""
    past_buf, valid = 64, 10
    inp = _inputs(2, S, [valid + S - 1, valid + S - 1], 32, 8, 128, past_buffer=past_buf, seed=S)
    before_k = inp["past_k"].copy()
    attn, prk, prv = _run(cuda, inp, 32, 8, present_len=past_buf, in_place=True)
    _check(inp, attn, prk, prv, 32, 8)
    assert np.array_equal(prk[:, :, valid + S:], before_k[:, :, valid + S:])


def test_shared_convention_separate_buffers(cuda):
    """present_len == past buffer extent but a separate present buffer: the past is copied."""
    inp = _inputs(1, 2, [12], 8, 2, 32, past_buffer=32, seed=8)
    _check(inp, *_run(cuda, inp, 8, 2, present_len=32), 8, 2)


def test_repeat_is_deterministic(cuda):
    inp = _inputs(1, 1, [700], 32, 8, 128, past_buffer=700, seed=9)
    a = _run(cuda, inp, 32, 8)
    b = _run(cuda, inp, 32, 8)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_session_host_io(cuda):
    """mnb_session_run_gqa with every tensor in host memory, growing then shared in place."""
    import mnb

    lib = mnb.load()
    Nq, Nkv, D = 8, 2, 32
    inp = _inputs(2, 3, [7, 5], Nq, Nkv, D, past_buffer=8, rotary_dim=16, max_seq=64, seed=10)
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    caches = C.c_void_p()
    try:
        node = mnb.gqa_problem(0, 0, 0, 0, 64, Nq, Nkv, D, 16)
        cos, sin = inp["cos"], inp["sin"]
        mnb.check(lib.mnb_gqa_caches_upload(sess, C.byref(node), cos.ctypes.data, cos.nbytes,
                                            sin.ctypes.data, sin.nbytes, C.byref(caches)))
        B, S = 2, 3
        attn = np.empty((B, S, Nq * D), np.float16)
        prk = np.zeros((B, Nkv, 8 + S, D), np.float16)
        prv = np.zeros((B, Nkv, 8 + S, D), np.float16)
        shape = mnb.gqa_problem(B, S, 8, 8 + S, 64, Nq, Nkv, D, 16)
        mnb.check(lib.mnb_session_run_gqa(sess, caches, C.byref(shape), inp["qkv"].ctypes.data,
                                          inp["past_k"].ctypes.data, inp["past_v"].ctypes.data,
                                          inp["seqlens_k"].ctypes.data, None, None,
                                          attn.ctypes.data, prk.ctypes.data, prv.ctypes.data, 0))
        _check(inp, attn, prk, prv, Nq, Nkv)
        # shared buffer, host memory, in place
        pk, pv = inp["past_k"].copy(), inp["past_v"].copy()
        shape = mnb.gqa_problem(B, S, 8, 8, 64, Nq, Nkv, D, 16)
        inp2 = dict(inp, seqlens_k=np.array([4, 2], np.int32))
        mnb.check(lib.mnb_session_run_gqa(sess, caches, C.byref(shape), inp["qkv"].ctypes.data,
                                          pk.ctypes.data, pv.ctypes.data,
                                          inp2["seqlens_k"].ctypes.data, None, None,
                                          attn.ctypes.data, pk.ctypes.data, pv.ctypes.data, 0))
        _check(inp2, attn, pk, pv, Nq, Nkv)
    finally:
        if caches.value:
            lib.mnb_gqa_caches_release(caches)
        lib.mnb_session_destroy(sess)


def test_session_per_call_caches(cuda):
    """A node without resident caches (cos/sin are graph inputs, as in the reference's
    tests/ops/test_gqa.py): the caches come with each call, from host or device memory."""
    import mnb
    import torch

    lib = mnb.load()
    Nq, Nkv, D = 8, 2, 32
    inp = _inputs(1, 1, [4], Nq, Nkv, D, past_buffer=4, rotary_dim=16, max_seq=64, seed=11)
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    rec = C.c_void_p()
    try:
        node = mnb.gqa_problem(0, 0, 0, 0, 64, Nq, Nkv, D, 16)
        mnb.check(lib.mnb_gqa_caches_upload(sess, C.byref(node), None, 0, None, 0, C.byref(rec)))
        shape = mnb.gqa_problem(1, 1, 4, 5, 64, Nq, Nkv, D, 16)
        attn = np.empty((1, 1, Nq * D), np.float16)
        prk = np.zeros((1, Nkv, 5, D), np.float16)
        prv = np.zeros((1, Nkv, 5, D), np.float16)
        args = [inp["qkv"].ctypes.data, inp["past_k"].ctypes.data, inp["past_v"].ctypes.data,
                inp["seqlens_k"].ctypes.data]
        # resident caches absent and none passed: refused
        assert lib.mnb_session_run_gqa(sess, rec, C.byref(shape), *args, None, None,
                                       attn.ctypes.data, prk.ctypes.data, prv.ctypes.data, 0) != 0
        mnb.check(lib.mnb_session_run_gqa(sess, rec, C.byref(shape), *args, inp["cos"].ctypes.data,
                                          inp["sin"].ctypes.data, attn.ctypes.data,
                                          prk.ctypes.data, prv.ctypes.data, 0))
        _check(inp, attn, prk, prv, Nq, Nkv)
        cd, sd = _t(inp["cos"], cuda), _t(inp["sin"], cuda)
        attn2 = np.empty_like(attn)
        mnb.check(lib.mnb_session_run_gqa(sess, rec, C.byref(shape), *args, cd.data_ptr(),
                                          sd.data_ptr(), attn2.ctypes.data, prk.ctypes.data,
                                          prv.ctypes.data, mnb.GQA_ON_DEVICE_CACHES))
        torch.cuda.synchronize()
        assert np.array_equal(attn, attn2)
    finally:
        if rec.value:
            lib.mnb_gqa_caches_release(rec)
        lib.mnb_session_destroy(sess)
