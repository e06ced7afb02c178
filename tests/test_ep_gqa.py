"""com.microsoft::GroupQueryAttention through the plugin EP, driven by the mock ORT host.

CPU: the claim predicate — the reference's claimed form (rust/src/ops/attention.rs:172-269:
packed QKV, KV cache, seqlens_k, do_rotary=1 half-rotation RoPE from inputs 7/8, numerics
options off, inputs 10..15 absent) and the translate-time refusals (attention.rs:420-560: head
grouping, the rotary width from rotary_embedding_dim or cos_cache's second dimension, fp16).
GPU: Compile uploads constant cos/sin caches once; Compute runs the GQA kernels with every
tensor in host memory (or in HBM through the EP's allocator), checked against oracle/gqa.py at
the bars of test_gpu_gqa.py.  The models follow the reference's tests/ops/test_gqa.py (8 / 2
heads, head_dim 32, rotary 16, max_seq 64, present [B, 2, past + 1, 32]).
"""

from __future__ import annotations

import numpy as np
import pytest

import mock_host as mh
from oracle import gqa as og
from oracle import matmul_nbits as orc

REF = dict(num_heads=8, kv_num_heads=2, head_dim=32, rotary_dim=16, max_seq=64)


@pytest.fixture
def host():
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0, "an OrtStatus was leaked"
    assert mh.lib().mock_bad_status_release() == 0, "an OrtStatus was released twice"


def _caches(max_seq=64, rd=16):
    cos, sin = og.rope_caches(max_seq, rd)
    return {"cos": cos, "sin": sin}


def _claim(host, shape=None, **kw):
    host.reset()
    s = dict(REF, B=1, S=-1, past_shape_len=-1, present_len=-1)
    s.update(shape or {})
    mh.add_gqa(host, "gqa", _caches(s["max_seq"], s["rotary_dim"]), **s, **kw)
    return host.get_capability()


@pytest.mark.parametrize("shape,kw", [
    ({}, {}),                                                        # the reference's model
    ({"present_len": 5, "past_shape_len": 4, "S": 1}, {}),           # declared growing extent
    ({"present_len": 64, "past_shape_len": 64}, {}),                 # shared buffer
    (dict(num_heads=32, kv_num_heads=32, head_dim=96, rotary_dim=96, max_seq=4096), {}),  # Phi
    (dict(num_heads=32, kv_num_heads=8, head_dim=128, rotary_dim=128, max_seq=512), {}),  # Llama
    ({}, {"attrs_over": {"smooth_softmax": -1}}),                    # Phi-3.5's "unset" sentinel
    ({}, {"attrs_over": {"scale": 0.125, "rotary_embedding_dim": 16}}),
    ({}, {"const_caches": False}),                                   # caches as graph inputs
])
def test_claimed(host, shape, kw):
    assert host.create_ep(-1) == 0
    assert _claim(host, shape, **kw) == (1, ["gqa:drop"])


@pytest.mark.parametrize("case,shape,kw", [
    ("separate_kv", {}, {"separate_kv": True}),
    ("no_rotary", {}, {"attrs_over": {"do_rotary": 0}}),
    ("interleaved", {}, {"attrs_over": {"rotary_interleaved": 1}}),
    ("window", {}, {"attrs_over": {"local_window_size": 128}}),
    ("softcap", {}, {"attrs_over": {"softcap": 30.0}}),
    ("smooth_softmax", {}, {"attrs_over": {"smooth_softmax": 1}}),
    ("qk_output", {}, {"attrs_over": {"qk_output": 1}}),
    ("kv_bits", {}, {"attrs_over": {"kv_cache_bit_width": 8}}),
    ("k_quant", {}, {"attrs_over": {"k_quant_type": "PER_TENSOR"}}),
    ("grouping", dict(num_heads=6, kv_num_heads=4), {}),
    ("head_dim_40", dict(head_dim=40, rotary_dim=40), {}),
    ("rotary_wider_than_head", {}, {"attrs_over": {"rotary_embedding_dim": 64}}),
    ("odd_rotary", {}, {"attrs_over": {"rotary_embedding_dim": 15}}),
    ("qkv_fp32", {}, {"qkv_elem": mh.FLOAT}),
    ("seqlens_fp32", {}, {"seqlens_elem": mh.FLOAT}),
    ("attention_bias", {}, {"extra_inputs": [("gqa_bias@10", mh.FLOAT16, (1, 8, 1, 1))]}),
    ("q_norm", {}, {"extra_inputs": [("gqa_qn@14", mh.FLOAT16, (32,))]}),
    ("output_qk", {}, {"outputs": ["gqa_out", "gqa_present_k", "gqa_present_v", "gqa_qk"]}),
    ("no_present", {}, {"outputs": ["gqa_out", "", ""]}),
    ("cache_width_mismatch", {}, {"attrs_over": {"rotary_embedding_dim": 8}}),
])
def test_declined(host, case, shape, kw):
    assert host.create_ep(-1) == 0
    host.reset()
    host.value("gqa_qk", mh.FLOAT16, (1, 8, 1, 1))
    s = dict(REF, B=1, S=-1, past_shape_len=-1, present_len=-1)
    s.update(shape)
    mh.add_gqa(host, "gqa", _caches(s["max_seq"], s["rotary_dim"]), **s, **kw)
    n, claimed = host.get_capability()
    assert n == 0 and claimed == [], case


def test_unrecoverable_rotary_width_is_declined(host):
    """No rotary_embedding_dim and a cos_cache without a second dimension: the reference refuses
    rather than assume head_dim (attention.rs:450-470)."""
    assert host.create_ep(-1) == 0
    host.reset()
    mh.add_gqa(host, "gqa", _caches(), **dict(REF, B=1, S=1, past_shape_len=4, present_len=5),
               cos_rank2=False)
    assert host.get_capability() == (0, [])


# ---- GPU: Compile + Compute ---------------------------------------------------------------------

@pytest.fixture
def gpu_host(cuda):
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    assert h.supported_devices(n_amd=1) == 1
    assert h.create_ep(0) == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0
    assert mh.lib().mock_bad_status_release() == 0


def _data(B, S, past, Nq, Nkv, D, rd, max_seq, seqlens=None, seed=0):
    rng = np.random.default_rng(seed)
    d = {"qkv": rng.standard_normal((B, S, (Nq + 2 * Nkv) * D), dtype=np.float32).astype(np.float16),
         "past_k": (0.1 * rng.standard_normal((B, Nkv, past, D), dtype=np.float32)).astype(np.float16),
         "past_v": (0.1 * rng.standard_normal((B, Nkv, past, D), dtype=np.float32)).astype(np.float16),
         "seqlens_k": np.asarray(seqlens if seqlens is not None else [past + S - 1] * B, np.int32)}
    d.update(_caches(max_seq, rd))
    return d


def _check(d, attn, prk, prv, Nq, Nkv, rd, scale=None):
    B, S, _ = d["qkv"].shape
    want, wk, wv = og.gqa(d["qkv"], d["past_k"], d["past_v"], d["seqlens_k"],
                          d["past_k"].shape[2] + S, d["cos"], d["sin"], Nq, Nkv, scale=scale,
                          rotary_dim=rd, f16_points=True)
    attn = attn.astype(np.float64)
    assert orc.max_rel_err_significant(attn, want) <= 2e-3
    assert orc.max_err_rms_normalised(attn, want) <= 2e-3
    for b in range(B):
        pl = max(int(d["seqlens_k"][b]) + 1 - S, 0)
        assert np.array_equal(prk[b, :, :pl], d["past_k"][b, :, :pl])
        assert np.array_equal(prv[b, :, :pl], d["past_v"][b, :, :pl])
        assert np.array_equal(prv[b, :, pl:pl + S].astype(np.float64), wv[b, :, pl:pl + S])
        ref = wk[b, :, pl:pl + S]
        assert np.all(np.abs(prk[b, :, pl:pl + S] - ref) <= 2.0 ** -10 * np.abs(ref) + 2.0 ** -24)


def _feed_all(h, names, d, const_caches, device=False):
    feed = h.feed_device if device else h.feed
    feed(names["qkv"], d["qkv"])
    feed(names["past_k"], d["past_k"])
    feed(names["past_v"], d["past_v"])
    feed(names["seqlens"], d["seqlens_k"])
    h.feed(names["total"], np.array(d["past_k"].shape[2] + d["qkv"].shape[1], np.int32))
    if not const_caches:
        feed(names["cos"], d["cos"])
        feed(names["sin"], d["sin"])


@pytest.mark.gpu
@pytest.mark.parametrize("past,const_caches", [(0, True), (4, True), (16, True), (4, False)])
def test_reference_model_matches_oracle(gpu_host, past, const_caches):
    """tests/ops/test_gqa.py's one-node model: decode, growing present [1, 2, past + 1, 32]."""
    print(f"[gpu] ep gqa reference model past={past} const={const_caches}", flush=True)
    d = _data(1, 1, past, 8, 2, 32, 16, 64, seed=past)
    gpu_host.reset()
    names = mh.add_gqa(gpu_host, "gqa", d, **dict(REF, B=-1, S=-1, past_shape_len=past,
                                                  present_len=past + 1),
                       const_caches=const_caches)
    assert gpu_host.get_capability() == (1, ["gqa:drop"])
    assert gpu_host.compile() == 0, mh.err()
    before = mh.EP_COUNT()
    _feed_all(gpu_host, names, d, const_caches)
    assert gpu_host.compute(0) == 0, mh.err()
    assert mh.EP_COUNT() == before + 1
    attn = gpu_host.fetch(names["out"], np.float16, 8 * 32)
    prk = gpu_host.fetch(names["present_k"], np.float16, 2 * (past + 1) * 32)
    prv = gpu_host.fetch(names["present_v"], np.float16, 2 * (past + 1) * 32)
    assert attn.shape == (1, 1, 256) and prk.shape == (1, 2, past + 1, 32) == prv.shape
    _check(d, attn, prk, prv, 8, 2, 16)


@pytest.mark.gpu
def test_prefill_symbolic_present_grows(gpu_host):
    """Llama-3 heads (32 / 8, head_dim 128), a symbolic present extent: present = past + S."""
    print("[gpu] ep gqa prefill symbolic present", flush=True)
    B, S, past = 2, 37, 20
    d = _data(B, S, past, 32, 8, 128, 128, 256, seed=3)
    gpu_host.reset()
    names = mh.add_gqa(gpu_host, "gqa", d, num_heads=32, kv_num_heads=8, head_dim=128,
                       rotary_dim=128, max_seq=256, B=-1, S=-1, past_shape_len=-1, present_len=-1)
    assert gpu_host.get_capability() == (1, ["gqa:drop"])
    assert gpu_host.compile() == 0, mh.err()
    _feed_all(gpu_host, names, d, True)
    assert gpu_host.compute(0) == 0, mh.err()
    attn = gpu_host.fetch(names["out"], np.float16, B * S * 32 * 128)
    n = B * 8 * (past + S) * 128
    prk = gpu_host.fetch(names["present_k"], np.float16, n)
    prv = gpu_host.fetch(names["present_v"], np.float16, n)
    assert prk.shape == (B, 8, past + S, 128)
    _check(d, attn, prk, prv, 32, 8, 128)


@pytest.mark.gpu
def test_declared_shared_buffer(gpu_host):
    """present declared with the past buffer's extent (shared-buffer convention), ragged valid
    lengths inside it; ORT hands separate buffers, so the past is copied."""
    print("[gpu] ep gqa shared buffer", flush=True)
    B, S, buf = 2, 2, 32
    d = _data(B, S, buf, 8, 2, 32, 16, 64, seqlens=[9, 20], seed=4)
    gpu_host.reset()
    names = mh.add_gqa(gpu_host, "gqa", d, **dict(REF, B=B, S=S, past_shape_len=buf,
                                                  present_len=buf))
    assert gpu_host.get_capability() == (1, ["gqa:drop"])
    assert gpu_host.compile() == 0, mh.err()
    _feed_all(gpu_host, names, d, True)
    assert gpu_host.compute(0) == 0, mh.err()
    attn = gpu_host.fetch(names["out"], np.float16, B * S * 256)
    prk = gpu_host.fetch(names["present_k"], np.float16, B * 2 * buf * 32)
    prv = gpu_host.fetch(names["present_v"], np.float16, B * 2 * buf * 32)
    assert prk.shape == (B, 2, buf, 32)
    _check(d, attn, prk, prv, 8, 2, 16)


@pytest.mark.gpu
def test_wrong_past_shape_is_invalid_argument(gpu_host):
    d = _data(1, 1, 4, 8, 2, 32, 16, 64)
    gpu_host.reset()
    names = mh.add_gqa(gpu_host, "gqa", d, **dict(REF, B=-1, S=-1, past_shape_len=-1,
                                                  present_len=-1))
    assert gpu_host.get_capability()[0] == 1
    assert gpu_host.compile() == 0, mh.err()
    _feed_all(gpu_host, names, d, True)
    gpu_host.feed(names["past_k"], np.zeros((1, 3, 4, 32), np.float16))   # 3 KV heads, not 2
    assert gpu_host.compute(0) == mh.ORT_INVALID_ARGUMENT


@pytest.fixture
def dm_host(cuda, monkeypatch):
    monkeypatch.setenv("MI355X_EP_DEVICE_MEMORY", "1")
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    assert h.supported_devices(n_amd=1) == 1
    assert h.create_ep(0) == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0
    assert mh.lib().mock_live_memory_infos() == 0


@pytest.mark.gpu
def test_device_resident_io(dm_host):
    """qkv, the KV cache and seqlens_k in HBM through the EP's allocator; outputs allocated in
    HBM; Phi-3.5 heads (32 / 32, head_dim 96)."""
    print("[gpu] ep gqa device I/O", flush=True)
    B, S, past = 1, 1, 300
    d = _data(B, S, past, 32, 32, 96, 96, 512, seed=6)
    dm_host.reset()
    names = mh.add_gqa(dm_host, "gqa", d, num_heads=32, kv_num_heads=32, head_dim=96,
                       rotary_dim=96, max_seq=512, B=-1, S=-1, past_shape_len=-1, present_len=-1)
    assert dm_host.get_capability() == (1, ["gqa:drop"])
    assert dm_host.compile() == 0, mh.err()
    assert dm_host.device_io_setup(0) == 0, mh.err()
    _feed_all(dm_host, names, d, True, device=True)
    assert dm_host.compute(0) == 0, mh.err()
    attn = dm_host.fetch(names["out"], np.float16, 32 * 96)
    n = 32 * (past + 1) * 96
    prk = dm_host.fetch(names["present_k"], np.float16, n)
    prv = dm_host.fetch(names["present_v"], np.float16, n)
    _check(d, attn, prk, prv, 32, 32, 96)
