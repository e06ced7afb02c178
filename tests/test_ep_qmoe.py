"""com.microsoft::QMoE through the plugin EP, driven by the mock ORT host.

CPU: the claim predicate (the reference's fingerprint, rust/src/ops/moe.rs:40-118, widened to
top-k <= 8 and narrowed to SwiGLU; the gpt-oss attribute set of docs/OP_COVERAGE.md:831-835 is
claimed) and its declines, read through ORT's int, float and string attribute calls.
GPU: Compile uploads the expert tensors once (per-channel or block scales), Compute runs the
fused QMoE on host tensors; checked against oracle/qmoe.py at the bars of test_gpu_qmoe.py
(parity against ORT's QMoE is unpinned: ORT is absent).
"""

from __future__ import annotations

import numpy as np
import pytest

import mock_host as mh
from oracle import matmul_nbits as orc
from oracle import qmoe as oq


@pytest.fixture
def host():
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0, "an OrtStatus was leaked"
    assert mh.lib().mock_bad_status_release() == 0, "an OrtStatus was released twice"


def _inputs(per_channel=False, bias=True, E=8, H=256, I=128, bs=32):
    return oq.make_qmoe_inputs(4, H, I, E, block_size=bs, per_channel=per_channel, bias=bias,
                               seed=21)


def _claim(host, inp, **kw):
    host.reset()
    mh.add_qmoe(host, "moe", inp, **kw)
    return host.get_capability()


def test_gpt_oss_attribute_set_is_claimed(host):
    assert host.create_ep(-1) == 0
    assert _claim(host, _inputs(), k=4, x_shape=(4, 256)) == (1, ["moe:drop"])


@pytest.mark.parametrize("per_channel,bias,router", [(True, True, mh.FLOAT16),
                                                     (False, False, mh.FLOAT),
                                                     (True, False, mh.FLOAT)])
def test_claimed_forms(host, per_channel, bias, router):
    assert host.create_ep(-1) == 0
    inp = _inputs(per_channel=per_channel, bias=bias)
    assert _claim(host, inp, k=2, x_shape=(-1, 256), router_elem=router)[0] == 1


def test_gpt_oss_recorded_form_is_claimed_when_asked(host):
    """gpt-oss-20b's QMoE as recorded (docs/OP_COVERAGE.md:831-835): 11 declared inputs, 8
    occupied, swiglu_fusion = 0, per-channel scales.  Read as fc1's 2I channels holding the
    interleaved gate/linear pairs, it runs as fusion 1 (ORT's CPU kernel refuses the attribute
    value, docs/OP_COVERAGE.md:2199-2204, and the reference's census asks for a re-export with 1
    over the same weights, tests/ops/test_phi35.py:1445-1453).  That reading is an inference with
    parity unpinned, so it is claimed only under ep.qmoe_unfused_as_interleaved=1 and declined
    by default."""
    host.option("ep.qmoe_unfused_as_interleaved", "1")
    assert host.create_ep(-1) == 0
    assert _claim(host, _inputs(per_channel=True), k=4, x_shape=(4, 256),
                  extra_inputs=["", "", ""], attrs_over={"swiglu_fusion": 0}) == (1, ["moe:drop"])


def test_gpt_oss_recorded_form_is_declined_by_default(host):
    assert host.create_ep(-1) == 0
    assert _claim(host, _inputs(per_channel=True), k=4, x_shape=(4, 256),
                  extra_inputs=["", "", ""], attrs_over={"swiglu_fusion": 0}) == (0, [])


def test_concatenated_swiglu_and_no_limit_are_claimed(host):
    assert host.create_ep(-1) == 0
    inp = _inputs()
    assert _claim(host, inp, k=1, x_shape=(4, 256),
                  attrs_over={"swiglu_fusion": 2, "swiglu_limit": None})[0] == 1


@pytest.mark.parametrize("case,kw", [
    ("top9", dict(k=9)),
    ("k_above_experts", dict(k=5, inp={"E": 4})),
    ("relu", dict(attrs_over={"activation_type": "relu"})),
    ("silu", dict(attrs_over={"activation_type": "silu"})),
    ("unfused_swiglu_with_fc3", dict(attrs_over={"swiglu_fusion": 0},
                                     extra_inputs=["moe_fc1", "moe_fc1_scales"])),
    ("swiglu_fusion_3", dict(attrs_over={"swiglu_fusion": 3})),
    ("sparse_mixer", dict(attrs_over={"use_sparse_mixer": 1})),
    ("eight_bit", dict(attrs_over={"expert_weight_bits": 8})),
    ("fp4", dict(attrs_over={"quant_type": "fp4"})),
    ("block16", dict(attrs_over={"block_size": 16})),
    ("prepacked", dict(attrs_over={"weights_prepacked": 1})),
    ("x_not_h", dict(x_shape=(4, 128))),
    ("int_router", dict(router_elem=mh.INT32)),
    ("non_constant_weights", dict(const_weights=False)),
    ("fc3_present", dict(extra_inputs=["moe_fc1"])),
])
def test_declines(host, case, kw):
    assert host.create_ep(-1) == 0
    args = dict(k=4, x_shape=(4, 256))
    args.update(kw)
    inp = _inputs(**args.pop("inp", {}))
    n, claimed = _claim(host, inp, **args)
    assert n == 0 and claimed == [], case


def test_missing_k_is_declined(host):
    assert host.create_ep(-1) == 0
    inp = _inputs()
    host.reset()
    mh.add_qmoe(host, "moe", inp, k=4, x_shape=(4, 256), attrs_over={"k": None})
    assert host.get_capability()[0] == 0


def test_qmoe_and_matmul_nbits_fuse_one_island_each(host):
    assert host.create_ep(-1) == 0
    host.reset()
    mh.add_qmoe(host, "moe", _inputs(), k=4, x_shape=(4, 256))
    mm = orc.make_inputs(4, 32, 256, with_zp=True, seed=2)
    mh.add_matmul_nbits(host, "mm", mm, 32, 256, 4, 32, (4, 256))
    n, claimed = host.get_capability()
    assert n == 2 and sorted(claimed) == ["mm:drop", "moe:drop"]


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


@pytest.mark.gpu
@pytest.mark.parametrize("lead,H,I,E,k,per_channel,fusion", [
    ((4,), 256, 128, 8, 2, False, 1),
    ((2, 5), 512, 256, 16, 4, True, 2),
    ((64,), 2880, 2880, 32, 4, True, 1),               # gpt-oss-20b expert block
    ((64,), 2880, 2880, 32, 4, True, 0),               # ... with its recorded swiglu_fusion = 0
])
def test_ep_qmoe_matches_oracle(gpu_host, lead, H, I, E, k, per_channel, fusion):
    print(f"[gpu] ep qmoe lead={lead} H={H} I={I} E={E} k={k} pc={per_channel} f={fusion}",
          flush=True)
    T = int(np.prod(lead))
    inp = oq.make_qmoe_inputs(T, H, I, E, per_channel=per_channel, seed=T + E)
    if fusion == 0:
        # the inferred interleaved reading of the recorded form is opt-in: a second EP on the
        # same host, created after the option is set
        gpu_host.option("ep.qmoe_unfused_as_interleaved", "1")
        assert gpu_host.create_ep(0) == 0, mh.err()
    gpu_host.reset()
    x_name, r_name, y_name = mh.add_qmoe(gpu_host, "moe", inp, k=k, x_shape=lead + (H,),
                                         attrs_over={"swiglu_fusion": fusion},
                                         extra_inputs=["", "", ""] if fusion == 0 else ())
    assert gpu_host.get_capability() == (1, ["moe:drop"])
    assert gpu_host.compile() == 0, mh.err()
    before = mh.EP_COUNT()
    gpu_host.feed(x_name, inp["x"].reshape(lead + (H,)))
    gpu_host.feed(r_name, inp["logits"])
    assert gpu_host.compute(0) == 0, mh.err()
    assert mh.EP_COUNT() == before + 1
    y = gpu_host.fetch(y_name, np.float16, T * H)
    assert y.shape == lead + (H,)
    kw = dict(k=k, inter=I, block_size=32, fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"],
              fusion=fusion or 1)                 # fusion 0 (gpt-oss) runs interleaved
    args = (inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"], inp["fc2_scales"])
    ref16 = oq.qmoe(*args, f16_points=True, **kw)
    ref = oq.qmoe(*args, **kw)
    y = y.reshape(T, H).astype(np.float32)
    assert orc.max_err_rms_normalised(y, ref16) <= 2e-3
    assert orc.max_rel_err_significant(y, ref16) <= 1e-2
    assert orc.max_err_rms_normalised(y, ref) <= 5e-3


@pytest.mark.gpu
def test_ep_qmoe_strip_major_weights_option(gpu_host):
    """ep.strip_major_weights (on by default): Compile also keeps strip-major copies of the expert weights
    (mnb_qmoe_weights_prepack); Compute's output is bit-identical to an EP with the option off."""
    print("[gpu] ep qmoe strip-major option T=64 H=I=2880 E=32 k=4", flush=True)
    T, H, I, E, k = 64, 2880, 2880, 32, 4
    inp = oq.make_qmoe_inputs(T, H, I, E, per_channel=True, seed=4321)
    ys = []
    for opt in ("0", "1"):
        gpu_host.option("ep.strip_major_weights", opt)
        assert gpu_host.create_ep(0) == 0, mh.err()
        gpu_host.reset()
        x_name, r_name, y_name = mh.add_qmoe(gpu_host, "moe", inp, k=k, x_shape=(T, H))
        assert gpu_host.get_capability() == (1, ["moe:drop"])
        assert gpu_host.compile() == 0, mh.err()
        gpu_host.feed(x_name, inp["x"])
        gpu_host.feed(r_name, inp["logits"])
        assert gpu_host.compute(0) == 0, mh.err()
        ys.append(gpu_host.fetch(y_name, np.float16, T * H))
    assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
    assert np.isfinite(ys[1].astype(np.float32)).all()
