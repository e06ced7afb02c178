"""(Skip)SimplifiedLayerNormalization through the plugin EP, driven by the mock ORT host.

CPU: the claim predicate (the reference's rows, rust/src/ops/norm.rs:53-140: the skip form with
its residual-sum output slot 3, the plain form in com.microsoft and in the default domain the
ORT GenAI builder uses) and its declines (unwritten output slots, another axis, a broadcast
skip, non-constant gamma, sizes outside the kernel).  GPU: Compile uploads gamma (and bias)
once; Compute writes output 0 and the residual sum; checked against oracle/rmsnorm.py with the
bars of test_gpu_rmsnorm.py.
"""

from __future__ import annotations

import numpy as np
import pytest

import mock_host as mh
from oracle import matmul_nbits as orc
from oracle import rmsnorm as rn


@pytest.fixture
def host():
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0, "an OrtStatus was leaked"
    assert mh.lib().mock_bad_status_release() == 0, "an OrtStatus was released twice"


def _inp(H=3072, dtype=np.float16):
    return rn.make_inputs(2, H, dtype=dtype, seed=4)


def _cap(host, **kw):
    host.reset()
    mh.add_norm(host, "norm", _inp(kw.pop("H", 3072), kw.pop("dtype", np.float16)), **kw)
    return host.get_capability()


@pytest.mark.parametrize("kw", [
    dict(x_shape=(1, 1, 3072)),                              # Phi-3.5: 3 inputs, slots 0 and 3
    dict(x_shape=(-1, 3072), bias=True),
    dict(x_shape=(4, 3072), with_sum=False),
    dict(x_shape=(4, 3072), skip=False, domain=""),           # the GenAI builder's spelling
    dict(x_shape=(4, 3072), skip=False, domain="com.microsoft", attrs_over={"axis": -1}),
    dict(x_shape=(2, 2880), H=2880),                          # gpt-oss hidden size
    dict(x_shape=(2, 1024), H=1024, dtype=np.float32, elem=mh.FLOAT),
])
def test_claimed(host, kw):
    assert host.create_ep(-1) == 0
    assert _cap(host, **kw) == (1, ["norm:drop"])


@pytest.mark.parametrize("case,kw", [
    ("inv_std_output", dict(x_shape=(4, 3072), outputs=["norm_y", "", "norm_y2"])),
    ("mean_output", dict(x_shape=(4, 3072), outputs=["norm_y", "norm_y2"])),
    ("plain_inv_std", dict(x_shape=(4, 3072), skip=False, outputs=["norm_y", "norm_y2"])),
    ("middle_axis", dict(x_shape=(4, 3072), skip=False, attrs_over={"axis": 0})),
    ("stash_double", dict(x_shape=(4, 3072), skip=False, attrs_over={"stash_type": 11})),
    ("symbolic_hidden", dict(x_shape=(4, -1))),
    ("too_wide", dict(x_shape=(1, 16384), H=16384)),
    ("odd_hidden", dict(x_shape=(1, 100), H=100)),
    ("non_constant_gamma", dict(x_shape=(4, 3072), const_gamma=False)),
    ("other_domain", dict(x_shape=(4, 3072), domain="ai.onnx.ml")),
])
def test_declined(host, case, kw):
    assert host.create_ep(-1) == 0
    host.reset()
    H = kw.pop("H", 3072)
    inp = _inp(H)
    host.value("norm_y2", mh.FLOAT16, (4, 3072))
    mh.add_norm(host, "norm", inp, **kw)
    n, claimed = host.get_capability()
    assert n == 0 and claimed == [], case


def test_broadcast_skip_is_declined(host):
    assert host.create_ep(-1) == 0
    host.reset()
    inp = _inp()
    host.value("x", mh.FLOAT16, (4, 3072))
    host.value("k", mh.FLOAT16, (1, 3072))
    host.value("g", mh.FLOAT16, (3072,), inp["gamma"])
    host.value("y", mh.FLOAT16, (4, 3072))
    host.node("SkipSimplifiedLayerNormalization", "com.microsoft", "n", ["x", "k", "g"], ["y"],
              {"epsilon": 1e-5})
    assert host.get_capability()[0] == 0


# ---- GPU ---------------------------------------------------------------------------------------

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
@pytest.mark.parametrize("lead,H,skip,bias,with_sum,dtype", [
    ((1, 1), 3072, True, False, True, np.float16),       # Phi-3.5 decode
    ((2, 7), 2880, True, True, True, np.float16),
    ((5,), 3072, False, False, False, np.float16),
    ((3,), 1024, True, False, False, np.float32),
])
def test_ep_norm_matches_oracle(gpu_host, lead, H, skip, bias, with_sum, dtype):
    print(f"[gpu] ep norm lead={lead} H={H} skip={skip} bias={bias} sum={with_sum}", flush=True)
    rows = int(np.prod(lead))
    inp = rn.make_inputs(rows, H, dtype=dtype, seed=rows + H)
    elem = mh.FLOAT16 if dtype == np.float16 else mh.FLOAT
    gpu_host.reset()
    x_name, k_name, y_name, s_name = mh.add_norm(gpu_host, "norm", inp, lead + (H,), skip=skip,
                                                 bias=bias, with_sum=with_sum, elem=elem,
                                                 domain="com.microsoft" if skip else "")
    assert gpu_host.get_capability() == (1, ["norm:drop"])
    assert gpu_host.compile() == 0, mh.err()
    gpu_host.feed(x_name, inp["x"].reshape(lead + (H,)))
    if skip:
        gpu_host.feed(k_name, inp["skip"].reshape(lead + (H,)))
    assert gpu_host.compute(0) == 0, mh.err()
    y = gpu_host.fetch(y_name, dtype, rows * H)
    assert y.shape == lead + (H,)
    ref, r = rn.skip_rmsnorm(inp["x"], inp["gamma"], inp["skip"] if skip else None,
                             inp["bias"] if bias else None, 1e-5)
    tol = 2e-3 if dtype == np.float16 else 1e-5
    y = y.reshape(rows, H).astype(np.float64)
    assert orc.max_rel_err_significant(y, ref) <= tol
    assert orc.max_err_rms_normalised(y, ref) <= tol
    if skip and with_sum:
        sm = gpu_host.fetch(s_name, dtype, rows * H).reshape(rows, H)
        want = inp["x"].astype(np.float32) + inp["skip"].astype(np.float32)
        if bias:
            want = want + inp["bias"].astype(np.float32)
        assert np.array_equal(sm, want.astype(dtype))       # fp32 adds, stored in the type
