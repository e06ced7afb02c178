"""GPU parity of the fused QMoE (mnb_qmoe, mnb_session_run_qmoe) against oracle/qmoe.py.

Bars, against the oracle evaluated with fp16 rounding at the points where the HIP path stores
intermediates (h, act, and act W2^T, all before their biases):
  * max |y - y_ref| / max(|y_ref|, RMS(y_ref)) <= 2e-3 over every element;
  * max relative error <= 1e-2 over significant elements (|y_ref| >= 0.1 RMS).  Looser than the
    MatMulNBits bar because a stored fp16 intermediate that sits on a rounding boundary may
    round one way in the fp32-accumulated kernel and the other in the fp64 oracle; the one-ulp
    difference (4.9e-4 of that value) reaches the output through the weighted sum, where
    cancellation can leave a small output element;
and against the oracle with no intermediate rounding: RMS-normalised error <= 5e-3.  fp16
output rounding alone contributes up to 4.9e-4.  Parity of the op against ONNX Runtime's QMoE is
unpinned (ORT is absent; see oracle/qmoe.py).
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import matmul_nbits as orc
from oracle import qmoe as oq

TOL_RMS = 2e-3
TOL_SIGNIFICANT = 1e-2
TOL_EXACT_RMS = 5e-3

# (T, H, I, E, k, block, fusion, bias, limit, normalize, router_f32)
CASES = [
    (1, 256, 128, 8, 2, 32, 1, True, 7.0, True, False),
    (5, 256, 128, 8, 4, 32, 2, False, None, False, True),
    (64, 512, 256, 32, 4, 32, 1, True, 7.0, True, False),
    (17, 384, 192, 16, 1, 64, 2, True, None, True, False),
    (33, 256, 256, 4, 4, 128, 1, True, 7.0, True, False),
    (8, 2880, 2880, 32, 4, 32, 1, True, 7.0, True, False),
    # T*k > 1024: per-token routing kernel and the separate counting sort; row-tiled GEMVs
    (300, 256, 128, 16, 4, 32, 1, True, 7.0, True, False),
    # E > 64: the k-round arg-max routing; SwiGLU in the strip GEMV's stores
    (20, 256, 128, 96, 4, 32, 1, True, 7.0, True, True),
    (3, 512, 256, 64, 8, 64, 1, False, None, False, False),
]


def _t(a, dev):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _refs(inp, k, I, bs, fusion, limit, normalize, alpha=1.702, beta=1.0):
    kw = dict(k=k, inter=I, block_size=bs, fc1_bias=inp["fc1_bias"], fc2_bias=inp["fc2_bias"],
              fusion=fusion, alpha=alpha, beta=beta, limit=limit, normalize=normalize)
    args = (inp["x"], inp["logits"], inp["fc1"], inp["fc1_scales"], inp["fc2"], inp["fc2_scales"])
    return oq.qmoe(*args, f16_points=True, **kw), oq.qmoe(*args, **kw)


def _check(y, ref16, ref):
    assert np.isfinite(y).all()
    e_rms16 = orc.max_err_rms_normalised(y, ref16)
    e_sig16 = orc.max_rel_err_significant(y, ref16)
    e_rms = orc.max_err_rms_normalised(y, ref)
    errs = (e_rms16, e_sig16, e_rms)
    print(f"[gpu] qmoe errors: rms16={e_rms16:.3e} sig16={e_sig16:.3e} rms={e_rms:.3e}", flush=True)
    assert e_rms16 <= TOL_RMS, errs
    assert e_sig16 <= TOL_SIGNIFICANT, errs
    assert e_rms <= TOL_EXACT_RMS, errs


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_qmoe_matches_oracle(cuda, case):
    import mnb
    import torch

    T, H, I, E, k, bs, fusion, bias, limit, normalize, r32 = case
    inp = oq.make_qmoe_inputs(T, H, I, E, block_size=bs, bias=bias, seed=1000 + T + E)
    if r32:
        inp["logits"] = inp["logits"].astype(np.float32)
    if T >= 5:
        inp["logits"][1] = 0                     # a token whose logits all tie
        inp["logits"][2, ::2] = -0.0             # ... and one whose ties mix -0 and +0
        inp["logits"][2, 1::2] = 0.0
    ref16, ref = _refs(inp, k, I, bs, fusion, limit, normalize)
    d = {key: _t(v, cuda) for key, v in inp.items()}
    y = mnb.qmoe(d["x"], d["logits"], d["fc1"], d["fc1_scales"], d["fc2"], d["fc2_scales"], k=k,
                 inter=I, block_size=bs, fc1_bias=d["fc1_bias"], fc2_bias=d["fc2_bias"],
                 fusion=fusion, normalize=normalize, limit=limit)
    torch.cuda.synchronize()
    _check(y.float().cpu().numpy(), ref16, ref)


def _skewed_logits(T, E, heavy=3, heavy_rows=40, odd=7, odd_rows=17):
    """Router logits under which expert `heavy` takes exactly `heavy_rows` tokens (three 16-row
    tiles) and expert `odd` exactly `odd_rows` (one more than a tile); every other token's second
    choice is spread over experts 8..12."""
    rng = np.random.default_rng(4040)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[:, heavy] = -8.0
    lg[:, odd] = -8.0
    for t in range(T):
        lg[t, 8 + t % 5] = 4.0
        if t < heavy_rows:
            lg[t, heavy] = 8.0
        elif t < heavy_rows + odd_rows:
            lg[t, odd] = 8.0
    return lg.astype(np.float16)


@pytest.mark.gpu
def test_qmoe_skewed_routing_spans_several_row_tiles(cuda):
    """fc1 finds its own rows (interleaved SwiGLU, T*k <= 1024, E <= 64) with the row-tile hint at
    T*k/E = 8: an expert with 40 rows spans three 16-row tiles (the tiles past the first read
    their window of the expert's ranked rows) and one with 17 rows spans two."""
    import mnb
    import torch

    T, H, I, E, k = 64, 256, 128, 16, 2
    inp = oq.make_qmoe_inputs(T, H, I, E, block_size=32, bias=True, seed=4041)
    inp["logits"] = _skewed_logits(T, E)
    experts, _ = oq.route(inp["logits"], k)
    counts = np.bincount(experts.reshape(-1), minlength=E)
    assert counts[3] == 40 and counts[7] == 17 and counts.max() == 40
    print(f"[gpu] qmoe skewed routing T={T} E={E} k={k} counts {counts.tolist()}", flush=True)
    ref16, ref = _refs(inp, k, I, 32, 1, 7.0, True)
    d = {key: _t(v, cuda) for key, v in inp.items()}
    y = mnb.qmoe(d["x"], d["logits"], d["fc1"], d["fc1_scales"], d["fc2"], d["fc2_scales"], k=k,
                 inter=I, block_size=32, fc1_bias=d["fc1_bias"], fc2_bias=d["fc2_bias"],
                 fusion=1, normalize=True, limit=7.0)
    torch.cuda.synchronize()
    _check(y.float().cpu().numpy(), ref16, ref)


@pytest.mark.gpu
def test_qmoe_is_deterministic(cuda):
    import mnb
    import torch

    inp = oq.make_qmoe_inputs(64, 512, 256, 32, seed=5)
    d = {key: _t(v, cuda) for key, v in inp.items()}
    outs = []
    for _ in range(3):
        y = mnb.qmoe(d["x"], d["logits"], d["fc1"], d["fc1_scales"], d["fc2"], d["fc2_scales"],
                     k=4, inter=256, fc1_bias=d["fc1_bias"], fc2_bias=d["fc2_bias"])
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().tobytes())
    assert outs[0] == outs[1] == outs[2]


def test_qmoe_rejects_unsupported_problems():
    import mnb

    lib = mnb.load()
    for kw in (dict(k=9), dict(k=5, experts=4), dict(fusion=0), dict(block_size=16),
               dict(hidden=100), dict(rows=5000, k=4)):
        args = dict(rows=4, hidden=256, inter=128, experts=8, k=2, block_size=32, fusion=1)
        args.update(kw)
        p = mnb.qmoe_problem(**args)
        assert lib.mnb_qmoe_check(C.byref(p)) != 0, kw


@pytest.mark.gpu
def test_session_qmoe_per_channel_scales_host_io(cuda):
    """The session path: weights uploaded once with per-channel scales (expanded to blocks),
    host x / logits / y staged through HBM."""
    import mnb

    T, H, I, E, k = 12, 512, 256, 16, 4
    inp = oq.make_qmoe_inputs(T, H, I, E, per_channel=True, seed=77)
    ref16, ref = _refs(inp, k, I, 32, 1, 7.0, True)
    lib = mnb.load()
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    w = C.c_void_p()
    p = mnb.qmoe_problem(0, H, I, E, k, 32, 1, True)
    arrs = [np.ascontiguousarray(inp[n]) for n in ("fc1", "fc1_scales", "fc1_bias", "fc2",
                                                    "fc2_scales", "fc2_bias")]
    try:
        mnb.check(lib.mnb_qmoe_weights_upload(sess, C.byref(p), 1,
                                              *[v for a in arrs for v in (a.ctypes.data, a.nbytes)],
                                              C.byref(w)))
        x = np.ascontiguousarray(inp["x"])
        lg = np.ascontiguousarray(inp["logits"])
        y = np.empty((T, H), dtype=np.float16)
        for _ in range(2):                       # the second call reuses every buffer
            y[:] = np.nan
            mnb.check(lib.mnb_session_run_qmoe(sess, w, T, x.ctypes.data, 0, lg.ctypes.data, 0,
                                               y.ctypes.data, 0))
            _check(y.astype(np.float32), ref16, ref)
    finally:
        if w.value:
            lib.mnb_qmoe_weights_release(w)
        lib.mnb_session_destroy(sess)


@pytest.mark.gpu
@pytest.mark.parametrize("T,H,I,E,k,bs,fusion", [
    (64, 2880, 2880, 32, 4, 32, 1),      # K = 2880 ends in a partial quad
    (8, 512, 256, 32, 4, 32, 1),
    (5, 256, 128, 8, 4, 64, 2),
    (20, 256, 128, 96, 4, 32, 1),        # E > 64
    (300, 256, 128, 16, 4, 32, 1),       # row-tiled GEMVs: the copy is not read
])
def test_session_qmoe_strip_major(cuda, T, H, I, E, k, bs, fusion):
    """mnb_qmoe_weights_prepack: the expert-grouped strip GEMV reads strip-major copies of fc1
    and fc2 (chunks past K zero); the output is bit-identical to the same node without them,
    and within the bars above of the oracle."""
    import mnb
    import torch

    print(f"[gpu] qmoe strip-major T={T} H={H} I={I} E={E} k={k} bs={bs} f={fusion}", flush=True)
    inp = oq.make_qmoe_inputs(T, H, I, E, seed=T + 3 * E, block_size=bs)
    ref16, ref = _refs(inp, k, I, bs, fusion, 7.0, True)
    lib = mnb.load()
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    arrs = [np.ascontiguousarray(inp[n]) for n in ("fc1", "fc1_scales", "fc1_bias", "fc2",
                                                    "fc2_scales", "fc2_bias")]
    ws, ys = [], []
    try:
        for pack in (False, True):
            w = C.c_void_p()
            p = mnb.qmoe_problem(0, H, I, E, k, bs, fusion, True)
            mnb.check(lib.mnb_qmoe_weights_upload(
                sess, C.byref(p), 0, *[v for a in arrs for v in (a.ctypes.data, a.nbytes)],
                C.byref(w)))
            ws.append(w)
            if pack:
                nb = C.c_int64(0)
                mnb.check(lib.mnb_qmoe_weights_prepack(w, C.byref(nb)))
                assert nb.value == E * 1024 * (-(-2 * I // 16) * -(-H // 128) +
                                               -(-H // 16) * -(-I // 128))
            x, lg = _t(inp["x"], cuda), _t(inp["logits"], cuda)
            y = torch.empty(T, H, dtype=torch.float16, device=cuda)
            mnb.check(lib.mnb_session_run_qmoe(sess, w, T, x.data_ptr(), 1, lg.data_ptr(), 1,
                                               y.data_ptr(), 1))
            torch.cuda.synchronize()
            ys.append(y.cpu().numpy())
        assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
        _check(ys[1].astype(np.float32), ref16, ref)
    finally:
        for w in ws:
            lib.mnb_qmoe_weights_release(w)
        lib.mnb_session_destroy(sess)
