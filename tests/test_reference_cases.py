"""The reference's own MatMulNBits node forms, read from its case models, through the plugin EP.

`tests/golden/reference_cases/` holds the six one-node models the reference keeps as evidence
(`evidence/cases/matmulnbits_{f16,f32}_scales[_zp][_dyn].onnx`, written by
`rust/tools/ledger_case_models.py:45-100,376-420`; sha256 in `PROVENANCE.md` there).  They are
read as data with `onnx_reader` (no onnx import) and bring forms no synthetic test declares:
zero points as the flat 1-D tensor `[N * ceil(bpc / 2)]` (`ledger_case_models.py:73-77`), a
symbolic leading dim `N` on A and Y (the `_dyn` models), and fp32 activations and scales.

CPU: the reader is pinned by the generator's own draws (each initializer equals what
`default_rng(seed)` produces in the generator's order), the forms are asserted, and the plugin
claims every model.  GPU: every model runs through GetCapability / Compile / Compute against the
oracle (fp16 bar 2e-3, fp32 bar 1e-5), the symbolic models at several row counts; and the
reference's fp16 three-input symbolic-batch regression case (`tests/ops/test_matmulnbits.py:
510-551`, inputs drawn as `tests/ops/_models.py:2527-2553` draws them) must give non-zero,
oracle-matching, run-to-run identical output.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import mock_host as mh
import onnx_reader
from oracle import matmul_nbits as orc

CASES_DIR = Path(__file__).resolve().parent / "golden" / "reference_cases"
CASES = sorted(CASES_DIR.glob("matmulnbits_*.onnx"))
F16_TOL, F32_TOL = 2e-3, 1e-5


def _case(path: Path) -> dict:
    g = onnx_reader.load(path)
    assert len(g.nodes) == 1
    node = g.nodes[0]
    x, y = g.inputs[0], g.outputs[0]
    a = node.attrs
    ini = g.initializers
    c = {"graph": g, "node": node, "x": x, "y": y, "K": a["K"], "N": a["N"], "bits": a["bits"],
         "bs": a["block_size"], "acc": a.get("accuracy_level"), "B": ini[node.inputs[1]].array,
         "scales": ini[node.inputs[2]].array,
         "zp": ini[node.inputs[3]].array if len(node.inputs) > 3 and node.inputs[3] else None,
         "dtype": np.float16 if x.elem == mh.FLOAT16 else np.float32}
    return c


def _generator_draws(name: str, N: int, K: int, bs: int, dtype, with_zp: bool):
    """The initializers as the generator draws them: `_matmulnbits` (seed 20260801) for the
    static fp16 pair, `_matmulnbits_typed` (seed 20260802) for the rest; packed weights, then
    scales, then the 1-D zero points."""
    typed = name not in ("matmulnbits_f16_scales", "matmulnbits_f16_scales_zp")
    rng = np.random.default_rng(20260802 if typed else 20260801)
    bpc = (K + bs - 1) // bs
    packed = rng.integers(0, 256, size=[N, bpc, bs * 4 // 8], dtype=np.uint8)
    scale = rng.uniform(0.001, 0.1, size=[N * bpc]).astype(dtype)
    zp = rng.integers(0, 256, size=[N * ((bpc + 1) // 2)], dtype=np.uint8) if with_zp else None
    return packed, scale, zp


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_reader_is_pinned_by_the_generators_draws(path):
    c = _case(path)
    packed, scale, zp = _generator_draws(path.stem, c["N"], c["K"], c["bs"], c["dtype"],
                                         c["zp"] is not None)
    assert np.array_equal(c["B"], packed)
    assert c["scales"].dtype == scale.dtype and np.array_equal(c["scales"].view(np.uint8),
                                                               scale.view(np.uint8))
    if zp is not None:
        assert np.array_equal(c["zp"], zp)


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_case_forms(path):
    c = _case(path)
    node = c["node"]
    assert (node.op_type, node.domain) == ("MatMulNBits", "com.microsoft")
    assert (c["K"], c["N"], c["bits"], c["bs"], c["acc"]) == (32, 32, 4, 32, 1)
    assert c["B"].shape == (32, 1, 16) and c["scales"].shape == (32,)
    stem = path.stem
    assert (c["zp"] is not None) == ("_zp" in stem)
    if c["zp"] is not None:
        assert c["zp"].shape == (32 * 1,)          # flat [N * ceil(bpc / 2)], not [N, zpb]
    lead = c["x"].dims[0]
    assert isinstance(lead, str) == stem.endswith("_dyn")
    assert c["x"].dims[1] == 32 and c["y"].dims[1] == 32
    assert c["dtype"] == (np.float32 if "_f32_" in stem else np.float16)
    assert c["graph"].opsets.get("com.microsoft") == 1


def _build(host, c: dict):
    """The case model's graph in the mock host: symbolic dims as -1, initializers as
    constants."""
    host.reset()
    dims = lambda v: tuple(-1 if isinstance(d, str) or d is None else d for d in v.dims)
    host.value(c["x"].name, c["x"].elem, dims(c["x"]))
    host.value(c["y"].name, c["y"].elem, dims(c["y"]))
    for name, t in c["graph"].initializers.items():
        host.value(name, t.dtype, tuple(t.dims), t.array)
    n = c["node"]
    host.node(n.op_type, n.domain, n.name, n.inputs, n.outputs, n.attrs)


@pytest.fixture
def cpu_host():
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_case_models_are_claimed(cpu_host, path):
    assert cpu_host.create_ep(-1) == 0
    c = _case(path)
    _build(cpu_host, c)
    n, claimed = cpu_host.get_capability()
    assert n == 1 and claimed == [f"{c['node'].name}:drop"], claimed


# ---- on the GPU ---------------------------------------------------------------------------------

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


def _run(host, c, rows, seed=20260801):
    x = np.random.default_rng(seed).standard_normal((rows, c["K"])).astype(c["dtype"])
    host.feed(c["x"].name, x)
    assert host.compute(0) == 0, mh.err()
    y = host.fetch(c["y"].name, c["dtype"], rows * c["N"]).reshape(rows, c["N"])
    return x, y


def _check(y, ref, tol, what):
    assert np.isfinite(y).all(), what
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert e1 <= tol and e2 <= tol, f"{what}: rel_sig={e1:.3e} rms_norm={e2:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_case_models_match_the_oracle(gpu_host, path):
    c = _case(path)
    print(f"[gpu] reference case {path.stem}", flush=True)
    _build(gpu_host, c)
    assert gpu_host.get_capability()[0] == 1
    assert gpu_host.compile() == 0, mh.err()
    row_counts = (1, 3, 17) if path.stem.endswith("_dyn") else (1,)
    tol = F16_TOL if c["dtype"] == np.float16 else F32_TOL
    for rows in row_counts:
        x, y = _run(gpu_host, c, rows)
        ref = orc.matmul_nbits(x, c["B"], c["scales"], c["zp"], c["N"], c["K"], c["bits"], c["bs"])
        _check(y, ref, tol, f"{path.stem} rows={rows}")


@pytest.mark.gpu
def test_fp16_symbolic_batch_regression_case(gpu_host):
    # tests/ops/test_matmulnbits.py:510-551: K=256, N=64, one row, fp16, three inputs (no zero
    # points), symbolic batch; inputs drawn in _models.py's order (packed, activation, scales)
    K, N, bs = 256, 64, 32
    rng = np.random.default_rng(42)
    bpc = K // bs
    packed = rng.integers(0, 256, size=[N, bpc, bs * 4 // 8], dtype=np.uint8)
    act = rng.standard_normal((1, K)).astype(np.float16)
    scale = rng.uniform(0.001, 0.1, size=[N * bpc]).astype(np.float16)
    h = gpu_host
    h.reset()
    h.value("X", mh.FLOAT16, (-1, K))
    h.value("Y", mh.FLOAT16, (-1, N))
    h.value("B", mh.UINT8, packed.shape, packed)
    h.value("scales", mh.FLOAT16, scale.shape, scale)
    h.node("MatMulNBits", "com.microsoft", "mm", ["X", "B", "scales"], ["Y"],
           {"K": K, "N": N, "bits": 4, "block_size": bs, "accuracy_level": 1})
    assert h.get_capability()[0] == 1
    assert h.compile() == 0, mh.err()
    ref = orc.matmul_nbits(act, packed, scale, None, N, K, 4, bs)
    outs = []
    for _ in range(3):                                   # the multirun form (:554-)
        h.feed("X", act)
        assert h.compute(0) == 0, mh.err()
        outs.append(h.fetch("Y", np.float16, N).reshape(1, N).copy())
    assert np.any(np.abs(outs[0]) > 1e-4), "all-zero output"
    _check(outs[0], ref, F16_TOL, "fp16 symbolic batch")
    assert all(np.array_equal(outs[0].view(np.uint16), o.view(np.uint16)) for o in outs[1:])
