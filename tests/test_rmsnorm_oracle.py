"""Pin the RMSNorm restatement (oracle/rmsnorm.py) before it checks the GPU.

Against a library routine (torch.nn.functional.rms_norm in float64), closed forms, and a
pure-Python brute force; each is chosen so that a plausible mistake (mean vs sum of squares,
epsilon outside the root, the residual left out, gamma applied twice) fails one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import rmsnorm as rn


def test_matches_torch_rms_norm():
    import torch

    inp = rn.make_inputs(5, 96, dtype=np.float32, seed=3)
    y, r = rn.skip_rmsnorm(inp["x"], inp["gamma"], inp["skip"], inp["bias"], 1e-5)
    rt = (torch.from_numpy(inp["x"]).double() + torch.from_numpy(inp["skip"]).double()
          + torch.from_numpy(inp["bias"]).double())
    want = torch.nn.functional.rms_norm(rt, (96,), torch.from_numpy(inp["gamma"]).double(), 1e-5)
    assert np.max(np.abs(y - want.numpy())) < 1e-12
    assert np.max(np.abs(r - rt.numpy())) == 0.0


def test_closed_forms():
    h = 64
    c = np.full((1, h), 3.0)
    y, _ = rn.skip_rmsnorm(c, np.ones(h), epsilon=0.0)
    assert np.allclose(y, 1.0, rtol=0, atol=1e-15)             # c / |c|
    y, _ = rn.skip_rmsnorm(c, np.ones(h), epsilon=7.0)
    assert np.allclose(y, 3.0 / math.sqrt(9.0 + 7.0), rtol=0, atol=1e-15)
    # scale invariance with epsilon 0, gamma linearity
    inp = rn.make_inputs(3, h, dtype=np.float32, seed=5, bias=False)
    y1, _ = rn.skip_rmsnorm(inp["x"], inp["gamma"], inp["skip"], epsilon=0.0)
    y2, _ = rn.skip_rmsnorm(4.0 * inp["x"], inp["gamma"], 4.0 * inp["skip"], epsilon=0.0)
    assert np.max(np.abs(y1 - y2)) < 1e-12
    y3, _ = rn.skip_rmsnorm(inp["x"], 2.0 * inp["gamma"], inp["skip"], epsilon=0.0)
    assert np.max(np.abs(2.0 * y1 - y3)) < 1e-12


def test_brute_force():
    inp = rn.make_inputs(2, 16, dtype=np.float16, seed=7)
    y, r = rn.skip_rmsnorm(inp["x"], inp["gamma"], inp["skip"], inp["bias"], 1e-5)
    for i in range(2):
        rr = [float(inp["x"][i, j]) + float(inp["skip"][i, j]) + float(inp["bias"][j])
              for j in range(16)]
        ms = sum(v * v for v in rr) / 16
        for j in range(16):
            assert abs(r[i, j] - rr[j]) == 0.0
            assert abs(y[i, j] - rr[j] / math.sqrt(ms + 1e-5) * float(inp["gamma"][j])) < 1e-12
