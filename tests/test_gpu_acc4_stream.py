"""GPU parity of the accuracy_level=4 strip-per-workgroup int8 GEMV (up to 16 fp16 rows; planner
kernel ACC4_STREAM) through the C ABI, against the CPU oracle.

The kernel follows the int8 quantiser (bit-exact against the oracle, tests/test_gpu_acc4_moe.py):
a workgroup of K / (128 r) wavefronts owns one 16-column strip over all of K, each wavefront r
quads of 128, and the partial tiles are added in LDS in wavefront order.  Bars: outputs match the
oracle's level-4 definition (`oracle/matmul_nbits.py matmul_nbits_acc4`: exact int32 block dots,
scaled by a_scale * b_scale, summed in fp64) within max relative error 2e-3 over significant
elements and 2e-3 of max(|y_ref|, RMS) everywhere -- fp16 output rounding dominates; repeated
calls are bit-identical; the strip GEMV (MNB_FORCE_KERNEL=strip) on the same inputs agrees within
the same bar.  Covers every quads-per-wavefront instantiation (1, 2, 4, 8), 1 to 16 wavefronts,
rows 1..16, ragged last strips, a single strip, zero points on and off, all three block sizes,
an all-zero activation block and a tiny activation; and the shapes the planner leaves to the
strip GEMV (K above 8192, K / block not a multiple of 4, K % 128 != 0).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu
F16_TOL = 2e-3


def _dev(x, device):
    import torch
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device)


def _check(y, ref, what, tol=F16_TOL):
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert np.isfinite(y).all(), what
    assert e1 <= tol and e2 <= tol, f"{what}: rel_sig={e1:.3e} rms_norm={e2:.3e}"


def _expected_geometry(M, N, K, bs):
    """(quads per wavefront, wavefronts) the planner is expected to pick, or None when the shape
    is left to the strip GEMV: K % 128 == 0, (K / bs) % 4 == 0, the codes of 16 rows plus the
    scales and partial tiles within 160 KiB of LDS."""
    if not (1 <= M <= 16) or K % 128 or (K // bs) % 4:
        return None
    quads = K // 128
    for r in (8, 4, 2, 1):
        if quads % r == 0 and (quads // r >= 8 or r == 1) and quads // r <= 16:
            w = quads // r
            lds = 16 * (128 * quads + 16) + (K // bs) * 64 + 16 + w * 1024
            return (r, w) if lds <= 160 * 1024 else None
    return None


def _run(inp, N, K, bs, cuda, force="", workspace=None):
    import mnb
    import torch
    M = inp["A"].shape[0]
    old = os.environ.get("MNB_FORCE_KERNEL")
    os.environ["MNB_FORCE_KERNEL"] = force
    try:
        info = mnb.plan(mnb.problem(M, N, K, 4, bs, inp["zp"] is not None, mnb.DTYPE_F16, 4))
        y = mnb.matmul_nbits(_dev(inp["A"], cuda), _dev(inp["B"], cuda), _dev(inp["scales"], cuda),
                             _dev(inp["zp"], cuda), N, K, 4, bs, accuracy_level=4,
                             workspace=workspace)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        else:
            os.environ["MNB_FORCE_KERNEL"] = old
    return info, y.cpu().numpy()


SHAPES = [
    # (M, N, K, bs, zp)
    (16, 3072, 8192, 128, True),       # 8 wavefronts of 8 quads
    (1, 256, 8192, 32, True),          # block 32 at K = 8192: 155 KiB of LDS
    (1, 64, 512, 128, True),           # 4 quads: 4 wavefronts of one quad
    (2, 48, 1024, 64, False),          # 8 wavefronts of one quad; 3 strips
    (5, 200, 2048, 32, True),          # 8 of 2; ragged last strip (200 = 12.5 strips)
    (8, 100, 3072, 128, False),        # 12 of 2
    (16, 16, 4096, 64, True),          # 8 of 4; a single strip
    (3, 1000, 6144, 32, True),         # 12 of 4
    (12, 520, 1536, 128, True),        # 12 of 1
]


@pytest.mark.parametrize("M,N,K,bs,zp", SHAPES)
def test_acc4_stream_matches_level_4_definition(cuda, M, N, K, bs, zp):
    import mnb
    print(f"[gpu] acc4 stream M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    geo = _expected_geometry(M, N, K, bs)
    assert geo is not None
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=7100 + M + N)
    inp["A"][0, :bs] = 0                       # an all-zero block: scale 0, codes 0
    inp["A"][M - 1, 5] = np.float16(1e-3)      # a tiny value next to normal ones
    info, y = _run(inp, N, K, bs, cuda)
    assert info.kernel == mnb.KERNEL_ACC4_STREAM
    assert (info.grid_x, info.waves_per_group) == ((N + 15) // 16, geo[1])
    ref4 = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(y, ref4, f"acc4 stream M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,bs", [(16, 256, 16384, 128),   # codes beyond 160 KiB of LDS
                                      (4, 64, 384, 128),        # 3 blocks per column
                                      (5, 100, 2880, 32)])      # K % 128 != 0
def test_shapes_left_to_the_strip_gemv(cuda, M, N, K, bs):
    import mnb
    print(f"[gpu] acc4 strip fallback M={M} N={N} K={K} bs={bs}", flush=True)
    assert _expected_geometry(M, N, K, bs) is None
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=True, seed=88 + K)
    info, y = _run(inp, N, K, bs, cuda)
    assert info.kernel == mnb.KERNEL_ACC4_I8
    ref4 = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(y, ref4, f"acc4 strip fallback M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,bs,zp", [(16, 3072, 8192, 128, True), (5, 200, 2048, 32, True)])
def test_acc4_stream_repeatable_and_agrees_with_strip_gemv(cuda, M, N, K, bs, zp):
    import mnb
    import torch
    print(f"[gpu] acc4 stream repeat M={M} N={N} K={K}", flush=True)
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=4242)
    ws = torch.empty(mnb.workspace_bytes(mnb.problem(M, N, K, 4, bs, zp, mnb.DTYPE_F16, 4)),
                     dtype=torch.uint8, device=cuda)
    _, y1 = _run(inp, N, K, bs, cuda, workspace=ws)
    _, y2 = _run(inp, N, K, bs, cuda, workspace=ws)
    assert np.array_equal(y1.view(np.uint16), y2.view(np.uint16))
    info, ys = _run(inp, N, K, bs, cuda, force="strip")
    assert info.kernel == mnb.KERNEL_ACC4_I8
    _check(y1, ys.astype(np.float64), "acc4 stream vs strip GEMV")
