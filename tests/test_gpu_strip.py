"""GPU parity of the strip GEMV (at most 16 rows per group, activations held in registers across
a run of 16-column strips) through the C ABI, against the CPU oracle.

Covers the dense planner path (5..16 rows), the expert-grouped path (one expert above 16 rows,
empty experts), the fused accuracy_level=4 quantiser, runs of several strips, wavefronts with no
K share, sub-aligned scale and zero-point pointers (byte-wise staging) and run-to-run bit
identity.  Bars as in the rest of the suite: fp16 outputs within max relative error 2e-3 over
significant elements (|y_ref| >= 0.1 RMS) and within 2e-3 of max(|y_ref|, RMS) everywhere,
against the fp64-accumulated oracle; level-4 outputs against the oracle's level-4 definition
(parity with ORT's own int8 quantiser is unpinned: ORT is absent and the reference declines
the level).
"""

from __future__ import annotations

import ctypes as C

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


def _forced(kernel):
    """Context manager setting MNB_FORCE_KERNEL (read on every plan) for the block."""
    import contextlib
    import os

    @contextlib.contextmanager
    def cm():
        old = os.environ.get("MNB_FORCE_KERNEL")
        os.environ["MNB_FORCE_KERNEL"] = kernel
        try:
            yield
        finally:
            if old is None:
                os.environ.pop("MNB_FORCE_KERNEL", None)
            else:
                os.environ["MNB_FORCE_KERNEL"] = old
    return cm()


STRIP_SHAPES = [
    # (M, N, K, bs, zp, strip): strip = the strip kernel takes the shape when asked for
    # (MNB_FORCE_KERNEL=strip; by default the batched decode kernel takes K % 128 == 0)
    (5, 64, 256, 32, True, True),
    (8, 104, 2880, 32, False, True),     # gpt-oss K: a partial last quad; N ragged (6.5 strips)
    (8, 100, 2880, 32, True, True),      # 45-byte zero-point rows: staged without 16-byte pieces
    (16, 3072, 3072, 32, False, True),
    (12, 48, 512, 64, True, True),
    (16, 96, 1024, 128, False, True),
    (9, 130, 384, 128, True, True),
    (6, 64, 128, 32, True, True),        # one quad: three of four wavefronts hold no K share
    (16, 9216, 3072, 32, True, True),    # Phi-3.5 qkv at a 16-row batch
    (7, 40000, 256, 32, False, True),    # runs of several strips per workgroup
]


@pytest.mark.parametrize("M,N,K,bs,zp,strip", STRIP_SHAPES)
def test_strip_gemv_parity(cuda, M, N, K, bs, zp, strip):
    import mnb
    import torch
    print(f"[gpu] strip M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    with _forced("strip" if strip else "group"):
        info = mnb.plan(mnb.problem(M, N, K, 4, bs, zp))
        assert info.kernel == (mnb.KERNEL_STRIP_MFMA if strip else mnb.KERNEL_GROUP_MFMA)
        inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=M + 7 * N)
        y = mnb.matmul_nbits(_dev(inp["A"], cuda), _dev(inp["B"], cuda),
                             _dev(inp["scales"], cuda), _dev(inp["zp"], cuda), N, K, 4, bs)
        torch.cuda.synchronize()
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(y.cpu().numpy(), ref, f"strip M={M} N={N} K={K}")


def test_strip_runs_of_several_strips():
    import mnb
    # the planner groups strips into runs when there are many more strips than workgroups
    with _forced("strip"):
        info = mnb.plan(mnb.problem(7, 40000, 256, 4, 32, False))
    assert info.kernel == mnb.KERNEL_STRIP_MFMA and info.tile_n >= 32


def test_strip_bit_identical_runs(cuda):
    import mnb
    import torch
    M, N, K, bs = 16, 4096, 2880, 32
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=True, seed=11)
    t = [_dev(inp[k], cuda) for k in ("A", "B", "scales", "zp")]
    outs = []
    for _ in range(3):
        y = mnb.matmul_nbits(*t, N, K, 4, bs)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().view(np.uint16))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_strip_sub_aligned_scales_and_zero_points(cuda):
    # scales one fp16 and zero points one byte into their buffers: the run's copy into LDS
    # takes the element-wise path
    import mnb
    import torch
    M, N, K, bs = 8, 200, 1024, 32
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=True, seed=3)
    sbuf = _dev(np.concatenate([np.zeros(1, np.float16), inp["scales"].ravel()]), cuda)
    zbuf = _dev(np.concatenate([np.zeros(1, np.uint8), inp["zp"].ravel()]), cuda)
    y = mnb.matmul_nbits(_dev(inp["A"], cuda), _dev(inp["B"], cuda), sbuf[1:], zbuf[1:], N, K,
                         4, bs)
    torch.cuda.synchronize()
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(y.cpu().numpy(), ref, "strip sub-aligned scales")


def _run_moe(cuda, A, offsets, rows, B, S, Z, N, K, bs):
    import mnb
    import torch
    E = len(offsets) - 1
    counts = np.diff(offsets)
    p = mnb.MoeProblem(E, int(offsets[-1]), int(counts.max()), A.shape[0], N, K, 4, bs,
                       int(Z is not None), mnb.DTYPE_F16)
    Y = torch.empty(int(offsets[-1]), N, dtype=torch.float16, device=cuda)
    ta, tr, to = _dev(A, cuda), _dev(rows.astype(np.int32), cuda), _dev(offsets.astype(np.int32), cuda)
    tb, ts, tz = _dev(B, cuda), _dev(S, cuda), _dev(Z, cuda)
    s = int(torch.cuda.current_stream().cuda_stream)
    mnb.check(mnb.load().mnb_moe_grouped(C.byref(p), ta.data_ptr(), tr.data_ptr(), to.data_ptr(),
                                         tb.data_ptr(), ts.data_ptr(),
                                         None if tz is None else tz.data_ptr(), Y.data_ptr(), s))
    torch.cuda.synchronize()
    return Y.cpu().numpy()


@pytest.mark.parametrize("N,K,bs,zp", [(96, 2880, 32, False), (40, 512, 64, True)])
def test_strip_moe_uneven_experts(cuda, N, K, bs, zp):
    # rows per expert 0, 3, 20, 5, 1, 0, 9, 2: the mean keeps the strip kernel, the expert with
    # 20 rows takes a second 16-row tile, empty experts launch nothing that stores
    counts = np.array([0, 3, 20, 5, 1, 0, 9, 2])
    E = len(counts)
    T = 24
    rng = np.random.default_rng(17)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    rows = rng.integers(0, T, size=int(offsets[-1]))
    ws = [orc.make_inputs(1, N, K, bits=4, block_size=bs, with_zp=zp, seed=100 + e) for e in range(E)]
    A = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16)
    B = np.stack([w["B"] for w in ws])
    S = np.stack([w["scales"] for w in ws])
    Z = np.stack([w["zp"] for w in ws]) if zp else None
    print(f"[gpu] strip moe N={N} K={K} bs={bs} zp={zp}", flush=True)
    y = _run_moe(cuda, A, offsets, rows, B, S, Z, N, K, bs)
    ref = orc.moe_grouped_matmul_nbits(A, rows, offsets, B, S, Z, N, K, 4, bs)
    _check(y, ref, "strip moe")


@pytest.mark.parametrize("M,N,K,bs,zp", [
    (16, 3072, 8192, 128, True),
    (8, 200, 2048, 64, True),
    (3, 100, 4096, 128, False),
    (16, 48, 1024, 32, True),
    (5, 100, 2880, 32, False),       # a partial last quad
])
def test_strip_accuracy_level_4(cuda, M, N, K, bs, zp):
    import mnb
    import os
    import torch
    print(f"[gpu] strip acc4 M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=900 + M)
    # an all-zero activation block and a tiny value exercise the quantiser's edge cases
    inp["A"][0, :bs] = 0
    inp["A"][M - 1, 5] = np.float16(1e-3)
    # MNB_FORCE_KERNEL=strip: the strip GEMV instead of the strip-per-wavefront int8 kernel
    old = os.environ.get("MNB_FORCE_KERNEL")
    os.environ["MNB_FORCE_KERNEL"] = "strip"
    try:
        assert mnb.plan(mnb.problem(M, N, K, 4, bs, zp, mnb.DTYPE_F16, 4)).kernel == \
            mnb.KERNEL_ACC4_I8
        y = mnb.matmul_nbits(_dev(inp["A"], cuda), _dev(inp["B"], cuda), _dev(inp["scales"], cuda),
                             _dev(inp["zp"], cuda), N, K, 4, bs, accuracy_level=4)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        else:
            os.environ["MNB_FORCE_KERNEL"] = old
    ref4 = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(y.cpu().numpy(), ref4, "strip acc4 vs level-4 definition")
