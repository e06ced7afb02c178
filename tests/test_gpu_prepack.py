"""GPU parity of the upload-time strip-major weight layout (mnb_weights_prepack).

A prepacked node's session calls that plan the batched decode kernel (4 to 16 fp16 rows) or, at
accuracy_level 4, the strip-per-workgroup int8 GEMV read the strip-major copy of B; every other
plan reads ORT's layout.  The copy holds the same bytes in
another order and the kernel does the same arithmetic on them, so the bar is bit-identical
output against the same node uploaded without the copy, plus the fp16 bar of the rest of the
suite against the oracle (max relative error 2e-3 over significant elements, |y_ref| >= 0.1 RMS).
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu

F16_TOL = 2e-3


def _upload(lib, mnb, s, inp, N, K, bs, zp):
    p = mnb.problem(0, N, K, 4, bs, zp)
    w = C.c_void_p()
    B, S, Z = inp["B"], inp["scales"], inp["zp"]
    mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes, S.ctypes.data,
                                     S.nbytes, Z.ctypes.data if zp else None,
                                     Z.nbytes if zp else 0, C.byref(w)))
    return w


@pytest.mark.parametrize("M,N,K,bs,zp", [
    (16, 3072, 3072, 32, True),     # Phi-3.5 o_proj: one strip per workgroup
    (16, 9216, 3072, 32, True),     # qkv_proj: three strips per workgroup
    (8, 3000, 8192, 128, True),     # N past the last whole strip, K = 8192 (16 wavefronts)
    (4, 1000, 2048, 64, False),     # implied zero point, partial last strip
    (12, 768, 768, 32, False),      # one quad per wavefront, six wavefronts
    (1, 3072, 3072, 32, True),      # one row: the streaming GEMV, ORT's layout
])
def test_prepacked_matches_ort_layout(cuda, M, N, K, bs, zp):
    import mnb
    import torch

    lib = mnb.load()
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=31 * M + N)
    plan = mnb.plan(mnb.problem(M, N, K, 4, bs, zp)).kernel
    if M >= 4:
        assert plan == mnb.KERNEL_BATCH_STREAM, f"plan {plan}: the test would not read the copy"
    print(f"[gpu] prepack M={M} N={N} K={K} bs={bs} zp={zp} (plan {plan})", flush=True)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        w_ort = _upload(lib, mnb, s, inp, N, K, bs, zp)
        w_pk = _upload(lib, mnb, s, inp, N, K, bs, zp)
        nb = C.c_int64(0)
        mnb.check(lib.mnb_weights_prepack(w_pk, C.byref(nb)))
        assert nb.value == -(-N // 16) * (K // 128) * 1024
        mnb.check(lib.mnb_weights_prepack(w_pk, None))          # a second call: nothing to do
        A = torch.from_numpy(np.ascontiguousarray(inp["A"])).to(cuda)
        ys = []
        for w in (w_ort, w_pk, w_pk):
            y = torch.empty(M, N, dtype=torch.float16, device=cuda)
            mnb.check(lib.mnb_session_run(s, w, M, A.data_ptr(), 1, y.data_ptr(), 1))
            ys.append(y.cpu().numpy())
        assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
        assert np.array_equal(ys[1].view(np.uint16), ys[2].view(np.uint16))
        ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
        assert np.isfinite(ys[1]).all()
        assert orc.max_rel_err_significant(ys[1], ref) <= F16_TOL
        assert orc.max_err_rms_normalised(ys[1], ref) <= F16_TOL
        mnb.check(lib.mnb_weights_release(w_ort))
        mnb.check(lib.mnb_weights_release(w_pk))
    finally:
        lib.mnb_session_destroy(s)


def _strip_plan(mnb, M, N, K, bs, zp):
    """The kernel a session call of a prepacked node runs: the planner's, except that a
    streaming-GEMV plan at 3 or 4 rows moves to the batched kernel, which then reads the copy."""
    import os
    plan = mnb.plan(mnb.problem(M, N, K, 4, bs, zp)).kernel
    if plan == mnb.KERNEL_GEMV_STREAM and M >= 3:
        os.environ["MNB_FORCE_KERNEL"] = "batch"
        try:
            forced = mnb.plan(mnb.problem(M, N, K, 4, bs, zp))
        finally:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        if forced.kernel == mnb.KERNEL_BATCH_STREAM:
            return mnb.KERNEL_BATCH_STREAM
    return plan


@pytest.mark.parametrize("M,N,K", [(3, 9216, 3072), (4, 3072, 8192), (3, 3072, 3072),
                                   (2, 9216, 3072)])
def test_prepacked_small_row_routing(cuda, M, N, K):
    """A prepacked node's 3- and 4-row calls take the batched kernel on the copy (the streaming
    GEMV is slower there on every Phi-3.5 node), 2-row calls keep the streaming GEMV:
    bit-identical to the ORT-layout node run on the same kernel (MNB_FORCE_KERNEL), and within
    the bar of the oracle."""
    import os
    import mnb
    import torch

    lib = mnb.load()
    inp = orc.make_inputs(M, N, K, bits=4, block_size=32, with_zp=True, seed=11 * M + N)
    want = _strip_plan(mnb, M, N, K, 32, True)
    assert want == (mnb.KERNEL_BATCH_STREAM if M >= 3 else mnb.KERNEL_GEMV_STREAM)
    print(f"[gpu] prepack routing M={M} N={N} K={K} -> kernel {want}", flush=True)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        w_ort = _upload(lib, mnb, s, inp, N, K, 32, True)
        w_pk = _upload(lib, mnb, s, inp, N, K, 32, True)
        mnb.check(lib.mnb_weights_prepack(w_pk, None))
        A = torch.from_numpy(np.ascontiguousarray(inp["A"])).to(cuda)
        ys = []
        for w, force in ((w_pk, None), (w_ort, "batch" if want == mnb.KERNEL_BATCH_STREAM else None)):
            if force:
                os.environ["MNB_FORCE_KERNEL"] = force
            try:
                y = torch.empty(M, N, dtype=torch.float16, device=cuda)
                mnb.check(lib.mnb_session_run(s, w, M, A.data_ptr(), 1, y.data_ptr(), 1))
                ys.append(y.cpu().numpy())
            finally:
                os.environ.pop("MNB_FORCE_KERNEL", None)
        assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
        ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, 32)
        assert orc.max_rel_err_significant(ys[0], ref) <= F16_TOL
        mnb.check(lib.mnb_weights_release(w_ort))
        mnb.check(lib.mnb_weights_release(w_pk))
    finally:
        lib.mnb_session_destroy(s)


@pytest.mark.parametrize("bits,bs,K,level", [(8, 32, 3072, 0), (4, 16, 3072, 0),
                                              (4, 32, 3040, 0), (4, 128, 16384, 4)])
def test_prepack_refuses_nodes_the_batched_kernel_never_runs(cuda, bits, bs, K, level):
    import mnb

    lib = mnb.load()
    N = 256
    inp = orc.make_inputs(1, N, K, bits=bits, block_size=bs, with_zp=True, seed=5)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        p = mnb.problem(0, N, K, bits, bs, True, mnb.DTYPE_F16, level)
        w = C.c_void_p()
        B, S, Z = inp["B"], inp["scales"], inp["zp"]
        mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes, S.ctypes.data,
                                         S.nbytes, Z.ctypes.data, Z.nbytes, C.byref(w)))
        nb = C.c_int64(-1)
        assert lib.mnb_weights_prepack(w, C.byref(nb)) == mnb.MNB_ERR_UNSUPPORTED
        assert nb.value == 0
        assert b"strip-major" in lib.mnb_last_error()
        mnb.check(lib.mnb_weights_release(w))
    finally:
        lib.mnb_session_destroy(s)


@pytest.mark.parametrize("M,N,K,bs,zp", [(16, 3072, 8192, 128, True),
                                         (5, 500, 1024, 32, False),
                                         (9, 1040, 2048, 64, True)])
def test_prepacked_accuracy_level_4(cuda, M, N, K, bs, zp):
    """accuracy_level 4 at up to 16 fp16 rows: the int8 GEMV reads the strip-major copy;
    bit-identical to the node without it, and the level-4 oracle at the fp16 bar."""
    import mnb
    import torch

    lib = mnb.load()
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=3 * M + N)
    p4 = mnb.problem(M, N, K, 4, bs, zp, mnb.DTYPE_F16, 4)
    assert mnb.plan(p4).kernel == mnb.KERNEL_ACC4_STREAM
    print(f"[gpu] prepack acc4 M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        ws = []
        for pack in (False, True):
            p = mnb.problem(0, N, K, 4, bs, zp, mnb.DTYPE_F16, 4)
            w = C.c_void_p()
            B, S, Z = inp["B"], inp["scales"], inp["zp"]
            mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes,
                                             S.ctypes.data, S.nbytes,
                                             Z.ctypes.data if zp else None,
                                             Z.nbytes if zp else 0, C.byref(w)))
            if pack:
                mnb.check(lib.mnb_weights_prepack(w, None))
            ws.append(w)
        A = torch.from_numpy(np.ascontiguousarray(inp["A"])).to(cuda)
        ys = []
        for w in ws:
            y = torch.empty(M, N, dtype=torch.float16, device=cuda)
            mnb.check(lib.mnb_session_run(s, w, M, A.data_ptr(), 1, y.data_ptr(), 1))
            ys.append(y.cpu().numpy())
        assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
        ref = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
        assert orc.max_rel_err_significant(ys[1], ref) <= F16_TOL
        for w in ws:
            mnb.check(lib.mnb_weights_release(w))
    finally:
        lib.mnb_session_destroy(s)
