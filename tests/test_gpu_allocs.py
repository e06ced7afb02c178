"""Steady-state calls allocate no device memory: the library's device-allocation counter
(mnb_device_alloc_count) is unchanged across repeated decode calls through the session layer and
through the plugin's Compute, once the weights are uploaded and the session's staging has grown
to the largest call.  Counterpart of the reference's AllocRecorder tests
(rust/src/ops/quant.rs:1496-1547); the host-only half is tests/test_decode_allocs.py.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import mock_host as mh
from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _check(y, ref, what):
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert e1 <= TOL and e2 <= TOL, f"{what}: {e1:.3e} {e2:.3e}"


def _upload(lib, mnb, s, inp, N, K, bs, acc=0):
    p = mnb.problem(0, N, K, 4, bs, inp["zp"] is not None, mnb.DTYPE_F16, acc)
    w = C.c_void_p()
    B, S, Z = inp["B"], inp["scales"], inp["zp"]
    mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes, S.ctypes.data,
                                     S.nbytes, Z.ctypes.data if Z is not None else None,
                                     Z.nbytes if Z is not None else 0, C.byref(w)))
    return w


def test_session_decode_calls_allocate_nothing(cuda):
    """qkv (fp16 decode) and the accuracy_level = 4 node of BASELINE configs[4], on host and on
    device tensors, at 1..16 rows: after one call at the largest M per node, 48 further calls
    leave the counter where it was, and the last outputs match the oracle."""
    import mnb
    import torch
    print("[gpu] session steady-state allocations", flush=True)
    lib = mnb.load()
    K1, N1, K2, N2, MMAX = 3072, 9216, 8192, 3072, 16
    w1 = orc.make_inputs(MMAX, N1, K1, bits=4, block_size=32, with_zp=True, seed=71)
    w2 = orc.make_inputs(MMAX, N2, K2, bits=4, block_size=128, with_zp=True, seed=72)
    s = C.c_void_p()
    before_upload = mnb.device_alloc_count()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        u1 = _upload(lib, mnb, s, w1, N1, K1, 32)
        u2 = _upload(lib, mnb, s, w2, N2, K2, 128, acc=4)
        assert mnb.device_alloc_count() > before_upload     # uploads are counted
        A1, A2 = np.ascontiguousarray(w1["A"]), np.ascontiguousarray(w2["A"])
        dA1, dA2 = torch.from_numpy(A1).to(cuda), torch.from_numpy(A2).to(cuda)
        dY1 = torch.empty(MMAX, N1, dtype=torch.float16, device=cuda)
        dY2 = torch.empty(MMAX, N2, dtype=torch.float16, device=cuda)
        Y1 = np.empty((MMAX, N1), dtype=np.float16)
        Y2 = np.empty((MMAX, N2), dtype=np.float16)
        torch.cuda.synchronize()

        def call(m, dev):
            if dev:
                mnb.check(lib.mnb_session_run(s, u1, m, dA1.data_ptr(), 1, dY1.data_ptr(), 1))
                mnb.check(lib.mnb_session_run(s, u2, m, dA2.data_ptr(), 1, dY2.data_ptr(), 1))
            else:
                mnb.check(lib.mnb_session_run(s, u1, m, A1.ctypes.data, 0, Y1.ctypes.data, 0))
                mnb.check(lib.mnb_session_run(s, u2, m, A2.ctypes.data, 0, Y2.ctypes.data, 0))

        call(MMAX, False)                          # staging and workspace grow once
        call(MMAX, True)
        steady = mnb.device_alloc_count()
        launches = mnb.launch_count()
        for i in range(12):
            for m in (1, 2, 4, 16):
                call(m, i % 2 == 1)
        torch.cuda.synchronize()
        assert mnb.device_alloc_count() == steady, "a steady-state call allocated device memory"
        assert mnb.launch_count() > launches
        call(MMAX, False)
        _check(Y1, orc.matmul_nbits(A1, w1["B"], w1["scales"], w1["zp"], N1, K1, 4, 32), "qkv")
        _check(Y2, orc.matmul_nbits_acc4(A2, w2["B"], w2["scales"], w2["zp"], N2, K2, 4, 128),
               "level 4")
        mnb.check(lib.mnb_weights_release(u1))
        mnb.check(lib.mnb_weights_release(u2))
    finally:
        lib.mnb_session_destroy(s)


def test_ep_compute_allocates_nothing_after_the_first_call(cuda):
    """Through the plugin: Compile uploads (the counter moves, so it sees the plugin's library),
    the first Compute sizes the staging, and ten more Computes allocate nothing."""
    import mnb
    print("[gpu] ep steady-state allocations", flush=True)
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    assert h.supported_devices(n_amd=1) == 1
    assert h.create_ep(0) == 0, mh.err()
    try:
        M, N, K = 1, 9216, 3072
        inp = orc.make_inputs(M, N, K, bits=4, block_size=32, with_zp=True, seed=73)
        h.reset()
        a_name, y_name = mh.add_matmul_nbits(h, "qkv", inp, N, K, 4, 32, (M, K))
        assert h.get_capability() == (1, ["qkv:drop"])
        c0 = mnb.device_alloc_count()
        assert h.compile() == 0, mh.err()
        assert mnb.device_alloc_count() > c0, "the plugin's uploads are not seen by the counter"
        h.feed(a_name, inp["A"])
        assert h.compute(0) == 0, mh.err()
        steady = mnb.device_alloc_count()
        for _ in range(10):
            h.feed(a_name, inp["A"])
            assert h.compute(0) == 0, mh.err()
        assert mnb.device_alloc_count() == steady, "a steady-state Compute allocated device memory"
        y = h.fetch(y_name, np.float16, M * N).reshape(M, N)
        _check(y, orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, 32), "ep")
    finally:
        assert h.close() == 0
