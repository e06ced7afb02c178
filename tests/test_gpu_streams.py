"""GPU tests of the stream layer behind the EP's OrtSyncStreamImpl, through the C ABI.

An async session (mnb_session_set_async) returns from a call with device tensors once its work
is enqueued; a call with a host tensor still returns after the stream has finished.  Events order
one stream after another (mnb_event_record / mnb_stream_wait_event) and the host after a stream
(mnb_event_synchronize); mnb_memcpy_on_stream orders a copy on a stream.  Each result is checked
against the CPU oracle at the fp16 bar (2e-3, as in the rest of the suite) or bit for bit against
the synchronous session on the same inputs.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _check(y, ref, what):
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert e1 <= TOL and e2 <= TOL, f"{what}: {e1:.3e} {e2:.3e}"


def _upload(lib, mnb, s, inp, N, K, bs):
    p = mnb.problem(0, N, K, 4, bs, inp["zp"] is not None)
    w = C.c_void_p()
    B, S, Z = inp["B"], inp["scales"], inp["zp"]
    mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes, S.ctypes.data,
                                     S.nbytes, Z.ctypes.data if Z is not None else None,
                                     Z.nbytes if Z is not None else 0, C.byref(w)))
    return w


def test_async_session_chain_and_events(cuda):
    """Two chained nodes on one async session (the second reads the first's output), run for two
    inputs without a host wait; a second async session waits on an event recorded after them and
    copies the result on its own stream; the host waits on a final event.  Every output matches
    the synchronous session bit for bit and the oracle at the fp16 bar."""
    import mnb
    import torch
    print("[gpu] async session chain + events", flush=True)
    lib = mnb.load()
    M, K, N1, N2 = 8, 2048, 768, 512
    w1 = orc.make_inputs(M, N1, K, bits=4, block_size=32, with_zp=True, seed=41)
    w2 = orc.make_inputs(M, N2, N1, bits=4, block_size=128, with_zp=True, seed=42)
    rng = np.random.default_rng(43)
    xs = [rng.standard_normal((M, K), dtype=np.float32).astype(np.float16) for _ in range(2)]
    sync_s, a_s, b_s = C.c_void_p(), C.c_void_p(), C.c_void_p()
    for s in (sync_s, a_s, b_s):
        mnb.check(lib.mnb_session_create(0, C.byref(s)))
    ev1, ev2 = C.c_void_p(), C.c_void_p()
    try:
        mnb.check(lib.mnb_session_set_async(a_s, 1))
        mnb.check(lib.mnb_session_set_async(b_s, 1))
        u1, u2 = _upload(lib, mnb, sync_s, w1, N1, K, 32), _upload(lib, mnb, sync_s, w2, N2, N1, 128)
        dx = [torch.from_numpy(x).to(cuda) for x in xs]
        y1 = [torch.empty(M, N1, dtype=torch.float16, device=cuda) for _ in xs]
        y2 = [torch.empty(M, N2, dtype=torch.float16, device=cuda) for _ in xs]
        copy = [torch.empty(M, N2, dtype=torch.float16, device=cuda) for _ in xs]
        torch.cuda.synchronize()
        for i in range(2):                           # enqueued back to back, no host wait
            mnb.check(lib.mnb_session_run(a_s, u1, M, dx[i].data_ptr(), 1, y1[i].data_ptr(), 1))
            mnb.check(lib.mnb_session_run(a_s, u2, M, y1[i].data_ptr(), 1, y2[i].data_ptr(), 1))
        mnb.check(lib.mnb_event_create(0, C.byref(ev1)))
        mnb.check(lib.mnb_event_record(ev1, lib.mnb_session_stream(a_s)))
        b_stream = lib.mnb_session_stream(b_s)
        mnb.check(lib.mnb_stream_wait_event(b_stream, ev1))
        for i in range(2):                           # ordered after the chain by the event
            mnb.check(lib.mnb_memcpy_on_stream(0, copy[i].data_ptr(), y2[i].data_ptr(),
                                               M * N2 * 2, mnb.COPY_DEVICE_TO_DEVICE, b_stream))
        mnb.check(lib.mnb_event_create(0, C.byref(ev2)))
        mnb.check(lib.mnb_event_record(ev2, b_stream))
        mnb.check(lib.mnb_event_synchronize(ev2))    # the host waits for the copies only
        for i, x in enumerate(xs):
            h1 = np.empty((M, N1), dtype=np.float16)
            h2 = np.empty((M, N2), dtype=np.float16)
            mnb.check(lib.mnb_session_run(sync_s, u1, M, x.ctypes.data, 0, h1.ctypes.data, 0))
            mnb.check(lib.mnb_session_run(sync_s, u2, M, h1.ctypes.data, 0, h2.ctypes.data, 0))
            got1 = y1[i].cpu().numpy()
            got2 = copy[i].cpu().numpy()
            assert np.array_equal(got1.view(np.uint16), h1.view(np.uint16)), f"mm1 run {i}"
            assert np.array_equal(got2.view(np.uint16), h2.view(np.uint16)), f"mm2 run {i}"
            _check(got1, orc.matmul_nbits(x, w1["B"], w1["scales"], w1["zp"], N1, K, 4, 32), "mm1")
            _check(got2, orc.matmul_nbits(got1, w2["B"], w2["scales"], w2["zp"], N2, N1, 4, 128),
                   "mm2")
        mnb.check(lib.mnb_weights_release(u1))
        mnb.check(lib.mnb_weights_release(u2))
    finally:
        lib.mnb_event_destroy(ev1)
        lib.mnb_event_destroy(ev2)
        for s in (sync_s, a_s, b_s):
            lib.mnb_session_destroy(s)


def test_async_session_with_host_tensors_still_returns_complete(cuda):
    """A host output is complete when an async session's call returns (the call waits for the
    stream whenever host memory is involved)."""
    import mnb
    print("[gpu] async session host I/O", flush=True)
    lib = mnb.load()
    M, N, K = 3, 640, 1536
    inp = orc.make_inputs(M, N, K, bits=4, block_size=64, with_zp=False, seed=44)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        mnb.check(lib.mnb_session_set_async(s, 1))
        u = _upload(lib, mnb, s, inp, N, K, 64)
        A = np.ascontiguousarray(inp["A"])
        for _ in range(3):
            Y = np.zeros((M, N), dtype=np.float16)
            mnb.check(lib.mnb_session_run(s, u, M, A.ctypes.data, 0, Y.ctypes.data, 0))
            _check(Y, orc.matmul_nbits(A, inp["B"], inp["scales"], None, N, K, 4, 64), "host I/O")
        mnb.check(lib.mnb_weights_release(u))
    finally:
        lib.mnb_session_destroy(s)
