"""mnb_matmul_nbits_noalloc against mnb_matmul_nbits with a caller-allocated workspace.

The allocation-free entry point runs the same kernels with the library's own per-GPU scratch
array in place of the workspace, so its outputs must be bit-identical to the workspace entry
point's on the same inputs.  Two calls in a row, the second with a smaller problem, show that the
scratch is reused correctly (the int8 path's split-K counters are cleared by the call); a prefill
GEMM whose K-split partials fit uses the scratch, one that does not runs unsplit; accuracy_level 4
beyond the scratch is refused before anything is launched.  No call of the allocation-free entry
point changes the library's device-allocation counter, and a call recorded in a HIP graph
(accuracy_level 4 and the batched decode kernel) replays bit-identically to its eager run, with
other calls on the same scratch between the replays.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu


def _dev(x, device):
    import torch

    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device)


def _both(cuda, M, N, K, bs, zp, level, seed, a_dtype=np.float16):
    """Y from the workspace entry point and from the allocation-free one (same inputs)."""
    import mnb
    import torch

    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=seed, a_dtype=a_dtype)
    t = {k: _dev(v, cuda) for k, v in inp.items()}
    f16 = a_dtype == np.float16
    p = mnb.problem(M, N, K, 4, bs, zp, mnb.DTYPE_F16 if f16 else mnb.DTYPE_F32, level)
    tdt = torch.float16 if f16 else torch.float32
    lib = mnb.load()
    st = int(torch.cuda.current_stream().cuda_stream)
    ws_bytes = mnb.workspace_bytes(p)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=cuda)
    y_ws = torch.full((M, N), float("nan"), dtype=tdt, device=cuda)
    y_na = torch.full((M, N), float("nan"), dtype=tdt, device=cuda)
    zptr = t["zp"].data_ptr() if zp else None
    mnb.check(lib.mnb_matmul_nbits(C.byref(p), t["A"].data_ptr(), t["B"].data_ptr(),
                                   t["scales"].data_ptr(), zptr, y_ws.data_ptr(), ws.data_ptr(),
                                   ws_bytes, st))
    torch.cuda.synchronize()
    allocs = mnb.device_alloc_count()
    mnb.check(lib.mnb_matmul_nbits_noalloc(C.byref(p), t["A"].data_ptr(), t["B"].data_ptr(),
                                           t["scales"].data_ptr(), zptr, y_na.data_ptr(), st))
    torch.cuda.synchronize()
    assert mnb.device_alloc_count() == allocs, "the allocation-free entry point allocated"
    return inp, y_ws.cpu().numpy(), y_na.cpu().numpy(), ws_bytes


def _same(a, b):
    u = np.uint16 if a.dtype == np.float16 else np.uint32
    return np.array_equal(a.view(u), b.view(u))


def test_scratch_size_is_stated():
    import mnb

    assert mnb.load().mnb_noalloc_scratch_bytes() == 48 << 20


def test_accuracy_level_4_twice_second_smaller(cuda):
    """BASELINE configs[4] (the int8 activations and their scales in the scratch), then a smaller
    level-4 problem on the same scratch."""
    import mnb

    print("[gpu] noalloc acc4 M=16 N=3072 K=8192 bs128 zp, then M=5 N=200 K=1024 bs64", flush=True)
    inp, y_ws, y_na, wsb = _both(cuda, 16, 3072, 8192, 128, True, 4, 71)
    assert 0 < wsb <= mnb.load().mnb_noalloc_scratch_bytes()
    assert np.isfinite(y_na).all() and _same(y_ws, y_na)
    ref = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], 3072, 8192, 4, 128)
    assert orc.max_rel_err_significant(y_na, ref) <= 2e-3
    inp, y_ws, y_na, _ = _both(cuda, 5, 200, 1024, 64, True, 4, 72)
    assert np.isfinite(y_na).all() and _same(y_ws, y_na)
    ref = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], 200, 1024, 4, 64)
    assert orc.max_rel_err_significant(y_na, ref) <= 2e-3


def test_level_4_k_split_counters_reused(cuda):
    """A level-4 shape whose int8 GEMV splits K over workgroups (fp32 activations take the
    row-tiled int8 GEMV; its partials and arrival counters live in the scratch), twice: a counter
    left non-zero by the first call would corrupt the second."""
    import mnb

    print("[gpu] noalloc acc4 K-split fp32 M=1 N=256 K=8192 bs32, twice", flush=True)
    p = mnb.problem(1, 256, 8192, 4, 32, True, mnb.DTYPE_F32, 4)
    assert mnb.plan(p).grid_x > (256 + 15) // 16          # more workgroups than strips: K split
    for seed in (73, 74):
        inp, y_ws, y_na, _ = _both(cuda, 1, 256, 8192, 32, True, 4, seed, np.float32)
        assert _same(y_ws, y_na)
        ref = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], 256, 8192, 4, 32)
        assert orc.max_err_rms_normalised(y_na, ref) <= 1e-5


def test_prefill_split_and_unsplit(cuda):
    """Prefill GEMMs: K-split partials in the scratch (M=256, BASELINE configs[2]; and an uneven
    split), then a decode-shaped call that needs no scratch."""
    import mnb

    print("[gpu] noalloc gemm M=256 N=8192 K=3072; M=129 N=300 K=1600; M=1", flush=True)
    for (M, N, K) in ((256, 8192, 3072), (129, 300, 1600)):
        p = mnb.problem(M, N, K, 4, 32, False)
        assert mnb.plan(p).kernel == mnb.KERNEL_GEMM_MFMA
        _, y_ws, y_na, wsb = _both(cuda, M, N, K, 32, False, 0, M + N)
        assert 0 < wsb <= mnb.load().mnb_noalloc_scratch_bytes()
        assert np.isfinite(y_na).all() and _same(y_ws, y_na)
    _, y_ws, y_na, wsb = _both(cuda, 1, 3072, 3072, 32, True, 0, 9)
    assert wsb == 0 and _same(y_ws, y_na)


def test_level_4_beyond_scratch_is_refused(cuda):
    import mnb

    M, N, K = 8192, 64, 8192            # 64 MiB of int8 activations alone
    p = mnb.problem(M, N, K, 4, 32, False, mnb.DTYPE_F16, 4)
    assert mnb.workspace_bytes(p) > mnb.load().mnb_noalloc_scratch_bytes()
    rc = mnb.load().mnb_matmul_nbits_noalloc(C.byref(p), None, None, None, None, None, None)
    assert rc == mnb.MNB_ERR_UNSUPPORTED
    assert b"scratch" in mnb.load().mnb_last_error()


@pytest.mark.parametrize("M,N,K,bs,zp,level,kernel", [
    (16, 3072, 8192, 128, True, 4, "ACC4_STREAM"),      # quantiser + GEMV
    (8, 3072, 3072, 32, True, 0, "BATCH_STREAM"),       # batched decode (no scratch needed)
    (256, 8192, 3072, 32, False, 0, "GEMM_MFMA"),       # prefill K split: partials in scratch
])
def test_graph_replays_match_eager(cuda, M, N, K, bs, zp, level, kernel):
    """The allocation-free call recorded into a HIP graph (torch.cuda.CUDAGraph stream capture),
    replayed three times with an eager allocation-free call of another shape between replays (it
    overwrites the shared scratch): every replay equals the eager output bit for bit, and neither
    the capture nor the replays allocate."""
    import mnb
    import torch

    print(f"[gpu] noalloc graph {kernel} M={M} N={N} K={K} bs{bs} level {level}", flush=True)
    p = mnb.problem(M, N, K, 4, bs, zp, mnb.DTYPE_F16, level)
    assert mnb.plan(p).kernel == getattr(mnb, "KERNEL_" + kernel)
    lib = mnb.load()
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=M + K)
    t = {k: _dev(v, cuda) for k, v in inp.items()}
    zptr = t["zp"].data_ptr() if zp else None
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)

    def call(stream_ptr):
        mnb.check(lib.mnb_matmul_nbits_noalloc(C.byref(p), t["A"].data_ptr(), t["B"].data_ptr(),
                                               t["scales"].data_ptr(), zptr, y.data_ptr(),
                                               stream_ptr))

    # another shape on the same scratch (level 4 at 16 rows: codes and scales of other values)
    o_inp = orc.make_inputs(16, 512, 4096, bits=4, block_size=64, with_zp=True, seed=5)
    o_t = {k: _dev(v, cuda) for k, v in o_inp.items()}
    o_p = mnb.problem(16, 512, 4096, 4, 64, True, mnb.DTYPE_F16, 4)
    o_y = torch.empty(16, 512, dtype=torch.float16, device=cuda)

    def other():
        mnb.check(lib.mnb_matmul_nbits_noalloc(
            C.byref(o_p), o_t["A"].data_ptr(), o_t["B"].data_ptr(), o_t["scales"].data_ptr(),
            o_t["zp"].data_ptr(), o_y.data_ptr(), int(torch.cuda.current_stream().cuda_stream)))

    call(int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    assert np.isfinite(eager).all()
    allocs = mnb.device_alloc_count()
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cs):
        call(int(cs.cuda_stream))
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(float("nan"))
        other()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert _same(y.cpu().numpy(), eager), f"replay {rep} differs from the eager call"
    assert mnb.device_alloc_count() == allocs
    del g
