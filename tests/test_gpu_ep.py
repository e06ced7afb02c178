"""The plugin EP end to end on the GPU, driven through the mock ORT host.

CreateEpFactories -> GetSupportedDevices (the MI355X is advertised) -> CreateEp -> GetCapability
-> Compile (constant weights uploaded to HBM once) -> Compute (host A in, one HIP launch, host Y
out), checked against the oracle at the fp16 bar (max rel err 2e-3 over significant elements and
RMS-normalised), with the reference's own Compute behaviours: leading dims of A fold into rows
(tests/ops/test_matmulnbits.py:510-551), repeated runs are bit-identical (:558-653), weights that
are graph inputs are re-read on every call, and a forced failure surfaces as a status
(rust/src/ep.rs:2409-2424).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import mock_host as mh
from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture
def host(cuda):
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    n = h.supported_devices(n_amd=1)
    assert n == 1, "the MI355X was not advertised"
    assert h.device_meta(0, "mi355x.arch").startswith("gfx950")
    assert h.create_ep(0) == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0
    assert mh.lib().mock_bad_status_release() == 0


def _check(y, ref, what):
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert e1 <= TOL and e2 <= TOL, f"{what}: {e1:.3e} {e2:.3e}"


@pytest.mark.parametrize("lead,N,K,bits,bs,zp", [
    ((1,), 3072, 3072, 4, 32, False),
    ((1,), 9216, 3072, 4, 32, True),           # configs[1] qkv
    ((2, 3), 160, 1024, 4, 64, True),          # leading dims fold into M = 6
    ((7,), 48, 256, 8, 16, False),
    ((33,), 96, 512, 4, 128, True),            # MFMA GEMV row tiles
    ((2, 4), 3072, 3072, 4, 32, True),         # batched decode: 8 rows of o_proj
])
def test_compute_matches_oracle(host, lead, N, K, bits, bs, zp):
    print(f"[gpu] ep lead={lead} N={N} K={K} bits={bits} bs={bs} zp={zp}", flush=True)
    M = int(np.prod(lead))
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=M + N)
    host.reset()
    a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, bits, bs, lead + (K,))
    assert host.get_capability() == (1, ["mm:drop"])
    assert host.compile() == 0, mh.err()
    before = mh.EP_COUNT()
    A = inp["A"].reshape(lead + (K,))
    host.feed(a_name, A)
    assert host.compute(0) == 0, mh.err()
    assert mh.EP_COUNT() == before + 1
    y = host.fetch(y_name, np.float16, M * N)
    assert y.shape == lead + (N,)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    _check(y.reshape(M, N), ref, "ep")


@pytest.mark.parametrize("lead,N,K,bs,zp,a_dtype", [
    ((16,), 3072, 8192, 128, True, np.float16),
    ((1,), 512, 1024, 32, True, np.float32),        # the shape of the reference's level-4 record
    ((2, 3), 96, 512, 64, False, np.float16),       # leading dims fold into M = 6
])
def test_compute_accuracy_level_4(host, lead, N, K, bs, zp, a_dtype):
    """A node with accuracy_level = 4 is claimed, compiled and computed with int8 activations
    (the plugin's Compute runs the quantiser and the int8 MFMA GEMV), matching the oracle's
    level-4 definition at the output dtype's bar."""
    print(f"[gpu] ep acc4 lead={lead} N={N} K={K} bs={bs} zp={zp} {a_dtype.__name__}", flush=True)
    M = int(np.prod(lead))
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=4 * M + N,
                          a_dtype=a_dtype)
    host.reset()
    a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, 4, bs, lead + (K,),
                                         a_dtype=a_dtype, acc_level=4)
    assert host.get_capability() == (1, ["mm:drop"])
    assert host.compile() == 0, mh.err()
    before = mh.EP_COUNT()
    host.feed(a_name, inp["A"].reshape(lead + (K,)))
    assert host.compute(0) == 0, mh.err()
    assert mh.EP_COUNT() == before + 1
    y = host.fetch(y_name, a_dtype, M * N).reshape(M, N)
    ref4 = orc.matmul_nbits_acc4(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    if a_dtype == np.float16:
        _check(y, ref4, "ep acc4")
    else:
        # fp32 output: only the fp32 combination of exact int32 block dots differs
        assert orc.max_err_rms_normalised(y, ref4) <= 1e-5
    # the level-1 result differs by the int8 quantisation noise of A (about 0.6 % of RMS(y))
    ref1 = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    rms = float(np.sqrt(np.mean(ref1.astype(np.float64) ** 2)))
    assert float(np.sqrt(np.mean((y.astype(np.float64) - ref1) ** 2))) <= 1.2e-2 * rms


def test_three_runs_bit_identical_and_row_count_changes(host):
    N, K = 512, 2048
    inp = orc.make_inputs(4, N, K, with_zp=True, seed=5)
    host.reset()
    a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, 4, 32, (-1, K))
    host.get_capability()
    assert host.compile() == 0, mh.err()
    outs = []
    for _ in range(3):
        host.feed(a_name, inp["A"])
        assert host.compute(0) == 0, mh.err()
        outs.append(host.fetch(y_name, np.float16, 4 * N).copy())
    assert all(np.array_equal(outs[0].view(np.uint16), o.view(np.uint16)) for o in outs[1:])
    assert not np.array_equal(outs[0][0], outs[0][1])
    # a different row count through the same compiled node (symbolic batch): one row runs the
    # streaming GEMV, four rows the batched MFMA kernel, which sums in another order -- equal
    # to the fp16 bar, not bit for bit
    host.feed(a_name, inp["A"][:1])
    assert host.compute(0) == 0, mh.err()
    y1 = host.fetch(y_name, np.float16, N)
    _check(y1.reshape(1, N), outs[0][0].reshape(1, N).astype(np.float64), "one row vs four")
    ref = orc.matmul_nbits(inp["A"][:1], inp["B"], inp["scales"], inp["zp"], N, K, 4, 32)
    _check(y1.reshape(1, N), ref, "one row")
    # zero rows: an empty output, no launch
    host.feed(a_name, inp["A"][:0])
    assert host.compute(0) == 0, mh.err()


def test_weights_as_graph_inputs_are_read_every_call(host):
    N, K = 64, 256
    inp = orc.make_inputs(2, N, K, with_zp=True, seed=9)
    inp2 = orc.make_inputs(2, N, K, with_zp=True, seed=10)
    host.reset()
    a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, 4, 32, (2, K), const_weights=False)
    assert host.get_capability()[1] == ["mm:keep"]
    assert host.compile() == 0, mh.err()
    for d in (inp, inp2):
        host.feed(a_name, inp["A"])
        host.feed("mm_B", d["B"])
        host.feed("mm_scales", d["scales"])
        host.feed("mm_zp", d["zp"])
        assert host.compute(0) == 0, mh.err()
        y = host.fetch(y_name, np.float16, 2 * N)
        _check(y, orc.matmul_nbits(inp["A"], d["B"], d["scales"], d["zp"], N, K, 4, 32), "inputs")


@pytest.mark.parametrize("M,N,K,bits,bs,zp", [
    (3, 40, 512, 4, 32, True),        # fp32 streaming GEMV, one row-tile
    (1, 3072, 3072, 4, 32, False),    # BASELINE configs[0]'s shape with fp32 activations
    (24, 300, 1024, 8, 64, True),     # row-tiled fp32 streaming GEMV
    (200, 512, 2048, 4, 32, True),    # fp32 MFMA GEMM
])
def test_fp32_node(host, M, N, K, bits, bs, zp):
    """fp32 activations through the plugin's Compute: the fp32 kernels the planner takes at each
    row count, against the oracle at the fp32 bar."""
    import mnb
    kern = mnb.plan(mnb.problem(M, N, K, bits, bs, zp, mnb.DTYPE_F32)).kernel
    print(f"[gpu] ep fp32 M={M} N={N} K={K} bits={bits} bs={bs} zp={zp} kernel {kern}", flush=True)
    assert kern == (mnb.KERNEL_GEMV_STREAM if M <= 64 else mnb.KERNEL_GEMM_MFMA)
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=11 + M,
                          a_dtype=np.float32)
    host.reset()
    a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, bits, bs, (M, K), a_dtype=np.float32)
    host.get_capability()
    assert host.compile() == 0, mh.err()
    host.feed(a_name, inp["A"])
    assert host.compute(0) == 0, mh.err()
    y = host.fetch(y_name, np.float32, M * N)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    assert orc.max_rel_err_significant(y, ref) <= 1e-5


def test_forced_compute_failure_is_a_status(host):
    inp = orc.make_inputs(1, 32, 64, seed=2)
    host.reset()
    a_name, _ = mh.add_matmul_nbits(host, "mm", inp, 32, 64, 4, 32, (1, 64))
    host.get_capability()
    assert host.compile() == 0, mh.err()
    host.feed(a_name, inp["A"])
    os.environ["MI355X_EP_FORCE_COMPUTE_FAILURE"] = "1"
    try:
        assert host.compute(0) == mh.ORT_EP_FAIL
        assert "forced Compute failure" in mh.err()
    finally:
        del os.environ["MI355X_EP_FORCE_COMPUTE_FAILURE"]
    assert host.compute(0) == 0, mh.err()


def test_wrong_activation_width_is_rejected(host):
    inp = orc.make_inputs(1, 32, 64, seed=2)
    host.reset()
    a_name, _ = mh.add_matmul_nbits(host, "mm", inp, 32, 64, 4, 32, (1, -1))
    host.get_capability()
    assert host.compile() == 0, mh.err()
    host.feed(a_name, np.zeros((1, 128), np.float16))
    assert host.compute(0) == mh.ORT_INVALID_ARGUMENT


@pytest.fixture
def dm_host(cuda, monkeypatch):
    # MI355X_EP_DEVICE_MEMORY=1: ORT-style device I/O through the EP's allocator and data transfer
    monkeypatch.setenv("MI355X_EP_DEVICE_MEMORY", "1")
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    assert h.supported_devices(n_amd=1) == 1
    n, (t, vendor, dev) = h.allocator_infos(0)
    assert n == 1 and t == mh.MEM_GPU and vendor == mh.AMD, "HBM was not advertised"
    assert h.create_ep(0) == 0, mh.err()
    assert h.default_memory_device()[0] == 1
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0
    assert mh.lib().mock_live_memory_infos() == 0


@pytest.mark.parametrize("M,N,K,bs,zp", [(1, 9216, 3072, 32, True), (16, 3072, 8192, 128, True),
                                          (300, 512, 1024, 32, False)])
def test_device_resident_io_matches_oracle(dm_host, M, N, K, bs, zp):
    print(f"[gpu] ep device I/O M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=M + 3 * N)
    dm_host.reset()
    a_name, y_name = mh.add_matmul_nbits(dm_host, "mm", inp, N, K, 4, bs, (M, K))
    assert dm_host.get_capability() == (1, ["mm:drop"])
    assert dm_host.compile() == 0, mh.err()
    assert dm_host.device_io_setup(0) == 0, mh.err()
    before = mh.EP_COUNT()
    dm_host.feed_device(a_name, inp["A"])            # A in HBM, Y allocated in HBM
    assert dm_host.compute(0) == 0, mh.err()
    assert mh.EP_COUNT() == before + 1
    y = dm_host.fetch(y_name, np.float16, M * N)     # read back through the data transfer
    _check(y, orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs),
           "device I/O")


def test_device_resident_weights_as_graph_inputs(dm_host):
    N, K = 64, 256
    inp = orc.make_inputs(3, N, K, with_zp=True, seed=12)
    dm_host.reset()
    a_name, y_name = mh.add_matmul_nbits(dm_host, "mm", inp, N, K, 4, 32, (3, K),
                                         const_weights=False)
    assert dm_host.get_capability()[1] == ["mm:keep"]
    assert dm_host.compile() == 0, mh.err()
    assert dm_host.device_io_setup(0) == 0, mh.err()
    dm_host.feed_device(a_name, inp["A"])
    dm_host.feed_device("mm_B", inp["B"])
    dm_host.feed_device("mm_scales", inp["scales"])
    dm_host.feed_device("mm_zp", inp["zp"])
    assert dm_host.compute(0) == 0, mh.err()
    y = dm_host.fetch(y_name, np.float16, 3 * N)
    _check(y, orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, 32),
           "device-resident weights")


def test_stream_aware_chain_matches_oracle(dm_host):
    """Stream-aware mode (ORT's OrtSyncStreamImpl): ORT creates one stream for the device through
    CreateSyncStreamForDevice, the input copy, two chained MatMulNBits islands (the second reads
    the first's HBM output) and the output copy are ordered on it with no host wait in between,
    and OnSessionRunEnd finishes the run.  Three runs (x, y, x): each matches the oracle (the
    second node against the oracle applied to the first node's own output), the first and third
    are bit-identical."""
    print("[gpu] ep stream-aware chain", flush=True)
    M, K, N1, N2 = 4, 1024, 512, 256
    w1 = orc.make_inputs(M, N1, K, bits=4, block_size=32, with_zp=True, seed=31)
    w2 = orc.make_inputs(M, N2, N1, bits=4, block_size=64, with_zp=False, seed=32)
    dm_host.reset()
    a_name, y1_name = mh.add_matmul_nbits(dm_host, "mm1", w1, N1, K, 4, 32, (M, K))
    # the second node's input is the first's output
    _, y2_name = mh.add_matmul_nbits(dm_host, "mm2", w2, N2, N1, 4, 64, (M, N1), a_name=y1_name)
    assert dm_host.get_capability()[0] == 2
    assert dm_host.compile() == 0, mh.err()
    assert dm_host.device_io_setup(0) == 0, mh.err()
    assert dm_host.is_stream_aware() == 1
    assert dm_host.stream_setup() == 1, mh.err()
    assert dm_host.stream_handle()
    rng = np.random.default_rng(33)
    xs = [rng.standard_normal((M, K), dtype=np.float32).astype(np.float16) for _ in range(2)]
    outs = []
    for x in (xs[0], xs[1], xs[0]):
        dm_host.feed_device(a_name, x)
        assert dm_host.compute(0) == 0, mh.err()
        assert dm_host.compute(1) == 0, mh.err()
        assert dm_host.run_end() == 0, mh.err()
        y1 = dm_host.fetch(y1_name, np.float16, M * N1).reshape(M, N1)
        y2 = dm_host.fetch(y2_name, np.float16, M * N2).reshape(M, N2)
        _check(y1, orc.matmul_nbits(x, w1["B"], w1["scales"], w1["zp"], N1, K, 4, 32), "stream mm1")
        _check(y2, orc.matmul_nbits(y1, w2["B"], w2["scales"], None, N2, N1, 4, 64), "stream mm2")
        outs.append(y2)
    assert np.array_equal(outs[0].view(np.uint16), outs[2].view(np.uint16))
    assert dm_host.notification_roundtrip() == 0, mh.err()



@pytest.mark.parametrize("M,N,K,bs,zp", [(16, 3072, 3072, 32, True), (8, 3000, 8192, 128, False),
                                         (1, 3072, 3072, 32, True)])
def test_strip_major_weights_option(host, M, N, K, bs, zp):
    """ep.strip_major_weights (on by default): Compile also keeps each node's strip-major copy of B
    (mnb_weights_prepack), which Compute reads when the plan is the batched decode kernel; the
    output is bit-identical to the same node on an EP with the option off, and within the bar of
    the oracle."""
    print(f"[gpu] ep strip-major M={M} N={N} K={K} bs={bs} zp={zp}", flush=True)
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=7 * M + N)
    ys = []
    for opt in ("0", "1"):
        host.option("ep.strip_major_weights", opt)
        assert host.create_ep(0) == 0, mh.err()
        host.reset()
        a_name, y_name = mh.add_matmul_nbits(host, "mm", inp, N, K, 4, bs, (M, K))
        assert host.get_capability() == (1, ["mm:drop"])
        assert host.compile() == 0, mh.err()
        host.feed(a_name, inp["A"])
        assert host.compute(0) == 0, mh.err()
        ys.append(host.fetch(y_name, np.float16, M * N).reshape(M, N))
    assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check(ys[1], ref, "ep strip-major")
