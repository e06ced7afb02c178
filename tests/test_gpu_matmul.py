"""GPU parity of the MatMulNBits HIP kernels against the CPU oracle, through the C ABI.

Bars (stated per test): dequant is bit-exact in fp16; integer-exact known answers are exact;
fp16 outputs are within max relative error 2e-3 over significant elements (|y_ref| >= 0.1 RMS,
the reference's own denominator, docs/PERF.md:4350-4372) of the fp64-accumulated oracle, and
within 2e-3 of it when normalised by max(|y_ref|, RMS) over every element; fp32 outputs within
1e-5.  fp16 output rounding alone contributes up to 4.9e-4.
"""

from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import pytest

from oracle import matmul_nbits as orc

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
F16_TOL = 2e-3
F32_TOL = 1e-5


def _load(name):
    d = np.load(GOLDEN / name)
    return {k: d[k] for k in d.files}


def _dev(x, device):
    import torch
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device)


# MNB_FORCE_KERNEL values and the planner kernel each one selects.
FORCED = {"stream": 5, "gemv": 1, "gemm": 2, "generic": 3, "group": 6, "strip": 7, "batch": 9}


def _forced_kernel(M, N, K, bits, bs, zp, kernel):
    """The kernel the planner picks for this shape with MNB_FORCE_KERNEL=kernel (host only)."""
    import mnb

    old = os.environ.get("MNB_FORCE_KERNEL")
    os.environ["MNB_FORCE_KERNEL"] = kernel
    try:
        return mnb.plan(mnb.problem(M, N, K, bits, bs, zp)).kernel
    finally:
        if old is None:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        else:
            os.environ["MNB_FORCE_KERNEL"] = old


def _forcible(shapes):
    """(shape..., kernel) for every forced kernel that really runs on the shape: a kernel that
    cannot take a shape is left out instead of silently re-running the default kernel."""
    return [(*sh, k) for sh in shapes for k in FORCED
            if _forced_kernel(*sh, k) == FORCED[k]]


def _run(inp, N, K, bits, bs, device, kernel=None, acc=0):
    import mnb
    import torch
    old = os.environ.get("MNB_FORCE_KERNEL")
    try:
        if kernel:
            os.environ["MNB_FORCE_KERNEL"] = kernel
            M = int(np.prod(inp["A"].shape[:-1]))
            got = mnb.plan(mnb.problem(M, N, K, bits, bs, inp.get("zp") is not None)).kernel
            assert got == FORCED[kernel], f"{kernel} forced, planner chose {got}"
        else:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        y = mnb.matmul_nbits(_dev(inp["A"], device), _dev(inp["B"], device),
                             _dev(inp["scales"], device), _dev(inp.get("zp"), device), N, K,
                             bits, bs, accuracy_level=acc)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        else:
            os.environ["MNB_FORCE_KERNEL"] = old
    return y.cpu().numpy()


def _check_f16(y, ref, what):
    e1 = orc.max_rel_err_significant(y, ref)
    e2 = orc.max_err_rms_normalised(y, ref)
    assert np.isfinite(y).all(), what
    assert e1 <= F16_TOL and e2 <= F16_TOL, f"{what}: rel_sig={e1:.3e} rms_norm={e2:.3e}"


KATS = sorted(p.name for p in GOLDEN.glob("kat_*.npz"))
DEQUANTS = sorted(p.name for p in GOLDEN.glob("dequant_*.npz"))


@pytest.mark.parametrize("name", DEQUANTS)
def test_dequant_bit_exact(cuda, name):
    import mnb
    import torch
    d = _load(name)
    N, K, bits, bs, hz = (int(v) for v in d["meta"])
    print(f"[gpu] dequant {name}", flush=True)
    W = mnb.dequantize_f16(_dev(d["B"], cuda), _dev(d["scales"], cuda), _dev(d.get("zp"), cuda),
                           N, K, bits, bs)
    torch.cuda.synchronize()
    got = W.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, d["W_bits"]), f"{np.count_nonzero(got != d['W_bits'])} mismatches"


def _kat_cases():
    out = []
    for name in KATS:
        M, N, K, bits, bs, hz = (int(v) for v in _load(name)["meta"])
        out += [(name, k) for k in FORCED if _forced_kernel(M, N, K, bits, bs, bool(hz), k) == FORCED[k]]
    return out


@pytest.mark.parametrize("name,kernel", _kat_cases())
def test_integer_exact_kat(cuda, name, kernel):
    d = _load(name)
    M, N, K, bits, bs, hz = (int(v) for v in d["meta"])
    print(f"[gpu] kat {name} {kernel}", flush=True)
    y = _run(d, N, K, bits, bs, cuda, kernel)
    assert np.array_equal(y.view(np.uint16), d["Y"].view(np.uint16)), \
        f"max |diff| = {np.abs(y.astype(np.float64) - d['Y_exact']).max()}"


SHAPES = [
    # (M, N, K, bits, bs, zp)
    (1, 64, 256, 4, 32, False),
    (1, 4096, 16384, 4, 32, True),     # 512 chunks per column: the widest register budget
    (1, 100, 8192, 8, 64, True),
    (2, 77, 4096, 8, 16, True),
    (3, 50, 2048, 4, 16, True),
    (4, 64, 4096, 4, 128, False),
    (1, 33, 256, 4, 32, True),         # odd N, partial column tile
    (1, 200, 2048, 8, 32, True),       # int8, two chunks per lane: lanes load their own scales
    (1, 96, 2048, 4, 16, True),        # block 16: two segments per chunk, lane-loaded scales
    (1, 32064, 3072, 4, 32, True),     # more wavefronts than the CUs hold: smallest workgroups
    (1, 47, 512, 4, 16, False),
    (1, 65, 1024, 4, 64, True),
    (1, 96, 2048, 4, 128, True),
    (2, 128, 3072, 4, 32, False),
    (3, 48, 2880, 4, 32, True),        # K not a multiple of the 128-weight wave step
    (4, 80, 640, 8, 32, True),
    (4, 96, 8192, 4, 32, True),        # four int4 rows at K=8192: two row-tiles of two rows
    (2, 72, 8192, 8, 32, True),        # int8 at K=8192: one-row tiles
    (3, 40, 8192, 4, 64, False),       # three rows, four chunks per lane
    (4, 48, 16384, 4, 32, True),       # four one-row tiles
    (5, 64, 512, 8, 16, False),
    (5, 9216, 3072, 4, 32, True),      # qkv at five rows: the batched decode kernel
    (4, 9216, 3072, 4, 32, True),      # qkv at four rows: batched, one strip per workgroup
    (4, 16400, 1024, 4, 32, False),    # four rows, 1025 workgroups, last strip whole
    (7, 40, 1024, 4, 64, True),
    (12, 33, 2048, 4, 128, False),     # partial strip
    (16, 3072, 8192, 4, 32, True),     # sixteen wavefronts of four quads
    (6, 8200, 1024, 4, 64, True),      # last strip partial
    (9, 16400, 512, 4, 32, False),
    (7, 8320, 1024, 4, 64, False),
    (8, 768, 768, 4, 32, True),        # batched, one quad per wavefront
    (16, 3072, 2304, 4, 32, True),     # batched, three quads per wavefront (Gemma-2's hidden size)
    (8, 2000, 768, 4, 64, True),       # block 64: six scales, three zp bytes per wavefront
    (8, 20000, 1920, 4, 32, False),    # two strips of three quads per wavefront
    (7, 32, 256, 8, 64, True),
    (8, 160, 1024, 8, 128, False),
    (9, 64, 4096, 4, 32, True),
    (16, 128, 3072, 4, 32, False),
    (17, 64, 512, 4, 32, True),        # two 16-row MFMA tiles
    (32, 96, 1024, 4, 64, False),
    (33, 64, 512, 4, 16, True),        # four-tile path
    (64, 64, 256, 8, 32, True),
    (100, 48, 256, 4, 32, False),      # several row groups
]


@pytest.mark.parametrize("M,N,K,bits,bs,zp,kernel", _forcible(SHAPES))
def test_random_parity_f16(cuda, M, N, K, bits, bs, zp, kernel):
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=M * 1000 + N + K)
    print(f"[gpu] parity M={M} N={N} K={K} bits={bits} bs={bs} zp={zp} {kernel}", flush=True)
    y = _run(inp, N, K, bits, bs, cuda, kernel)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    _check_f16(y, ref, f"{kernel} M={M} N={N} K={K} b{bits} bs{bs} zp={zp}")


# Every (strips per workgroup S, quads per wavefront R) the batched decode kernel is built for
# (S R <= 8), as its planner chooses them, with whole and short last workgroups, partial strips,
# blocks 32 / 64 and with and without zero points: (M, N, K, bits, bs, zp, S, R).
BATCH_GEOMETRY = [
    (8, 768, 768, 4, 32, True, 1, 1),
    (4, 16400, 1024, 4, 32, False, 1, 2),
    (16, 3072, 2304, 4, 32, True, 1, 3),
    (16, 3072, 8192, 4, 32, True, 1, 4),
    (4, 65000, 256, 4, 32, True, 2, 1),       # last workgroup one strip, partial strip
    (4, 24008, 2048, 4, 32, True, 2, 2),      # partial strip
    (8, 20000, 1920, 4, 32, False, 2, 3),
    (4, 4100, 8192, 4, 32, True, 2, 4),       # last workgroup one partial strip
    (12, 8320, 1920, 4, 32, True, 3, 1),      # last workgroup one strip
    (4, 33000, 1024, 4, 64, False, 3, 2),     # last workgroup two strips, the second partial
    (4, 65000, 512, 4, 32, True, 4, 1),       # last workgroup three strips, the third partial
    (4, 65000, 1024, 4, 64, False, 4, 2),
]


@pytest.mark.parametrize("M,N,K,bits,bs,zp,S,R", BATCH_GEOMETRY)
def test_batch_geometry_parity(cuda, M, N, K, bits, bs, zp, S, R):
    import mnb
    info = mnb.plan(mnb.problem(M, N, K, bits, bs, zp))
    assert info.kernel == mnb.KERNEL_BATCH_STREAM
    assert (info.tile_n // 16, (K // 128) // info.waves_per_group) == (S, R)
    assert info.grid_x == -(-(-(-N // 16)) // S)
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=7 * M + N + K)
    print(f"[gpu] batch geometry M={M} N={N} K={K} bs={bs} zp={zp} S={S} R={R}", flush=True)
    y = _run(inp, N, K, bits, bs, cuda)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    _check_f16(y, ref, f"batch S={S} R={R} M={M} N={N} K={K}")


# The first four run the generic kernel's forms (and the fp32 streaming GEMV at M <= 4); the rest
# are fp32 decode shapes of the streaming GEMV: the Phi-3.5 nodes at one to four rows, int8,
# blocks 16-128, a column count that leaves the last workgroup partial.
F32_SHAPES = [(1, 40, 256, 4, 32, True), (6, 24, 512, 8, 64, False), (3, 17, 128, 4, 16, True),
              (9, 50, 1024, 4, 128, False),
              (1, 9216, 3072, 4, 32, True), (1, 3072, 8192, 4, 32, True), (2, 3072, 8192, 4, 32, True),
              (4, 1000, 3072, 4, 32, False), (3, 16384, 3072, 4, 32, True), (1, 640, 2048, 8, 64, True),
              (2, 500, 1024, 8, 16, False), (4, 300, 4096, 4, 128, True), (1, 2880, 2880, 4, 16, False),
              (4, 3072, 8192, 4, 32, True), (16, 3072, 3072, 4, 32, True), (37, 700, 2048, 8, 32, True),
              (64, 256, 8192, 4, 64, False), (70, 48, 512, 4, 32, True),
              (256, 3072, 3072, 4, 32, True), (130, 1000, 2048, 8, 64, False), (300, 257, 1024, 4, 16, True),
              (2048, 384, 3072, 4, 32, False), (97, 8192, 512, 8, 128, True),
              (512, 8192, 512, 4, 32, True), (1024, 4096, 1024, 8, 64, False)]   # 128-row tiles


@pytest.mark.parametrize("M,N,K,bits,bs,zp", F32_SHAPES)
def test_random_parity_f32(cuda, M, N, K, bits, bs, zp):
    import mnb
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=7 + M, a_dtype=np.float32)
    kern = mnb.plan(mnb.problem(M, N, K, bits, bs, zp, mnb.DTYPE_F32)).kernel
    print(f"[gpu] parity f32 M={M} N={N} K={K} bits={bits} bs={bs} zp={zp} kernel {kern}", flush=True)
    assert kern == (mnb.KERNEL_GEMV_STREAM if M <= 64 else mnb.KERNEL_GEMM_MFMA)
    y = _run(inp, N, K, bits, bs, cuda)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    assert orc.max_rel_err_significant(y, ref) <= F32_TOL
    assert orc.max_err_rms_normalised(y, ref) <= F32_TOL


@pytest.mark.parametrize("M,N,K,bits,bs,zp", [(1, 64, 32768, 4, 32, True), (2, 100, 16384, 8, 32, False)])
def test_wide_k_parity_f32(cuda, M, N, K, bits, bs, zp):
    """A few fp32 rows whose staged activations exceed the streaming GEMV's LDS (K = 16-32 K):
    the planner takes the fp32 GEMM (one 64-row tile) instead."""
    import mnb
    assert mnb.plan(mnb.problem(M, N, K, bits, bs, zp, mnb.DTYPE_F32)).kernel == mnb.KERNEL_GEMM_MFMA
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=23 + M, a_dtype=np.float32)
    print(f"[gpu] parity f32 wide K M={M} N={N} K={K}", flush=True)
    y = _run(inp, N, K, bits, bs, cuda)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    assert orc.max_rel_err_significant(y, ref) <= F32_TOL
    assert orc.max_err_rms_normalised(y, ref) <= F32_TOL


@pytest.mark.parametrize("M,N,K,bits,bs,zp", [(6, 24, 512, 8, 64, False), (9, 50, 1024, 4, 128, False),
                                              (2, 40, 256, 4, 16, True)])
def test_generic_parity_f32(cuda, M, N, K, bits, bs, zp):
    """The generic kernel's fp32 form (forced: the planner sends these shapes to the streaming
    GEMV), against the same oracle and bar."""
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=17 + M, a_dtype=np.float32)
    print(f"[gpu] parity f32 generic M={M} N={N} K={K}", flush=True)
    y = _run(inp, N, K, bits, bs, cuda, "generic")
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    assert orc.max_rel_err_significant(y, ref) <= F32_TOL
    assert orc.max_err_rms_normalised(y, ref) <= F32_TOL


# BASELINE configs 1 and 2 (Phi-3.5 decode layer set), full size, through the default planner.
CONFIGS = [
    ("cfg1", 1, 3072, 3072, False),
    ("cfg2_qkv", 1, 9216, 3072, True),
    ("cfg2_o", 1, 3072, 3072, True),
    ("cfg2_gate_up", 1, 16384, 3072, True),
    ("cfg2_down", 1, 3072, 8192, True),
    ("cfg5_shape_fp", 16, 3072, 8192, True),
]


@pytest.mark.parametrize("name,M,N,K,zp", CONFIGS)
def test_baseline_configs_full_size(cuda, name, M, N, K, zp):
    bs = 32 if name != "cfg5_shape_fp" else 128
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=20260801)
    print(f"[gpu] {name} M={M} N={N} K={K}", flush=True)
    y = _run(inp, N, K, 4, bs, cuda)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    _check_f16(y, ref, name)


GEMM_SHAPES = [
    # (M, N, K, bits, bs, zp): tile edges in M and N, every block size and both weight widths
    (65, 64, 256, 4, 32, False),
    (128, 256, 512, 4, 32, True),
    (129, 300, 1024, 4, 64, False),
    (256, 8192, 3072, 4, 32, False),   # BASELINE configs[2], M=256
    (300, 130, 2048, 4, 128, True),
    (512, 512, 3072, 4, 32, True),
    (777, 1000, 768, 4, 64, True),
    (100, 200, 512, 4, 16, True),      # block 16: two scale dwords per column and step
    (300, 96, 1024, 4, 16, False),
    (2048, 2880, 2880, 8, 32, True),   # gpt-oss 8-bit node at prefill size
    (129, 136, 1024, 8, 16, True),     # 8-bit, block 16: a zero-point dword per step
    (300, 260, 2048, 8, 64, False),
    (65, 128, 1536, 8, 128, True),
]


@pytest.mark.parametrize("M,N,K,bits,bs,zp", GEMM_SHAPES)
def test_gemm_parity(cuda, M, N, K, bits, bs, zp):
    inp = orc.make_inputs(M, N, K, bits=bits, block_size=bs, with_zp=zp, seed=M + 7 * N + K)
    print(f"[gpu] gemm M={M} N={N} K={K} bits={bits} bs={bs} zp={zp}", flush=True)
    y = _run(inp, N, K, bits, bs, cuda, "gemm")
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, bits, bs)
    _check_f16(y, ref, f"gemm M={M} N={N} K={K} bits={bits} bs={bs}")


def test_gemm_uneven_k_split(cuda):
    """K split whose last split is shorter: K = 1600 is 25 steps of 64, over 3 workgroups per tile
    (9, 9 and 7 steps).  Checked against the oracle, and against the same GEMM run unsplit (no
    workspace) at the same bar."""
    import mnb
    import torch

    M, N, K = 129, 300, 1600
    p = mnb.problem(M, N, K, 4, 32, False)
    info = mnb.plan(p)
    tiles = -(-M // info.tile_m) * -(-N // info.tile_n)
    assert info.kernel == mnb.KERNEL_GEMM_MFMA and info.grid_x == 3 * tiles
    assert mnb.workspace_bytes(p) == 3 * M * N * 4
    inp = orc.make_inputs(M, N, K, bits=4, block_size=32, with_zp=False, seed=1600)
    print(f"[gpu] gemm uneven split M={M} N={N} K={K}", flush=True)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], None, N, K, 4, 32)
    split = _run(inp, N, K, 4, 32, cuda)
    _check_f16(split, ref, "uneven split")
    t = {k: _dev(v, cuda) for k, v in inp.items() if v is not None}
    unsplit = torch.empty(M, N, dtype=torch.float16, device=cuda)
    import ctypes as C
    mnb.check(mnb.load().mnb_matmul_nbits(C.byref(p), t["A"].data_ptr(), t["B"].data_ptr(),
                                          t["scales"].data_ptr(), None, unsplit.data_ptr(), None,
                                          0, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    _check_f16(unsplit.cpu().numpy(), ref, "unsplit")


@pytest.mark.parametrize("M", [512, 2048])
def test_prefill_config_full_size(cuda, M):
    # K=3072, N=8192, int4 bs32, implicit zero point, through the planner
    import mnb
    N, K = 8192, 3072
    assert mnb.plan(mnb.problem(M, N, K, 4, 32, False)).kernel == mnb.KERNEL_GEMM_MFMA
    inp = orc.make_inputs(M, N, K, bits=4, block_size=32, with_zp=False, seed=20260801)
    print(f"[gpu] prefill M={M}", flush=True)
    y = _run(inp, N, K, 4, 32, cuda)
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], None, N, K, 4, 32)
    _check_f16(y, ref, f"prefill M={M}")


def test_gemm_k_split_plan():
    import mnb
    # M=256 and 512 (64 and 128 row tiles of 256 x 128 for 256 CUs) split K over 4 and 2
    # workgroups per tile, with fp32 partials in the workspace; M=2048 fills the GPU unsplit
    for m, ks in ((256, 4), (512, 2), (2048, 1)):
        info = mnb.plan(mnb.problem(m, 8192, 3072, 4, 32, False))
        assert info.kernel == mnb.KERNEL_GEMM_MFMA
        assert info.grid_x == (m + 255) // 256 * 64 * ks
        assert info.workspace_bytes == (ks * m * 8192 * 4 if ks > 1 else 0)


def test_gemm_k_split_graph_replays(cuda):
    """A K-split GEMM (the split launch and the partial sum) recorded in a graph: each replay
    (eager work and a synchronisation between them) is bit-identical to the eager call."""
    import mnb
    import torch

    M, N, K = 512, 4096, 3072                          # 64 tiles, four K splits each
    p = mnb.problem(M, N, K, 4, 32, True)
    assert mnb.plan(p).grid_x == 4 * 64
    inp = orc.make_inputs(M, N, K, bits=4, block_size=32, with_zp=True, seed=4096)
    t = {k: _dev(inp[k], cuda) for k in ("A", "B", "scales", "zp")}
    ws = torch.empty(mnb.workspace_bytes(p), dtype=torch.uint8, device=cuda)
    y = torch.empty(M, N, dtype=torch.float16, device=cuda)
    print("[gpu] gemm K split in a graph, 3 replays", flush=True)
    eager = mnb.matmul_nbits(t["A"], t["B"], t["scales"], t["zp"], N, K, 4, 32).cpu().numpy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mnb.matmul_nbits(t["A"], t["B"], t["scales"], t["zp"], N, K, 4, 32, out=y, workspace=ws,
                         stream=s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mnb.matmul_nbits(t["A"], t["B"], t["scales"], t["zp"], N, K, 4, 32, out=y, workspace=ws,
                         stream=s.cuda_stream)
    for r in range(3):
        y.fill_(0)
        mnb.matmul_nbits(t["A"][:1], t["B"], t["scales"], t["zp"], N, K, 4, 32)   # eager work
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint16), eager.view(np.uint16)), f"replay {r}"


@pytest.mark.parametrize("M,N,K,bs,zp", [(256, 8192, 3072, 32, False), (300, 130, 2048, 128, True),
                                         (129, 300, 1024, 64, False)])
def test_gemm_k_split_and_unsplit_runs(cuda, M, N, K, bs, zp):
    # the split launch (workspace given) and the one-pass launch (no workspace) both meet the
    # bar against the oracle, and the split is run-to-run bit-identical
    import ctypes as C
    import mnb
    import torch
    inp = orc.make_inputs(M, N, K, bits=4, block_size=bs, with_zp=zp, seed=5 + M)
    p = mnb.problem(M, N, K, 4, bs, zp)
    assert mnb.workspace_bytes(p) > 0
    print(f"[gpu] gemm split/unsplit M={M} N={N} K={K}", flush=True)
    t = {k: _dev(inp[k], cuda) for k in ("A", "B", "scales", "zp")}
    ys = [mnb.matmul_nbits(t["A"], t["B"], t["scales"], t["zp"], N, K, 4, bs) for _ in range(2)]
    y1 = torch.empty(M, N, dtype=torch.float16, device=cuda)
    s = int(torch.cuda.current_stream().cuda_stream)
    mnb.check(mnb.load().mnb_matmul_nbits(C.byref(p), t["A"].data_ptr(), t["B"].data_ptr(),
                                          t["scales"].data_ptr(),
                                          t["zp"].data_ptr() if zp else None, y1.data_ptr(),
                                          None, 0, s))
    torch.cuda.synchronize()
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], inp["zp"], N, K, 4, bs)
    split = [y.cpu().numpy() for y in ys]
    assert np.array_equal(split[0].view(np.uint16), split[1].view(np.uint16))
    _check_f16(split[0], ref, f"split M={M}")
    _check_f16(y1.cpu().numpy(), ref, f"unsplit M={M}")


def test_three_runs_bit_identical(cuda):
    # tests/ops/test_matmulnbits.py:558-653: repeated runs in one session are bit-identical
    inp = orc.make_inputs(4, 1000, 3072, bits=4, block_size=32, with_zp=True, seed=42)
    print("[gpu] determinism", flush=True)
    ys = [_run(inp, 1000, 3072, 4, 32, cuda) for _ in range(3)]
    assert all(np.array_equal(ys[0].view(np.uint16), y.view(np.uint16)) for y in ys[1:])
    # negative control: the rows are distinct (tests/ops/test_matmulnbits.py:454-478)
    assert not np.array_equal(ys[0][0], ys[0][1])


def test_m_zero_is_a_no_op(cuda):
    import mnb
    import torch
    A = torch.empty(0, 256, dtype=torch.float16, device=cuda)
    inp = orc.make_inputs(1, 32, 256, seed=1)
    y = mnb.matmul_nbits(A, _dev(inp["B"], cuda), _dev(inp["scales"], cuda), None, 32, 256, 4, 32)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, 32)


def test_unaligned_activation_view_falls_back(cuda):
    import mnb
    import torch
    inp = orc.make_inputs(2, 64, 256, seed=3)
    flat = torch.zeros(2 * 256 + 1, dtype=torch.float16, device=cuda)
    flat[1:] = torch.from_numpy(inp["A"].reshape(-1)).to(cuda)
    A = flat[1:].view(2, 256)                       # 2-byte aligned, not 16
    y = mnb.matmul_nbits(A, _dev(inp["B"], cuda), _dev(inp["scales"], cuda), None, 64, 256, 4, 32)
    torch.cuda.synchronize()
    ref = orc.matmul_nbits(inp["A"], inp["B"], inp["scales"], None, 64, 256, 4, 32)
    _check_f16(y.cpu().numpy(), ref, "unaligned")


def test_session_host_io_path(cuda):
    """Weights uploaded once, then host A in / host Y out (the reference's Compute data flow)."""
    import ctypes as C
    import mnb
    lib = mnb.load()
    inp = orc.make_inputs(3, 96, 512, bits=4, block_size=32, with_zp=True, seed=77)
    s = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(s)))
    try:
        p = mnb.problem(0, 96, 512, 4, 32, True)
        w = C.c_void_p()
        B, S, Z = inp["B"], inp["scales"], inp["zp"]
        mnb.check(lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes, S.ctypes.data,
                                         S.nbytes, Z.ctypes.data, Z.nbytes, C.byref(w)))
        before = mnb.launch_count()
        for _ in range(2):
            Y = np.zeros((3, 96), dtype=np.float16)
            A = np.ascontiguousarray(inp["A"])
            mnb.check(lib.mnb_session_run_host(s, w, 3, A.ctypes.data, Y.ctypes.data))
            ref = orc.matmul_nbits(A, B, S, Z, 96, 512, 4, 32)
            _check_f16(Y, ref, "session")
        assert mnb.launch_count() == before + 2
        # a wrong byte count is rejected, not read past
        w2 = C.c_void_p()
        rc = lib.mnb_weights_upload(s, C.byref(p), B.ctypes.data, B.nbytes - 1, S.ctypes.data,
                                    S.nbytes, Z.ctypes.data, Z.nbytes, C.byref(w2))
        assert rc == mnb.MNB_ERR_INVALID
        mnb.check(lib.mnb_weights_release(w))
    finally:
        lib.mnb_session_destroy(s)
