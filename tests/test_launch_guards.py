"""Host-side guards of the HIP library (nothing here reaches a device): launch shapes against the
workgroup sizes the kernels are compiled for, and forms the library refuses before launching.

A workgroup larger than the thread count a kernel was compiled for (its __launch_bounds__) does
not run: the launch fails as an unspecified launch failure.  The launchers therefore refuse such
a shape before any HIP call, returning hipErrorInvalidValue.  The decode launcher takes its shape
as a StreamConfig (internal C++ API of libmnb_hip.so, bound here by its mangled name).
"""

from __future__ import annotations

import ctypes as C

HIP_ERROR_INVALID_VALUE = 1
LAUNCH_STREAM_CFG = "_ZN3mnb22launch_gemv_stream_cfgERKNS_12StreamConfigEPKvPKhS4_S6_PvllliiP12ihipStream_t"


class StreamConfig(C.Structure):
    # mnb::StreamConfig (csrc/kernels/mnb_launch.hpp)
    _fields_ = [("mr", C.c_int), ("g", C.c_int), ("cpl", C.c_int), ("u", C.c_int),
                ("waves_per_group", C.c_int), ("vec_s", C.c_int), ("vec_z", C.c_int),
                ("groups", C.c_int64), ("lds", C.c_int64)]


def _launcher():
    import mnb

    f = getattr(mnb.load(), LAUNCH_STREAM_CFG)
    f.restype = C.c_int
    f.argtypes = [C.POINTER(StreamConfig)] + [C.c_void_p] * 5 + [C.c_int64] * 3 + \
        [C.c_int, C.c_int, C.c_void_p]
    return f


def _cfg(**kw) -> StreamConfig:
    # a shape for qkv at M=1 (K=3072, N=9216): 32 lanes per column, 3 chunks each
    base = dict(mr=1, g=32, cpl=3, u=1, waves_per_group=4, vec_s=0, vec_z=0, groups=0, lds=0)
    base.update(kw)
    return StreamConfig(**base)


def _call(cfg: StreamConfig) -> int:
    fake = C.c_void_p(0x1000)          # never dereferenced: the guard returns first
    return _launcher()(C.byref(cfg), fake, fake, fake, fake, fake, 1, 9216, 3072, 4, 32, None)


def test_stream_launch_refuses_workgroups_above_compiled_bound():
    # 17 wavefronts = 1088 threads; gemv_stream is compiled for 1024
    assert _call(_cfg(waves_per_group=17)) == HIP_ERROR_INVALID_VALUE
    assert _call(_cfg(waves_per_group=32)) == HIP_ERROR_INVALID_VALUE
    assert _call(_cfg(waves_per_group=0)) == HIP_ERROR_INVALID_VALUE


def test_stream_launch_refuses_malformed_shapes():
    assert _call(_cfg(g=8)) == HIP_ERROR_INVALID_VALUE
    assert _call(_cfg(cpl=2)) == HIP_ERROR_INVALID_VALUE          # 32 * 2 chunks < 96
    assert _call(_cfg(mr=5)) == HIP_ERROR_INVALID_VALUE
    assert _call(_cfg(u=3)) == HIP_ERROR_INVALID_VALUE
    assert _call(_cfg(cpl=9)) == HIP_ERROR_INVALID_VALUE          # above the instantiated 8
    assert _call(_cfg(u=2)) == HIP_ERROR_INVALID_VALUE            # one column per lane group
    assert _call(_cfg(mr=2, u=2)) == HIP_ERROR_INVALID_VALUE


def test_planner_shapes_stay_within_compiled_bounds():
    """Every plan the planner makes for the decode, strip, group and GEMV kernels uses a
    workgroup no larger than that kernel family's compiled bound."""
    import mnb

    bounds = {mnb.KERNEL_GEMV_STREAM: 1024, mnb.KERNEL_GROUP_MFMA: 512,
              mnb.KERNEL_GEMV_MFMA: 1024, mnb.KERNEL_GEMM_MFMA: 512, mnb.KERNEL_ACC4_I8: 1024,
              mnb.KERNEL_STRIP_MFMA: 1024, mnb.KERNEL_GENERIC: 256,
              mnb.KERNEL_ACC4_STREAM: 1024, mnb.KERNEL_BATCH_STREAM: 1024}
    for m in (1, 2, 3, 4, 5, 8, 16, 17, 33, 64, 65, 256, 2048):
        for k, n in ((3072, 9216), (8192, 3072), (9216, 3072), (2880, 2880), (128, 48)):
            for bits in (4, 8):
                for bs in (16, 32, 64, 128):
                    for level in (0, 4):
                        p = mnb.problem(m, n, k, bits, bs, True, mnb.DTYPE_F16, level)
                        try:
                            info = mnb.plan(p)
                        except mnb.MnbError:
                            continue
                        bound = bounds[info.kernel]
                        if info.kernel == mnb.KERNEL_ACC4_STREAM and (k // 128) // info.waves_per_group == 8:
                            bound = 512                  # 8 quads per wavefront: compiled for 8 wavefronts
                        assert 64 * info.waves_per_group <= bound, (m, k, n, bits, bs, level, info.kernel, info.waves_per_group)


def test_noalloc_refuses_level_4_beyond_its_scratch():
    """The allocation-free entry point refuses an accuracy_level 4 problem whose workspace is
    larger than its scratch array, before any device work (the pointers are never read)."""
    import mnb

    lib = mnb.load()
    p = mnb.problem(8192, 64, 8192, 4, 32, False, mnb.DTYPE_F16, 4)
    assert mnb.workspace_bytes(p) > lib.mnb_noalloc_scratch_bytes() == 48 << 20
    assert lib.mnb_matmul_nbits_noalloc(C.byref(p), None, None, None, None, None, None) == \
        mnb.MNB_ERR_UNSUPPORTED
    assert b"scratch" in lib.mnb_last_error()


def test_rmsnorm_refuses_wide_fp32_rows():
    """fp32 rows above 4096 elements (and fp16 above 8192) are refused with a message, before
    anything reaches a device."""
    import mnb

    lib = mnb.load()
    for dtype, hidden, ok in ((mnb.DTYPE_F32, 4096, True), (mnb.DTYPE_F32, 8192, False),
                              (mnb.DTYPE_F16, 8192, True), (mnb.DTYPE_F16, 8200, False)):
        p = mnb.RmsNormProblem(5, hidden, 1e-5, 1, 0, 1, dtype)
        rc = lib.mnb_rmsnorm_check(C.byref(p))
        if ok:
            assert rc == mnb.MNB_OK
        else:
            assert rc == mnb.MNB_ERR_UNSUPPORTED
            assert b"hidden" in lib.mnb_last_error()
        rc = lib.mnb_skip_rmsnorm(C.byref(p), None, None, None, None, None, None, None)
        assert (rc == mnb.MNB_ERR_INVALID) if ok else (rc == mnb.MNB_ERR_UNSUPPORTED)


def test_decode_routing_by_rows_and_strips():
    """Host planning of the Phi-3.5 decode nodes (int4, block 32, zero points): up to three rows
    stream the weights once per row-tile on gemv_stream; from four rows on the batched kernel
    takes every node."""
    import mnb

    nodes = {"qkv": (3072, 9216), "o": (3072, 3072), "gate_up": (3072, 16384), "down": (8192, 3072)}
    for name, (k, n) in nodes.items():
        for m in (1, 2, 3):
            assert mnb.plan(mnb.problem(m, n, k, 4, 32, True)).kernel == mnb.KERNEL_GEMV_STREAM, (name, m)
        for m in (4, 5, 8, 16):
            assert mnb.plan(mnb.problem(m, n, k, 4, 32, True)).kernel == mnb.KERNEL_BATCH_STREAM, (name, m)


def test_fp32_decode_routing():
    """fp32 activations at 1-64 rows take the fp32 streaming GEMV (reported as the streaming
    kernel): row-tiles of the most rows, up to four, whose staged fp32 chunks fit in 96 KB of
    LDS, each tile with the fp16 kernel's launch shape for that row count; above 64 rows the fp32
    MFMA GEMM."""
    import mnb

    f32 = mnb.DTYPE_F32
    for k, n in ((3072, 9216), (3072, 3072), (3072, 16384), (8192, 3072)):
        for m in (1, 2, 3, 4, 5, 8, 16, 33, 64):
            for bits in (4, 8):
                for bs in (16, 32, 64, 128):
                    info = mnb.plan(mnb.problem(m, n, k, bits, bs, True, f32))
                    wpc = 128 // bits                    # weights per staged 16-byte chunk
                    mr = max(r for r in range(1, min(m, 4) + 1)
                             if r * (k // wpc) * (4 * wpc + 16) <= 96 * 1024)
                    assert info.kernel == mnb.KERNEL_GEMV_STREAM, (m, n, k, bits, bs)
                    assert (info.tile_m, info.grid_y) == (mr, -(-m // mr)), (m, n, k, bits, bs)
                    assert 64 * info.waves_per_group <= 1024
                    f16 = mnb.plan(mnb.problem(mr, n, k, bits, bs, True))
                    if f16.kernel == mnb.KERNEL_GEMV_STREAM:   # (at four rows fp16 may batch)
                        assert (info.waves_per_group, info.tile_n, info.grid_x) == \
                            (f16.waves_per_group, f16.tile_n, f16.grid_x), (m, n, k, bits, bs)
    # above 64 rows the fp32 MFMA GEMM: 128 x 128 tiles of four wavefronts (64 x 128 where the
    # 128-row tiles would number fewer than the 256 CUs), no workspace
    for m, bm in ((65, 64), (256, 64), (512, 128), (2048, 128)):
        info = mnb.plan(mnb.problem(m, 8192, 3072, 4, 32, True, f32))
        assert info.kernel == mnb.KERNEL_GEMM_MFMA and info.waves_per_group == 4
        assert info.tile_m == bm and info.grid_x == -(-m // bm) * 64 and info.workspace_bytes == 0
    # K not a multiple of the GEMM's 32-k step: the generic kernel
    assert mnb.plan(mnb.problem(65, 64, 48, 4, 16, True, f32)).kernel == mnb.KERNEL_GENERIC


# (M, N, K, bs, zp) -> (strips per workgroup S, quads per wavefront R) of the batched decode
# kernel.  The first twelve are the GPU parity shapes of tests/test_gpu_matmul.py
# (BATCH_GEOMETRY), one per instantiated (S, R) with S R <= 8; the rest are the Phi-3.5 decode
# nodes at 4 / 8 / 16 rows, at the geometries measured fastest on MI355X.
BATCH_PLANS = {
    (8, 768, 768, 32, True): (1, 1),
    (4, 16400, 1024, 32, False): (1, 2),
    (16, 3072, 2304, 32, True): (1, 3),
    (16, 3072, 8192, 32, True): (1, 4),
    (4, 65000, 256, 32, True): (2, 1),
    (4, 24008, 2048, 32, True): (2, 2),
    (8, 20000, 1920, 32, False): (2, 3),
    (4, 4100, 8192, 32, True): (2, 4),
    (12, 8320, 1920, 32, True): (3, 1),
    (4, 33000, 1024, 64, False): (3, 2),
    (4, 65000, 512, 32, True): (4, 1),
    (4, 65000, 1024, 64, False): (4, 2),
    (4, 9216, 3072, 32, True): (1, 3),       # qkv
    (8, 9216, 3072, 32, True): (3, 2),
    (16, 9216, 3072, 32, True): (3, 2),
    (4, 3072, 3072, 32, True): (1, 2),       # o_proj
    (8, 3072, 3072, 32, True): (1, 2),
    (16, 3072, 3072, 32, True): (1, 4),
    (4, 16384, 3072, 32, True): (2, 2),      # gate_up
    (8, 16384, 3072, 32, True): (2, 2),
    (16, 16384, 3072, 32, True): (4, 2),
    (8, 3072, 8192, 32, True): (1, 4),       # down_proj
}


def test_batched_decode_geometry():
    """The planner's batched-decode geometry: S = tile_n / 16, R = (K / 128) / waves_per_group,
    and one workgroup per S strips."""
    import mnb

    for (m, n, k, bs, zp), (s, r) in BATCH_PLANS.items():
        info = mnb.plan(mnb.problem(m, n, k, 4, bs, zp))
        assert info.kernel == mnb.KERNEL_BATCH_STREAM, (m, n, k)
        assert (info.tile_n // 16, (k // 128) // info.waves_per_group) == (s, r), (m, n, k)
        assert info.grid_x == -(-((n + 15) // 16) // s), (m, n, k)
        assert (k // 128) % r == 0 and info.waves_per_group <= 16 and s * r <= 8


def test_level4_stream_kernel_k_limit():
    """accuracy_level 4 at 16 fp16 rows: K = 8192 takes the strip-per-workgroup int8 kernel with
    8 quads per wavefront (8 wavefronts, the most it is compiled for at that depth); K = 9216 with
    block 128 would need 9 such wavefronts and goes to the int8 strip GEMV instead."""
    import mnb

    p = mnb.problem(16, 3072, 8192, 4, 128, True, mnb.DTYPE_F16, 4)
    info = mnb.plan(p)
    assert info.kernel == mnb.KERNEL_ACC4_STREAM and info.waves_per_group == 8
    p = mnb.problem(16, 3072, 9216, 4, 128, True, mnb.DTYPE_F16, 4)
    assert mnb.plan(p).kernel == mnb.KERNEL_ACC4_I8
