"""The decode path allocates nothing: the structural form of the reference's AllocRecorder tests
(rust/src/ops/quant.rs:1496-1547, "the GEMV materialises no dequantised weight" and "GEMV
allocation is independent of the reduction extent").

Host-only: the planner's workspace figure (mnb_workspace_bytes, what a caller must provide and
what a session allocates) for the decode and small-batch plans, with no GPU.  The GPU half
(tests/test_gpu_allocs.py) shows that steady-state calls leave the library's device-allocation
counter unchanged.
"""

from __future__ import annotations

import pytest

import mnb

PHI35 = [("qkv_proj", 3072, 9216), ("o_proj", 3072, 3072), ("gate_up_proj", 3072, 16384),
         ("down_proj", 8192, 3072)]


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("name,k,n", PHI35)
def test_fp16_decode_and_small_batch_plans_need_no_workspace(name, k, n, m):
    for bits, bs, zp in ((4, 32, True), (4, 128, False), (8, 32, True), (4, 16, True)):
        p = mnb.problem(m, n, k, bits, bs, zp)
        assert mnb.workspace_bytes(p) == 0, (name, m, bits, bs, zp)
        assert mnb.plan(p).workspace_bytes == 0


@pytest.mark.parametrize("m", [1, 16])
def test_workspace_is_independent_of_the_reduction_extent(m):
    """Anything proportional to K in a GEMV's scratch is what an expanded weight looks like."""
    got = {k: mnb.workspace_bytes(mnb.problem(m, 3072, k, 4, 32, True))
           for k in (1024, 3072, 8192, 16384, 32768)}
    assert set(got.values()) == {0}, got


def test_int8_path_scratch_holds_activations_only():
    """accuracy_level = 4 at decode and batched-decode sizes (<= 16 rows) needs scratch for A's
    int8 codes and block scales only: exactly M x K code bytes plus the fp32 scales of 16 rows,
    each part 256-byte aligned, whatever N is -- far below a dequantised weight (2 N K bytes)."""
    def a256(x):
        return (x + 255) // 256 * 256
    for m, k in ((1, 1024), (1, 3072), (4, 3072), (8, 4096), (16, 2048), (16, 8192)):
        for n in (512, 3072, 12288):
            p = mnb.problem(m, n, k, 4, 128, True, mnb.DTYPE_F16, 4)
            assert mnb.plan(p).kernel == mnb.KERNEL_ACC4_STREAM, (m, k, n)
            ws = mnb.workspace_bytes(p)
            assert ws == a256(m * k) + a256(16 * (k // 128) * 4), (m, k, n, ws)
            assert ws < n * k // 2                    # below even the packed int4 weight
