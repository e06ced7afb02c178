"""The MFMA calibration kernel bench.py uses to state the chip's fp16 MFMA ceiling.

Checked by closed forms: with constant operands (A = 1, B = 0) every accumulator stays 0; with
operands whose products are exact small integers the per-thread sum of the eight accumulators is
known exactly (every MFMA adds the same integer to each element).  Argument errors are rejected
before anything is launched.
"""

from __future__ import annotations

import pytest


def test_calibrate_rejects_bad_arguments():
    import mnb

    lib = mnb.load()
    assert lib.mnb_calibrate_mfma(0, 10, None, None, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_mfma(4, 0, None, None, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_mfma(4, 10, None, None, None) == mnb.MNB_ERR_INVALID


@pytest.mark.gpu
def test_calibrate_constant_operands_sum_to_zero(cuda):
    import mnb
    import torch

    lib = mnb.load()
    wgs, iters = 8, 50
    out = torch.full((wgs * 256,), float("nan"), dtype=torch.float32, device=cuda)
    mnb.check(lib.mnb_calibrate_mfma(wgs, iters, None, out.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.gpu
def test_calibrate_integer_operands_closed_form(cuda):
    """All A operands 1 and all B operands 2: each MFMA adds 16 * 1 * 2 = 32 to every element of
    its accumulator, so a thread's 16 accumulators x 16 elements sum to 16 * 16 * 32 * iters."""
    import mnb
    import torch

    lib = mnb.load()
    wgs, iters = 4, 37
    ops = torch.empty(wgs * 256, 8, 8, dtype=torch.float16, device=cuda)
    ops[:, :4, :] = 1.0
    ops[:, 4:, :] = 2.0
    out = torch.empty(wgs * 256, dtype=torch.float32, device=cuda)
    mnb.check(lib.mnb_calibrate_mfma(wgs, iters, ops.data_ptr(), out.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    expect = 16 * 16 * 32 * iters
    assert torch.all(out == expect).item(), (out.min().item(), out.max().item(), expect)


def test_read_floor_rejects_bad_arguments():
    import ctypes as C

    import mnb

    lib = mnb.load()
    buf = (C.c_uint8 * 4096)()
    out = (C.c_uint32 * 1024)()
    src = C.addressof(buf) + (-C.addressof(buf)) % 16
    assert lib.mnb_calibrate_read(None, 1024, 1, 4, 1, out, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_read(src, 1000, 1, 4, 1, out, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_read(src + 8, 1024, 1, 4, 1, out, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_read(src, 1024, 3, 4, 1, out, None) == mnb.MNB_ERR_INVALID
    # more than the 1024 threads per workgroup the kernel is compiled for
    assert lib.mnb_calibrate_read(src, 1024, 1, 17, 1, out, None) == mnb.MNB_ERR_INVALID
    assert lib.mnb_calibrate_read(src, 1024, 1, 0, 1, out, None) == mnb.MNB_ERR_INVALID


@pytest.mark.gpu
@pytest.mark.parametrize("loads,wpg,contig", [(1, 4, 1), (2, 4, 1), (4, 16, 0), (16, 1, 0)])
def test_read_floor_reads_every_unit(cuda, loads, wpg, contig):
    """Each thread XORs its `loads` 16-byte units; the result equals the kernel's marker exactly
    when every unit the thread was given was read.  Units of marker / zero chosen so that each
    thread's XOR is the marker: thread slot j of every 1 KB run holds the marker in its first
    unit only (contiguous runs) or in run 0 of the grid stride only."""
    import mnb
    import torch

    lib = mnb.load()
    magic = 0x9E3779B9
    waves = 64
    runs = waves * loads
    units = torch.zeros(runs, 64, 4, dtype=torch.int64)
    if contig:
        units.view(waves, loads, 64, 4)[:, 0, :, 0] = magic     # first run of each wavefront
    else:
        units[:waves, :, 0] = magic                             # runs 0 .. waves-1 (j = 0)
    src = torch.from_numpy(units.numpy().astype("uint32")).to(cuda)
    out = torch.zeros(1024, dtype=torch.int32, device=cuda)
    mnb.check(lib.mnb_calibrate_read(src.data_ptr(), src.numel() * 4, loads, wpg, contig,
                                     out.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.all(o[:64 * wpg] == 1), o[:64 * wpg]
    assert torch.all(o[64 * wpg:] == 0)
