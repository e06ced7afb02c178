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
