"""GroupQueryAttention C-ABI argument checks (no GPU: mnb_gqa_check and the workspace query are
host code, and mnb_gqa rejects bad arguments before any launch).

The declines mirror the reference's translate_gqa (rust/src/ops/attention.rs:388-560): a head
count that does not group, an odd or oversized rotary_dim, and a present length that is neither
the shared-buffer nor the growing-cache extent.
"""

from __future__ import annotations

import ctypes as C

import pytest

ERR_INVALID, ERR_UNSUPPORTED = 1, 2


@pytest.fixture(scope="module")
def lib():
    import mnb
    return mnb.load()


def _p(**kw):
    import mnb
    a = dict(batch=1, seq_len=2, past_len_max=4, present_len=6, max_seq=64, num_heads=8,
             kv_num_heads=2, head_dim=32, rotary_dim=16)
    a.update(kw)
    scale = a.pop("scale", None)
    return mnb.gqa_problem(scale=scale, **a)


def test_accepts_both_cache_conventions(lib):
    assert lib.mnb_gqa_check(C.byref(_p())) == 0                      # growing
    assert lib.mnb_gqa_check(C.byref(_p(present_len=4))) == 0         # shared buffer
    assert lib.mnb_gqa_check(C.byref(_p(present_len=100))) == 0       # larger growing buffer
    assert lib.mnb_gqa_check(C.byref(_p(past_len_max=0, present_len=2))) == 0


@pytest.mark.parametrize("kw,code", [
    ({"num_heads": 6, "kv_num_heads": 4}, ERR_UNSUPPORTED),
    ({"kv_num_heads": 0}, ERR_UNSUPPORTED),
    ({"head_dim": 40}, ERR_UNSUPPORTED),
    ({"head_dim": 272}, ERR_UNSUPPORTED),
    ({"rotary_dim": 15}, ERR_INVALID),
    ({"rotary_dim": 0}, ERR_INVALID),
    ({"rotary_dim": 34}, ERR_INVALID),
    ({"present_len": 5}, ERR_INVALID),
    ({"present_len": 3}, ERR_INVALID),
    ({"max_seq": 0}, ERR_INVALID),
    ({"batch": -1}, ERR_INVALID),
    ({"scale": float("nan")}, ERR_INVALID),
])
def test_rejects(lib, kw, code):
    p = _p(**kw)
    assert lib.mnb_gqa_check(C.byref(p)) == code
    assert lib.mnb_last_error()
    ws = C.c_size_t(123)
    assert lib.mnb_gqa_workspace_bytes(C.byref(p), C.byref(ws)) == code
    assert ws.value == 0


def test_rejects_dtype(lib):
    p = _p()
    p.dtype = 2                                          # fp32
    assert lib.mnb_gqa_check(C.byref(p)) == ERR_UNSUPPORTED


def test_workspace_covers_rotated_q_and_new_kv(lib):
    p = _p(batch=2, seq_len=3, past_len_max=8, present_len=11)
    ws = C.c_size_t()
    assert lib.mnb_gqa_workspace_bytes(C.byref(p), C.byref(ws)) == 0
    q = 2 * 8 * 3 * 32
    kv = 2 * 2 * 3 * 32
    assert ws.value >= q * 4 + 2 * kv * 2


def test_null_and_alias_rejected_before_launch(lib):
    p = _p()
    buf = (C.c_uint8 * 4096)()
    a = C.addressof(buf)
    # seqlens_k NULL
    assert lib.mnb_gqa(C.byref(p), a, a + 512, a + 1024, None, a, a, a, a + 1536, a + 2048,
                       a, 4096, None) == ERR_INVALID
    # present_key aliases past_key but present_value does not alias past_value
    assert lib.mnb_gqa(C.byref(p), a, a + 512, a + 1024, a, a, a, a, a + 512, a + 2048, a,
                       4096, None) == ERR_INVALID
    # aliasing with a growing present length
    assert lib.mnb_gqa(C.byref(p), a, a + 512, a + 1024, a, a, a, a, a + 512, a + 1024, a,
                       4096, None) == ERR_INVALID
