"""ctypes binding of ``libmnb_hip.so`` (the C ABI in ``include/mnb_hip.h``).

This is the Python host's view of the MI355X MatMulNBits library: tests and ``bench.py`` call
the HIP kernels through exactly the C entry points an ORT plugin or any other FFI host binds.
PyTorch is used only as device-memory and stream plumbing (``tensor.data_ptr()``,
``torch.cuda.current_stream().cuda_stream``).  Loading fails loudly when the library has not
been built; there is no CPU fallback.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_DIR = PKG / "lib"
HIP_LIB = LIB_DIR / "libmnb_hip.so"
EP_LIB = LIB_DIR / "libonnxruntime_mi355x_ep.so"

MNB_OK = 0
MNB_ERR_INVALID = 1
MNB_ERR_UNSUPPORTED = 2
MNB_ERR_HIP = 3
MNB_ERR_NOMEM = 4

COPY_HOST_TO_DEVICE = 1
COPY_DEVICE_TO_HOST = 2
COPY_DEVICE_TO_DEVICE = 3

DTYPE_F16 = 1
DTYPE_F32 = 2

KERNEL_GEMV_MFMA = 1
KERNEL_GEMM_MFMA = 2
KERNEL_GENERIC = 3
KERNEL_ACC4_I8 = 4
KERNEL_GEMV_STREAM = 5
KERNEL_GROUP_MFMA = 6
KERNEL_STRIP_MFMA = 7
KERNEL_ACC4_STREAM = 8
KERNEL_BATCH_STREAM = 9
KERNEL_NAMES = {1: "gemv_mfma", 2: "gemm_mfma", 3: "generic", 4: "acc4_i8", 5: "gemv_stream",
                6: "group_mfma", 7: "strip_mfma", 8: "acc4_stream", 9: "batch_stream"}


class Problem(C.Structure):
    _fields_ = [
        ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("bits", C.c_int32), ("block_size", C.c_int32), ("has_zero_points", C.c_int32),
        ("dtype", C.c_int32), ("accuracy_level", C.c_int32), ("reserved", C.c_int32),
    ]


class PlanInfo(C.Structure):
    _fields_ = [
        ("kernel", C.c_int32), ("waves_per_group", C.c_int32), ("tile_n", C.c_int32),
        ("tile_m", C.c_int32), ("grid_x", C.c_int64), ("grid_y", C.c_int64),
        ("workspace_bytes", C.c_int64),
    ]


class MoeProblem(C.Structure):
    _fields_ = [
        ("num_experts", C.c_int64), ("total_rows", C.c_int64), ("max_rows_per_expert", C.c_int64),
        ("a_rows", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("bits", C.c_int32), ("block_size", C.c_int32), ("has_zero_points", C.c_int32),
        ("dtype", C.c_int32),
    ]


class QmoeProblem(C.Structure):
    _fields_ = [
        ("rows", C.c_int64), ("hidden", C.c_int64), ("inter", C.c_int64),
        ("num_experts", C.c_int64), ("k", C.c_int32), ("block_size", C.c_int32),
        ("swiglu_fusion", C.c_int32), ("normalize_routing", C.c_int32),
        ("activation_alpha", C.c_float), ("activation_beta", C.c_float),
        ("swiglu_limit", C.c_float), ("has_swiglu_limit", C.c_int32),
        ("router_dtype", C.c_int32), ("dtype", C.c_int32),
    ]


class RmsNormProblem(C.Structure):
    _fields_ = [
        ("rows", C.c_int64), ("hidden", C.c_int64), ("epsilon", C.c_float),
        ("has_skip", C.c_int32), ("has_bias", C.c_int32), ("want_sum", C.c_int32),
        ("dtype", C.c_int32),
    ]


class GqaProblem(C.Structure):
    _fields_ = [
        ("batch", C.c_int64), ("seq_len", C.c_int64), ("past_len_max", C.c_int64),
        ("present_len", C.c_int64), ("max_seq", C.c_int64), ("num_heads", C.c_int32),
        ("kv_num_heads", C.c_int32), ("head_dim", C.c_int32), ("rotary_dim", C.c_int32),
        ("scale", C.c_float), ("dtype", C.c_int32),
    ]


GQA_ON_DEVICE_QKV, GQA_ON_DEVICE_PAST, GQA_ON_DEVICE_SEQLENS = 1, 2, 4
GQA_ON_DEVICE_OUT, GQA_ON_DEVICE_PRESENT, GQA_ON_DEVICE_CACHES = 8, 16, 32


class MnbError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"mnb error {code}: {msg}")
        self.code = code


_lib = None


def load() -> C.CDLL:
    """Load ``libmnb_hip.so`` (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not HIP_LIB.exists():
        raise FileNotFoundError(
            f"{HIP_LIB} is missing: build it with `python onnxruntime-ep-vulkan_amd/build.py`")
    lib = C.CDLL(str(HIP_LIB), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    vp, i64, i32, sz = C.c_void_p, C.c_int64, C.c_int32, C.c_size_t
    sig = {
        "mnb_last_error": (C.c_char_p, []),
        "mnb_version": (C.c_int, []),
        "mnb_check_problem": (C.c_int, [C.POINTER(Problem)]),
        "mnb_plan": (C.c_int, [C.POINTER(Problem), C.POINTER(PlanInfo)]),
        "mnb_workspace_bytes": (C.c_int, [C.POINTER(Problem), C.POINTER(sz)]),
        "mnb_matmul_nbits": (C.c_int, [C.POINTER(Problem), vp, vp, vp, vp, vp, vp, sz, vp]),
        "mnb_matmul_nbits_noalloc": (C.c_int, [C.POINTER(Problem), vp, vp, vp, vp, vp, vp]),
        "mnb_noalloc_scratch_bytes": (sz, []),
        "mnb_dequantize_f16": (C.c_int, [i64, i64, i32, i32, vp, vp, vp, vp, vp]),
        "mnb_quantize_a_int8": (C.c_int, [i64, i64, i32, i32, vp, vp, vp, vp, vp]),
        "mnb_moe_grouped": (C.c_int, [C.POINTER(MoeProblem), vp, vp, vp, vp, vp, vp, vp, vp]),
        "mnb_device_count": (C.c_int, [C.POINTER(C.c_int)]),
        "mnb_device_arch": (C.c_int, [C.c_int, C.c_char_p, sz]),
        "mnb_session_create": (C.c_int, [C.c_int, C.POINTER(vp)]),
        "mnb_session_destroy": (C.c_int, [vp]),
        "mnb_session_stream": (vp, [vp]),
        "mnb_session_synchronize": (C.c_int, [vp]),
        "mnb_session_set_async": (C.c_int, [vp, C.c_int]),
        "mnb_memcpy_on_stream": (C.c_int, [C.c_int, vp, vp, C.c_size_t, C.c_int, vp]),
        "mnb_stream_synchronize": (C.c_int, [C.c_int, vp]),
        "mnb_device_synchronize": (C.c_int, [C.c_int]),
        "mnb_event_create": (C.c_int, [C.c_int, C.POINTER(vp)]),
        "mnb_event_destroy": (C.c_int, [vp]),
        "mnb_event_record": (C.c_int, [vp, vp]),
        "mnb_stream_wait_event": (C.c_int, [vp, vp]),
        "mnb_event_synchronize": (C.c_int, [vp]),
        "mnb_weights_upload": (C.c_int, [vp, C.POINTER(Problem), vp, sz, vp, sz, vp, sz,
                                         C.POINTER(vp)]),
        "mnb_weights_release": (C.c_int, [vp]),
        "mnb_weights_prepack": (C.c_int, [vp, C.POINTER(i64)]),
        "mnb_session_run_device": (C.c_int, [vp, vp, i64, vp, vp]),
        "mnb_session_run_host": (C.c_int, [vp, vp, i64, vp, vp]),
        "mnb_session_run": (C.c_int, [vp, vp, i64, vp, C.c_int, vp, C.c_int]),
        "mnb_device_malloc": (C.c_int, [C.c_int, sz, C.POINTER(vp)]),
        "mnb_device_free": (C.c_int, [C.c_int, vp]),
        "mnb_memcpy": (C.c_int, [C.c_int, vp, vp, sz, C.c_int]),
        "mnb_launch_count": (C.c_uint64, []),
        "mnb_device_alloc_count": (C.c_uint64, []),
        "mnb_calibrate_mfma": (C.c_int, [i32, i32, vp, vp, vp]),
        "mnb_calibrate_read": (C.c_int, [vp, sz, i32, i32, i32, vp, vp]),
        "mnb_qmoe_check": (C.c_int, [C.POINTER(QmoeProblem)]),
        "mnb_qmoe_workspace_bytes": (C.c_int, [C.POINTER(QmoeProblem), C.POINTER(sz)]),
        "mnb_qmoe": (C.c_int, [C.POINTER(QmoeProblem), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                               sz, vp]),
        "mnb_qmoe_weights_upload": (C.c_int, [vp, C.POINTER(QmoeProblem), i32, vp, sz, vp, sz,
                                              vp, sz, vp, sz, vp, sz, vp, sz, C.POINTER(vp)]),
        "mnb_qmoe_weights_release": (C.c_int, [vp]),
        "mnb_qmoe_weights_prepack": (C.c_int, [vp, C.POINTER(i64)]),
        "mnb_session_run_qmoe": (C.c_int, [vp, vp, i64, vp, C.c_int, vp, C.c_int, vp, C.c_int]),
        "mnb_rmsnorm_check": (C.c_int, [C.POINTER(RmsNormProblem)]),
        "mnb_skip_rmsnorm": (C.c_int, [C.POINTER(RmsNormProblem), vp, vp, vp, vp, vp, vp, vp]),
        "mnb_rmsnorm_weights_upload": (C.c_int, [vp, C.POINTER(RmsNormProblem), vp, sz, vp, sz,
                                                 C.POINTER(vp)]),
        "mnb_rmsnorm_weights_release": (C.c_int, [vp]),
        "mnb_session_run_rmsnorm": (C.c_int, [vp, vp, i64, vp, C.c_int, vp, C.c_int, vp, C.c_int,
                                              vp, C.c_int]),
        "mnb_gqa_check": (C.c_int, [C.POINTER(GqaProblem)]),
        "mnb_gqa_workspace_bytes": (C.c_int, [C.POINTER(GqaProblem), C.POINTER(sz)]),
        "mnb_gqa": (C.c_int, [C.POINTER(GqaProblem), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz,
                              vp]),
        "mnb_gqa_caches_upload": (C.c_int, [vp, C.POINTER(GqaProblem), vp, sz, vp, sz,
                                            C.POINTER(vp)]),
        "mnb_gqa_caches_release": (C.c_int, [vp]),
        "mnb_session_run_gqa": (C.c_int, [vp, vp, C.POINTER(GqaProblem), vp, vp, vp, vp, vp, vp,
                                          vp, vp, vp, C.c_uint32]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != MNB_OK:
        raise MnbError(rc, load().mnb_last_error().decode(errors="replace"))


def problem(m, n, k, bits=4, block_size=32, has_zp=False, dtype=DTYPE_F16,
            accuracy_level=0) -> Problem:
    return Problem(int(m), int(n), int(k), int(bits), int(block_size), int(bool(has_zp)),
                   int(dtype), int(accuracy_level), 0)


def plan(p: Problem) -> PlanInfo:
    info = PlanInfo()
    check(load().mnb_plan(C.byref(p), C.byref(info)))
    return info


def workspace_bytes(p: Problem) -> int:
    v = C.c_size_t(0)
    check(load().mnb_workspace_bytes(C.byref(p), C.byref(v)))
    return int(v.value)


# ---- torch conveniences (device-pointer plumbing only) ---------------------------------------

def _ptr(t) -> int | None:
    return None if t is None else int(t.data_ptr())


def _stream(stream) -> int | None:
    if stream is not None:
        return int(stream)
    import torch
    return int(torch.cuda.current_stream().cuda_stream)


def matmul_nbits(A, B, scales, zp, N: int, K: int, bits: int = 4, block_size: int = 32,
                 accuracy_level: int = 0, out=None, workspace=None, stream=None):
    """Run MatMulNBits on CUDA tensors through the C ABI; returns ``out`` ``[.., N]``."""
    import torch
    lead = tuple(A.shape[:-1])
    m = 1
    for d in lead:
        m *= int(d)
    dtype = DTYPE_F16 if A.dtype == torch.float16 else DTYPE_F32
    p = problem(m, N, K, bits, block_size, zp is not None, dtype, accuracy_level)
    if out is None:
        out = torch.empty(*lead, N, dtype=A.dtype, device=A.device)
    ws = workspace_bytes(p)
    if ws and workspace is None:
        workspace = torch.empty(ws, dtype=torch.uint8, device=A.device)
    check(load().mnb_matmul_nbits(C.byref(p), _ptr(A), _ptr(B), _ptr(scales), _ptr(zp),
                                  _ptr(out), _ptr(workspace), ws, _stream(stream)))
    return out


def dequantize_f16(B, scales, zp, N: int, K: int, bits: int = 4, block_size: int = 32,
                   out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty(N, K, dtype=torch.float16, device=B.device)
    check(load().mnb_dequantize_f16(N, K, bits, block_size, _ptr(B), _ptr(scales), _ptr(zp),
                                    _ptr(out), _stream(stream)))
    return out


def qmoe_problem(rows, hidden, inter, experts, k, block_size=32, fusion=1, normalize=True,
                 alpha=1.702, beta=1.0, limit=7.0, router_f32=False) -> QmoeProblem:
    return QmoeProblem(int(rows), int(hidden), int(inter), int(experts), int(k), int(block_size),
                       int(fusion), int(bool(normalize)), float(alpha), float(beta),
                       float(limit if limit is not None else 0.0), int(limit is not None),
                       DTYPE_F32 if router_f32 else DTYPE_F16, DTYPE_F16)


def qmoe(x, logits, fc1, fc1_scales, fc2, fc2_scales, *, k: int, inter: int, block_size: int = 32,
         fc1_bias=None, fc2_bias=None, fusion: int = 1, normalize: bool = True,
         alpha: float = 1.702, beta: float = 1.0, limit: float | None = 7.0, out=None,
         workspace=None, stream=None):
    """Fused QMoE on CUDA tensors through the C ABI (block scales ``[E, N, K/bs]``)."""
    import torch
    rows, hidden = int(x.shape[0]), int(x.shape[1])
    p = qmoe_problem(rows, hidden, inter, int(logits.shape[1]), k, block_size, fusion, normalize,
                     alpha, beta, limit, logits.dtype == torch.float32)
    if out is None:
        out = torch.empty(rows, hidden, dtype=torch.float16, device=x.device)
    ws = C.c_size_t(0)
    check(load().mnb_qmoe_workspace_bytes(C.byref(p), C.byref(ws)))
    if workspace is None:
        workspace = torch.empty(max(int(ws.value), 1), dtype=torch.uint8, device=x.device)
    check(load().mnb_qmoe(C.byref(p), _ptr(x), _ptr(logits), _ptr(fc1), _ptr(fc1_scales),
                          _ptr(fc1_bias), _ptr(fc2), _ptr(fc2_scales), _ptr(fc2_bias), _ptr(out),
                          _ptr(workspace), int(workspace.numel()), _stream(stream)))
    return out


def skip_rmsnorm(x, gamma, *, skip=None, bias=None, epsilon: float = 1e-5, want_sum=False,
                 out=None, sum_out=None, stream=None):
    """(Skip)SimplifiedLayerNormalization on CUDA tensors over the last axis; returns
    ``(y, residual_sum or None)``."""
    import torch
    hidden = int(x.shape[-1])
    rows = x.numel() // hidden if hidden else 0
    p = RmsNormProblem(rows, hidden, float(epsilon), int(skip is not None), int(bias is not None),
                       int(bool(want_sum)), DTYPE_F16 if x.dtype == torch.float16 else DTYPE_F32)
    if out is None:
        out = torch.empty_like(x)
    if want_sum and sum_out is None:
        sum_out = torch.empty_like(x)
    check(load().mnb_skip_rmsnorm(C.byref(p), _ptr(x), _ptr(skip), _ptr(gamma), _ptr(bias),
                                  _ptr(out), _ptr(sum_out) if want_sum else None, _stream(stream)))
    return out, (sum_out if want_sum else None)


def gqa_problem(batch: int, seq_len: int, past_len_max: int, present_len: int, max_seq: int,
                num_heads: int, kv_num_heads: int, head_dim: int, rotary_dim: int,
                scale: float | None = None) -> GqaProblem:
    if scale is None:
        scale = head_dim ** -0.5
    return GqaProblem(batch, seq_len, past_len_max, present_len, max_seq, num_heads, kv_num_heads,
                      head_dim, rotary_dim, float(scale), DTYPE_F16)


def gqa(qkv, past_k, past_v, seqlens_k, cos, sin, *, num_heads: int, kv_num_heads: int,
        scale: float | None = None, rotary_dim: int | None = None, present_len: int | None = None,
        present_k=None, present_v=None, stream=None):
    """GroupQueryAttention (packed QKV, fused RoPE) on CUDA tensors; returns
    ``(attn_out, present_key, present_value)``.  ``present_k``/``present_v`` may be the past
    tensors themselves (shared-buffer convention, updated in place)."""
    import torch
    B, S, P = (int(x) for x in qkv.shape)
    D = P // (num_heads + 2 * kv_num_heads)
    past = int(past_k.shape[2]) if past_k is not None else 0
    if present_len is None:
        present_len = int(present_k.shape[2]) if present_k is not None else past + S
    rd = rotary_dim if rotary_dim is not None else 2 * int(cos.shape[1])
    p = gqa_problem(B, S, past, present_len, int(cos.shape[0]), num_heads, kv_num_heads, D, rd,
                    scale)
    dev = qkv.device
    out = torch.empty((B, S, num_heads * D), dtype=torch.float16, device=dev)
    if present_k is None:
        present_k = torch.zeros((B, kv_num_heads, present_len, D), dtype=torch.float16, device=dev)
    if present_v is None:
        present_v = torch.zeros((B, kv_num_heads, present_len, D), dtype=torch.float16, device=dev)
    lib = load()
    ws_bytes = C.c_size_t()
    check(lib.mnb_gqa_workspace_bytes(C.byref(p), C.byref(ws_bytes)))
    ws = torch.empty(max(int(ws_bytes.value), 1), dtype=torch.uint8, device=dev)
    check(lib.mnb_gqa(C.byref(p), _ptr(qkv), _ptr(past_k), _ptr(past_v), _ptr(seqlens_k),
                      _ptr(cos), _ptr(sin), _ptr(out), _ptr(present_k), _ptr(present_v),
                      _ptr(ws), int(ws_bytes.value), _stream(stream)))
    return out, present_k, present_v


def launch_count() -> int:
    return int(load().mnb_launch_count())


def device_alloc_count() -> int:
    """Device allocations the library has made on its own behalf (uploads, staging growth)."""
    return int(load().mnb_device_alloc_count())
