"""ctypes driver for the mock ONNX Runtime host (tests/mock_ort/mock_ort.cpp) — test helper.

The mock host dlopens the plugin EP and plays ORT's side of the plugin-EP ABI over an in-memory
graph.  This module wraps it so a test can build a one-node (or larger) graph of MatMulNBits
nodes, run GetCapability / Compile / Compute, and read the output tensors.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
# The sanitizer lane (tests/test_ep_sanitizers.py) points these at its ASan/UBSan builds.
MOCK_SO = Path(os.environ.get("MI355X_TEST_MOCK_SO") or
               Path(__file__).resolve().parent / "mock_ort" / "build" / "libmock_ort.so")
EP_SO = Path(os.environ.get("MI355X_TEST_EP_SO") or
             ROOT / "onnxruntime-ep-vulkan_amd" / "lib" / "libonnxruntime_mi355x_ep.so")

FLOAT, UINT8, INT32, FLOAT16 = 1, 2, 6, 10
NP_ELEM = {np.dtype(np.float32): FLOAT, np.dtype(np.uint8): UINT8, np.dtype(np.int32): INT32,
           np.dtype(np.float16): FLOAT16}
ORT_INVALID_ARGUMENT = 2
MEM_CPU, MEM_GPU = 0, 1          # OrtMemoryInfoDeviceType
AMD, NVIDIA = 0x1002, 0x10DE
ORT_EP_FAIL = 11   # onnxruntime_error_code.h: OK=0, FAIL, INVALID_ARGUMENT, ..., INVALID_GRAPH=10, EP_FAIL=11

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not MOCK_SO.exists():
            raise FileNotFoundError(f"{MOCK_SO} is missing: run `make -C tests/mock_ort`")
        L = C.CDLL(str(MOCK_SO))
        i64p = C.POINTER(C.c_int64)
        sig = {
            "mock_last_error": (C.c_char_p, []),
            "mock_live_statuses": (C.c_long, []),
            "mock_created_statuses": (C.c_long, []),
            "mock_bad_status_release": (C.c_int, []),
            "mock_init": (C.c_int, [C.c_char_p, C.c_uint]),
            "mock_factory_info": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t,
                                            C.POINTER(C.c_uint), C.POINTER(C.c_uint)]),
            "mock_supported_devices": (C.c_int, [C.c_int, C.c_int]),
            "mock_device_meta": (C.c_char_p, [C.c_int, C.c_char_p]),
            "mock_session_option": (None, [C.c_char_p, C.c_char_p]),
            "mock_create_ep": (C.c_int, [C.c_int]),
            "mock_create_ep_n": (C.c_int, [C.c_int]),
            "mock_ep_name": (C.c_char_p, []),
            "mock_graph_reset": (None, []),
            "mock_add_value": (C.c_int, [C.c_char_p, C.c_int, C.c_int, i64p, C.c_void_p, C.c_size_t]),
            "mock_add_node": (C.c_int, [C.c_char_p] * 6),
            "mock_get_capability": (C.c_int, [C.c_int, C.c_char_p, C.c_size_t]),
            "mock_compile": (C.c_int, []),
            "mock_feed": (C.c_int, [C.c_char_p, C.c_int, C.c_int, i64p, C.c_void_p, C.c_size_t]),
            "mock_compute": (C.c_int, [C.c_int]),
            "mock_fetch": (C.c_int, [C.c_char_p, C.c_void_p, C.c_size_t, i64p, C.c_int]),
            "mock_shutdown": (C.c_int, []),
            "mock_live_memory_infos": (C.c_long, []),
            "mock_allocator_infos": (C.c_int, [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_uint),
                                               C.POINTER(C.c_int)]),
            "mock_create_allocator_for": (C.c_int, [C.c_int, C.c_uint, C.c_int, C.c_int]),
            "mock_can_copy": (C.c_int, [C.c_int, C.c_uint, C.c_int, C.c_uint]),
            "mock_default_memory_device": (C.c_int, [C.POINTER(C.c_int), C.POINTER(C.c_uint),
                                                     C.POINTER(C.c_int)]),
            "mock_device_io_setup": (C.c_int, [C.c_int]),
            "mock_feed_device": (C.c_int, [C.c_char_p, C.c_int, C.c_int, i64p, C.c_void_p,
                                           C.c_size_t]),
            "mock_is_stream_aware": (C.c_int, []),
            "mock_stream_setup": (C.c_int, []),
            "mock_stream_handle": (C.c_void_p, []),
            "mock_run_end": (C.c_int, []),
            "mock_notification_roundtrip": (C.c_int, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def EP_COUNT() -> int:
    """OrtEpMi355xGetComputeCount of the EP library (MatMulNBits Computes that launched)."""
    import ctypes
    f = ctypes.CDLL(str(EP_SO)).OrtEpMi355xGetComputeCount
    f.restype = ctypes.c_uint64
    return int(f())


def err() -> str:
    return lib().mock_last_error().decode(errors="replace")


def _dims(shape):
    arr = (C.c_int64 * max(1, len(shape)))(*[int(d) for d in shape])
    return arr


class Host:
    """One mock ORT process-level environment with the EP library loaded."""

    def __init__(self, api_version: int = 28, ep_path: Path = EP_SO):
        self.L = lib()
        self._keep = []
        rc = self.L.mock_init(str(ep_path).encode(), api_version)
        self.init_rc = rc
        if rc:
            self.init_error = err()

    def close(self):
        rc = self.L.mock_shutdown()
        self._keep.clear()
        return rc

    # ---- factory / device ----
    def factory_info(self):
        name = C.create_string_buffer(128)
        vendor = C.create_string_buffer(128)
        vid, ver = C.c_uint(), C.c_uint()
        assert self.L.mock_factory_info(name, 128, vendor, 128, C.byref(vid), C.byref(ver)) == 0
        return name.value.decode(), vendor.value.decode(), vid.value, ver.value

    def supported_devices(self, n_amd=1, n_other=0) -> int:
        return self.L.mock_supported_devices(n_amd, n_other)

    def device_meta(self, i, key):
        v = self.L.mock_device_meta(i, key.encode())
        return None if v is None else v.decode()

    def option(self, key, value):
        self.L.mock_session_option(key.encode(), str(value).encode())

    def create_ep(self, device: int = 0) -> int:
        return self.L.mock_create_ep(device)

    # ---- graph ----
    def reset(self):
        self.L.mock_graph_reset()
        self._keep.clear()

    def value(self, name, elem, shape, data: np.ndarray | None = None):
        ptr, nbytes = None, 0
        if data is not None:
            data = np.ascontiguousarray(data)
            self._keep.append(data)
            ptr, nbytes = data.ctypes.data, data.nbytes
        assert self.L.mock_add_value(name.encode(), elem, len(shape), _dims(shape), ptr, nbytes) == 0

    def node(self, op, domain, name, inputs, outputs, attrs: dict):
        def fmt(k, v):
            if isinstance(v, str):
                return f"{k}:s={v}"
            if isinstance(v, float):
                return f"{k}:f={v!r}"
            return f"{k}={int(v)}"
        a = ",".join(fmt(k, v) for k, v in attrs.items())
        rc = self.L.mock_add_node(op.encode(), domain.encode(), name.encode(),
                                  ",".join(inputs).encode(), ",".join(outputs).encode(), a.encode())
        assert rc == 0, err()

    def get_capability(self, nested=False):
        buf = C.create_string_buffer(4096)
        n = self.L.mock_get_capability(int(nested), buf, 4096)
        claimed = [s for s in buf.value.decode().split(";") if s]
        return n, claimed

    def compile(self) -> int:
        return self.L.mock_compile()

    def feed(self, name, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        self._keep.append(arr)
        assert self.L.mock_feed(name.encode(), NP_ELEM[arr.dtype], arr.ndim, _dims(arr.shape),
                                arr.ctypes.data, arr.nbytes) == 0

    def feed_device(self, name, arr: np.ndarray):
        """A graph input placed in device memory through the EP's allocator and data transfer."""
        arr = np.ascontiguousarray(arr)
        rc = self.L.mock_feed_device(name.encode(), NP_ELEM[arr.dtype], arr.ndim, _dims(arr.shape),
                                     arr.ctypes.data, arr.nbytes)
        assert rc == 0, err()

    # ---- device memory ----
    def allocator_infos(self, i):
        t, v, d = C.c_int(), C.c_uint(), C.c_int()
        n = self.L.mock_allocator_infos(i, C.byref(t), C.byref(v), C.byref(d))
        return n, (t.value, v.value, d.value)

    def create_allocator_for(self, type_, vendor, device_id, mem=0) -> int:
        return self.L.mock_create_allocator_for(type_, vendor, device_id, mem)

    def can_copy(self, src, dst) -> int:
        return self.L.mock_can_copy(src[0], src[1], dst[0], dst[1])

    def default_memory_device(self):
        t, v, d = C.c_int(), C.c_uint(), C.c_int()
        r = self.L.mock_default_memory_device(C.byref(t), C.byref(v), C.byref(d))
        return r, (t.value, v.value, d.value)

    def device_io_setup(self, i=0) -> int:
        return self.L.mock_device_io_setup(i)

    def is_stream_aware(self) -> int:
        return lib().mock_is_stream_aware()

    def stream_setup(self) -> int:
        """ORT's stream set-up for a stream-aware factory (after device_io_setup): 1 when a
        stream was created, 0 when the factory is not stream-aware."""
        return lib().mock_stream_setup()

    def stream_handle(self):
        return lib().mock_stream_handle()

    def run_end(self) -> int:
        return lib().mock_run_end()

    def notification_roundtrip(self) -> int:
        return lib().mock_notification_roundtrip()

    def compute(self, group=0) -> int:
        return self.L.mock_compute(group)

    def fetch(self, name, dtype, max_elems):
        out = np.empty(max_elems, dtype=dtype)
        dims = (C.c_int64 * 8)()
        r = self.L.mock_fetch(name.encode(), out.ctypes.data, out.nbytes, dims, 8)
        assert r >= 0, err()
        shape = tuple(dims[i] for i in range(r))
        n = int(np.prod(shape)) if shape else 1
        return out[:n].reshape(shape)


def add_matmul_nbits(h: Host, name: str, inp: dict, N: int, K: int, bits: int, bs: int,
                     a_shape, a_dtype=np.float16, const_weights=True, acc_level=None,
                     extra_inputs=(), y_name=None, a_name=None):
    """Adds one MatMulNBits node with inputs from an oracle make_inputs() dict; `a_name` names
    an existing value (another node's output) as A."""
    el = FLOAT16 if np.dtype(a_dtype) == np.float16 else FLOAT
    if a_name is None:
        a_name = f"{name}_A"
        h.value(a_name, el, a_shape)
    y_name = y_name or f"{name}_Y"
    h.value(y_name, el, tuple(a_shape[:-1]) + (N,))
    ins = [a_name]
    for role, arr, elem in (("B", inp["B"], UINT8), ("scales", inp["scales"], el),
                            ("zp", inp.get("zp"), UINT8)):
        if arr is None:
            if role == "zp" and extra_inputs:
                ins.append("")
            continue
        vn = f"{name}_{role}"
        h.value(vn, elem, arr.shape, arr if const_weights else None)
        ins.append(vn)
    ins.extend(extra_inputs)
    attrs = {"K": K, "N": N, "bits": bits, "block_size": bs}
    if acc_level is not None:
        attrs["accuracy_level"] = acc_level
    h.node("MatMulNBits", "com.microsoft", name, ins, [y_name], attrs)
    return a_name, y_name


def add_qmoe(h: Host, name: str, inp: dict, *, k: int, x_shape, router_elem=FLOAT16,
             attrs_over: dict | None = None, const_weights=True, extra_inputs=(),
             y_name=None):
    """Adds one com.microsoft::QMoE node (gpt-oss attribute set) from an oracle
    make_qmoe_inputs() dict: input, router_probs, fc1 weights/scales/bias, fc2
    weights/scales/bias.  Per-channel scales ([E, N]) leave block_size out."""
    x_name, r_name, y_name = f"{name}_x", f"{name}_router", y_name or f"{name}_y"
    E = inp["fc1"].shape[0]
    rows = int(np.prod(x_shape[:-1])) if all(d >= 0 for d in x_shape[:-1]) else -1
    h.value(x_name, FLOAT16, x_shape)
    h.value(r_name, router_elem, (rows, E))
    h.value(y_name, FLOAT16, x_shape)
    ins = [x_name, r_name]
    for role in ("fc1", "fc1_scales", "fc1_bias", "fc2", "fc2_scales", "fc2_bias"):
        arr = inp.get(role)
        if arr is None:
            ins.append("")
            continue
        vn = f"{name}_{role}"
        elem = UINT8 if role in ("fc1", "fc2") else FLOAT16
        h.value(vn, elem, arr.shape, arr if const_weights else None)
        ins.append(vn)
    ins.extend(extra_inputs)
    attrs = {"k": k, "activation_type": "swiglu", "activation_alpha": 1.702,
             "activation_beta": 1.0, "swiglu_limit": 7.0, "swiglu_fusion": 1,
             "normalize_routing_weights": 1, "use_sparse_mixer": 0, "expert_weight_bits": 4}
    if inp["fc1_scales"].ndim == 3:
        attrs["block_size"] = inp["fc1"].shape[2] * 2 // inp["fc1_scales"].shape[2]
    attrs.update(attrs_over or {})
    attrs = {a: v for a, v in attrs.items() if v is not None}
    h.node("QMoE", "com.microsoft", name, ins, [y_name], attrs)
    return x_name, r_name, y_name


def add_norm(h: Host, name: str, inp: dict, x_shape, *, skip=True, bias=False, with_sum=True,
             epsilon=1e-5, domain="com.microsoft", elem=FLOAT16, attrs_over: dict | None = None,
             outputs=None, const_gamma=True):
    """Adds a SkipSimplifiedLayerNormalization (skip=True) or SimplifiedLayerNormalization node
    from an oracle/rmsnorm make_inputs() dict; `outputs` overrides the output slot names."""
    H = x_shape[-1]
    x_name, k_name, y_name, s_name = (f"{name}_x", f"{name}_skip", f"{name}_y", f"{name}_sum")
    h.value(x_name, elem, x_shape)
    h.value(y_name, elem, x_shape)
    h.value(f"{name}_gamma", elem, (H,), inp["gamma"] if const_gamma else None)
    ins = [x_name]
    if skip:
        h.value(k_name, elem, x_shape)
        ins.append(k_name)
    ins.append(f"{name}_gamma")
    if skip and bias:
        h.value(f"{name}_bias", elem, (H,), inp["bias"])
        ins.append(f"{name}_bias")
    if outputs is None:
        if skip:
            h.value(s_name, elem, x_shape)
            outputs = [y_name, "", "", s_name] if with_sum else [y_name]
        else:
            outputs = [y_name]
    attrs = {"epsilon": float(epsilon)}
    attrs.update(attrs_over or {})
    op = "SkipSimplifiedLayerNormalization" if skip else "SimplifiedLayerNormalization"
    h.node(op, domain, name, ins, outputs, attrs)
    return x_name, k_name, y_name, s_name


def add_gqa(h: Host, name: str, inp: dict, *, num_heads: int, kv_num_heads: int, B, S,
            past_shape_len, present_len, max_seq: int, rotary_dim: int, head_dim: int,
            const_caches=True, attrs_over: dict | None = None, separate_kv=False,
            extra_inputs=(), outputs=None, qkv_elem=FLOAT16, seqlens_elem=INT32,
            cos_rank2=True):
    """Adds a com.microsoft::GroupQueryAttention node in the packed-QKV form (the reference's
    tests/ops/test_gqa.py model).  B, S, past_shape_len and present_len are declared extents
    (-1 = symbolic); `inp` holds cos/sin when `const_caches` (then initializers)."""
    D = head_dim
    P = (num_heads + 2 * kv_num_heads) * D
    n = lambda s: f"{name}_{s}"
    h.value(n("qkv"), qkv_elem, (B, S, P))
    h.value(n("past_k"), FLOAT16, (B, kv_num_heads, past_shape_len, D))
    h.value(n("past_v"), FLOAT16, (B, kv_num_heads, past_shape_len, D))
    h.value(n("seqlens"), seqlens_elem, (B,))
    h.value(n("total"), INT32, ())
    cshape = (max_seq, rotary_dim // 2) if cos_rank2 else (max_seq * rotary_dim // 2,)
    h.value(n("cos"), FLOAT16, cshape, inp["cos"] if const_caches else None)
    h.value(n("sin"), FLOAT16, cshape, inp["sin"] if const_caches else None)
    ins = [n("qkv"), "", "", n("past_k"), n("past_v"), n("seqlens"), n("total"), n("cos"),
           n("sin")]
    if separate_kv:
        h.value(n("k"), FLOAT16, (B, S, kv_num_heads * D))
        ins[1] = n("k")
    for nm, elem, shape in extra_inputs:
        while len(ins) < 16 and len(ins) < int(nm.split("@")[1]):
            ins.append("")
        h.value(nm.split("@")[0], elem, shape)
        ins.append(nm.split("@")[0])
    h.value(n("out"), FLOAT16, (B, S, num_heads * D))
    h.value(n("present_k"), FLOAT16, (B, kv_num_heads, present_len, D))
    h.value(n("present_v"), FLOAT16, (B, kv_num_heads, present_len, D))
    if outputs is None:
        outputs = [n("out"), n("present_k"), n("present_v")]
    attrs = {"num_heads": num_heads, "kv_num_heads": kv_num_heads, "do_rotary": 1,
             "rotary_interleaved": 0, "local_window_size": -1}
    attrs.update(attrs_over or {})
    attrs = {k: v for k, v in attrs.items() if v is not None}
    h.node("GroupQueryAttention", "com.microsoft", name, ins, outputs, attrs)
    return {k: n(k) for k in ("qkv", "past_k", "past_v", "seqlens", "total", "cos", "sin", "out",
                              "present_k", "present_v")}
