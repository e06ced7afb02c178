"""A minimal reader of ONNX model files (protobuf wire format) -- test helper.

The `onnx` package is not installed here or on the GPU boxes, so the reference's MatMulNBits
case models (`evidence/cases/matmulnbits_*.onnx`, written by
`rust/tools/ledger_case_models.py:45-100,376-420`) are read as data: the ModelProto fields a
one-node graph uses -- its nodes (op type, domain, inputs, outputs, int/float/string attributes),
initializers (dims, element type, raw_data or the typed repeated fields) and the declared inputs
and outputs (element type and dims, a symbolic dim as its name) -- decoded from the wire format
(field numbers of onnx.proto3).  Nothing in a file is executed.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

# TensorProto.DataType -> numpy
_DTYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 5: np.int16, 6: np.int32, 7: np.int64,
           10: np.float16, 11: np.float64, 12: np.uint32, 13: np.uint64}


def _varint(buf: bytes, i: int) -> tuple[int, int]:
    v, shift = 0, 0
    while True:
        b = buf[i]
        i += 1
        v |= (b & 0x7F) << shift
        if b < 0x80:
            return v, i
        shift += 7
        if shift > 63:
            raise ValueError("varint too long")


def _fields(buf: bytes):
    """Yields (field number, wire type, value) over one message; length-delimited values are
    bytes, varints int, fixed32 / fixed64 raw bytes."""
    i, n = 0, len(buf)
    while i < n:
        key, i = _varint(buf, i)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            v, i = buf[i:i + 8], i + 8
        elif wt == 2:
            ln, i = _varint(buf, i)
            v, i = buf[i:i + ln], i + ln
        elif wt == 5:
            v, i = buf[i:i + 4], i + 4
        else:
            raise ValueError(f"unsupported wire type {wt} (field {fno})")
        if i > n:
            raise ValueError("truncated message")
        yield fno, wt, v


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _packed_varints(v, wt) -> list[int]:
    if wt == 0:
        return [_signed(v)]
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(_signed(x))
    return out


@dataclass
class Tensor:
    name: str
    dtype: int
    dims: list[int]
    array: np.ndarray


@dataclass
class ValueInfo:
    name: str
    elem: int
    dims: list            # ints, or the dim_param string of a symbolic dim


@dataclass
class Node:
    op_type: str
    domain: str
    name: str
    inputs: list[str]
    outputs: list[str]
    attrs: dict = field(default_factory=dict)


@dataclass
class Graph:
    nodes: list[Node]
    initializers: dict[str, Tensor]
    inputs: list[ValueInfo]
    outputs: list[ValueInfo]
    opsets: dict[str, int]


def _tensor(buf: bytes) -> Tensor:
    dims, dtype, name, raw = [], 0, "", None
    typed: dict[int, list] = {}
    for fno, wt, v in _fields(buf):
        if fno == 1:
            dims.extend(_packed_varints(v, wt))
        elif fno == 2:
            dtype = v
        elif fno == 8:
            name = v.decode()
        elif fno == 9:
            raw = v
        elif fno in (5, 7):                              # int32_data / int64_data
            typed.setdefault(fno, []).extend(_packed_varints(v, wt))
        elif fno == 4:                                   # float_data (packed or single)
            typed.setdefault(4, []).extend(struct.unpack(f"<{len(v) // 4}f", v))
    np_t = _DTYPES.get(dtype)
    if np_t is None:
        raise ValueError(f"tensor {name}: data type {dtype} is not handled")
    if raw is not None:
        arr = np.frombuffer(raw, dtype=np.dtype(np_t).newbyteorder("<")).astype(np_t)
    elif 4 in typed:
        arr = np.asarray(typed[4], dtype=np_t)
    elif 5 in typed:
        # int32_data carries fp16 as its bit patterns and the small integer types as values
        vals = np.asarray(typed[5], dtype=np.int64)
        arr = vals.astype(np.uint16).view(np.float16) if dtype == 10 else vals.astype(np_t)
    elif 7 in typed:
        arr = np.asarray(typed[7], dtype=np_t)
    else:
        arr = np.zeros(0, dtype=np_t)
    n = int(np.prod(dims)) if dims else 1
    if arr.size != n:
        raise ValueError(f"tensor {name}: {arr.size} elements for dims {dims}")
    return Tensor(name, dtype, dims, arr.reshape(dims) if dims else arr.reshape(()))


def _value_info(buf: bytes) -> ValueInfo:
    name, elem, dims = "", 0, []
    for fno, _, v in _fields(buf):
        if fno == 1:
            name = v.decode()
        elif fno == 2:                                   # TypeProto
            for f2, _, v2 in _fields(v):
                if f2 != 1:                              # tensor_type only
                    continue
                for f3, _, v3 in _fields(v2):
                    if f3 == 1:
                        elem = v3
                    elif f3 == 2:                        # TensorShapeProto
                        for f4, _, v4 in _fields(v3):
                            if f4 != 1:
                                continue
                            d = None
                            for f5, _, v5 in _fields(v4):
                                if f5 == 1:
                                    d = _signed(v5)
                                elif f5 == 2:
                                    d = v5.decode()
                            dims.append(d)
    return ValueInfo(name, elem, dims)


def _attribute(buf: bytes):
    name, val, ints = "", None, []
    for fno, wt, v in _fields(buf):
        if fno == 1:
            name = v.decode()
        elif fno == 2:
            val = struct.unpack("<f", v)[0]
        elif fno == 3:
            val = _signed(v)
        elif fno == 4:
            val = v.decode()
        elif fno == 8:
            ints.extend(_packed_varints(v, wt))
    if val is None and ints:
        val = ints
    return name, val


def _node(buf: bytes) -> Node:
    n = Node("", "", "", [], [])
    for fno, _, v in _fields(buf):
        if fno == 1:
            n.inputs.append(v.decode())
        elif fno == 2:
            n.outputs.append(v.decode())
        elif fno == 3:
            n.name = v.decode()
        elif fno == 4:
            n.op_type = v.decode()
        elif fno == 7:
            n.domain = v.decode()
        elif fno == 5:
            k, val = _attribute(v)
            n.attrs[k] = val
    return n


def load(path: str | Path) -> Graph:
    """The main graph of an ONNX model file."""
    buf = Path(path).read_bytes()
    graph_buf, opsets = None, {}
    for fno, _, v in _fields(buf):
        if fno == 7:
            graph_buf = v
        elif fno == 8:                                   # OperatorSetIdProto
            dom, ver = "", 0
            for f2, _, v2 in _fields(v):
                if f2 == 1:
                    dom = v2.decode()
                elif f2 == 2:
                    ver = v2
            opsets[dom] = ver
    if graph_buf is None:
        raise ValueError(f"{path}: no graph")
    g = Graph([], {}, [], [], opsets)
    for fno, _, v in _fields(graph_buf):
        if fno == 1:
            g.nodes.append(_node(v))
        elif fno == 5:
            t = _tensor(v)
            g.initializers[t.name] = t
        elif fno == 11:
            g.inputs.append(_value_info(v))
        elif fno == 12:
            g.outputs.append(_value_info(v))
    return g
