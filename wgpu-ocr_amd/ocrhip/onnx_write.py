"""A minimal ONNX (ModelProto) writer: protobuf wire format by hand, no `onnx` package.

It writes exactly what the model loader reads (the subset the reference's loader reads at
src/onnx.rs:88-123): graph nodes with attributes, float and int64 initializers, the graph
input and output value infos. Field numbers follow onnx.proto (IR version 8, opset 17).
"""
from __future__ import annotations

import struct

import numpy as np

FLOAT = 1
INT64 = 7

# AttributeProto.AttributeType
ATTR_FLOAT, ATTR_INT, ATTR_STRING, ATTR_TENSOR, ATTR_FLOATS, ATTR_INTS = 1, 2, 3, 4, 6, 7


def _varint(v: int) -> bytes:
    if v < 0:
        v += 1 << 64
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field: int, wire: int) -> bytes:
    return _varint((field << 3) | wire)


def _len(field: int, payload: bytes) -> bytes:
    return _key(field, 2) + _varint(len(payload)) + payload


def _int(field: int, v: int) -> bytes:
    return _key(field, 0) + _varint(int(v))


def _str(field: int, s: str | bytes) -> bytes:
    return _len(field, s.encode() if isinstance(s, str) else s)


def _packed_int64(field: int, vals) -> bytes:
    return _len(field, b"".join(_varint(int(v)) for v in vals))


def tensor(name: str, arr: np.ndarray) -> bytes:
    """TensorProto with raw little-endian data (float32 or int64)."""
    arr = np.asarray(arr)
    if arr.dtype == np.float32:
        dtype = FLOAT
    elif arr.dtype == np.int64:
        dtype = INT64
    else:
        raise TypeError(f"unsupported dtype {arr.dtype}")
    out = b"".join(_int(1, d) for d in arr.shape)  # dims (unpacked, both forms are legal)
    out += _int(2, dtype)
    out += _str(8, name)
    out += _len(9, np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes())
    return out


def attribute(name: str, value) -> bytes:
    out = _str(1, name)
    if isinstance(value, float):
        out += _key(2, 5) + struct.pack("<f", value) + _int(20, ATTR_FLOAT)
    elif isinstance(value, bool) or isinstance(value, (int, np.integer)):
        out += _int(3, int(value)) + _int(20, ATTR_INT)
    elif isinstance(value, str):
        out += _str(4, value) + _int(20, ATTR_STRING)
    elif isinstance(value, np.ndarray):
        out += _len(5, tensor("", value)) + _int(20, ATTR_TENSOR)
    elif isinstance(value, (list, tuple)) and all(isinstance(v, (int, np.integer)) for v in value):
        out += _packed_int64(8, value) + _int(20, ATTR_INTS)
    elif isinstance(value, (list, tuple)):
        out += _len(7, struct.pack(f"<{len(value)}f", *value)) + _int(20, ATTR_FLOATS)
    else:
        raise TypeError(f"attribute {name}: {type(value)}")
    return out


def node(op: str, inputs, outputs, name: str = "", **attrs) -> bytes:
    out = b"".join(_str(1, i) for i in inputs)
    out += b"".join(_str(2, o) for o in outputs)
    if name:
        out += _str(3, name)
    out += _str(4, op)
    for k in sorted(attrs):
        out += _len(5, attribute(k, attrs[k]))
    return out


def value_info(name: str, shape) -> bytes:
    dims = b""
    for d in shape:
        dims += _len(1, _int(1, d) if isinstance(d, int) else _str(2, d))
    tensor_type = _int(1, FLOAT) + _len(2, dims)
    return _str(1, name) + _len(2, _len(1, tensor_type))


class Graph:
    """Collects nodes and initializers, then serialises a ModelProto."""

    def __init__(self, name: str):
        self.name = name
        self.nodes: list[bytes] = []
        self.inits: list[bytes] = []
        self.counter = 0

    def fresh(self, stem: str) -> str:
        self.counter += 1
        return f"{stem}_{self.counter}"

    def init(self, name: str, arr: np.ndarray) -> str:
        self.inits.append(tensor(name, arr))
        return name

    def add(self, op: str, inputs, n_out: int = 1, **attrs):
        outs = [self.fresh(op.lower()) for _ in range(n_out)]
        self.nodes.append(node(op, inputs, outs, name=outs[0], **attrs))
        return outs[0] if n_out == 1 else outs

    def model(self, inp: str, in_shape, out: str, out_shape) -> bytes:
        g = b"".join(_len(1, n) for n in self.nodes)
        g += _str(2, self.name)
        g += b"".join(_len(5, t) for t in self.inits)
        g += _len(11, value_info(inp, in_shape))
        g += _len(12, value_info(out, out_shape))
        m = _int(1, 8)  # ir_version
        m += _str(2, "ocrhip-synth")
        m += _len(7, g)
        m += _len(8, _str(1, "") + _int(2, 17))  # opset_import: default domain, opset 17
        return m
