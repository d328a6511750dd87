"""ORACLE (test infrastructure only): a protobuf reader for ONNX ModelProto.

Independent of the product's C++ reader. It keeps what the reference's loader keeps
(src/onnx.rs:88-123): float and int64 initializers and `Constant` nodes become weights or
integer lists, nodes keep their attributes, the input is the first graph input that is not an
initializer and the output is the first graph output.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np


def _varint(buf: bytes, i: int):
    v = 0
    shift = 0
    while True:
        b = buf[i]
        i += 1
        v |= (b & 0x7F) << shift
        if b < 0x80:
            return v, i
        shift += 7


def _fields(buf: bytes):
    """Yield (field number, wire type, value) with value bytes for wire type 2."""
    i = 0
    while i < len(buf):
        key, i = _varint(buf, i)
        f, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            v = buf[i: i + 8]
            i += 8
        elif wt == 2:
            n, i = _varint(buf, i)
            v = buf[i: i + n]
            i += n
        elif wt == 5:
            v = buf[i: i + 4]
            i += 4
        else:
            raise ValueError(f"wire type {wt}")
        yield f, wt, v


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _ints(wt, v):
    if wt == 0:
        return [_signed(v)]
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(_signed(x))
    return out


def parse_tensor(buf: bytes):
    dims, dtype, name, raw, floats, int64s = [], 0, "", None, [], []
    for f, wt, v in _fields(buf):
        if f == 1:
            dims += _ints(wt, v)
        elif f == 2:
            dtype = v
        elif f == 8:
            name = v.decode()
        elif f == 9:
            raw = v
        elif f == 4:
            floats += list(struct.unpack(f"<{len(v) // 4}f", v)) if wt == 2 else [struct.unpack("<f", v)[0]]
        elif f == 7:
            int64s += _ints(wt, v)
    if dtype == 1:
        arr = np.frombuffer(raw, "<f4").astype(np.float32) if raw is not None else np.array(floats, np.float32)
    elif dtype == 7:
        arr = np.frombuffer(raw, "<i8").astype(np.int64) if raw is not None else np.array(int64s, np.int64)
    else:
        arr = None
    if arr is not None:
        arr = arr.reshape(dims)
    return name, arr


@dataclass
class Node:
    op: str
    inputs: list
    outputs: list
    attrs: dict = field(default_factory=dict)


def _parse_attr(buf: bytes):
    name, val, ints, floats = "", None, [], []
    for f, wt, v in _fields(buf):
        if f == 1:
            name = v.decode()
        elif f == 2:
            val = struct.unpack("<f", v)[0]
        elif f == 3:
            val = _signed(v)
        elif f == 4:
            val = v.decode()
        elif f == 5:
            val = parse_tensor(v)[1]
        elif f == 7:
            floats += list(struct.unpack(f"<{len(v) // 4}f", v)) if wt == 2 else [struct.unpack("<f", v)[0]]
        elif f == 8:
            ints += _ints(wt, v)
    if ints:
        val = ints
    elif floats:
        val = floats
    return name, val


@dataclass
class Model:
    nodes: list
    weights: dict
    ints: dict
    input: str
    output: str


def load(path: str) -> Model:
    data = open(path, "rb").read()
    graph = None
    for f, _, v in _fields(data):
        if f == 7:
            graph = v
    if graph is None:
        raise ValueError("model has no graph")
    nodes, weights, ints, inputs, outputs = [], {}, {}, [], []

    def add(name, arr):
        if arr is None:
            return
        if arr.dtype == np.float32:
            weights[name] = arr
        else:
            ints[name] = arr

    for f, _, v in _fields(graph):
        if f == 1:
            ins, outs, op, attrs = [], [], "", {}
            for g, _, w in _fields(v):
                if g == 1:
                    ins.append(w.decode())
                elif g == 2:
                    outs.append(w.decode())
                elif g == 4:
                    op = w.decode()
                elif g == 5:
                    k, val = _parse_attr(w)
                    attrs[k] = val
            if op == "Constant":
                if outs and isinstance(attrs.get("value"), np.ndarray):
                    add(outs[0], attrs["value"])
                continue
            nodes.append(Node(op, ins, outs, attrs))
        elif f == 5:
            name, arr = parse_tensor(v)
            add(name, arr)
        elif f == 11:
            inputs.append(next(w.decode() for g, _, w in _fields(v) if g == 1))
        elif f == 12:
            outputs.append(next(w.decode() for g, _, w in _fields(v) if g == 1))
    inp = next(i for i in inputs if i not in weights and i not in ints)
    return Model(nodes, weights, ints, inp, outputs[0])
