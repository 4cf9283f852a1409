"""A minimal ONNX ModelProto writer for the loader tests (protobuf wire
format, no ``onnx`` package): nodes with int / ints attributes, initializers
as raw_data, inline typed lists or external data in a companion file."""
import struct

import numpy as np

DTYPE = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3,
         np.dtype(np.int32): 6, np.dtype(np.int64): 7, np.dtype(np.float16): 10}


def _varint(v):
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(no, wt):
    return _varint((no << 3) | wt)


def f_varint(no, v):
    return _key(no, 0) + _varint(v)


def f_bytes(no, b):
    if isinstance(b, str):
        b = b.encode()
    return _key(no, 2) + _varint(len(b)) + bytes(b)


def f_packed(no, vals):
    return f_bytes(no, b"".join(_varint(int(v)) for v in vals))


def tensor(name, arr, mode="raw", external=None):
    """TensorProto.  mode: "raw" (raw_data), "inline" (int32_data for
    8/16-bit and int32 types, float_data for float32), or "external" with
    external = (location, offset, length) (length None: field omitted)."""
    arr = np.asarray(arr)
    out = f_packed(1, arr.shape) if arr.ndim else b""
    out += f_varint(2, DTYPE[arr.dtype]) + f_bytes(8, name)
    if mode == "raw":
        out += f_bytes(9, np.ascontiguousarray(arr).tobytes())
    elif mode == "inline":
        if arr.dtype == np.float32:
            out += f_bytes(4, np.ascontiguousarray(arr).tobytes())
        elif arr.dtype == np.float16:
            out += f_packed(5, arr.view(np.uint16).ravel())
        else:
            out += f_packed(5, arr.astype(np.int64).ravel())
    else:
        loc, off, ln = external
        ent = f_bytes(13, f_bytes(1, "location") + f_bytes(2, loc))
        ent += f_bytes(13, f_bytes(1, "offset") + f_bytes(2, str(off)))
        if ln is not None:
            ent += f_bytes(13, f_bytes(1, "length") + f_bytes(2, str(ln)))
        out += ent + f_varint(14, 1)
    return out


def node(op, inputs, outputs, name="", domain="", **attrs):
    out = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    if name:
        out += f_bytes(3, name)
    out += f_bytes(4, op)
    if domain:
        out += f_bytes(7, domain)
    for k, v in attrs.items():
        if isinstance(v, (list, tuple)):
            a = f_bytes(1, k) + f_packed(8, v) + f_varint(20, 7)    # INTS
        else:
            a = f_bytes(1, k) + f_varint(3, int(v)) + f_varint(20, 2)  # INT
        out += f_bytes(5, a)
    return out


def model(nodes, initializers):
    graph = b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, "g")
    graph += b"".join(f_bytes(5, t) for t in initializers)
    opset = f_bytes(8, f_bytes(1, "") + f_varint(2, 17))
    opset += f_bytes(8, f_bytes(1, "com.microsoft") + f_varint(2, 1))
    return f_varint(1, 8) + opset + f_bytes(7, graph)


class ExternalFile:
    """Collects arrays for a companion data file; returns (location, offset,
    length) for each."""

    def __init__(self, location, align=64):
        self.location = location
        self.data = bytearray()
        self.align = align

    def add(self, arr):
        pad = (-len(self.data)) % self.align
        self.data += b"\0" * pad
        off = len(self.data)
        raw = np.ascontiguousarray(arr).tobytes()
        self.data += raw
        return self.location, off, len(raw)
