"""Quantized weights of an ONNX model file as resident device packs.

Host-side mirror of the weight loading in the reference's ``loadOnnxModel``
(lib/onnx_runtime_dart_io.dart:19-42) and ``tensorFromProto``
(lib/src/onnx_proto_loader.dart:80-243), restricted to the quantized nodes
of this path: ``mmnb_model_load`` (include/mmnb.h) walks the graph and packs
the weights of every MatMulNBits, MatMulInteger, QLinearMatMul, ConvInteger
and QLinearConv whose weight inputs are initializers, reading raw and
external data in place (memory-mapped).  Nodes are then run by name with
their activations; the arithmetic is the ops of ``ops.py``.

Errors follow ``ops.py``: ``ValueError`` for the reference's
``FormatException`` / ``ArgumentError`` (malformed files, unsafe external
paths, out-of-range external data), ``NotImplementedError`` for
``UnsupportedError``.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, ptr
from .ops import _zp_array


def check_external_ref(location, offset, length, file_len):
    """The external-data guard (checkExternalRef,
    onnx_runtime_dart_io.dart:44-69); raises ValueError when rejected."""
    lib = _lib.load()
    loc = None if location is None else location.encode()
    check(lib.mmnb_check_external_ref(loc, int(offset), int(length), int(file_len)))


class LoadedModel:
    """Resident packs of one model file, keyed by node name (a node without
    a name is keyed by its first output)."""

    def __init__(self, path, ctx=None):
        self.ctx = ctx if ctx is not None else _lib.default_context()
        h = ctypes.c_void_p()
        check(self.ctx.lib.mmnb_model_load(self.ctx.handle, str(path).encode(),
                                           ctypes.byref(h)))
        self.handle = h
        self.nodes = {}
        lib = self.ctx.lib
        for i in range(int(lib.mmnb_model_pack_count(h))):
            op, name, pk = ctypes.c_char_p(), ctypes.c_char_p(), ctypes.c_void_p()
            check(lib.mmnb_model_pack_info(h, i, ctypes.byref(op), ctypes.byref(name),
                                           ctypes.byref(pk)))
            k, n, b = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
            check(lib.mmnb_pack_dims(pk, ctypes.byref(k), ctypes.byref(n), ctypes.byref(b)))
            self.nodes[name.value.decode()] = (op.value.decode(), pk.value, k.value, n.value,
                                               b.value)

    def op_type(self, name):
        return self.nodes[name][0]

    def _node(self, name, *ops):
        if name not in self.nodes:
            raise ValueError(f"model: no packed node named {name}")
        op, pk, k, n, b = self.nodes[name]
        if op not in ops:
            raise ValueError(f"model: {name} is a {op} node")
        return pk, k, n, b

    def matmul_nbits(self, name, a):
        pk, k, n, _ = self._node(name, "MatMulNBits")
        af = np.ascontiguousarray(a, dtype=np.float32)
        if af.ndim == 0 or af.shape[-1] != k:
            raise ValueError(f"MatMulNBits: A's last dimension must be K={k}, got {af.shape}")
        m = af.size // k
        y = np.empty(m * n, np.float32)
        if m:
            check(self.ctx.lib.mmnb_matmul_nbits(self.ctx.handle, pk, ptr(af), m, ptr(y)))
        return y.reshape(list(af.shape[:-1]) + [n])

    def _integer_rows(self, a, k):
        a = np.ascontiguousarray(a)
        if a.dtype not in (np.uint8, np.int8):
            raise NotImplementedError(f"A must be uint8 or int8, got {a.dtype}")
        if a.ndim < 2 or a.shape[-1] != k:
            raise ValueError("MatMulInteger inner dim mismatch")
        m = a.shape[-2]
        return a, m, a.size // (m * k) if m * k else 1

    def matmul_integer(self, name, a, a_zp=None):
        pk, k, n, b = self._node(name, "MatMulInteger")
        a, m, a_batch = self._integer_rows(a, k)
        batch = max(a_batch, b)
        z = _zp_array(a_zp)
        y = np.empty(batch * m * n, np.int32)
        if m and n:
            check(self.ctx.lib.mmnb_matmul_integer(self.ctx.handle, pk, ptr(a.view(np.uint8)),
                                                   int(a.dtype == np.int8), a_batch, m, ptr(z),
                                                   0 if z is None else z.size, ptr(y)))
        return y.astype(np.int64).reshape(list(a.shape[:-2]) + [m, n] if a_batch >= b
                                          else [batch, m, n])

    def qlinear_matmul(self, name, a, a_scale, a_zp, b_scale, y_scale, y_zp, *, lo, hi):
        pk, k, n, b = self._node(name, "QLinearMatMul")
        a, m, a_batch = self._integer_rows(a, k)
        batch = max(a_batch, b)
        z = _zp_array(a_zp)
        signed = lo < 0
        y = np.empty(batch * m * n, np.int8 if signed else np.uint8)
        yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])

        def f(v):
            arr = np.asarray(v, np.float32).ravel()
            if arr.size != 1:
                raise NotImplementedError("QLinearMatMul: only per-tensor scales supported")
            return float(arr[0])
        if m and n:
            check(self.ctx.lib.mmnb_qlinear_matmul(
                self.ctx.handle, pk, ptr(a.view(np.uint8)), int(a.dtype == np.int8), a_batch, m,
                ptr(z), 0 if z is None else z.size, f(a_scale), f(b_scale), f(y_scale), yz,
                int(signed), ptr(y)))
        return y.astype(np.int64).reshape(list(a.shape[:-2]) + [m, n] if a_batch >= b
                                          else [batch, m, n])

    def _conv(self, name, op, x, strides, pads, dilations):
        pk, _, mo, _ = self._node(name, op)
        x = np.ascontiguousarray(x)
        if x.dtype not in (np.uint8, np.int8):
            raise NotImplementedError(f"conv: input must be uint8 or int8, got {x.dtype}")
        squeeze = x.ndim == 3
        if squeeze:
            x = x.reshape(x.shape[0], x.shape[1], 1, x.shape[2])
            strides = [1, strides[0] if strides else 1]
            pads = None if pads is None else [0, pads[0], 0, pads[1]]
            dilations = [1, dilations[0] if dilations else 1]
        prm = _lib.ConvParams()
        for i, v in enumerate(strides or [1, 1]):
            prm.strides[i] = int(v)
        for i, v in enumerate(dilations or [1, 1]):
            prm.dilations[i] = int(v)
        for i, v in enumerate(pads or [0, 0, 0, 0]):
            prm.pads[i] = int(v)
        oh, ow = ctypes.c_int64(), ctypes.c_int64()
        check(self.ctx.lib.mmnb_conv_output_shape(pk, *[int(v) for v in x.shape],
                                                  ctypes.byref(prm), ctypes.byref(oh),
                                                  ctypes.byref(ow)))
        return pk, mo, x, prm, oh.value, ow.value, squeeze

    def conv_integer(self, name, x, x_zp=None, *, strides=None, pads=None, dilations=None):
        pk, mo, x4, prm, oh, ow, squeeze = self._conv(name, "ConvInteger", x, strides, pads,
                                                      dilations)
        xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
        y = np.empty(x4.shape[0] * mo * oh * ow, np.int32)
        if y.size:
            check(self.ctx.lib.mmnb_conv_integer(self.ctx.handle, pk, ptr(x4.view(np.uint8)),
                                                 int(x4.dtype == np.int8),
                                                 *[int(v) for v in x4.shape], xz,
                                                 ctypes.byref(prm), ptr(y)))
        y = y.astype(np.int64).reshape(x4.shape[0], mo, oh, ow)
        return y.reshape(x4.shape[0], mo, ow) if squeeze else y

    def qlinear_conv(self, name, x, x_scale, x_zp, w_scale, y_scale, y_zp, bias=None, *, lo,
                     hi, strides=None, pads=None, dilations=None):
        pk, mo, x4, prm, oh, ow, _ = self._conv(name, "QLinearConv", x, strides, pads,
                                                dilations)
        xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
        yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
        ws = np.ascontiguousarray(np.asarray(w_scale, np.float32).ravel())
        bi = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.int32))
        signed = lo < 0
        y = np.empty(x4.shape[0] * mo * oh * ow, np.int8 if signed else np.uint8)
        if y.size:
            check(self.ctx.lib.mmnb_qlinear_conv(
                self.ctx.handle, pk, ptr(x4.view(np.uint8)), int(x4.dtype == np.int8),
                *[int(v) for v in x4.shape], xz, float(np.asarray(x_scale, np.float32).ravel()[0]),
                ptr(ws), ws.size, float(np.asarray(y_scale, np.float32).ravel()[0]), yz,
                int(signed), ptr(bi), ctypes.byref(prm), ptr(y)))
        return y.astype(np.int64).reshape(x4.shape[0], mo, oh, ow)

    def free(self):
        if self.handle:
            self.ctx.lib.mmnb_model_free(self.handle)
            self.handle = None
            self.nodes = {}
