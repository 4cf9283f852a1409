"""Host-side mirror of the reference's quantized operator functions, running
on the MI355X through libmmnb's C ABI.

Same names (snake_case), argument meaning, output types and error behaviour
as the Dart functions they replace:

* ``op_matmul_nbits``    <- ``opMatMulNBits``  (lib/src/onnx_qlinear_ops.dart:114-156)
* ``op_matmul_integer``  <- ``opMatMulInteger`` (lib/src/onnx_qlinear_ops.dart:30-79)
* ``op_dynamic_quantize_linear`` <- ``opDynamicQuantizeLinear``
  (lib/src/onnx_ops.dart:2556-2583)
* ``op_qlinear_matmul``  <- ``opQLinearMatMul`` (lib/src/onnx_qlinear_ops.dart:83-106)
* ``op_conv_integer``    <- ``opConvInteger`` (lib/src/onnx_qlinear_ops.dart:235-267)
* ``op_qlinear_conv``    <- ``opQLinearConv`` (lib/src/onnx_qlinear_ops.dart:270-308)
* ``dispatch``           <- the ``_dispatch`` arms of these operators
  (lib/src/onnx_graph.dart:1561-1609)

Tensors are numpy arrays (shape + dtype + row-major data, like the Dart
``Tensor``).  Exceptions: ``NotImplementedError`` where the reference throws
``UnsupportedError``, ``ValueError`` for ``ArgumentError``/``AssertionError``.

Weight packs are uploaded once and cached per weight object, the way a Dart
binding caches them in an ``Expando`` keyed on the initializer ``Tensor``
(initializers keep their identity across runs, onnx_graph.dart:90-93, :553).
"""
import ctypes
import threading
import weakref

import numpy as np

from . import _lib
from ._lib import check, ptr


class _PackCache:
    """Device packs keyed by the identity of the host arrays they came from;
    a pack is freed when any of its source arrays is garbage collected."""

    def __init__(self):
        self._packs = {}
        self._lock = threading.Lock()

    def get(self, key_objs, extra, make):
        key = tuple(id(o) for o in key_objs) + tuple(extra)
        with self._lock:
            hit = self._packs.get(key)
            if hit is not None:
                refs, pack = hit
                if all(r() is o for r, o in zip(refs, key_objs)):
                    return pack
                self._drop(key)
        pack = make()
        refs = []
        for o in key_objs:
            try:
                refs.append(weakref.ref(o, lambda _r, k=key: self.evict(k)))
            except TypeError:
                refs.append(lambda o=o: o)  # not weak-referenceable: keep alive
        with self._lock:
            self._packs[key] = (refs, pack)
        return pack

    def evict(self, key):
        with self._lock:
            self._drop(key)

    def _drop(self, key):
        hit = self._packs.pop(key, None)
        if hit is not None:
            hit[1].free()

    def clear(self):
        with self._lock:
            for key in list(self._packs):
                self._drop(key)


_CACHE = _PackCache()


class Pack:
    """An uploaded weight pack (device memory owned by libmmnb)."""

    def __init__(self, ctx, handle, kind, **meta):
        self.ctx = ctx
        self.handle = handle
        self.kind = kind
        self.__dict__.update(meta)

    @property
    def device_bytes(self):
        return int(self.ctx.lib.mmnb_pack_device_bytes(self.handle))

    def free(self):
        if self.handle:
            check(self.ctx.lib.mmnb_pack_free(self.handle))
            self.handle = None


def _ctx(ctx):
    return ctx if ctx is not None else _lib.default_context()


# --------------------------------------------------------------- MatMulNBits

def pack_nbits(b_q, scales, zero_points, *, k, n, bits, block_size, ctx=None):
    """Upload a MatMulNBits weight (B, scales, optional packed zero points)."""
    ctx = _ctx(ctx)
    b = np.ascontiguousarray(b_q)
    if b.dtype != np.uint8:
        # the reference re-packs non-uint8 B through asIntList (:124)
        b = np.ascontiguousarray(np.asarray(b, dtype=np.int64).astype(np.uint8))
    s = np.ascontiguousarray(scales, dtype=np.float32)
    z = None if zero_points is None else np.ascontiguousarray(zero_points)
    if z is not None and z.dtype != np.uint8:
        # float zero points are not byte data: the reference reads them as 8
        # (zeroPoints?.u8 is null, :124, :132)
        z = None
    h = ctypes.c_void_p()
    check(ctx.lib.mmnb_pack_nbits(ctx.handle, ptr(b), b.size, ptr(s), s.size, ptr(z),
                                  0 if z is None else z.size, int(k), int(n), int(bits),
                                  int(block_size), ctypes.byref(h)))
    return Pack(ctx, h, "nbits", k=int(k), n=int(n), block=int(block_size))


def op_matmul_nbits(a, b_q, scales, zero_points, *, k, n, bits, block_size, ctx=None):
    """``y = A . dequant(B)^T``; A fp32 ``[..., K]``, returns fp32 ``[..., N]``.

    Mirrors opMatMulNBits (onnx_qlinear_ops.dart:114-156): ``bits != 4`` is
    unsupported, ``m = len(A) / K``."""
    if bits != 4:
        raise NotImplementedError(f"MatMulNBits: only bits=4 supported, got {bits}")
    ctx = _ctx(ctx)
    keys = [b_q, scales] + ([zero_points] if zero_points is not None else [])
    pack = _CACHE.get(keys, (k, n, bits, block_size, ctx.device),
                      lambda: pack_nbits(b_q, scales, zero_points, k=k, n=n, bits=bits,
                                         block_size=block_size, ctx=ctx))
    af = np.ascontiguousarray(a, dtype=np.float32)
    if af.ndim == 0 or af.shape[-1] != k:
        raise ValueError(f"MatMulNBits: A's last dimension must be K={k}, got {af.shape}")
    m = af.size // k
    y = np.empty(m * n, dtype=np.float32)
    if m:
        check(ctx.lib.mmnb_matmul_nbits(ctx.handle, pack.handle, ptr(af), m, ptr(y)))
    return y.reshape(list(af.shape[:-1]) + [n])


# ----------------------------------- MatMulNBits as ORT-exported models use it

_FLOAT_TYPES = {np.dtype(np.float32): _lib.DT_F32, np.dtype(np.float16): _lib.DT_F16}


def _float_arg(x, what):
    arr = np.ascontiguousarray(x)
    if arr.dtype not in _FLOAT_TYPES:
        arr = np.ascontiguousarray(arr, dtype=np.float32)
    return arr, _FLOAT_TYPES[arr.dtype]


def pack_nbits_ex(b_q, scales, zero_points=None, g_idx=None, bias=None, *, k, n, bits,
                  block_size, ctx=None):
    """Upload a MatMulNBits weight with the inputs and types ORT exports use
    and the reference rejects (onnx_graph.dart:1585-1588): bits 4 or 8,
    uint8 zero points in the flat layout (1-D) or per column ([N, bytes] 2-D),
    float / fp16 zero points, fp16 scales, g_idx [K] and bias [N]."""
    ctx = _ctx(ctx)
    b = np.ascontiguousarray(b_q)
    if b.dtype != np.uint8:
        b = np.ascontiguousarray(np.asarray(b, dtype=np.int64).astype(np.uint8))
    s, st = _float_arg(scales, "scales")
    d = _lib.NBitsDesc()
    d.k, d.n, d.bits, d.block_size = int(k), int(n), int(bits), int(block_size)
    d.b_q, d.b_q_len = ptr(b), b.size
    d.scales, d.scales_len, d.scales_type = ptr(s), s.size, st
    keep = [b, s]
    if zero_points is not None:
        z = np.ascontiguousarray(zero_points)
        if z.dtype == np.uint8:
            d.zero_points_type = _lib.DT_U8
            d.zero_points_layout = _lib.ZP_PER_COLUMN if z.ndim == 2 else _lib.ZP_FLAT
        else:
            z, d.zero_points_type = _float_arg(z, "zero_points")
        d.zero_points, d.zero_points_len = ptr(z), z.size
        keep.append(z)
    if g_idx is not None:
        gi = np.ascontiguousarray(np.asarray(g_idx).astype(np.int32).ravel())
        d.g_idx, d.g_idx_len = ptr(gi), gi.size
        keep.append(gi)
    if bias is not None:
        bb, d.bias_type = _float_arg(np.asarray(bias).ravel(), "bias")
        d.bias, d.bias_len = ptr(bb), bb.size
        keep.append(bb)
    h = ctypes.c_void_p()
    check(ctx.lib.mmnb_pack_nbits_ex(ctx.handle, ctypes.byref(d), ctypes.byref(h)))
    return Pack(ctx, h, "nbits", k=int(k), n=int(n), block=int(block_size))


def op_matmul_nbits_ex(a, b_q, scales, zero_points=None, g_idx=None, bias=None, *, k, n,
                       bits, block_size, ctx=None):
    """MatMulNBits with ORT's full input list (A, B, scales, zero_points,
    g_idx, bias): ``W[k, n] = (q - zp[n, g]) * scale[n, g]`` with
    ``g = g_idx[k]`` (or ``k / block_size``), ``y = A W + bias``."""
    if bits not in (4, 8):
        raise NotImplementedError(f"MatMulNBits: bits must be 4 or 8, got {bits}")
    ctx = _ctx(ctx)
    keys = [b_q, scales] + [t for t in (zero_points, g_idx, bias) if t is not None]
    extra = (k, n, bits, block_size, ctx.device, "ex",
             zero_points is not None, g_idx is not None, bias is not None)
    pack = _CACHE.get(keys, extra,
                      lambda: pack_nbits_ex(b_q, scales, zero_points, g_idx, bias, k=k, n=n,
                                            bits=bits, block_size=block_size, ctx=ctx))
    af = np.ascontiguousarray(a, dtype=np.float32)
    if af.ndim == 0 or af.shape[-1] != k:
        raise ValueError(f"MatMulNBits: A's last dimension must be K={k}, got {af.shape}")
    m = af.size // k
    y = np.empty(m * n, dtype=np.float32)
    if m:
        check(ctx.lib.mmnb_matmul_nbits(ctx.handle, pack.handle, ptr(af), m, ptr(y)))
    return y.reshape(list(af.shape[:-1]) + [n])


# ---------------------------------------------------- DynamicQuantizeLinear

def op_dynamic_quantize_linear(x, ctx=None):
    """Returns ``[y uint8 (x.shape), scale float32 (shape ()), zero_point int64
    (shape ())]`` like opDynamicQuantizeLinear (onnx_ops.dart:2556-2583)."""
    ctx = _ctx(ctx)
    xf = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(xf.shape, dtype=np.uint8)
    sc = ctypes.c_float()
    zp = ctypes.c_int64()
    check(ctx.lib.mmnb_dynamic_quantize_linear(ctx.handle, ptr(xf), xf.size, ptr(y),
                                               ctypes.byref(sc), ctypes.byref(zp)))
    return [y, np.array(sc.value, dtype=np.float32), np.array(zp.value, dtype=np.int64)]


# ------------------------------------------------------------- MatMulInteger

def _zp_array(zp):
    if zp is None:
        return None
    return np.ascontiguousarray(np.asarray(zp).astype(np.int64).ravel())


def pack_integer(b, b_zp, ctx=None):
    """Upload a MatMulInteger right-hand operand ``[..., K, N]`` (uint8/int8)."""
    ctx = _ctx(ctx)
    b = np.ascontiguousarray(b)
    if b.dtype not in (np.uint8, np.int8):
        raise NotImplementedError(f"MatMulInteger: B must be uint8 or int8, got {b.dtype}")
    if b.ndim < 2:
        raise ValueError("MatMulInteger: B must have rank >= 2")
    k, n = b.shape[-2], b.shape[-1]
    batch = b.size // (k * n) if k * n else 1
    z = _zp_array(b_zp)
    h = ctypes.c_void_p()
    check(ctx.lib.mmnb_pack_integer(ctx.handle, ptr(b.view(np.uint8)), int(b.dtype == np.int8),
                                    batch, k, n, ptr(z), 0 if z is None else z.size,
                                    ctypes.byref(h)))
    return Pack(ctx, h, "integer", k=k, n=n, batch=batch, batch_shape=b.shape[:-2])


def op_matmul_integer(a, b, a_zp, b_zp, ctx=None):
    """``y = (A - aZp) . (B - bZp)`` exact, returned as int64 like the
    reference (onnx_qlinear_ops.dart:30-79; int32 semantics)."""
    ctx = _ctx(ctx)
    a = np.ascontiguousarray(a)
    if a.dtype not in (np.uint8, np.int8):
        raise NotImplementedError(f"MatMulInteger: A must be uint8 or int8, got {a.dtype}")
    b_arr = np.asarray(b)
    if a.ndim < 2 or b_arr.ndim < 2:
        raise ValueError("MatMulInteger: operands must have rank >= 2")
    m, k = a.shape[-2], a.shape[-1]
    if b_arr.shape[-2] != k:
        raise ValueError("MatMulInteger inner dim mismatch")
    n = b_arr.shape[-1]
    keys = [b] + ([b_zp] if b_zp is not None and not np.isscalar(b_zp) else [])
    extra = (ctx.device,) + ((int(b_zp),) if b_zp is not None and np.isscalar(b_zp) else ())
    pack = _CACHE.get(keys, extra, lambda: pack_integer(b, b_zp, ctx))
    a_batch = a.size // (m * k) if m * k else 1
    batch = max(a_batch, pack.batch)
    z = _zp_array(a_zp)
    y = np.empty(batch * m * n, dtype=np.int32)
    if m and n:
        check(ctx.lib.mmnb_matmul_integer(ctx.handle, pack.handle, ptr(a.view(np.uint8)),
                                          int(a.dtype == np.int8), a_batch, m, ptr(z),
                                          0 if z is None else z.size, ptr(y)))
    batch_shape = a.shape[:-2] if a_batch >= pack.batch else pack.batch_shape
    return y.astype(np.int64).reshape(list(batch_shape) + [m, n])


# ------------------------------------------------------------ QLinearMatMul

def _scalar_f(t, what):
    arr = np.asarray(t, dtype=np.float32).ravel()
    if arr.size != 1:
        raise NotImplementedError(f"{what}: only per-tensor scales supported")
    return float(arr[0])


def op_qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, *, lo, hi, ctx=None):
    """MatMulInteger + requantisation with ``fl32(fl32(aS*bS)/yS)``, saturating
    to ``[lo, hi]`` (opQLinearMatMul, onnx_qlinear_ops.dart:83-106).  Returns
    int64 like the reference."""
    if (np.asarray(a_scale).size != 1 or np.asarray(b_scale).size != 1
            or np.asarray(y_scale).size != 1):
        raise NotImplementedError("QLinearMatMul: only per-tensor scales supported")
    if (lo, hi) not in ((-128, 127), (0, 255)):
        raise ValueError("QLinearMatMul: output range must be int8 or uint8")
    ctx = _ctx(ctx)
    a = np.ascontiguousarray(a)
    if a.dtype not in (np.uint8, np.int8):
        raise NotImplementedError(f"QLinearMatMul: A must be uint8 or int8, got {a.dtype}")
    b_arr = np.asarray(b)
    if a.ndim < 2 or b_arr.ndim < 2:
        raise ValueError("MatMulInteger: operands must have rank >= 2")
    m, k = a.shape[-2], a.shape[-1]
    if b_arr.shape[-2] != k:
        raise ValueError("MatMulInteger inner dim mismatch")
    n = b_arr.shape[-1]
    keys = [b] + ([b_zp] if b_zp is not None and not np.isscalar(b_zp) else [])
    extra = (ctx.device,) + ((int(b_zp),) if b_zp is not None and np.isscalar(b_zp) else ())
    pack = _CACHE.get(keys, extra, lambda: pack_integer(b, b_zp, ctx))
    a_batch = a.size // (m * k) if m * k else 1
    batch = max(a_batch, pack.batch)
    z = _zp_array(a_zp)
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    signed = lo < 0
    y = np.empty(batch * m * n, dtype=np.int8 if signed else np.uint8)
    if m and n:
        check(ctx.lib.mmnb_qlinear_matmul(
            ctx.handle, pack.handle, ptr(a.view(np.uint8)), int(a.dtype == np.int8), a_batch, m,
            ptr(z), 0 if z is None else z.size, _scalar_f(a_scale, "QLinearMatMul"),
            _scalar_f(b_scale, "QLinearMatMul"), _scalar_f(y_scale, "QLinearMatMul"), yz,
            int(signed), ptr(y)))
    batch_shape = a.shape[:-2] if a_batch >= pack.batch else pack.batch_shape
    return y.astype(np.int64).reshape(list(batch_shape) + [m, n])


# -------------------------------------------------------------- convolutions

def pack_conv(w, w_zp, group, ctx=None):
    """Upload a convolution weight ``[M, C/group, kh, kw]`` (uint8/int8)."""
    ctx = _ctx(ctx)
    w = np.ascontiguousarray(w)
    if w.dtype not in (np.uint8, np.int8):
        raise NotImplementedError(f"conv: weight must be uint8 or int8, got {w.dtype}")
    if w.ndim != 4:
        raise ValueError("conv: weight must be [M, C/group, kh, kw]")
    z = _zp_array(w_zp)
    h = ctypes.c_void_p()
    check(ctx.lib.mmnb_pack_conv(ctx.handle, ptr(w.view(np.uint8)), int(w.dtype == np.int8),
                                 *[int(d) for d in w.shape], int(group), ptr(z),
                                 0 if z is None else z.size, ctypes.byref(h)))
    return Pack(ctx, h, "conv", m=int(w.shape[0]))


def _conv_prep(x, w, w_zp, strides, pads, dilations, group, ctx):
    """The reference's 1-D -> 2-D reshape (onnx_qlinear_ops.dart:238-252) and
    defaults; returns (x4, w4, params, squeeze, pack)."""
    x = np.ascontiguousarray(x)
    w_arr = np.asarray(w)
    if x.dtype not in (np.uint8, np.int8):
        raise NotImplementedError(f"conv: input must be uint8 or int8, got {x.dtype}")
    squeeze = False
    if x.ndim == 3:
        x = x.reshape(x.shape[0], x.shape[1], 1, x.shape[2])
        if w_arr.ndim == 3:
            w_arr = w_arr.reshape(w_arr.shape[0], w_arr.shape[1], 1, w_arr.shape[2])
        strides = [1, (strides[0] if strides else 1)]
        pads = None if pads is None else [0, pads[0], 0, pads[1]]
        dilations = [1, (dilations[0] if dilations else 1)]
        squeeze = True
    if x.ndim != 4 or w_arr.ndim != 4:
        raise ValueError("ConvInteger implemented for 1-D/2-D convs")
    prm = _lib.ConvParams()
    s = list(strides) if strides else [1, 1]
    p = list(pads) if pads else [0, 0, 0, 0]
    d = list(dilations) if dilations else [1, 1]
    for i in range(2):
        prm.strides[i] = int(s[i])
        prm.dilations[i] = int(d[i])
    for i in range(4):
        prm.pads[i] = int(p[i])
    keys = [w] + ([w_zp] if w_zp is not None and not np.isscalar(w_zp) else [])
    extra = (ctx.device, int(group), "conv") + \
        ((int(w_zp),) if w_zp is not None and np.isscalar(w_zp) else ())
    pack = _CACHE.get(keys, extra, lambda: pack_conv(w_arr, w_zp, group, ctx))
    return x, prm, squeeze, pack


def _conv_out_shape(ctx, pack, x, prm):
    oh, ow = ctypes.c_int64(), ctypes.c_int64()
    check(ctx.lib.mmnb_conv_output_shape(pack.handle, *[int(v) for v in x.shape],
                                         ctypes.byref(prm), ctypes.byref(oh), ctypes.byref(ow)))
    return oh.value, ow.value


def op_conv_integer(x, w, x_zp, w_zp, *, strides=None, pads=None, dilations=None, group=1,
                    ctx=None):
    """``acc[n, m, oy, ox] = sum (x - xZp)(w - wZp[m])`` exact, int64 out like
    opConvInteger (onnx_qlinear_ops.dart:235-267); 1-D convs run as 2-D."""
    ctx = _ctx(ctx)
    x4, prm, squeeze, pack = _conv_prep(x, w, w_zp, strides, pads, dilations, group, ctx)
    oh, ow = _conv_out_shape(ctx, pack, x4, prm)
    xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
    n = x4.shape[0]
    y = np.empty(n * pack.m * oh * ow, dtype=np.int32)
    if y.size:
        check(ctx.lib.mmnb_conv_integer(ctx.handle, pack.handle, ptr(x4.view(np.uint8)),
                                        int(x4.dtype == np.int8), *[int(v) for v in x4.shape],
                                        xz, ctypes.byref(prm), ptr(y)))
    y = y.astype(np.int64).reshape(n, pack.m, oh, ow)
    return y.reshape(n, pack.m, ow) if squeeze else y


def op_qlinear_conv(x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, bias, *, strides=None,
                    pads=None, dilations=None, group=1, lo, hi, ctx=None):
    """Integer conv + int32 bias + per-channel requantisation in double
    (opQLinearConv, onnx_qlinear_ops.dart:270-308); 2-D only."""
    if np.asarray(x).ndim != 4:
        raise ValueError("QLinearConv implemented for 2-D convs")
    if (lo, hi) not in ((-128, 127), (0, 255)):
        raise ValueError("QLinearConv: output range must be int8 or uint8")
    ctx = _ctx(ctx)
    x4, prm, _, pack = _conv_prep(x, w, w_zp, strides, pads, dilations, group, ctx)
    oh, ow = _conv_out_shape(ctx, pack, x4, prm)
    xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    ws = np.ascontiguousarray(np.asarray(w_scale, dtype=np.float32).ravel())
    bi = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.int32).ravel())
    if bi is not None and bi.size != pack.m:
        raise ValueError("QLinearConv: bias must have M values")
    signed = lo < 0
    n = x4.shape[0]
    y = np.empty(n * pack.m * oh * ow, dtype=np.int8 if signed else np.uint8)
    if y.size:
        check(ctx.lib.mmnb_qlinear_conv(
            ctx.handle, pack.handle, ptr(x4.view(np.uint8)), int(x4.dtype == np.int8),
            *[int(v) for v in x4.shape], xz, float(np.asarray(x_scale, np.float32).ravel()[0]),
            ptr(ws), ws.size, float(np.asarray(y_scale, np.float32).ravel()[0]), yz, int(signed),
            ptr(bi), ctypes.byref(prm), ptr(y)))
    return y.astype(np.int64).reshape(n, pack.m, oh, ow)


# --------------------------------------------------------- dispatch arms

def dispatch(op_type, ins, attrs, ort_semantics=False):
    """The ``_dispatch`` arms for the quantized operators
    (onnx_graph.dart:1561-1609).  ``ins`` lists the node's positional inputs
    (None for an empty name); returns the output list.  The output range of
    QLinearMatMul / QLinearConv follows the y zero point's type (int8 ->
    [-128, 127], else [0, 255]; the reference reads the initializer's
    element type, :1578, :1598).

    ``ort_semantics=True`` lifts the reference's MatMulNBits restrictions:
    g_idx / bias inputs, bits = 8, float zero points and fp16 scales go to
    ``op_matmul_nbits_ex``; the default keeps the reference's behaviour."""
    def need(i):
        if i >= len(ins) or ins[i] is None:
            raise ValueError(f"{op_type}: missing input {i}")
        return ins[i]

    if op_type == "DynamicQuantizeLinear":
        return op_dynamic_quantize_linear(need(0))
    if op_type == "MatMulInteger":
        return [op_matmul_integer(need(0), need(1), ins[2] if len(ins) > 2 else None,
                                  ins[3] if len(ins) > 3 else None)]
    if op_type == "MatMulNBits" and ort_semantics:
        opt_in = [ins[i] if len(ins) > i else None for i in range(3, 6)]
        return [op_matmul_nbits_ex(need(0), need(1), need(2), *opt_in, k=attrs["K"],
                                   n=attrs["N"], bits=attrs.get("bits", 4),
                                   block_size=attrs["block_size"])]
    if op_type == "MatMulNBits":
        if len(ins) > 4:
            raise NotImplementedError("MatMulNBits: g_idx/bias inputs not supported")
        return [op_matmul_nbits(need(0), need(1), need(2), ins[3] if len(ins) > 3 else None,
                                k=attrs["K"], n=attrs["N"], bits=attrs.get("bits", 4),
                                block_size=attrs["block_size"])]
    def rng8(i):
        z = ins[i] if len(ins) > i else None
        return (-128, 127) if z is not None and np.asarray(z).dtype == np.int8 else (0, 255)

    def opt(i):
        return ins[i] if len(ins) > i else None

    if op_type == "ConvInteger":
        return [op_conv_integer(need(0), need(1), opt(2), opt(3), strides=attrs.get("strides"),
                                pads=attrs.get("pads"), dilations=attrs.get("dilations"),
                                group=attrs.get("group", 1))]
    if op_type == "QLinearMatMul":
        lo, hi = rng8(7)
        return [op_qlinear_matmul(need(0), need(1), opt(2), need(3), need(4), opt(5), need(6),
                                  opt(7), lo=lo, hi=hi)]
    if op_type == "QLinearConv":
        lo, hi = rng8(7)
        return [op_qlinear_conv(need(0), need(1), opt(2), need(3), need(4), opt(5), need(6),
                                opt(7), opt(8), strides=attrs.get("strides"),
                                pads=attrs.get("pads"), dilations=attrs.get("dilations"),
                                group=attrs.get("group", 1), lo=lo, hi=hi)]
    raise NotImplementedError(f"Unsupported op: {op_type}")


def clear_pack_cache():
    _CACHE.clear()
