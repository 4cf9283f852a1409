"""CPU oracle of QLinearMatMul, ConvInteger and QLinearConv.

TEST INFRASTRUCTURE ONLY: this module checks the GPU kernels.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product package never does.

Each function restates the reference's Dart arithmetic
(onnx_runtime_dart, ``lib/src/onnx_qlinear_ops.dart``) in numpy with exact
int64 accumulation; the requantisation keeps the reference's rounding
points (binary32 steps for QLinearMatMul, double for QLinearConv).
"""
import numpy as np

from oracle import refcpu


def round_even(v):
    """_roundEven (onnx_qlinear_ops.dart:17-24): round half to even of a
    double; numpy's rint is the same IEEE operation."""
    return np.rint(np.asarray(v, dtype=np.float64))


def qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, lo, hi):
    """opQLinearMatMul (onnx_qlinear_ops.dart:83-106): acc = MatMulInteger;
    mult = fl32(fl32(aS * bS) / yS); q = roundEven(fl32(acc * mult)) + yZp,
    clamped to [lo, hi].  Returns int64."""
    for s in (a_scale, b_scale, y_scale):
        if np.asarray(s).size != 1:
            raise NotImplementedError("QLinearMatMul: only per-tensor scales supported")
    acc = refcpu.matmul_integer(a, b, a_zp, b_zp)
    a_s = float(np.asarray(a_scale, np.float32).ravel()[0])
    b_s = float(np.asarray(b_scale, np.float32).ravel()[0])
    y_s = float(np.asarray(y_scale, np.float32).ravel()[0])
    mult = np.float32(np.float32(a_s * b_s) / y_s)         # two binary32 stores (:95-96)
    prod = (acc.astype(np.float64) * float(mult)).astype(np.float32)   # f32[0] = acc * mult
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    q = round_even(prod.astype(np.float64)) + yz
    return np.clip(q, lo, hi).astype(np.int64)


def _conv_shape(x, w, strides, pads, dilations):
    """_convOutSpatial (onnx_qlinear_ops.dart:222-231)."""
    out = []
    for a in range(2):
        window = dilations[a] * (w.shape[2 + a] - 1) + 1
        out.append((x.shape[2 + a] + pads[a] + pads[2 + a] - window) // strides[a] + 1)
    return out


def conv_int_acc(x, w, x_zp, w_zp_per_channel, strides, pads, dilations, group):
    """_convIntAcc (onnx_qlinear_ops.dart:160-220): acc[n, m, oy, ox] =
    sum over in-image taps of (x - xZp)(w - wZp[m]), int64.  Vectorised per
    tap: out-of-image taps contribute nothing, as in the reference."""
    x = np.asarray(x).astype(np.int64)
    w = np.asarray(w).astype(np.int64)
    n, c_in, h, wd = x.shape
    m, cg, kh, kw = w.shape
    oh, ow = _conv_shape(x, w, strides, pads, dilations)
    mg = m // group
    xs = x - int(x_zp)
    ws = w - np.asarray(w_zp_per_channel, np.int64).reshape(m, 1, 1, 1)
    out = np.zeros((n, m, oh, ow), np.int64)
    oy = np.arange(oh)
    ox = np.arange(ow)
    for ky in range(kh):
        iy = oy * strides[0] - pads[0] + ky * dilations[0]
        vy = (iy >= 0) & (iy < h)
        for kx in range(kw):
            ix = ox * strides[1] - pads[1] + kx * dilations[1]
            vx = (ix >= 0) & (ix < wd)
            if not vy.any() or not vx.any():
                continue
            tap = np.zeros((n, c_in, oh, ow), np.int64)
            tap[:, :, np.ix_(vy, vx)[0], np.ix_(vy, vx)[1]] = \
                xs[:, :, iy[vy]][:, :, :, ix[vx]]
            for g in range(group):
                xg = tap[:, g * cg:(g + 1) * cg]                 # [n, cg, oh, ow]
                wg = ws[g * mg:(g + 1) * mg, :, ky, kx]          # [mg, cg]
                out[:, g * mg:(g + 1) * mg] += np.einsum("nchw,mc->nmhw", xg, wg)
    return out


def conv_int_acc_loops(x, w, x_zp, w_zp_per_channel, strides, pads, dilations, group):
    """The same accumulator as plain loops in the reference's order
    (onnx_qlinear_ops.dart:183-216), for tiny cases only."""
    x = np.asarray(x).astype(np.int64)
    w = np.asarray(w).astype(np.int64)
    n, c_in, h, wd = x.shape
    m, cg, kh, kw = w.shape
    oh, ow = _conv_shape(x, w, strides, pads, dilations)
    mg = m // group
    out = np.zeros((n, m, oh, ow), np.int64)
    for b in range(n):
        for om in range(m):
            g = om // mg
            wz = int(w_zp_per_channel[om])
            for yy in range(oh):
                for xx in range(ow):
                    acc = 0
                    for c in range(cg):
                        for ky in range(kh):
                            iy = yy * strides[0] - pads[0] + ky * dilations[0]
                            if iy < 0 or iy >= h:
                                continue
                            for kx in range(kw):
                                ix = xx * strides[1] - pads[1] + kx * dilations[1]
                                if ix < 0 or ix >= wd:
                                    continue
                                acc += (int(x[b, g * cg + c, iy, ix]) - int(x_zp)) * \
                                    (int(w[om, c, ky, kx]) - wz)
                    out[b, om, yy, xx] = acc
    return out


def _defaults(strides, pads, dilations):
    return (list(strides) if strides else [1, 1], list(pads) if pads else [0, 0, 0, 0],
            list(dilations) if dilations else [1, 1])


def _wz(w, w_zp):
    m = w.shape[0]
    if w_zp is None:
        return np.zeros(m, np.int64)
    z = np.asarray(w_zp).astype(np.int64).ravel()
    if z.size != 1 and z.size != m:
        raise NotImplementedError("ConvInteger: weight zero point must be scalar or "
                                  "per-output-channel")
    return np.full(m, z[0]) if z.size == 1 else z


def conv_integer(x, w, x_zp, w_zp, strides=None, pads=None, dilations=None, group=1):
    """opConvInteger (onnx_qlinear_ops.dart:235-267), 1-D as 2-D with height 1."""
    x = np.asarray(x)
    w = np.asarray(w)
    if x.ndim == 3:
        y = conv_integer(x.reshape(x.shape[0], x.shape[1], 1, x.shape[2]),
                         w.reshape(w.shape[0], w.shape[1], 1, w.shape[2]), x_zp, w_zp,
                         [1, strides[0] if strides else 1],
                         None if pads is None else [0, pads[0], 0, pads[1]],
                         [1, dilations[0] if dilations else 1], group)
        return y.reshape(y.shape[0], y.shape[1], y.shape[3])
    s, p, d = _defaults(strides, pads, dilations)
    xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
    return conv_int_acc(x, w, xz, _wz(w, w_zp), s, p, d, group)


def qlinear_conv(x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, bias, strides=None,
                 pads=None, dilations=None, group=1, lo=0, hi=255):
    """opQLinearConv (onnx_qlinear_ops.dart:270-308): per channel
    mult = xs * wS[c] / ys and q = roundEven((acc + bias[c]) * mult) + yZp,
    in double, clamped to [lo, hi]."""
    x = np.asarray(x)
    w = np.asarray(w)
    s, p, d = _defaults(strides, pads, dilations)
    xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
    acc = conv_int_acc(x, w, xz, _wz(w, w_zp), s, p, d, group)
    m = w.shape[0]
    xs = float(np.asarray(x_scale, np.float32).ravel()[0])
    ys = float(np.asarray(y_scale, np.float32).ravel()[0])
    ws = np.asarray(w_scale, np.float32).ravel().astype(np.float64)
    mult = np.array([xs * (ws[0] if ws.size == 1 else ws[c]) / ys for c in range(m)])
    bv = np.zeros(m, np.int64) if bias is None else np.asarray(bias).astype(np.int64).ravel()
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    val = (acc + bv.reshape(1, m, 1, 1)).astype(np.float64) * mult.reshape(1, m, 1, 1)
    q = round_even(val) + yz
    return np.clip(q, lo, hi).astype(np.int64)
