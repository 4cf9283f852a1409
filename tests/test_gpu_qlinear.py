"""GPU parity of QLinearMatMul, ConvInteger and QLinearConv against the
oracle (oracle/qlinear.py), through the C ABI.  Integer outputs: the bar is
bit-exact.

Fixtures (qlinearmatmul, convinteger, convinteger_1d, qlinearconv_pertensor,
qlinearconv_perchannel_bias) go through the dispatch arms; random cases cover
int8/uint8 operand mixes, per-row / per-column / per-channel zero points,
batched QLinearMatMul, grouped convolutions with strides, pads and
dilations, several images, reduction lengths that are and are not multiples
of 16 (the two MatMulInteger kernels), saturation at both ends, and the
device entry points against the host ones.
"""
import ctypes

import numpy as np
import pytest

from oracle import qlinear as Q
from onnx_runtime_dart_amd import _lib, ops
from tests.helpers import load_golden, node_arg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


@pytest.mark.parametrize("case", ["qlinearmatmul", "convinteger", "convinteger_1d",
                                  "qlinearconv_pertensor", "qlinearconv_perchannel_bias"])
def test_golden_fixtures_through_dispatch(ctx, case):
    d, vals, exp = load_golden(case)
    ins = [node_arg(d, vals, i) for i in range(len(d["node_inputs"]))]
    y = ops.dispatch(d["op_type"], ins, d["attrs"])[0]
    np.testing.assert_array_equal(y, exp["out0"].astype(np.int64))


@pytest.mark.parametrize("m,k,n,a8,b8,y8,azp,bzp,batch", [
    (4, 6, 5, False, False, False, "s", "s", 1),
    (37, 100, 70, True, True, True, "row", "col", 1),    # K % 16 != 0: register path
    (64, 256, 96, False, True, False, "s", "col", 1),    # K % 16 == 0: LDS path
    (5, 48, 9, False, False, True, None, None, 3),       # batched A and B
    (130, 1024, 200, False, True, False, "s", "s", 1),
])
def test_qlinear_matmul_vs_oracle(ctx, m, k, n, a8, b8, y8, azp, bzp, batch):
    rng = np.random.default_rng(m * 7 + k + n)
    at = np.int8 if a8 else np.uint8
    bt = np.int8 if b8 else np.uint8
    lo_a, hi_a = (-128, 128) if a8 else (0, 256)
    lo_b, hi_b = (-128, 128) if b8 else (0, 256)
    shape_a = (batch, m, k) if batch > 1 else (m, k)
    shape_b = (batch, k, n) if batch > 1 else (k, n)
    a = rng.integers(lo_a, hi_a, shape_a).astype(at)
    b = rng.integers(lo_b, hi_b, shape_b).astype(bt)
    a_zp = {"s": at(rng.integers(lo_a, hi_a)), "row": rng.integers(lo_a, hi_a, m).astype(at),
            None: None}[azp]
    b_zp = {"s": bt(rng.integers(lo_b, hi_b)), "col": rng.integers(lo_b, hi_b, n).astype(bt),
            None: None}[bzp]
    a_s, b_s = np.float32(0.013), np.float32(0.021)
    y_s = np.float32(0.37 * np.sqrt(k) * 0.013 * 0.021 * 60)  # spreads over the range
    y_zp = np.int8(-3) if y8 else np.uint8(120)
    lo, hi = (-128, 127) if y8 else (0, 255)
    y = ops.op_qlinear_matmul(a, a_s, a_zp, b, b_s, b_zp, y_s, y_zp, lo=lo, hi=hi, ctx=ctx)
    want = Q.qlinear_matmul(a, a_s, a_zp, b, b_s, b_zp, y_s, y_zp, lo, hi)
    np.testing.assert_array_equal(y, want)
    assert np.any(y == lo) or np.any(y == hi) or m * n < 100  # saturation exercised


CONV = [
    # n, c, h, w, m, kh, kw, group, strides, pads, dilations, x8, w8
    (1, 3, 8, 9, 4, 3, 3, 1, [1, 1], [1, 1, 1, 1], [1, 1], False, True),   # K = 27
    (2, 4, 6, 6, 6, 3, 2, 2, [2, 1], [0, 1, 2, 0], [1, 2], True, True),
    (1, 6, 7, 6, 6, 1, 3, 3, [1, 2], [0, 0, 0, 0], [1, 1], False, False),
    (1, 16, 12, 12, 32, 3, 3, 1, [1, 1], [1, 1, 1, 1], [1, 1], False, True),  # K = 144
    (3, 32, 9, 9, 64, 1, 1, 2, [1, 1], [0, 0, 0, 0], [1, 1], False, True),    # K = 16
    (1, 64, 20, 23, 16, 3, 3, 1, [1, 1], [1, 1, 1, 1], [1, 1], False, True),  # K = 576
    (1, 8, 15, 31, 8, 3, 3, 2, [2, 2], [1, 2, 1, 0], [1, 1], True, True),
    (1, 512, 4, 30, 8, 3, 3, 1, [1, 1], [0, 0, 0, 0], [1, 12], False, True),  # K = 4608
]


def _conv_inputs(case):
    n, c, h, w, m, kh, kw, group, s, p, dl, x8, w8 = case
    rng = np.random.default_rng(n + c * 3 + h * 5 + m * 7 + kh)
    xt, wt = (np.int8 if x8 else np.uint8), (np.int8 if w8 else np.uint8)
    lx = (-128, 128) if x8 else (0, 256)
    lw = (-128, 128) if w8 else (0, 256)
    x = rng.integers(*lx, (n, c, h, w)).astype(xt)
    wt_ = rng.integers(*lw, (m, c // group, kh, kw)).astype(wt)
    xz = xt(rng.integers(*lx))
    wz = rng.integers(*lw, m).astype(wt)
    return x, wt_, xz, wz, dict(strides=s, pads=p, dilations=dl, group=group)


@pytest.mark.parametrize("case", CONV)
def test_conv_integer_vs_oracle(ctx, case):
    x, w, xz, wz, geo = _conv_inputs(case)
    y = ops.op_conv_integer(x, w, xz, wz, ctx=ctx, **geo)
    want = Q.conv_integer(x, w, xz, wz, geo["strides"], geo["pads"], geo["dilations"],
                          geo["group"])
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("case", CONV)
@pytest.mark.parametrize("y8", [False, True])
def test_qlinear_conv_vs_oracle(ctx, case, y8):
    x, w, xz, wz, geo = _conv_inputs(case)
    m = w.shape[0]
    rng = np.random.default_rng(m)
    x_s = np.float32(0.02)
    w_s = rng.uniform(0.005, 0.03, m).astype(np.float32)
    k = w[0].size
    y_s = np.float32(0.02 * 0.02 * np.sqrt(k) * 40)
    bias = rng.integers(-5000, 5000, m).astype(np.int32)
    y_zp = np.int8(5) if y8 else np.uint8(128)
    lo, hi = (-128, 127) if y8 else (0, 255)
    y = ops.op_qlinear_conv(x, x_s, xz, w, w_s, wz, y_s, y_zp, bias, lo=lo, hi=hi, ctx=ctx,
                            **geo)
    want = Q.qlinear_conv(x, x_s, xz, w, w_s, wz, y_s, y_zp, bias, geo["strides"], geo["pads"],
                          geo["dilations"], geo["group"], lo, hi)
    np.testing.assert_array_equal(y, want)


def test_conv_1d_matches_oracle(ctx):
    rng = np.random.default_rng(5)
    x = rng.integers(0, 256, (2, 3, 40)).astype(np.uint8)
    w = rng.integers(-128, 128, (5, 3, 7)).astype(np.int8)
    y = ops.op_conv_integer(x, w, np.uint8(17), np.int8(-4), strides=[2], pads=[3, 1],
                            dilations=[2], ctx=ctx)
    want = Q.conv_integer(x, w, np.uint8(17), np.int8(-4), [2], [3, 1], [2])
    np.testing.assert_array_equal(y, want)


def test_device_forms_match_host_forms(ctx):
    x, w, xz, wz, geo = _conv_inputs(CONV[1])
    pack = ops.pack_conv(w, wz, geo["group"], ctx)
    prm = _lib.ConvParams()
    for i in range(2):
        prm.strides[i] = geo["strides"][i]
        prm.dilations[i] = geo["dilations"][i]
    for i in range(4):
        prm.pads[i] = geo["pads"][i]
    oh, ow = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(ctx.lib.mmnb_conv_output_shape(pack.handle, *x.shape, ctypes.byref(prm),
                                              ctypes.byref(oh), ctypes.byref(ow)))
    n, m = x.shape[0], w.shape[0]
    dx = ctx.to_device(x.view(np.uint8))
    dy = ctx.alloc(n * m * oh.value * ow.value * 4)
    _lib.check(ctx.lib.mmnb_conv_integer_dev(ctx.handle, pack.handle, dx.ptr, 1, *x.shape,
                                             int(xz), ctypes.byref(prm), dy.ptr))
    ctx.synchronize()
    y_dev = dy.numpy(np.int32, (n, m, oh.value, ow.value))
    y_host = ops.op_conv_integer(x, w, xz, wz, ctx=ctx, **geo)
    np.testing.assert_array_equal(y_dev.astype(np.int64), y_host)
    # QLinearMatMul device form
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, (33, 80)).astype(np.uint8)
    b = rng.integers(-128, 128, (80, 40)).astype(np.int8)
    bp = ops.pack_integer(b, np.int8(3), ctx)
    da = ctx.to_device(a)
    dq = ctx.alloc(33 * 40)
    dz = ctx.to_device(np.array([9], np.int32))
    _lib.check(ctx.lib.mmnb_qlinear_matmul_dev(ctx.handle, bp.handle, da.ptr, 0, 1, 33, dz.ptr,
                                               1, 0.01, 0.02, 0.05, 7, 0, dq.ptr))
    ctx.synchronize()
    q_dev = dq.numpy(np.uint8, (33, 40))
    want = Q.qlinear_matmul(a, np.float32(0.01), np.uint8(9), b, np.float32(0.02), np.int8(3),
                            np.float32(0.05), np.uint8(7), 0, 255)
    np.testing.assert_array_equal(q_dev.astype(np.int64), want)
    for buf in (dx, dy, da, dq, dz):
        buf.free()
    pack.free()
    bp.free()


def test_argument_errors(ctx):
    x = np.zeros((1, 4, 5, 5), np.uint8)
    w = np.zeros((6, 2, 3, 3), np.int8)
    with pytest.raises(NotImplementedError):   # weight zp neither scalar nor per channel
        ops.op_conv_integer(x, w, None, np.zeros(4, np.int8), group=2, ctx=ctx)
    with pytest.raises(ValueError):            # channels != c_per_group * group
        ops.op_conv_integer(x, w, None, None, group=1, ctx=ctx)
    with pytest.raises(ValueError):            # window larger than the padded input
        ops.op_conv_integer(np.zeros((1, 2, 2, 2), np.uint8), np.zeros((1, 2, 3, 3), np.int8),
                            None, None, ctx=ctx)
    a = np.zeros((2, 3), np.uint8)
    b = np.zeros((3, 4), np.uint8)
    with pytest.raises(NotImplementedError):   # per-axis scales
        ops.op_qlinear_matmul(a, np.ones(2, np.float32), None, b, np.float32(1), None,
                              np.float32(1), None, lo=0, hi=255, ctx=ctx)
    with pytest.raises(ValueError):            # y_scale 0
        ops.op_qlinear_matmul(a, np.float32(1), None, b, np.float32(1), None,
                              np.float32(0), None, lo=0, hi=255, ctx=ctx)
