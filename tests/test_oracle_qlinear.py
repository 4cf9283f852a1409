"""The QLinearMatMul / ConvInteger / QLinearConv oracle (oracle/qlinear.py)
against the reference's golden vectors and what the arithmetic fixes.

Fixtures: qlinearmatmul, convinteger, convinteger_1d, qlinearconv_pertensor,
qlinearconv_perchannel_bias (tool/gen_fixtures.py:736-781, ORT CPU outputs),
compared exactly: the outputs are integers.  Beyond them: the vectorised
convolution against plain loops in the reference's order (groups, strides,
pads, dilations, per-channel zero points), QLinearConv with unit scales as
the clamped integer accumulator, and planted mistakes (requantising
QLinearMatMul in double only; dropping the input zero point at padded taps)
that the checks reject.
"""
import numpy as np
import pytest

from oracle import qlinear as Q
from tests.helpers import load_golden, node_arg


def _rng8(z):
    return (-128, 127) if z is not None and np.asarray(z).dtype == np.int8 else (0, 255)


def test_qlinearmatmul_golden():
    d, vals, exp = load_golden("qlinearmatmul")
    ins = [node_arg(d, vals, i) for i in range(8)]
    lo, hi = _rng8(ins[7])
    y = Q.qlinear_matmul(*ins, lo, hi)
    np.testing.assert_array_equal(y, exp["out0"].astype(np.int64))


@pytest.mark.parametrize("case", ["convinteger", "convinteger_1d"])
def test_convinteger_golden(case):
    d, vals, exp = load_golden(case)
    ins = [node_arg(d, vals, i) for i in range(4)]
    at = d["attrs"]
    y = Q.conv_integer(*ins, strides=at.get("strides"), pads=at.get("pads"),
                       dilations=at.get("dilations"), group=at.get("group", 1))
    np.testing.assert_array_equal(y, exp["out0"].astype(np.int64))


@pytest.mark.parametrize("case", ["qlinearconv_pertensor", "qlinearconv_perchannel_bias"])
def test_qlinearconv_golden(case):
    d, vals, exp = load_golden(case)
    ins = [node_arg(d, vals, i) for i in range(9)]
    at = d["attrs"]
    lo, hi = _rng8(ins[7])
    y = Q.qlinear_conv(*ins, strides=at.get("strides"), pads=at.get("pads"),
                       dilations=at.get("dilations"), group=at.get("group", 1), lo=lo, hi=hi)
    np.testing.assert_array_equal(y, exp["out0"].astype(np.int64))


CONV_CASES = [
    # n, c, h, w, m, kh, kw, group, strides, pads, dilations
    (1, 3, 6, 7, 4, 3, 3, 1, [1, 1], [1, 1, 1, 1], [1, 1]),
    (2, 4, 5, 5, 6, 3, 2, 2, [2, 1], [0, 1, 2, 0], [1, 2]),
    (1, 6, 7, 6, 6, 1, 3, 3, [1, 2], [0, 0, 0, 0], [1, 1]),
    (1, 2, 9, 4, 2, 2, 2, 1, [3, 1], [2, 1, 1, 2], [2, 1]),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_matches_reference_loops(case):
    n, c, h, w, m, kh, kw, group, s, p, dl = case
    rng = np.random.default_rng(sum(case[:8]))
    x = rng.integers(0, 256, (n, c, h, w)).astype(np.uint8)
    wt = rng.integers(-128, 128, (m, c // group, kh, kw)).astype(np.int8)
    xz = np.uint8(rng.integers(0, 256))
    wz = rng.integers(-128, 128, m).astype(np.int8)
    fast = Q.conv_integer(x, wt, xz, wz, s, p, dl, group)
    slow = Q.conv_int_acc_loops(x, wt, int(xz), wz.astype(np.int64), s, p, dl, group)
    np.testing.assert_array_equal(fast, slow)


def test_qlinearconv_unit_scales_is_clamped_accumulator():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 4, (1, 2, 4, 4)).astype(np.uint8)
    w = rng.integers(-2, 3, (3, 2, 2, 2)).astype(np.int8)
    bias = np.array([5, -7, 100], np.int32)
    one = np.float32(1.0)
    y = Q.qlinear_conv(x, one, np.uint8(1), w, one, np.int8(0), one, np.uint8(10), bias,
                       lo=0, hi=255)
    acc = Q.conv_integer(x, w, np.uint8(1), np.int8(0))
    want = np.clip(acc + bias.reshape(1, 3, 1, 1) + 10, 0, 255)
    np.testing.assert_array_equal(y, want)


def _product_with_acc(acc):
    """uint8 A [1, K] and int8 B [K, 1] whose exact product is acc >= 0."""
    q, r = divmod(acc, 255)
    t, u = divmod(q, 127)
    r1 = min(r, 127)
    a = np.array([[255] * (t + 1) + [1, 1]], np.uint8)
    b = np.array([[127]] * t + [[u], [r1], [r - r1]], np.int8)
    return a, b


def test_qlinearmatmul_binary32_steps_matter():
    """The reference requantises in binary32 steps (onnx_qlinear_ops.dart:91-101).
    Find an accumulator where fl32(acc * mult) lands on a .5 tie (or across
    one) that a double-only evaluation does not, build a product with that
    accumulator, and check the oracle follows the binary32 sequence."""
    found = None
    for y_s in (0.731, 0.419, 1.37, 2.9):
        a_s, b_s, y_s = np.float32(0.0173), np.float32(0.0091), np.float32(y_s)
        mult = np.float32(np.float32(float(a_s) * float(b_s)) / float(y_s))
        acc = np.arange(0, int(255 / float(mult)), dtype=np.int64)
        x64 = acc * float(mult)
        x32 = x64.astype(np.float32).astype(np.float64)
        diff = np.nonzero(np.rint(x64) != np.rint(x32))[0]
        if diff.size:
            found = (a_s, b_s, y_s, int(acc[diff[0]]), x64[diff[0]], x32[diff[0]])
            break
    assert found, "no tie case in range"
    a_s, b_s, y_s, target, v64, v32 = found
    a, b = _product_with_acc(target)
    y = Q.qlinear_matmul(a, a_s, None, b, b_s, None, y_s, np.uint8(0), 0, 255)
    assert int(y[0, 0]) == int(np.rint(v32))
    assert int(y[0, 0]) != int(np.rint(v64))


def test_padding_taps_use_the_input_zero_point():
    """A planted mistake -- padding with 0 instead of skipping the tap -- is
    caught by the 2-D fixture (x_zp != 0 there)."""
    d, vals, exp = load_golden("convinteger")
    x, w, xz, wz = (node_arg(d, vals, i) for i in range(4))
    assert int(xz) != 0
    xp = np.pad(x.astype(np.int64) - int(xz), ((0, 0), (0, 0), (1, 1), (1, 1)))
    wrong = Q.conv_int_acc_loops(np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1))), w, int(xz),
                                 np.full(w.shape[0], int(wz)), [1, 1], [0, 0, 0, 0], [1, 1], 1)
    right = Q.conv_int_acc_loops(xp + int(xz), w, int(xz), np.full(w.shape[0], int(wz)),
                                 [1, 1], [0, 0, 0, 0], [1, 1], 1)
    np.testing.assert_array_equal(right, exp["out0"])
    assert np.any(wrong != exp["out0"])


def test_weight_zero_point_shape_rejected():
    x = np.zeros((1, 2, 3, 3), np.uint8)
    w = np.zeros((4, 2, 1, 1), np.int8)
    with pytest.raises(NotImplementedError):
        Q.conv_integer(x, w, None, np.zeros(3, np.int8))


def test_qlinearmatmul_per_axis_scales_rejected():
    a = np.zeros((2, 3), np.uint8)
    b = np.zeros((3, 4), np.uint8)
    with pytest.raises(NotImplementedError):
        Q.qlinear_matmul(a, np.ones(2, np.float32), None, b, np.float32(1), None,
                         np.float32(1), None, 0, 255)
