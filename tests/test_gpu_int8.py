"""GPU parity of DynamicQuantizeLinear and MatMulInteger (+ the fused
fp32 rescale) against the CPU oracle: bit-exact."""
import ctypes

import numpy as np
import pytest

from oracle import refcpu
from onnx_runtime_dart_amd import _lib, ops, synth
from tests.helpers import load_golden, node_arg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


def dql_check(ctx, x):
    y, s, z = ops.op_dynamic_quantize_linear(x, ctx=ctx)
    ry, rs, rz = refcpu.dynamic_quantize_linear(x)
    assert y.shape == x.shape and y.dtype == np.uint8
    assert s.shape == () and z.shape == () and z.dtype == np.int64
    assert np.float32(s).tobytes() == np.float32(rs).tobytes()
    assert int(z) == rz
    np.testing.assert_array_equal(y, ry)
    return y, s, z


# ------------------------------------------------------------------- DQL
def test_dql_golden(ctx):
    d, vals, exp = load_golden("dynamicquantizelinear")
    y, s, z = ops.dispatch("DynamicQuantizeLinear", [vals["x"]], {})
    np.testing.assert_array_equal(y.astype(np.int64), exp["out0"])
    assert np.float32(s) == np.float32(exp["out1"]) and int(z) == int(exp["out2"])


def test_dql_int8_chain_input(ctx):
    x, _ = synth.int8_chain_problem()
    dql_check(ctx, x)


@pytest.mark.parametrize("n", [1, 3, 7, 64, 1023, 4097, 1 << 20, (1 << 22) + 5])
def test_dql_sizes(ctx, n):
    x = (np.random.default_rng(n).standard_normal(n) * 2.5).astype(np.float32)
    dql_check(ctx, x)


def test_dql_special_inputs(ctx):
    dql_check(ctx, np.zeros(1000, np.float32))                        # scale 0
    dql_check(ctx, np.abs(np.random.default_rng(0).standard_normal(999)).astype(np.float32))
    dql_check(ctx, -np.abs(np.random.default_rng(1).standard_normal(999)).astype(np.float32))
    # exact ties at scale 1: round half to even
    x = np.array([0.0, 255.0, 0.5, 1.5, 2.5, 3.5, 100.5, 101.5, 254.5], np.float32)
    y, s, z = dql_check(ctx, x)
    assert y.tolist() == [0, 255, 0, 2, 2, 4, 100, 102, 254]
    # unaligned view (offset by one float)
    base = np.random.default_rng(3).standard_normal(4099).astype(np.float32)
    dql_check(ctx, base[1:])


def test_dql_many_scales_match_double_sequence(ctx):
    rng = np.random.default_rng(42)
    for _ in range(40):
        x = (rng.standard_normal(333) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        dql_check(ctx, x)


@pytest.mark.parametrize("n", [5, 1000, 70001])
def test_dql_non_finite_input_is_rejected(ctx, n):
    # the reference's _roundEven throws on a NaN / infinite quotient
    # (onnx_ops.dart:2490-2497, :2574-2576): the host entry point returns
    # MMNB_ERR_UNSUPPORTED (NotImplementedError), like the oracle; the device
    # form writes a NaN scale as its marker
    rng = np.random.default_rng(n)
    for pos, bad in ((0, np.nan), (n - 1, np.inf), (n // 2, -np.inf)):
        x = rng.standard_normal(n).astype(np.float32)
        x[pos] = bad
        with pytest.raises(NotImplementedError):
            refcpu.dynamic_quantize_linear(x)
        with pytest.raises(NotImplementedError):
            ops.op_dynamic_quantize_linear(x, ctx=ctx)
        dx, dy, dsz = ctx.to_device(x), ctx.alloc(n), ctx.alloc(8)
        _lib.check(ctx.lib.mmnb_dynamic_quantize_linear_dev(ctx.handle, dx.ptr, n, dy.ptr,
                                                            dsz.ptr,
                                                            ctypes.c_void_p(dsz.ptr.value + 4)))
        ctx.synchronize()
        assert np.isnan(dsz.numpy(np.float32, (2,))[0])
        for bf in (dx, dy, dsz):
            bf.free()
    # NaN among zeros: scale 0, nothing rounded, zp everywhere (no error)
    x = np.zeros(n, np.float32)
    x[n // 3] = np.nan
    dql_check(ctx, x)


def test_dql_empty(ctx):
    y, s, z = ops.op_dynamic_quantize_linear(np.zeros((0,), np.float32), ctx=ctx)
    assert y.size == 0 and float(s) == 0.0 and int(z) == 0


# --------------------------------------------------------- MatMulInteger
@pytest.mark.parametrize("case", ["matmulinteger_u8i8", "matmulinteger_nozp",
                                  "matmulinteger_batched", "matmulinteger_percol_bzp"])
def test_mmi_golden(ctx, case):
    d, vals, exp = load_golden(case)
    ins = [node_arg(d, vals, i) for i in range(len(d["node_inputs"]))]
    y = ops.dispatch("MatMulInteger", ins, {})[0]
    assert y.dtype == np.int64
    np.testing.assert_array_equal(y, exp["out0"])


def test_mmi_hand_case(ctx):
    # compact_tensor_test.dart:48-58
    a = np.array([[10, 130, 250]], dtype=np.uint8)
    b = np.array([[-1, 2], [3, -4], [5, 6]], dtype=np.int8)
    y = ops.op_matmul_integer(a, b, np.array(10), np.array(1), ctx=ctx)
    assert y.tolist() == [[1200, 600]]


def test_mmi_int8_chain_shape(ctx):
    x, b = synth.int8_chain_problem()
    aq, s, z = dql_check(ctx, x)
    y = ops.op_matmul_integer(aq, b, z, np.array(0, np.int8), ctx=ctx)
    ref = refcpu.matmul_integer(aq, b, int(z), 0)
    np.testing.assert_array_equal(y, ref)


@pytest.mark.parametrize("adt,bdt,az,bz,ab,bb,m,k,n", [
    (np.uint8, np.int8, "s", "s", None, None, 70, 200, 90),
    (np.uint8, np.int8, "row", "col", None, None, 33, 128, 65),
    (np.uint8, np.uint8, None, None, None, None, 17, 64, 31),
    (np.int8, np.int8, "s", None, None, None, 64, 1024, 64),
    (np.int8, np.uint8, None, "col", None, None, 5, 77, 3),     # K % 16 != 0
    (np.uint8, np.int8, "s", "s", 3, None, 9, 48, 20),          # batched A, shared B
    (np.uint8, np.int8, None, "col", None, 2, 9, 48, 20),       # shared A, batched B
    (np.uint8, np.int8, "row", "s", 2, 2, 16, 96, 40),
    (np.uint8, np.int8, "s", "s", None, None, 1, 1024, 3072),   # M = 1
    (np.uint8, np.int8, "s", "s", None, None, 130, 4096, 1),    # N = 1
    # K % 16 == 0 up to 1024: all of K in one round trip; K steps not a
    # multiple of 4 (A pieces padded to whole swizzle groups), M and N ragged
    (np.uint8, np.int8, "row", "col", None, None, 100, 336, 200),
    (np.uint8, np.uint8, "s", "col", None, None, 70, 1008, 96),
    (np.int8, np.int8, None, "s", 2, None, 40, 720, 136),
])
def test_mmi_brute_force(ctx, adt, bdt, az, bz, ab, bb, m, k, n):
    rng = np.random.default_rng(m * 31 + k + n)
    ai, bi = np.iinfo(adt), np.iinfo(bdt)
    a = rng.integers(ai.min, ai.max + 1, ((ab,) if ab else ()) + (m, k)).astype(adt)
    b = rng.integers(bi.min, bi.max + 1, ((bb,) if bb else ()) + (k, n)).astype(bdt)
    azv = {None: None, "s": np.array(rng.integers(ai.min, ai.max + 1), adt),
           "row": rng.integers(ai.min, ai.max + 1, m).astype(adt)}[az]
    bzv = {None: None, "s": np.array(rng.integers(bi.min, bi.max + 1), bdt),
           "col": rng.integers(bi.min, bi.max + 1, n).astype(bdt)}[bz]
    y = ops.op_matmul_integer(a, b, azv, bzv, ctx=ctx)
    ref = refcpu.matmul_integer(a, b, azv, bzv)
    assert y.shape == ref.shape
    np.testing.assert_array_equal(y, ref)


def test_mmi_extreme_values_exact(ctx):
    # all-255 A against all -128 B with zero points at the opposite ends:
    # the largest magnitudes the int32 contract allows at this K
    m, k, n = 64, 4096, 64
    a = np.full((m, k), 255, np.uint8)
    b = np.full((k, n), -128, np.int8)
    y = ops.op_matmul_integer(a, b, np.array(0, np.uint8), np.array(127, np.int8), ctx=ctx)
    assert np.all(y == 255 * (-255) * k)


def test_mmi_rejects_bad_zero_points(ctx):
    a = np.zeros((4, 3), np.uint8)
    b = np.zeros((3, 5), np.int8)
    with pytest.raises(NotImplementedError):
        ops.op_matmul_integer(a, b, np.zeros(2, np.uint8), None, ctx=ctx)
    with pytest.raises(NotImplementedError):
        ops.op_matmul_integer(a, b, None, np.zeros(3, np.int8), ctx=ctx)


# ------------------------------------------------ fused dynamic chain
@pytest.mark.parametrize("m,k,n,per_col", [(512, 1024, 3072, False), (37, 200, 70, True),
                                           (1, 64, 16, False)])
def test_dynamic_matmul_chain_bit_exact(ctx, m, k, n, per_col):
    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    b_scale = (rng.uniform(0.001, 0.01, n if per_col else 1)).astype(np.float32)
    pack = ops.pack_integer(b, np.array(0, np.int8), ctx=ctx)
    dx = ctx.to_device(x)
    dbs = ctx.to_device(b_scale)
    daq = ctx.alloc(m * k)
    dsc = ctx.alloc(4)
    dzp = ctx.alloc(4)
    dacc = ctx.alloc(m * n * 4)
    dy = ctx.alloc(m * n * 4)
    _lib.check(ctx.lib.mmnb_dynamic_matmul_dev(ctx.handle, pack.handle, dx.ptr, m, dbs.ptr,
                                               b_scale.size, daq.ptr, dsc.ptr, dzp.ptr,
                                               dacc.ptr, dy.ptr))
    ctx.synchronize()
    aq = daq.numpy(np.uint8, (m, k))
    sc = dsc.numpy(np.float32, (1,))[0]
    zp = int(dzp.numpy(np.int32, (1,))[0])
    acc = dacc.numpy(np.int32, (m, n))
    y = dy.numpy(np.float32, (m, n))
    ry, rs, rz = refcpu.dynamic_quantize_linear(x)
    np.testing.assert_array_equal(aq, ry)
    assert sc == rs and zp == rz
    racc = refcpu.matmul_integer(ry, b, rz, 0)
    np.testing.assert_array_equal(acc.astype(np.int64), racc)
    ref = refcpu.rescale(racc, rs, b_scale)
    np.testing.assert_array_equal(y, ref)
    for buf in (dx, dbs, daq, dsc, dzp, dacc, dy):
        buf.free()
    pack.free()


@pytest.mark.parametrize("m,k,n,per_col", [(512, 1024, 3072, True), (65, 336, 130, False)])
def test_dynamic_matmul_chain_without_int32_output(ctx, m, k, n, per_col):
    # d_acc NULL: only the fp32 result leaves the kernel; still bit-exact
    rng = np.random.default_rng(3 * m + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    b_scale = (rng.uniform(0.001, 0.01, n if per_col else 1)).astype(np.float32)
    pack = ops.pack_integer(b, np.array(0, np.int8), ctx=ctx)
    dx, dbs = ctx.to_device(x), ctx.to_device(b_scale)
    daq, dsc, dzp, dy = ctx.alloc(m * k), ctx.alloc(4), ctx.alloc(4), ctx.alloc(m * n * 4)
    _lib.check(ctx.lib.mmnb_dynamic_matmul_dev(ctx.handle, pack.handle, dx.ptr, m, dbs.ptr,
                                               b_scale.size, daq.ptr, dsc.ptr, dzp.ptr, None,
                                               dy.ptr))
    ctx.synchronize()
    y = dy.numpy(np.float32, (m, n))
    ry, rs, rz = refcpu.dynamic_quantize_linear(x)
    np.testing.assert_array_equal(daq.numpy(np.uint8, (m, k)), ry)
    ref = refcpu.rescale(refcpu.matmul_integer(ry, b, rz, 0), rs, b_scale)
    np.testing.assert_array_equal(y, ref)
    for buf in (dx, dbs, daq, dsc, dzp, dy):
        buf.free()
    pack.free()
