"""GPU parity of MatMulNBits with bits = 8, g_idx, bias, float zero points,
fp16 scales and the per-column zero-point layout (mmnb_pack_nbits_ex)
against the extended oracle (oracle/nbits_ex.py).

Bar: normwise relative error <= 1e-5 against the oracle, and
|y - y64| <= gamma_{2K + n_blocks + 4} * sum|a| (|q| + |zp| + c) scale,
c = 272 for bits 8 (the hi/lo planes and the correction term) and 0 for
bits 4: the kernels split (q - zp) s into q s and a per-block correction,
so the error scales with the parts, not with their difference.  Cases
cover the GEMV (M = 1), the multi-row GEMV (M <= 8) and the GEMM (M > 8).
"""
import numpy as np
import pytest

from oracle import nbits_ex as X
from onnx_runtime_dart_amd import _lib, ops
from tests.helpers import normwise_rel_err

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
TOL = 1e-5


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


def _weights(rng, k, n, bits, bs):
    nb = (k + bs - 1) // bs
    b = rng.integers(0, 256, (n, nb, bs * bits // 8)).astype(np.uint8)
    s = rng.uniform(0.002, 0.02, n * nb).astype(np.float32)
    return b, s, nb


def _zp(rng, kind, n, nb, bits):
    if kind is None:
        return None
    if kind == "u8":
        if bits == 8:
            return rng.integers(0, 256, n * nb).astype(np.uint8)
        return rng.integers(0, 256, (n * nb + 1) // 2).astype(np.uint8)
    if kind == "col":
        return rng.integers(0, 256, (n, (nb + 1) // 2)).astype(np.uint8)
    hi = 15.0 if bits == 4 else 255.0
    z = rng.uniform(0, hi, (n, nb))
    return z.astype(np.float16 if kind == "f16" else np.float32)


CASES = [
    # m, k, n, bits, bs, zp, g_idx, bias, fp16 scales
    (1, 1024, 256, 8, 32, "u8", False, None, False),
    (4, 512, 100, 8, 64, None, False, None, False),
    (64, 1024, 256, 8, 128, "u8", False, None, False),
    (1, 200, 33, 8, 32, "f32", False, None, False),       # partial block
    (1, 1024, 512, 4, 32, "f32", False, None, False),
    (3, 256, 70, 4, 64, "f16", False, None, False),
    (70, 512, 130, 4, 32, "f32", False, None, False),
    (2, 96, 7, 4, 32, "col", False, None, False),          # odd n_blocks
    (1, 384, 300, 4, 128, "col", False, None, False),
    (1, 1024, 256, 4, 32, "u8", False, None, True),
    (1, 512, 128, 4, 64, "u8", True, None, False),
    (40, 256, 96, 4, 32, "f32", True, None, False),
    (1, 1024, 300, 4, 32, None, False, "f32", False),
    (9, 256, 40, 8, 32, "u8", False, "f16", True),
    (130, 1024, 64, 4, 64, "col", True, "f32", True),
]


@pytest.mark.parametrize("case", CASES)
def test_extended_matmul_nbits_vs_oracle(ctx, case):
    m, k, n, bits, bs, zkind, use_g, bkind, s16 = case
    rng = np.random.default_rng(m * 31 + k + n + bits)
    b, s, nb = _weights(rng, k, n, bits, bs)
    z = _zp(rng, zkind, n, nb, bits)
    g = rng.permutation(np.repeat(np.arange(nb), bs)) if use_g else None
    bias = None if bkind is None else rng.standard_normal(n).astype(
        np.float16 if bkind == "f16" else np.float32)
    if s16:
        s = s.astype(np.float16)
    a = rng.standard_normal((m, k)).astype(np.float32)
    y = ops.op_matmul_nbits_ex(a, b, s, z, g, bias, k=k, n=n, bits=bits, block_size=bs,
                               ctx=ctx)
    ref = X.matmul_nbits_ex(a, b, s, z, g, bias, k, n, bits, bs)
    assert normwise_rel_err(y, ref) <= TOL
    y64, _ = X.matmul_nbits_ex_f64(a, b, s, z, g, bias, k, n, bits, bs)
    q = X.unpack_q(b, k, n, bits, bs).astype(np.float64)
    zz = X.zero_points_per_block(z, n, nb, bits)
    gi = np.arange(k) // bs if g is None else g
    sc = np.asarray(s, np.float32).astype(np.float64).reshape(n, nb)[:, gi]
    part = (np.abs(q) + np.abs(zz[:, gi]) + (272.0 if bits == 8 else 0.0)) * sc
    scale = np.abs(a.astype(np.float64)) @ part.T
    if bias is not None:
        scale = scale + np.abs(np.asarray(bias, np.float32).astype(np.float64))
    kk = 2 * k + nb + 4
    gam = kk * U / (1 - kk * U)
    assert np.all(np.abs(y - y64) <= gam * scale + 1e-30)


def test_plain_inputs_through_ex_equal_the_reference_path(ctx):
    rng = np.random.default_rng(2)
    k, n, bs = 512, 96, 32
    b, s, nb = _weights(rng, k, n, 4, bs)
    z = rng.integers(0, 256, (n * nb + 1) // 2).astype(np.uint8)
    a = rng.standard_normal((3, k)).astype(np.float32)
    y1 = ops.op_matmul_nbits(a, b, s, z, k=k, n=n, bits=4, block_size=bs, ctx=ctx)
    y2 = ops.op_matmul_nbits_ex(a, b, s, z, k=k, n=n, bits=4, block_size=bs, ctx=ctx)
    np.testing.assert_array_equal(y1, y2)


def test_dispatch_with_ort_semantics(ctx):
    rng = np.random.default_rng(4)
    k, n, bs = 256, 40, 32
    b, s, nb = _weights(rng, k, n, 4, bs)
    bias = rng.standard_normal(n).astype(np.float32)
    g = np.arange(k) // bs
    a = rng.standard_normal((2, k)).astype(np.float32)
    attrs = {"K": k, "N": n, "bits": 4, "block_size": bs}
    y = ops.dispatch("MatMulNBits", [a, b, s, None, g, bias], attrs, ort_semantics=True)[0]
    ref = X.matmul_nbits_ex(a, b, s, None, g, bias, k, n, 4, bs)
    assert normwise_rel_err(y, ref) <= TOL
    with pytest.raises(NotImplementedError):  # the reference's behaviour by default
        ops.dispatch("MatMulNBits", [a, b, s, None, g, bias], attrs)


def test_argument_errors(ctx):
    rng = np.random.default_rng(5)
    k, n, bs = 128, 8, 32
    b, s, nb = _weights(rng, k, n, 4, bs)
    with pytest.raises(NotImplementedError):   # bits 2
        ops.pack_nbits_ex(b, s, k=k, n=n, bits=2, block_size=bs, ctx=ctx)
    with pytest.raises(ValueError):            # g_idx length != K
        ops.pack_nbits_ex(b, s, None, np.zeros(k - 1, np.int32), k=k, n=n, bits=4,
                          block_size=bs, ctx=ctx)
    with pytest.raises(ValueError):            # g_idx out of range
        ops.pack_nbits_ex(b, s, None, np.full(k, nb, np.int32), k=k, n=n, bits=4,
                          block_size=bs, ctx=ctx)
    with pytest.raises(NotImplementedError):   # groups of unequal size
        g = np.zeros(k, np.int32)
        g[-1] = 1
        ops.pack_nbits_ex(b, s, None, g, k=k, n=n, bits=4, block_size=bs, ctx=ctx)
    with pytest.raises(ValueError):            # bias too short
        ops.pack_nbits_ex(b, s, None, None, np.zeros(n - 1, np.float32), k=k, n=n, bits=4,
                          block_size=bs, ctx=ctx)
