"""The extended MatMulNBits oracle (oracle/nbits_ex.py) pinned against the
reference-faithful oracle and what the definitions fix.

The reference has no fixture for bits = 8, g_idx, bias, float zero points,
fp16 scales or the per-column zero-point layout (it rejects or ignores
them), so these are restated from the ORT operator definition and pinned
by: bit-identity with refcpu.matmul_nbits where the two overlap (bits 4,
flat uint8 zero points); integral float zero points equal to the uint8 ones;
the per-column layout equal to the flat one after re-indexing; fp16 scales
equal to their exact fp32 widening; identity g_idx equal to none and a
permuted g_idx equal to the same product with rows of A and W permuted;
bits = 8 against an int64 brute force; bias as an exact binary32 shift.
A planted mistake (per-column bytes read with the flat index) is rejected.
"""
import numpy as np
import pytest

from oracle import nbits_ex as X
from oracle import refcpu
from onnx_runtime_dart_amd import synth


def _problem(m, k, n, bs, zp, seed):
    return synth.mmnb_problem(m, k, n, bs, zp, seed=seed)


@pytest.mark.parametrize("m,k,n,bs,zp", [(3, 64, 6, 32, True), (2, 40, 5, 32, False),
                                         (4, 256, 33, 64, True)])
def test_overlap_with_reference_oracle_is_bitwise(m, k, n, bs, zp):
    p = _problem(m, k, n, bs, zp, seed=k + n)
    want = refcpu.matmul_nbits(p.a, p.b_q, p.scales, p.zero_points, k, n, 4, bs)
    got = X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, None, None, k, n, 4, bs)
    np.testing.assert_array_equal(got, want)


def _flat_to_per_column(zflat, n, nb):
    idx = np.arange(n * nb)
    nib = np.where(idx % 2 == 0, zflat[idx >> 1] & 0xF, zflat[idx >> 1] >> 4).reshape(n, nb)
    row = (nb + 1) // 2
    out = np.zeros((n, row), np.uint8)
    for b in range(nb):
        out[:, b // 2] |= (nib[:, b] << (4 * (b & 1))).astype(np.uint8)
    return out, nib


def test_per_column_layout_equals_flat_and_flat_indexing_of_it_differs():
    k, n, bs = 96, 7, 32        # n_blocks = 3 (odd): the layouts differ
    p = _problem(2, k, n, bs, True, seed=4)
    nb = 3
    zpc, nib = _flat_to_per_column(p.zero_points, n, nb)
    a = X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, None, None, k, n, 4, bs)
    b = X.matmul_nbits_ex(p.a, p.b_q, p.scales, zpc, None, None, k, n, 4, bs)
    np.testing.assert_array_equal(a, b)
    wrong = X.matmul_nbits_ex(p.a, p.b_q, p.scales, zpc.ravel(), None, None, k, n, 4, bs)
    assert np.any(wrong != a)


def test_integral_float_zero_points_equal_uint8_ones():
    k, n, bs = 128, 9, 32
    p = _problem(3, k, n, bs, True, seed=8)
    _, nib = _flat_to_per_column(p.zero_points, n, k // bs)
    for dt in (np.float32, np.float16):
        got = X.matmul_nbits_ex(p.a, p.b_q, p.scales, nib.astype(dt), None, None, k, n, 4, bs)
        want = X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, None, None, k, n, 4, bs)
        np.testing.assert_array_equal(got, want)


def test_fp16_scales_are_their_fp32_widening():
    k, n, bs = 64, 5, 16
    p = _problem(2, k, n, bs, False, seed=2)
    s16 = p.scales.astype(np.float16)
    got = X.matmul_nbits_ex(p.a, p.b_q, s16, None, None, None, k, n, 4, bs)
    want = X.matmul_nbits_ex(p.a, p.b_q, s16.astype(np.float32), None, None, None, k, n, 4, bs)
    np.testing.assert_array_equal(got, want)


def test_g_idx_identity_and_permutation():
    k, n, bs = 128, 6, 32
    p = _problem(3, k, n, bs, True, seed=6)
    ident = np.arange(k) // bs
    base = X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, None, None, k, n, 4, bs)
    np.testing.assert_array_equal(
        X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, ident, None, k, n, 4, bs), base)
    # act-order: rows permuted, group of row j is its block after sorting
    rng = np.random.default_rng(1)
    g = rng.permutation(np.repeat(np.arange(k // bs), bs))
    w = X.dequant(p.b_q, p.scales, p.zero_points, g, k, n, 4, bs).astype(np.float64)
    want = p.a.astype(np.float64) @ w
    got = X.matmul_nbits_ex(p.a, p.b_q, p.scales, p.zero_points, g, None, k, n, 4, bs)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # the weight of row j uses group g[j]: check one element by hand
    q = X.unpack_q(p.b_q, k, n, 4, bs)
    zz = X.zero_points_per_block(p.zero_points, n, k // bs, 4)
    j, c = 5, 2
    assert w[j, c] == np.float32((q[c, j] - zz[c, g[j]]) * p.scales.reshape(n, -1)[c, g[j]])


def test_bits8_brute_force():
    rng = np.random.default_rng(3)
    k, n, bs, m = 80, 5, 16, 3
    nb = k // bs
    q = rng.integers(0, 256, (n, k)).astype(np.uint8)
    s = rng.uniform(0.001, 0.01, n * nb).astype(np.float32)
    z = rng.integers(0, 256, n * nb).astype(np.uint8)
    a = rng.standard_normal((m, k)).astype(np.float32)
    got = X.matmul_nbits_ex(a, q, s, z, None, None, k, n, 8, bs)
    w = (q.astype(np.int64) - z.reshape(n, nb).repeat(bs, 1)) * s.reshape(n, nb).repeat(bs, 1)
    want = a.astype(np.float64) @ w.T.astype(np.float32).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    default = X.matmul_nbits_ex(a, q, s, None, None, None, k, n, 8, bs)
    want128 = a.astype(np.float64) @ ((q.astype(np.int64) - 128) *
                                      s.reshape(n, nb).repeat(bs, 1)).T
    assert np.max(np.abs(default - want128)) <= 1e-5 * np.max(np.abs(want128))


def test_bias_is_a_binary32_shift():
    k, n, bs = 64, 4, 32
    p = _problem(2, k, n, bs, False, seed=9)
    bias = np.array([1.5, -2.0, 0.25, 3.0], np.float32)
    base = X.matmul_nbits_ex(p.a, p.b_q, p.scales, None, None, None, k, n, 4, bs)
    got = X.matmul_nbits_ex(p.a, p.b_q, p.scales, None, None, bias, k, n, 4, bs)
    np.testing.assert_array_equal(got, (base + bias).astype(np.float32))
