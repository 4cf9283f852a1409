"""GPU parity of MatMulNBits (int4) against the CPU oracle, through the C ABI.

Float bar: normwise relative error max|y_gpu - y_ref| / max|y_ref| <= 1e-5
against the oracle (bit-faithful to the Dart native path), plus the
accumulation bound |y_gpu - y_exact| <= gamma_{K+2} * sum|a||W| against an
fp64 product (the GPU sums in a different order and applies each block's
scale to a partial sum instead of rounding every weight, hence K+2).
"""
import numpy as np
import pytest

from oracle import refcpu
from onnx_runtime_dart_amd import _lib, ops, synth
from tests.helpers import fixture_float_ok, load_golden, node_arg, normwise_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
U = 2.0 ** -24
THREADS = min(16, refcpu.host_threads())


def gamma(k):
    return k * U / (1 - k * U)


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


def run_gpu(ctx, p):
    return ops.op_matmul_nbits(p.a, p.b_q, p.scales, p.zero_points, k=p.k, n=p.n, bits=4,
                               block_size=p.block, ctx=ctx)


def oracle(p, rows=None):
    a = p.a if rows is None else p.a[rows]
    return refcpu.matmul_nbits(a, p.b_q, p.scales, p.zero_points, p.k, p.n, 4, p.block,
                               threads=THREADS)


def check_bound(p, y, rows=None):
    a = p.a if rows is None else p.a[rows]
    y64, absdot = refcpu.matmul_nbits_f64(a, p.b_q, p.scales, p.zero_points, p.k, p.n,
                                          p.block)
    err = np.abs(y.astype(np.float64) - y64)
    assert np.all(err <= gamma(p.k + 2) * absdot + 1e-30), float(np.max(err / (absdot + 1e-300)))


@pytest.mark.parametrize("case", ["matmulnbits_basic", "matmulnbits_zeropoints",
                                  "matmulnbits_partial_block"])
def test_golden_fixtures_through_dispatch(ctx, case):
    d, vals, exp = load_golden(case)
    ins = [node_arg(d, vals, i) for i in range(len(d["node_inputs"]))]
    y = ops.dispatch("MatMulNBits", ins, d["attrs"])[0]
    assert y.shape == exp["out0"].shape and y.dtype == np.float32
    ok, max_abs, cos = fixture_float_ok(y, exp["out0"])
    assert ok, (max_abs, cos)
    at = d["attrs"]
    ref = refcpu.matmul_nbits(ins[0], ins[1], ins[2], ins[3] if len(ins) > 3 else None,
                              at["K"], at["N"], 4, at["block_size"])
    assert normwise_rel_err(y, ref) <= TOL


def test_single_node_config(ctx):
    # M=1, K=N=1024, block 32, packed zero points
    p = synth.mmnb_problem(1, 1024, 1024, 32, True, seed=0)
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("kn", synth.DECODE_PROJECTIONS)
def test_decode_sweep(ctx, m, kn):
    k, n = kn
    p = synth.mmnb_problem(m, k, n, 128, False, seed=1, scale_range=(0.002, 0.02))
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


@pytest.mark.parametrize("block,zp", [(128, False), (32, True)])
def test_headline_gemv_4096(ctx, block, zp):
    p = synth.mmnb_problem(1, 4096, 4096, block, zp, seed=7)
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


@pytest.mark.parametrize("k,n,block,zp", [(16384, 16384, 128, False), (11008, 4096, 32, True),
                                          (8192, 14336, 64, True), (14336, 4096, 128, False)])
def test_gemv_long_k(ctx, k, n, block, zp):
    # Decode GEMV at full size with K > 4096 (2..4 chunks per lane)
    p = synth.mmnb_problem(1, k, n, block, zp, seed=5 + k // 1024)
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)
    np.testing.assert_array_equal(run_gpu(ctx, p), y)


@pytest.mark.parametrize("m,n,block", [(128, 4096, 32), (128, 4096, 128)])
def test_prefill_full_oracle(ctx, m, n, block):
    p = synth.mmnb_problem(m, 4096, n, block, True, seed=2, outlier_frac=0.01)
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


# Every (M, N, block) of the prefill sweep: M in {128, 512, 2048}, K = 4096,
# N in {4096, 14336}, block 32 and 128 with zero points (the launch shape --
# tile width, K slices -- differs across them).
C3 = [(m, n, b) for m in (128, 512, 2048) for n in (4096, 14336) for b in (32, 128)]


@pytest.mark.parametrize("m,n,block", C3)
def test_prefill_full_size_row_sample(ctx, m, n, block):
    # Rows are independent: the oracle on a sample of rows is the exact
    # reference for those rows of the full-size product.
    p = synth.mmnb_problem(m, 4096, n, block, True, seed=2, outlier_frac=0.01)
    y = run_gpu(ctx, p)
    assert np.all(np.isfinite(y))
    rows = np.array([0, 1, m // 3, m // 2 + 1, m - 2, m - 1])
    ref = oracle(p, rows)
    assert normwise_rel_err(y[rows], ref) <= TOL
    check_bound(p, y[rows], rows)


@pytest.mark.parametrize("m,k,n,block,zp", [
    (1, 40, 5, 32, False),      # partial block, n % 4 != 0 (double tail in the oracle)
    (2, 40, 5, 32, True),
    (3, 200, 37, 64, True),
    (1, 16, 3, 16, True),       # block 16
    (5, 256, 70, 256, False),   # block 256, K == block
    (9, 96, 33, 32, True),      # GEMM path, M not a multiple of the tile
    (65, 1000, 130, 128, True),  # GEMM path, K not a multiple of 64
    (8, 3000, 17, 64, False),
    (1, 4096, 1, 128, True),    # single column
    # M = 1 with K > 4096: several chunks per lane, the next chunk's loads
    # in flight during the current one's arithmetic
    (1, 9000, 33, 128, True),
    (1, 5000, 70, 16, True),    # block 16, K not a multiple of 64
    (1, 12288, 200, 32, False),
    (1, 4160, 9, 64, True),     # one chunk past a 4-wave workgroup's first pass
    # decode GEMV for 2 <= M <= 8 (activations staged in LDS)
    (2, 9000, 33, 128, True),   # K > 4096: several chunk iterations
    (4, 5000, 100, 16, True),   # block 16, iterations
    (7, 1000, 300, 32, True),
    (6, 64, 1000, 64, False),   # one chunk per column, many column groups
    (3, 3072, 1024, 128, False),
    (8, 8192, 40, 64, True),    # A too large for one workgroup's LDS: GEMM path
    # GEMM with K split over two wave groups (few tiles, K >= 1024)
    (64, 2000, 100, 16, True),  # block 16, K not a multiple of 64
    (33, 5000, 130, 256, True),  # block 256: group ranges aligned to 4 segments
    (128, 1024, 256, 512, False),  # block 512: 8 segments per block
    (100, 1100, 96, 32, True),
    # boundaries: the first M on the GEMM path, a small-batch prefill on the
    # headline's weights, one output column, K of a single block
    (9, 1000, 65, 32, True),
    (16, 4096, 4096, 32, True),
    (1, 1024, 1, 32, True),
    (20, 1024, 1, 64, False),
    (12, 16, 5, 16, False),
    (1, 32, 3, 32, True),
])
def test_edge_shapes(ctx, m, k, n, block, zp):
    p = synth.mmnb_problem(m, k, n, block, zp, seed=11 + m + n)
    y = run_gpu(ctx, p)
    assert y.shape == (m, n)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


@pytest.mark.parametrize("m,k,n,block,zp", [
    (100, 4096, 512, 32, True),    # 8 tiles: 8 K slices
    (64, 3072, 1024, 128, False),  # 4 slices (8 would pad K)
    (256, 2048, 1024, 128, True),  # decoder o projection shape: 4 slices
    (256, 1024, 4096, 128, True),  # decoder q|k|v shape: 2 slices
    (64, 2000, 100, 16, True),     # block 16, K not a multiple of 64
])
def test_gemm_k_slices(ctx, m, k, n, block, zp):
    # Few tiles: K is split across workgroups and the last slice of each tile
    # sums the partials in slice order, so repeated calls give the same bits.
    p = synth.mmnb_problem(m, k, n, block, zp, seed=21 + m + k)
    y = run_gpu(ctx, p)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)
    np.testing.assert_array_equal(run_gpu(ctx, p), y)


def test_batched_activation_shape(ctx):
    p = synth.mmnb_problem(6, 256, 48, 32, True, seed=5)
    a3 = p.a.reshape(2, 3, 256)
    y = ops.op_matmul_nbits(a3, p.b_q, p.scales, p.zero_points, k=256, n=48, bits=4,
                            block_size=32, ctx=ctx)
    assert y.shape == (2, 3, 48)
    assert normwise_rel_err(y.reshape(6, 48), oracle(p)) <= TOL


def test_zero_rows_and_tiny_magnitudes(ctx):
    p = synth.mmnb_problem(12, 512, 64, 32, True, seed=9)
    p.a[3] = 0.0
    p.a[5] *= np.float32(1e-30)
    p.a[7] *= np.float32(1e20)
    y = run_gpu(ctx, p)
    ref = oracle(p)
    assert np.all(y[3] == 0.0)
    for r in range(12):
        if r == 3:
            continue
        assert normwise_rel_err(y[r], ref[r]) <= TOL, r


def zero_point_grid(p):
    """[n, n_blocks] zero point of every (column, block): nibble
    col * n_blocks + blk of the packed input, low nibble first, or 8 without
    one (onnx_qlinear_ops.dart:132-137)."""
    nb = p.n_blocks
    if p.zero_points is None:
        return np.full((p.n, nb), 8, np.uint8)
    zi = np.arange(p.n * nb)
    return ((p.zero_points[zi >> 1] >> (4 * (zi & 1))) & 0xF).astype(np.uint8).reshape(p.n, nb)


def prune_to_zero_point(p, seed, dead_cols=0.125, dead_blocks=0.25, keep=None):
    """Sets nibbles to their block's zero point, so that W = (q - zp) * scale
    is exactly 0 there: whole columns (returned), whole (column, block)
    pairs and, with `keep`, all but that fraction of the other weights.
    Padding nibbles past K stay zero."""
    rng = np.random.default_rng(seed)
    n, nb, half = p.b_q.shape
    q = np.stack([p.b_q & 0xF, p.b_q >> 4], -1).reshape(n, nb, 2 * half)
    z = np.broadcast_to(zero_point_grid(p)[:, :, None], q.shape)
    dead = rng.random(q.shape) >= (1.0 if keep is None else keep)
    dead |= (rng.random((n, nb)) < dead_blocks)[:, :, None]
    cols = np.flatnonzero(rng.random(n) < dead_cols)
    dead[cols] = True
    q = np.where(dead, z, q)
    q = q.reshape(n, nb * 2 * half)
    q[:, p.k:] = 0
    q = q.reshape(n, nb, half, 2)
    p.b_q = (q[..., 0] | (q[..., 1] << 4)).astype(np.uint8)
    return cols


@pytest.mark.parametrize("m", [1, 4, 64])
@pytest.mark.parametrize("block,zp", [(128, False), (32, True), (64, True)])
@pytest.mark.parametrize("keep", [None, 0.001], ids=["blocks", "sparse"])
def test_weights_equal_to_zero_point(ctx, m, block, zp, keep):
    # Pruned weights: columns and blocks whose nibbles all equal the zero
    # point give W = 0 exactly in the reference, and so exactly 0 here; the
    # accumulation bound (sum |a||W| is small) catches a zero point folded in
    # after the products (scale * sum a q - scale * zp * sum a).
    p = synth.mmnb_problem(m, 4096, 512, block, zp, seed=31 + m + block)
    cols = prune_to_zero_point(p, seed=block + m, keep=keep)
    assert cols.size > 0
    y = run_gpu(ctx, p)
    assert np.all(y[:, cols] == 0.0)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


@pytest.mark.parametrize("k,block,zp", [(9000, 128, True), (12288, 32, False)])
def test_weights_equal_to_zero_point_long_k(ctx, k, block, zp):
    p = synth.mmnb_problem(1, k, 300, block, zp, seed=41)
    cols = prune_to_zero_point(p, seed=k, keep=0.002)
    y = run_gpu(ctx, p)
    assert np.all(y[:, cols] == 0.0)
    assert normwise_rel_err(y, oracle(p)) <= TOL
    check_bound(p, y)


def test_all_zero_nibbles_closed_form(ctx):
    # q = 0, zero point 8 -> W = -8 * scale: y = -8 * sum_k a_k scale[n, blk(k)]
    k, n, bs = 256, 16, 64
    nb = k // bs
    b = np.zeros((n, nb, bs // 2), np.uint8)
    s = np.random.default_rng(1).uniform(0.1, 1, (n, nb)).astype(np.float32)
    a = np.random.default_rng(2).standard_normal((3, k)).astype(np.float32)
    y = ops.op_matmul_nbits(a, b, s, None, k=k, n=n, bits=4, block_size=bs, ctx=ctx)
    want = -8.0 * (a.astype(np.float64).reshape(3, nb, bs).sum(-1) @ s.T.astype(np.float64))
    assert normwise_rel_err(y, want) <= TOL


def test_device_entry_point_matches_host_entry_point(ctx):
    # K a multiple of 64 (aligned path) and not (masked path)
    for (m, k, n, bs) in [(1, 1024, 256, 32), (4, 1000, 96, 8 * 16), (24, 320, 200, 64),
                          (5, 1001, 64, 32), (2, 4097, 48, 128)]:
        p = synth.mmnb_problem(m, k, n, bs, True, seed=k)
        pack = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4,
                              block_size=bs, ctx=ctx)
        da = ctx.to_device(p.a)
        dy = ctx.alloc(m * n * 4)
        _lib.check(ctx.lib.mmnb_matmul_nbits_dev(ctx.handle, pack.handle, da.ptr, m, dy.ptr))
        ctx.synchronize()
        y_dev = dy.numpy(np.float32, (m, n))
        y_host = run_gpu(ctx, p)
        np.testing.assert_array_equal(y_dev, y_host)
        da.free()
        dy.free()
        pack.free()


def test_pack_is_cached_and_resident(ctx):
    p = synth.mmnb_problem(1, 512, 128, 32, True, seed=3)
    ops.clear_pack_cache()
    y1 = run_gpu(ctx, p)
    y2 = run_gpu(ctx, p)
    np.testing.assert_array_equal(y1, y2)  # deterministic, same resident pack
    assert len(ops._CACHE._packs) == 1


def test_argument_errors(ctx):
    p = synth.mmnb_problem(1, 64, 8, 32, False, seed=3)
    with pytest.raises(ValueError):  # B too short
        ops.pack_nbits(p.b_q[:4], p.scales, None, k=64, n=8, bits=4, block_size=32, ctx=ctx)
    with pytest.raises(ValueError):  # scales too short
        ops.pack_nbits(p.b_q, p.scales[:2], None, k=64, n=8, bits=4, block_size=32, ctx=ctx)
    with pytest.raises(NotImplementedError):  # odd block size (the oracle refuses it too)
        ops.pack_nbits(np.zeros((8, 3, 1), np.uint8), np.ones(24, np.float32), None, k=9, n=8,
                       bits=4, block_size=3, ctx=ctx)
    with pytest.raises(NotImplementedError):  # block size 0
        ops.pack_nbits(p.b_q, p.scales, None, k=64, n=8, bits=4, block_size=0, ctx=ctx)
    with pytest.raises(ValueError):  # A's last dim != K
        ops.op_matmul_nbits(np.zeros((1, 63), np.float32), p.b_q, p.scales, None, k=64, n=8,
                            bits=4, block_size=32, ctx=ctx)


# ---------------------------------------------------------------------------
# Every even block size the reference accepts (onnx_qlinear_ops.dart:120-146).
# Multiples of 16 that are not powers of two run the fast kernels on a
# re-blocked pack (same tolerance and bound as above); the other even sizes
# run the generic kernel, which keeps the reference's per-weight rounding and
# k order: its results must equal the oracle bit for bit (including the
# double-precision tail columns of the M = 1 path when N % 4 != 0).
REBLOCKED = [48, 80, 96, 192, 320]
GENERIC = [2, 4, 6, 8, 10, 12, 14, 18, 20, 24, 30, 1000]


@pytest.mark.parametrize("block", REBLOCKED + GENERIC)
@pytest.mark.parametrize("m", [1, 3, 20])
@pytest.mark.parametrize("zp", [False, True])
def test_any_even_block_size(ctx, block, m, zp):
    k, n = 1000, 150  # K not a multiple of any block here but 2, 4, 8, 10, 20, 1000; N % 4 = 2
    p = synth.mmnb_problem(m, k, n, block, zp, seed=block * 7 + m)
    y = run_gpu(ctx, p)
    ref = oracle(p)
    if block in GENERIC:
        np.testing.assert_array_equal(y, ref)
    else:
        assert normwise_rel_err(y, ref) <= TOL
        check_bound(p, y)


@pytest.mark.parametrize("block", [48, 8])
def test_block_sizes_through_dispatch(ctx, block):
    # the MatMulNBits arm (onnx_graph.dart:1584-1596) with block sizes that are
    # not powers of two; M = 70 takes the prefill path, M = 1 the decode path
    for m in (1, 70):
        p = synth.mmnb_problem(m, 640, 96, block, True, seed=block + m)
        ins = [p.a.reshape(1, m, 640), p.b_q, p.scales, p.zero_points]
        y = ops.dispatch("MatMulNBits", ins, {"K": 640, "N": 96, "block_size": block})[0]
        assert y.shape == (1, m, 96) and y.dtype == np.float32
        ref = oracle(p)
        if block % 16:
            np.testing.assert_array_equal(y.reshape(m, 96), ref)
        else:
            assert normwise_rel_err(y.reshape(m, 96), ref) <= TOL


def test_reblocked_pack_equals_power_of_two_pack(ctx):
    # block 48 with every reference block's three 16-k thirds given the same
    # scale / zero point is the block-16 problem with repeated scales: the
    # re-blocked pack must give exactly the block-16 pack's bits
    k, n, m = 960, 64, 24
    p48 = synth.mmnb_problem(m, k, n, 48, True, seed=5)
    nb48 = k // 48
    s16 = np.repeat(p48.scales.reshape(n, nb48), 3, axis=1)
    zi = np.arange(n * nb48)
    z48 = (p48.zero_points[zi >> 1] >> (4 * (zi & 1))) & 0xF
    z16 = np.repeat(z48.reshape(n, nb48), 3, axis=1).ravel()
    zp16 = np.zeros((z16.size + 1) // 2, np.uint8)
    np.bitwise_or.at(zp16, np.arange(z16.size) >> 1, (z16 << (4 * (np.arange(z16.size) & 1))).astype(np.uint8))
    b16 = p48.b_q.reshape(n, k // 2).reshape(n, k // 16, 8)
    for mm in (1, m):
        y48 = ops.op_matmul_nbits(p48.a[:mm], p48.b_q, p48.scales, p48.zero_points, k=k, n=n,
                                  bits=4, block_size=48, ctx=ctx)
        y16 = ops.op_matmul_nbits(p48.a[:mm], b16, s16, zp16, k=k, n=n, bits=4, block_size=16,
                                  ctx=ctx)
        np.testing.assert_array_equal(y48, y16)


# ---------------------------------------------------------------------------
# Non-finite activations: the reference forms each a * W in binary32, so a row
# holding +-inf gives +-inf in a column where every infinite term has the same
# sign, and NaN where W is 0 at an infinite a (inf * 0), where infinite terms
# of both signs meet, or where the row holds a NaN (onnx_qlinear_ops.dart:146,
# gemm_kernel_simd.dart:89-104).  The GPU must give the same pattern; the
# finite rows keep the usual tolerance.
def check_non_finite(y, ref, bad_rows):
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    assert np.array_equal(np.isposinf(y), np.isposinf(ref))
    assert np.array_equal(np.isneginf(y), np.isneginf(ref))
    good = np.setdiff1d(np.arange(y.shape[0]), bad_rows)
    assert normwise_rel_err(y[good], ref[good]) <= TOL


@pytest.mark.parametrize("m", [1, 4, 64])
@pytest.mark.parametrize("block,zp", [(32, True), (128, False)])
def test_non_finite_activations(ctx, m, block, zp):
    k, n = 1024, 96
    p = synth.mmnb_problem(m, k, n, block, zp, seed=m + block)
    # W = 0 at k = 17 for a third of the columns (nibble = the block's zero
    # point), so an infinite a[., 17] yields NaN there and +-inf elsewhere
    zg = zero_point_grid(p)
    q = np.stack([p.b_q & 0xF, p.b_q >> 4], -1).reshape(n, -1)
    cols0 = np.arange(0, n, 3)
    q[cols0, 17] = zg[cols0, 17 // block]
    q = q.reshape(n, p.n_blocks, block // 2, 2)
    p.b_q = (q[..., 0] | (q[..., 1] << 4)).astype(np.uint8)
    bad = [0]
    p.a[0, 17] = np.inf
    if m > 1:
        p.a[1, 100] = -np.inf
        p.a[1, 700] = np.inf    # both signs in one row
        p.a[2, 5] = np.nan
        p.a[3, 17] = -np.inf
        bad = [0, 1, 2, 3]
    y = run_gpu(ctx, p)
    ref = oracle(p)
    assert np.isnan(ref[0, cols0]).all() and np.isinf(np.delete(ref[0], cols0)).any()
    check_non_finite(y, ref, bad)


@pytest.mark.parametrize("m", [1, 4, 32])
@pytest.mark.parametrize("block,zp", [(32, True), (128, False)])
def test_large_magnitude_activations(ctx, m, block, zp):
    # rows far from 1 in magnitude: the GEMVs carry a power of two in their
    # per-weight values (8 (q - zp) with zero points, (q - 8) / 16 without)
    # and fold its inverse into each block's scale, so the sums range like
    # the reference's terms; the GEMM scales every row by a power of two
    p = synth.mmnb_problem(m, 2048, 64, block, zp, seed=13 + m)
    f = np.array([1e33, 1e-33, 1e30, 1e-30] * m, np.float32)[:m]
    p.a *= f[:, None]
    y = run_gpu(ctx, p)
    ref = oracle(p)
    for r in range(m):
        assert normwise_rel_err(y[r], ref[r]) <= TOL, r
