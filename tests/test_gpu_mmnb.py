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
    with pytest.raises(NotImplementedError):  # block size not a power of two
        ops.pack_nbits(p.b_q, p.scales, None, k=64, n=8, bits=4, block_size=48, ctx=ctx)
    with pytest.raises(ValueError):  # A's last dim != K
        ops.op_matmul_nbits(np.zeros((1, 63), np.float32), p.b_q, p.scales, None, k=64, n=8,
                            bits=4, block_size=32, ctx=ctx)
