"""The allocation-free MatMulNBits entry point (mmnb_matmul_nbits_dev_noalloc)
against mmnb_matmul_nbits_dev, through the C ABI: the same kernels on a
fixed workspace instead of the context's grow-only scratch, so the results
must be identical bit for bit.  Two calls in a row per case, the second with
a smaller input (the workspace keeps the first call's contents), and the
GEMV, the plain GEMM and the K-sliced GEMM (whose tile counters live in the
workspace) all covered."""
import numpy as np
import pytest

from onnx_runtime_dart_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


def _run(ctx, fn, pack, a):
    m, k = a.shape
    da = ctx.to_device(np.ascontiguousarray(a))
    dy = ctx.alloc(m * pack.n * 4)
    try:
        _lib.check(fn(ctx.handle, pack.handle, da.ptr, m, dy.ptr))
        ctx.synchronize()
        return dy.numpy(np.float32, (m, pack.n))
    finally:
        da.free()
        dy.free()


@pytest.mark.parametrize("k,n,block,zp,ms", [
    (4096, 4096, 32, True, (512, 130)),    # GEMM, then a smaller GEMM
    (4096, 512, 32, True, (100, 40)),      # K-sliced GEMM (8 tiles), then fewer rows
    (1024, 3072, 128, False, (64, 1)),     # GEMM, then the M = 1 GEMV
    (3000, 700, 64, True, (8, 3)),         # multi-row GEMV, K not a multiple of 64
    (8192, 40, 64, True, (8, 5)),          # rows too long for the GEMV's LDS: the GEMM
])
def test_noalloc_matches_dev_entry_point(ctx, k, n, block, zp, ms):
    p = synth.mmnb_problem(max(ms), k, n, block, zp, seed=k + n)
    pack = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4, block_size=block,
                          ctx=ctx)
    try:
        for m in ms:  # second call smaller than the first
            a = p.a[:m]
            want = _run(ctx, ctx.lib.mmnb_matmul_nbits_dev, pack, a)
            got = _run(ctx, ctx.lib.mmnb_matmul_nbits_dev_noalloc, pack, a)
            np.testing.assert_array_equal(got, want)
            assert np.all(np.isfinite(got))
    finally:
        pack.free()


def test_noalloc_repeat_calls_identical(ctx):
    # K slices: the counters the last slice resets must start the next call
    # at zero, so back-to-back calls give the same bits
    p = synth.mmnb_problem(64, 3072, 1024, 128, False, seed=7)
    pack = ops.pack_nbits(p.b_q, p.scales, None, k=3072, n=1024, bits=4, block_size=128, ctx=ctx)
    try:
        first = _run(ctx, ctx.lib.mmnb_matmul_nbits_dev_noalloc, pack, p.a)
        for _ in range(3):
            np.testing.assert_array_equal(
                _run(ctx, ctx.lib.mmnb_matmul_nbits_dev_noalloc, pack, p.a), first)
    finally:
        pack.free()


def test_noalloc_rejects_oversized_and_extended(ctx):
    assert ctx.lib.mmnb_noalloc_workspace_bytes() == 64 << 20
    k, n = 4096, 64
    p = synth.mmnb_problem(1, k, n, 128, False, seed=3)
    pack = ops.pack_nbits(p.b_q, p.scales, None, k=k, n=n, bits=4, block_size=128, ctx=ctx)
    m = 8192  # prepared activations alone: 8192 x 4096 x 4 bytes > 64 MiB
    da = ctx.alloc(m * k * 4)
    dy = ctx.alloc(m * n * 4)
    try:
        with pytest.raises(NotImplementedError):
            _lib.check(ctx.lib.mmnb_matmul_nbits_dev_noalloc(ctx.handle, pack.handle, da.ptr, m,
                                                              dy.ptr))
    finally:
        da.free()
        dy.free()
        pack.free()
    bias = np.ones(n, np.float32)
    xp = ops.pack_nbits_ex(p.b_q, p.scales.ravel(), None, None, bias, k=k, n=n, bits=4,
                           block_size=128, ctx=ctx)
    da, dy = ctx.alloc(k * 4), ctx.alloc(n * 4)
    try:
        with pytest.raises(NotImplementedError):
            _lib.check(ctx.lib.mmnb_matmul_nbits_dev_noalloc(ctx.handle, xp.handle, da.ptr, 1,
                                                              dy.ptr))
    finally:
        da.free()
        dy.free()
        xp.free()


def test_noalloc_first_call_inside_graph_capture():
    # A fresh context (no scratch ever grown) whose FIRST MatMulNBits calls
    # are made under HIP graph capture through the no-alloc entry point: a
    # K-sliced GEMM (tile counters in the workspace, cleared by the prep
    # kernel) and an M <= 8 call that falls back to the GEMM (rows too long
    # for the multi-row GEMV's LDS; a GEMM of more than 64 KB of LDS, so a
    # hipFuncSetAttribute while capturing).  Nothing may allocate during capture; every replay,
    # with eager work and synchronisations in between, must give the bits of
    # mmnb_matmul_nbits_dev run outside capture.
    c = _lib.Context(0)
    cases = [(100, 4096, 512, 32, True), (5, 8192, 40, 64, True)]
    packs, bufs = [], []
    try:
        for m, k, n, block, zp in cases:
            p = synth.mmnb_problem(m, k, n, block, zp, seed=k + m)
            pk = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4,
                                block_size=block, ctx=c)
            da, dy = c.to_device(p.a), c.alloc(m * n * 4)
            packs.append(pk)
            bufs.append((m, n, da, dy))
        c.synchronize()
        c.graph_begin()
        for pk, (m, n, da, dy) in zip(packs, bufs):
            _lib.check(c.lib.mmnb_matmul_nbits_dev_noalloc(c.handle, pk.handle, da.ptr, m,
                                                            dy.ptr))
        g = c.graph_end()
        try:
            want = []
            for pk, (m, n, da, dy) in zip(packs, bufs):
                want.append(_run(c, c.lib.mmnb_matmul_nbits_dev, pk, da.numpy(np.float32,
                                                                              (m, pk.k))))
            for rep in range(3):
                for (m, n, da, dy) in bufs:
                    dy.upload(np.full((m, n), np.nan, np.float32))
                c.graph_launch(g)
                c.synchronize()
                for w, (m, n, da, dy) in zip(want, bufs):
                    np.testing.assert_array_equal(dy.numpy(np.float32, (m, n)), w, err_msg=str(rep))
                # eager work between replays (the entry points outside the graph)
                _run(c, c.lib.mmnb_matmul_nbits_dev_noalloc, packs[0],
                     bufs[0][2].numpy(np.float32, (bufs[0][0], packs[0].k)))
        finally:
            c.graph_destroy(g)
    finally:
        for (m, n, da, dy) in bufs:
            da.free()
            dy.free()
        for pk in packs:
            pk.free()
        c.close()
