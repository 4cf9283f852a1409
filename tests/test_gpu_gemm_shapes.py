"""The prefill GEMM under every launch shape it can take, against the oracle.

The library picks the tile width (128 or 256 columns), the LDS stages and the
number of K slices from the problem size; the MMNB_GEMM_* variables (read
when a context is created) force each choice, so every combination is
checked on shapes where the automatic choice would not take it.  Bar as in
test_gpu_mmnb.py: normwise relative error <= 1e-5 against the oracle, and
repeated calls give the same bits.
"""
import os

import numpy as np
import pytest

from oracle import refcpu
from onnx_runtime_dart_amd import _lib, ops, synth
from onnx_runtime_dart_amd._lib import check, ptr
from tests.helpers import normwise_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
THREADS = min(16, refcpu.host_threads())
SHAPES = [(64, 1024, 512, 32, True), (100, 2048, 300, 128, False), (192, 4096, 768, 64, True)]


@pytest.fixture(scope="module", params=[(1, 1, 2), (1, 2, 2), (1, 8, 2), (2, 1, 2), (2, 2, 2),
                                        (2, 4, 2), (1, 1, 3), (1, 4, 3)],
                ids=lambda p: f"cb{p[0]}-ks{p[1]}-st{p[2]}")
def forced_ctx(request):
    cb, ks, st = request.param
    names = ("MMNB_GEMM_CB", "MMNB_GEMM_KSPLIT", "MMNB_GEMM_STAGES")
    saved = {k: os.environ.get(k) for k in names}
    os.environ.update({"MMNB_GEMM_CB": str(cb), "MMNB_GEMM_KSPLIT": str(ks),
                       "MMNB_GEMM_STAGES": str(st)})
    try:
        ctx = _lib.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    yield ctx
    ctx.close()


@pytest.mark.parametrize("m,k,n,block,zp", SHAPES)
def test_forced_launch_shapes(forced_ctx, m, k, n, block, zp):
    p = synth.mmnb_problem(m, k, n, block, zp, seed=31 + m + n, outlier_frac=0.01)
    pack = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4, block_size=block,
                          ctx=forced_ctx)
    try:
        def run():
            y = np.empty(m * n, np.float32)
            check(forced_ctx.lib.mmnb_matmul_nbits(forced_ctx.handle, pack.handle, ptr(p.a), m,
                                                   ptr(y)))
            return y.reshape(m, n)
        y = run()
        ref = refcpu.matmul_nbits(p.a, p.b_q, p.scales, p.zero_points, k, n, 4, block,
                                  threads=THREADS)
        assert normwise_rel_err(y, ref) <= TOL
        np.testing.assert_array_equal(run(), y)
    finally:
        pack.free()
