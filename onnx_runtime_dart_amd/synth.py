"""Seeded synthetic tensors for the benchmark workloads and the parity tests.

Each tensor of a workload draws from its own ``numpy.random.default_rng``
stream seeded ``base_seed * 1000 + tensor_index``, so every tensor is
reproducible on its own:

* single node:  A ~ N(0,1) [1,1024]; nibbles uniform 0..15 packed
  [1024, 32, 16]; scales ~ U(0.005, 0.02) [1024, 32]; packed uint4 zero
  points [1024*32/2] uniform.
* decode GEMV:  M in {1,4,8}, block 128, symmetric (no zero-point input),
  scales ~ U(0.002, 0.02).
* prefill GEMM: M in {128, 512, 2048}, random packed zero points, A ~ N(0,1)
  with 1% of the K columns scaled by 20.
* int8 chain:   x ~ N(0,1) [512, 1024]; B int8 uniform in [-127, 127]
  [1024, 3072]; b_zero_point 0.
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np


def _rng(seed, idx):
    return np.random.default_rng(seed * 1000 + idx)


@dataclass
class MmnbProblem:
    a: np.ndarray            # float32 [m, k]
    b_q: np.ndarray          # uint8 [n, n_blocks, block/2]
    scales: np.ndarray       # float32 [n, n_blocks]
    zero_points: Optional[np.ndarray]  # uint8 [ceil(n*n_blocks/2)] or None
    m: int
    k: int
    n: int
    block: int

    @property
    def n_blocks(self):
        return (self.k + self.block - 1) // self.block

    def weight_bytes(self):
        zb = 0 if self.zero_points is None else self.zero_points.nbytes
        return self.b_q.nbytes + self.scales.nbytes + zb


def mmnb_weights(k, n, block, zp, seed, scale_range=(0.005, 0.02)):
    nb = (k + block - 1) // block
    b_q = _rng(seed, 1).integers(0, 256, size=(n, nb, block // 2), dtype=np.uint8)
    if k % block:
        # nibbles past k in the last blob are padding (zero, as ORT packs)
        valid = k - (nb - 1) * block
        tail = b_q[:, -1, :]
        keep = np.zeros(block // 2, dtype=np.uint8)
        keep[: valid // 2] = 0xFF
        if valid % 2:
            keep[valid // 2] = 0x0F
        b_q[:, -1, :] = tail & keep
    lo, hi = scale_range
    scales = _rng(seed, 2).uniform(lo, hi, size=(n, nb)).astype(np.float32)
    zps = None
    if zp:
        zps = _rng(seed, 3).integers(0, 256, size=((n * nb + 1) // 2,), dtype=np.uint8)
        if (n * nb) % 2:
            zps[-1] &= 0x0F
    return b_q, scales, zps


def activations(m, k, seed, outlier_frac=0.0, outlier_scale=20.0):
    a = _rng(seed, 0).standard_normal((m, k)).astype(np.float32)
    if outlier_frac > 0:
        cols = _rng(seed, 4).choice(k, size=max(1, int(round(k * outlier_frac))),
                                    replace=False)
        a[:, cols] *= np.float32(outlier_scale)
    return a


def mmnb_problem(m, k, n, block, zp, seed, scale_range=(0.005, 0.02),
                 outlier_frac=0.0):
    b_q, scales, zps = mmnb_weights(k, n, block, zp, seed, scale_range)
    a = activations(m, k, seed, outlier_frac)
    return MmnbProblem(a, b_q, scales, zps, m, k, n, block)


def int8_chain_problem(m=512, k=1024, n=3072, seed=3):
    x = _rng(seed, 0).standard_normal((m, k)).astype(np.float32)
    b = _rng(seed, 1).integers(-127, 128, size=(k, n)).astype(np.int8)
    return x, b


# Decode-shape projections of the decode sweep: (K, N)
DECODE_PROJECTIONS = [(1024, 2048), (1024, 1024), (1024, 6144), (3072, 1024)]
