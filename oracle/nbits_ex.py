"""CPU oracle of MatMulNBits with the inputs ORT exports use and the
reference rejects: bits = 8, g_idx, bias, float zero points, fp16 scales,
the per-column zero-point layout.

TEST INFRASTRUCTURE ONLY: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it.

The reference (lib/src/onnx_qlinear_ops.dart:114-156) implements bits = 4
with flat uint8 zero points only.  This restates the ORT contrib operator's
published definition (com.microsoft MatMulNBits: inputs A, B, scales,
zero_points, g_idx, bias; W[k, n] = (q[n, k] - zp[n, g]) * scale[n, g] with
g = g_idx[k], else k / block_size; Y = A W + bias) with the reference's own
arithmetic where they overlap: the dequantised weight rounded once to
binary32, the k-sequential fp32 GEMM of refcpu.matmul_kernel, the bias added
in binary32.  With bits = 4, flat uint8 zero points and neither g_idx nor
bias it is bit-identical to refcpu.matmul_nbits (tested).
"""
import numpy as np

from oracle import refcpu


def unpack_q(b_q, k, n, bits, block):
    """q[n, k] from B [n, ceil(k/bs), bs*bits/8] (low nibble first)."""
    nb = (k + block - 1) // block
    b = np.asarray(b_q, np.uint8).reshape(n, nb, block * bits // 8)
    if bits == 8:
        q = b.reshape(n, nb * block).astype(np.int64)
    else:
        q = np.stack([b & 0xF, b >> 4], axis=-1).reshape(n, nb * block).astype(np.int64)
    return q[:, :k]


def zero_points_per_block(zero_points, n, nb, bits):
    """zp[n, nb] as float64: default 8 / 128; uint8 packed (1-D: the
    reference's flat nibble order; 2-D: one byte row per column, ORT's
    layout); float / fp16 values as given."""
    if zero_points is None:
        return np.full((n, nb), 8.0 if bits == 4 else 128.0)
    z = np.asarray(zero_points)
    if z.dtype != np.uint8:
        return z.astype(np.float32).astype(np.float64).reshape(n, nb)
    if bits == 8:
        return z.reshape(n, nb).astype(np.float64)
    if z.ndim == 2:
        row = z.reshape(n, -1)
        nib = np.stack([row & 0xF, row >> 4], axis=-1).reshape(n, -1)[:, :nb]
        return nib.astype(np.float64)
    flat = z.ravel()
    idx = np.arange(n * nb)
    nib = np.where(idx % 2 == 0, flat[idx >> 1] & 0xF, flat[idx >> 1] >> 4)
    return nib.reshape(n, nb).astype(np.float64)


def dequant(b_q, scales, zero_points, g_idx, k, n, bits, block):
    """W^T [k, n] fp32: fl32((q - zp) * scale) per element."""
    nb = (k + block - 1) // block
    q = unpack_q(b_q, k, n, bits, block).astype(np.float64)
    s = np.asarray(scales).astype(np.float32).astype(np.float64).reshape(n, nb)
    z = zero_points_per_block(zero_points, n, nb, bits)
    g = np.arange(k) // block if g_idx is None else np.asarray(g_idx, np.int64).ravel()
    w = (q - z[:, g]) * s[:, g]                      # exact in double for integer zp
    return np.ascontiguousarray(w.astype(np.float32).T)


def matmul_nbits_ex(a, b_q, scales, zero_points, g_idx, bias, k, n, bits, block):
    a = np.ascontiguousarray(a, np.float32)
    m = a.size // k
    wt = dequant(b_q, scales, zero_points, g_idx, k, n, bits, block)
    y = refcpu.matmul_kernel(a.reshape(m, k), wt, m, k, n)
    if bias is not None:
        y = (y + np.asarray(bias).astype(np.float32).reshape(1, n)).astype(np.float32)
    return y.reshape(list(a.shape[:-1]) + [n])


def matmul_nbits_ex_f64(a, b_q, scales, zero_points, g_idx, bias, k, n, bits, block):
    """fp64 product with the binary32 dequantised weights, and sum|a||W| per
    output (the accumulation bound's scale)."""
    a = np.asarray(a, np.float64).reshape(-1, k)
    wt = dequant(b_q, scales, zero_points, g_idx, k, n, bits, block).astype(np.float64)
    y = a @ wt
    absdot = np.abs(a) @ np.abs(wt)
    if bias is not None:
        b = np.asarray(bias).astype(np.float32).astype(np.float64).reshape(1, n)
        y = y + b
        absdot = absdot + np.abs(b)
    return y, absdot
