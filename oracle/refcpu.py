"""ctypes front end of the CPU oracle (``oracle/librefcpu.so``).

TEST INFRASTRUCTURE ONLY: the oracle is the parity checker for the GPU
kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product package never does.

Every function restates the reference Dart arithmetic; see ``refcpu.c`` for
the file:line each one follows.
"""
import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "librefcpu.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
REF_ERR_UNSUPPORTED = -2  # refcpu.c: the reference throws UnsupportedError


def build():
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.ref_matmul_nbits.argtypes = [_f32p, _i64, _u8p, _f32p, _vp, _i64,
                                       _i64, _i64, _i64, _f32p]
        L.ref_matmul_nbits.restype = ctypes.c_int
        L.ref_matmul_nbits_mt.argtypes = [_f32p, _i64, _u8p, _f32p, _vp, _i64,
                                          _i64, _i64, _i64, _f32p, ctypes.c_int]
        L.ref_matmul_nbits_mt.restype = ctypes.c_int
        L.ref_matmul_nbits_f64.argtypes = [_f32p, _i64, _u8p, _f32p, _vp,
                                           _i64, _i64, _i64, _f64p, _f64p]
        L.ref_matmul_nbits_f64.restype = ctypes.c_int
        L.ref_mmnb_dequant.argtypes = [_u8p, _f32p, _vp, _i64, _i64, _i64, _f32p]
        L.ref_mmnb_dequant.restype = None
        L.ref_matmul_kernel.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64]
        L.ref_matmul_kernel.restype = ctypes.c_int
        L.ref_dql.argtypes = [_f32p, _i64, _u8p, ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_int64)]
        L.ref_dql.restype = ctypes.c_int
        L.ref_matmul_integer.argtypes = [_u8p, ctypes.c_int, _i64, _i64, _i64,
                                         _u8p, ctypes.c_int, _i64, _i64,
                                         _vp, _i64, _vp, _i64, _i64p]
        L.ref_matmul_integer.restype = ctypes.c_int
        L.ref_rescale.argtypes = [_i64p, _i64, _i64, ctypes.c_float, _f32p,
                                  _i64, _f32p]
        L.ref_rescale.restype = None
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _zp_ptr(zp):
    if zp is None:
        return None, None
    z = np.ascontiguousarray(zp, dtype=np.uint8).ravel()
    return z, z.ctypes.data_as(_vp)


def matmul_nbits(a, b_q, scales, zero_points, k, n, bits=4, block_size=32,
                 threads=1):
    """Reference ``opMatMulNBits`` (onnx_qlinear_ops.dart:114-156).

    ``a`` is any-shaped fp32 whose length is a multiple of ``k``; returns
    ``[..., n]`` fp32 bit-identical to the Dart native path."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    m = a.size // k
    af = a.ravel()[: m * k].copy()
    b = np.ascontiguousarray(b_q, dtype=np.uint8).ravel()
    s = np.ascontiguousarray(scales, dtype=np.float32).ravel()
    z, zp_p = _zp_ptr(zero_points)
    out = np.zeros(m * n, dtype=np.float32)
    if threads > 1:
        rc = lib().ref_matmul_nbits_mt(af, m, b, s, zp_p, k, n, bits,
                                       block_size, out, threads)
    else:
        rc = lib().ref_matmul_nbits(af, m, b, s, zp_p, k, n, bits, block_size,
                                    out)
    if rc != 0:
        raise OracleError(f"ref_matmul_nbits failed ({rc})")
    shape = list(a.shape[:-1]) + [n] if a.ndim >= 1 else [n]
    return out.reshape(shape)


def matmul_nbits_f64(a, b_q, scales, zero_points, k, n, block_size):
    """fp64 product of A with the reference's binary32 dequantized weights,
    plus sum |a||W| per output (for the gamma_K accumulation bound)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    m = a.size // k
    af = a.ravel()[: m * k].copy()
    b = np.ascontiguousarray(b_q, dtype=np.uint8).ravel()
    s = np.ascontiguousarray(scales, dtype=np.float32).ravel()
    z, zp_p = _zp_ptr(zero_points)
    y = np.zeros(m * n, dtype=np.float64)
    ad = np.zeros(m * n, dtype=np.float64)
    rc = lib().ref_matmul_nbits_f64(af, m, b, s, zp_p, k, n, block_size, y, ad)
    if rc != 0:
        raise OracleError(f"ref_matmul_nbits_f64 failed ({rc})")
    return y.reshape(m, n), ad.reshape(m, n)


def dequant(b_q, scales, zero_points, k, n, block_size):
    """W^T [k, n] fp32 exactly as onnx_qlinear_ops.dart:127-149 builds it."""
    b = np.ascontiguousarray(b_q, dtype=np.uint8).ravel()
    s = np.ascontiguousarray(scales, dtype=np.float32).ravel()
    z, zp_p = _zp_ptr(zero_points)
    bt = np.zeros(k * n, dtype=np.float32)
    lib().ref_mmnb_dequant(b, s, zp_p, k, n, block_size, bt)
    return bt.reshape(k, n)


def matmul_kernel(a, b, m, k, n):
    """The fp32 GEMM of gemm_kernel_simd.dart:27-309 (bit-faithful order)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()
    out = np.zeros(m * n, dtype=np.float32)
    rc = lib().ref_matmul_kernel(a, b, out, m, k, n)
    if rc != 0:
        raise OracleError(f"ref_matmul_kernel failed ({rc})")
    return out.reshape(m, n)


def dynamic_quantize_linear(x):
    """Reference ``opDynamicQuantizeLinear`` (onnx_ops.dart:2556-2583):
    returns (y uint8 same shape, scale float32, zero_point int)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    xf = x.ravel().copy()
    y = np.zeros(xf.size, dtype=np.uint8)
    sc = ctypes.c_float(0.0)
    zp = ctypes.c_int64(0)
    rc = lib().ref_dql(xf, xf.size, y, ctypes.byref(sc), ctypes.byref(zp))
    if rc == REF_ERR_UNSUPPORTED:
        # the reference's _roundEven calls toInt() on a NaN / infinite quotient
        raise NotImplementedError("DynamicQuantizeLinear: NaN or infinite input")
    return y.reshape(x.shape), np.float32(sc.value), int(zp.value)


def matmul_integer(a, b, a_zp=None, b_zp=None):
    """Reference ``opMatMulInteger`` (onnx_qlinear_ops.dart:30-79).

    ``a``/``b`` are uint8 or int8 numpy arrays of rank >= 2; zero points are
    None, scalars, per-row [M] (A) or per-column [N] (B).  Returns int64."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype not in (np.uint8, np.int8) or b.dtype not in (np.uint8, np.int8):
        raise TypeError("MatMulInteger operands must be uint8 or int8")
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    if b.shape[-2] != k:
        raise ValueError("MatMulInteger inner dim mismatch")
    a_batch = a.size // (m * k) if m * k else 1
    b_batch = b.size // (k * n) if k * n else 1
    batch = max(a_batch, b_batch)
    az = None if a_zp is None else np.ascontiguousarray(
        np.asarray(a_zp).astype(np.int64).ravel())
    bz = None if b_zp is None else np.ascontiguousarray(
        np.asarray(b_zp).astype(np.int64).ravel())
    out = np.zeros(batch * m * n, dtype=np.int64)
    rc = lib().ref_matmul_integer(
        a.view(np.uint8).ravel(), int(a.dtype == np.int8), a_batch, m, k,
        b.view(np.uint8).ravel(), int(b.dtype == np.int8), b_batch, n,
        None if az is None else az.ctypes.data_as(_vp), 0 if az is None else az.size,
        None if bz is None else bz.ctypes.data_as(_vp), 0 if bz is None else bz.size,
        out)
    if rc == -2:
        raise NotImplementedError("MatMulInteger: zero points must be scalar, "
                                  "per-row [M] for A or per-column [N] for B")
    if rc != 0:
        raise OracleError(f"ref_matmul_integer failed ({rc})")
    batch_shape = a.shape[:-2] if a_batch >= b_batch else b.shape[:-2]
    return out.reshape(list(batch_shape) + [m, n])


def rescale(acc, a_scale, b_scale):
    """Cast(to=FLOAT) -> Mul(a_scale, b_scale) -> Mul of the dynamic-quant
    export pattern: fl32(fl32(acc) * fl32(a_scale * b_scale[j]))."""
    acc = np.ascontiguousarray(acc, dtype=np.int64)
    n = acc.shape[-1]
    rows = acc.size // n if n else 0
    bs = np.ascontiguousarray(np.asarray(b_scale, dtype=np.float32).ravel())
    y = np.zeros(acc.size, dtype=np.float32)
    lib().ref_rescale(acc.ravel(), rows, n, float(np.float32(a_scale)), bs,
                      bs.size, y)
    return y.reshape(acc.shape)


def host_threads():
    """Cores available to this process (the CPU baseline's thread count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
