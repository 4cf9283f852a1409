"""CPU checks of the integer identities the fp32 GEMV kernels dequantise
with (dq_nibbles in onnx_runtime_dart_amd/csrc/mmnb_device.h), and of the
power of the accumulation-bound check used by the GPU parity tests.

The kernels turn a dword of 8 nibbles into 8 floats that hold the exact
(q - zp) scaled by a power of two:
  zero point 8:  x = w ^ 0x88888888, xh = x >> 4; the low nibble of byte b
                 of x (of xh) is the 4-bit two's complement of q - 8 for
                 nibble 2b (2b + 1), converted by v_cvt_off_f32_i4 (signed
                 4-bit value / 16, its documented table) to (q - 8) / 16
  zero point z:  lo = (((w << 3) & 0x78787878) + c) ^ 0x80808080,
                 hi = (((w >> 1) & 0x78787878) + c) ^ 0x80808080,
                 c = (128 - 8z) * 0x01010101; signed byte b reads 8 (q - z)
Checked here for every nibble value in every position and every z.
"""
import numpy as np
import pytest

from oracle import refcpu

U = 2.0 ** -24


def gamma(k):
    return k * U / (1 - k * U)


def _bytes_signed(v):
    v = np.asarray(v, np.uint32)
    return np.stack([((v >> (8 * b)) & 0xFF).astype(np.uint8).view(np.int8) for b in range(4)],
                    -1).astype(np.int64)


def _nibbles(w):
    w = np.asarray(w, np.uint32)
    return np.stack([((w >> (4 * e)) & 0xF) for e in range(8)], -1).astype(np.int64)


# v_cvt_off_f32_i4: bits 3:0 of the operand, as a signed 4-bit value, / 16
# (the instruction's table: 0b1000 -> -0.5, 0b1111 -> -0.0625, 0b0000 -> 0,
# 0b0111 -> 0.4375)
_CVT_OFF_I4 = {0b1000: -0.5, 0b1111: -0.0625, 0b0000: 0.0, 0b0111: 0.4375}


def _cvt_off_f32_i4(v):
    n = np.asarray(v, np.int64) & 0xF
    return np.where(n >= 8, n - 16, n) / 16.0


def test_cvt_off_table():
    for n, want in _CVT_OFF_I4.items():
        assert _cvt_off_f32_i4(n) == want
        # the byte select passes the whole byte; only bits 3:0 count
        assert _cvt_off_f32_i4(n | 0xA0) == want


def _dq_zp8(w):
    """The zero-point-8 kernel steps; [.., 8] floats in nibble order."""
    w = np.asarray(w, np.uint32)
    x = w ^ np.uint32(0x88888888)
    xh = x >> np.uint32(4)
    out = np.empty(w.shape + (8,), np.float64)
    for b in range(4):
        out[..., 2 * b] = _cvt_off_f32_i4((x >> np.uint32(8 * b)) & np.uint32(0xFF))
        out[..., 2 * b + 1] = _cvt_off_f32_i4((xh >> np.uint32(8 * b)) & np.uint32(0xFF))
    return out


def _dq(w, z):
    """The explicit-zero-point kernel steps; [.., 8] values in nibble order."""
    w = np.asarray(w, np.uint32)
    c = np.uint32(((128 - 8 * z) * 0x01010101) & 0xFFFFFFFF)
    lo = (((w << np.uint32(3)) & np.uint32(0x78787878)) + c) ^ np.uint32(0x80808080)
    hi = (((w >> np.uint32(1)) & np.uint32(0x78787878)) + c) ^ np.uint32(0x80808080)
    lb, hb = _bytes_signed(lo), _bytes_signed(hi)
    out = np.empty(w.shape + (8,), np.int64)
    out[..., 0::2] = lb
    out[..., 1::2] = hb
    return out


def _all_words():
    # every nibble value in every position: w = v * 0x11111111 for v in 0..15,
    # plus random words
    rng = np.random.default_rng(0)
    w = np.concatenate([np.arange(16, dtype=np.uint32) * np.uint32(0x11111111),
                        rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)])
    # and each position alone taking each value, the others at 0 and at 15
    for e in range(8):
        for v in range(16):
            for bg in (0, 0xFFFFFFFF):
                ww = (bg & ~(0xF << (4 * e))) | (v << (4 * e))
                w = np.append(w, np.uint32(ww))
    return w


def test_zero_point_8_identity():
    w = _all_words()
    np.testing.assert_array_equal(_dq_zp8(w), (_nibbles(w) - 8) / 16.0)


@pytest.mark.parametrize("z", range(16))
def test_explicit_zero_point_identity(z):
    w = _all_words()
    np.testing.assert_array_equal(_dq(w, z), 8 * (_nibbles(w) - z))


# ------------------------------------------------------ bound-check power
def _gemv_emulation(a, q, z, s, bs, fold):
    """binary32 emulation of one output of the M = 1 GEMV over 32-k chunks:
    per chunk d = sum a * v (v = q - z exact, or v = q with the zero point
    folded in afterwards: acc += s * d - (s * z) * sum a)."""
    f32 = np.float32
    acc = f32(0.0)
    for c0 in range(0, a.size, 32):
        blk = c0 // bs
        d, sa = f32(0.0), f32(0.0)
        for e in range(32):
            v = f32(q[c0 + e]) if fold else f32(int(q[c0 + e]) - int(z[blk]))
            d = f32(d + f32(a[c0 + e] * v))
            sa = f32(sa + a[c0 + e])
        acc = f32(acc + f32(s[blk] * d))
        if fold:
            acc = f32(acc - f32(f32(s[blk] * f32(z[blk])) * sa))
    return acc


def test_bound_check_rejects_a_folded_zero_point():
    # A column whose nibbles mostly equal the zero point: the reference's W
    # is exactly 0 there.  The folded form leaves rounding residue of order
    # u * zp * scale * sum|a|, far above gamma_K * sum|a||W|; the exact form
    # stays inside the bound.  This is what the GPU tests' bound check relies
    # on to catch a folded zero point.
    k, bs = 512, 32
    rng = np.random.default_rng(4)
    nb = k // bs
    a = rng.standard_normal(k).astype(np.float32)
    z = rng.integers(0, 16, nb)
    q = np.repeat(z, bs).astype(np.int64)
    live = np.argsort(np.abs(a))[:2]   # two live weights on small activations
    q[live] = (q[live] + 5) % 16
    s = rng.uniform(0.005, 0.02, nb).astype(np.float32)
    # reference bytes [n=1, nb, bs/2] and flat zero-point nibbles
    b_q = (q[0::2] | (q[1::2] << 4)).astype(np.uint8).reshape(1, nb, bs // 2)
    zp = np.zeros((nb + 1) // 2, np.uint8)
    for i, v in enumerate(z):
        zp[i >> 1] |= np.uint8(v << (4 * (i & 1)))
    y64, absdot = refcpu.matmul_nbits_f64(a[None], b_q, s, zp, k, 1, bs)
    bound = gamma(k + 2) * absdot[0, 0]
    exact = _gemv_emulation(a, q, z, s, bs, fold=False)
    folded = _gemv_emulation(a, q, z, s, bs, fold=True)
    assert abs(float(exact) - y64[0, 0]) <= bound
    assert abs(float(folded) - y64[0, 0]) > bound


def test_all_zero_point_column_is_exactly_zero_only_unfolded():
    k, bs = 256, 64
    rng = np.random.default_rng(5)
    a = rng.standard_normal(k).astype(np.float32)
    z = rng.integers(1, 16, k // bs)
    q = np.repeat(z, bs)
    s = rng.uniform(0.005, 0.02, k // bs).astype(np.float32)
    assert _gemv_emulation(a, q, z, s, bs, fold=False) == 0.0
    assert _gemv_emulation(a, q, z, s, bs, fold=True) != 0.0
