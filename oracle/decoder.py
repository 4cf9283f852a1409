"""CPU oracle of the decoder ops around MatMulNBits and of a Qwen3-shaped
int4 decoder built from them.

TEST INFRASTRUCTURE ONLY: this module checks the GPU decoder path.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product package never does.

Each function restates the reference's Dart arithmetic (onnx_runtime_dart,
``lib/src/onnx_ops.dart``), keeping its rounding points: Dart computes in
``double`` and stores into ``Float32List`` (one binary32 rounding per store),
and its fp32 GEMM is the sequential-k kernel restated in ``refcpu.c``
(``matmul_kernel``).
"""
from dataclasses import dataclass, field

import numpy as np

from oracle import refcpu

F32 = np.float32
F64 = np.float64


def rmsnorm(x, gamma, eps):
    """opRMSNorm, last-axis case (onnx_ops.dart:1436-1461): per row
    ss = sum(x^2) in double, inv = 1/sqrt(ss/d + eps), y = fl32(x*inv*g)."""
    x = np.asarray(x, F32)
    g = np.asarray(gamma, F32).astype(F64)
    d = x.shape[-1]
    if g.shape[-1] != d:
        raise ValueError("RMSNorm gamma length != last dim")
    x64 = x.astype(F64)
    ss = np.sum(x64 * x64, axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(ss / d + float(eps))
    return (x64 * inv * g).astype(F32)


def rotary(x, pos, cos_cache, sin_cache, interleaved=False, num_heads=0):
    """opRotaryEmbedding for 3-D x [b, s, heads*head] (onnx_ops.dart:2121-2181):
    rotated pairs in double, stored as binary32; the tail past the rotary
    dimension passes through."""
    x = np.asarray(x, F32)
    cos = np.asarray(cos_cache, F32).astype(F64)
    sin = np.asarray(sin_cache, F32).astype(F64)
    pos = np.asarray(pos, np.int64)
    half_rot = cos.shape[-1]
    rot = 2 * half_rot
    b, s, hidden = x.shape
    head = hidden // num_heads if num_heads > 0 else rot
    heads = hidden // head
    out = x.copy()
    xr = x.reshape(b, s, heads, head).astype(F64)
    o = out.reshape(b, s, heads, head)
    flat = pos.reshape(-1)
    for bi in range(b):
        for si in range(s):
            # positionIds rank 1: pos[s]; else pos[b*seq + s] (:2150)
            p = int(flat[si] if pos.ndim == 1 else flat[bi * s + si])
            c, sn = cos[p], sin[p]
            if interleaved:
                x0, x1 = xr[bi, si, :, 0:rot:2], xr[bi, si, :, 1:rot:2]
                o[bi, si, :, 0:rot:2] = (x0 * c - x1 * sn).astype(F32)
                o[bi, si, :, 1:rot:2] = (x1 * c + x0 * sn).astype(F32)
            else:
                h = rot // 2
                x0, x1 = xr[bi, si, :, :h], xr[bi, si, :, h:rot]
                o[bi, si, :, :h] = (x0 * c - x1 * sn).astype(F32)
                o[bi, si, :, h:rot] = (x1 * c + x0 * sn).astype(F32)
    return out


def gqa(q, k, v, num_heads, kv_heads, scale=None, past_k=None, past_v=None,
        cos_cache=None, sin_cache=None, do_rotary=False, interleaved=False, bias=None):
    """opGroupQueryAttention (onnx_ops.dart:1508-1640).  q [b, s, nh*hd],
    k/v [b, s, kvh*hd], past [b, kvh, P, hd].  Returns (out, present_k,
    present_v).  Scores and the context product use the reference's fp32
    GEMM; the softmax is in double with binary32 stores, as in Dart."""
    q = np.asarray(q, F32)
    k = np.asarray(k, F32)
    v = np.asarray(v, F32)
    b, s, _ = q.shape
    hd = q.shape[2] // num_heads
    group = num_heads // kv_heads
    P = past_k.shape[2] if past_k is not None else 0
    T = P + s
    if do_rotary:
        # positions are built as [1, seq] (:1537-1541) and RotaryEmbedding
        # indexes them pos[b*seq + s] (:2150): batch > 1 reads past the end
        # and the reference throws
        if b > 1:
            raise ValueError("GroupQueryAttention: rotary with batch > 1 is out of range")
        pos = np.arange(P, P + s, dtype=np.int64).reshape(1, s)
        q = rotary(q, pos, cos_cache, sin_cache, interleaved, num_heads)
        k = rotary(k, pos, cos_cache, sin_cache, interleaved, kv_heads)
    sc = (1.0 / np.sqrt(hd)) if scale is None else float(scale)
    pk = np.zeros((b, kv_heads, T, hd), F32)
    pv = np.zeros((b, kv_heads, T, hd), F32)
    if P:
        pk[:, :, :P] = past_k
        pv[:, :, :P] = past_v
    pk[:, :, P:] = k.reshape(b, s, kv_heads, hd).transpose(0, 2, 1, 3)
    pv[:, :, P:] = v.reshape(b, s, kv_heads, hd).transpose(0, 2, 1, 3)
    out = np.zeros((b, s, num_heads * hd), F32)
    bias = None if bias is None else np.asarray(bias, F32)
    for bi in range(b):
        for h in range(num_heads):
            kvh = h // group
            qh = q[bi, :, h * hd:(h + 1) * hd]
            kt = np.ascontiguousarray(pk[bi, kvh].T)
            scores = refcpu.matmul_kernel(qh, kt, s, hd, T)
            probs = np.zeros((s, T), F32)
            for i in range(s):
                last = P + i
                row = scores[i, :last + 1].astype(F64) * sc
                if bias is not None:
                    bh = h % bias.shape[1]
                    row = row + bias[bi, bh, i, :last + 1].astype(F64)
                row = row.astype(F32).astype(F64)      # stored into Float32List
                mx = row.max()
                e = np.exp(row - mx)
                ssum = 0.0
                for val in e:                          # sequential double sum
                    ssum += val
                inv = 1.0 / ssum
                probs[i, :last + 1] = (e.astype(F32).astype(F64) * inv).astype(F32)
            ctx = refcpu.matmul_kernel(probs, np.ascontiguousarray(pv[bi, kvh]), s, T, hd)
            out[bi, :, h * hd:(h + 1) * hd] = ctx
    return out, pk, pv


def silu_mul(gate, up):
    """The Sigmoid -> Mul -> Mul chain of a SwiGLU block: sigmoid as
    1/(1+exp(-x)) in double (onnx_ops.dart:1963-1964) stored as binary32,
    then two binary32 products (_arithFloatFast, :99-135)."""
    g = np.asarray(gate, F32)
    sig = (1.0 / (1.0 + np.exp(-g.astype(F64)))).astype(F32)
    return ((g * sig).astype(F32) * np.asarray(up, F32)).astype(F32)


def rope_tables(max_len, head_dim, theta):
    """cos/sin caches [max_len, head_dim/2] as a Qwen-style export stores
    them (inv_freq = theta^(-2i/d), angle = pos * inv_freq), binary32."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=F64) / head_dim))
    ang = np.arange(max_len, dtype=F64)[:, None] * inv[None, :]
    return np.cos(ang).astype(F32), np.sin(ang).astype(F32)


# ----------------------------------------------------------------------------
# Qwen3-shaped decoder (the per-layer node sequence of an int4 ONNX export:
# SimplifiedLayerNormalization, MatMulNBits q/k/v, per-head q/k RMSNorm,
# GroupQueryAttention with rotary and KV cache, MatMulNBits o, residual Add,
# SimplifiedLayerNormalization, MatMulNBits gate/up, SiLU*up, MatMulNBits
# down, residual Add; final norm and MatMulNBits lm_head).
# ----------------------------------------------------------------------------
@dataclass
class NBits:
    """One MatMulNBits weight in the reference byte format."""
    b_q: np.ndarray      # uint8 [n, k/bs, bs/2]
    scales: np.ndarray   # fp32 [n, k/bs]
    k: int
    n: int
    block: int

    def matmul(self, a):
        return refcpu.matmul_nbits(a, self.b_q, self.scales, None, self.k, self.n, 4,
                                   self.block, threads=min(16, refcpu.host_threads()))


@dataclass
class Layer:
    ln1: np.ndarray
    ln2: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray
    q: NBits
    k: NBits
    v: NBits
    o: NBits
    gate: NBits
    up: NBits
    down: NBits


@dataclass
class Model:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    eps: float
    embed: np.ndarray
    layers: list
    norm: np.ndarray
    lm_head: NBits
    cos: np.ndarray
    sin: np.ndarray
    cache_k: list = field(default_factory=list)
    cache_v: list = field(default_factory=list)

    def forward(self, tokens):
        """Run `tokens` (a prompt chunk or one decode token) through the
        decoder with the KV cache; returns logits [len(tokens), vocab]."""
        tokens = np.asarray(tokens, np.int64)
        s = len(tokens)
        x = self.embed[tokens]
        nh, kvh, hd = self.heads, self.kv_heads, self.head_dim
        if not self.cache_k:
            self.cache_k = [None] * len(self.layers)
            self.cache_v = [None] * len(self.layers)
        for li, L in enumerate(self.layers):
            h = rmsnorm(x, L.ln1, self.eps)
            q = rmsnorm(L.q.matmul(h).reshape(s, nh, hd), L.q_norm, self.eps).reshape(1, s, -1)
            k = rmsnorm(L.k.matmul(h).reshape(s, kvh, hd), L.k_norm, self.eps).reshape(1, s, -1)
            v = L.v.matmul(h).reshape(1, s, -1)
            out, pk, pv = gqa(q, k, v, nh, kvh, None, self.cache_k[li], self.cache_v[li],
                              self.cos, self.sin, do_rotary=True)
            self.cache_k[li], self.cache_v[li] = pk, pv
            x = (x + L.o.matmul(out.reshape(s, -1))).astype(F32)
            h = rmsnorm(x, L.ln2, self.eps)
            a = silu_mul(L.gate.matmul(h), L.up.matmul(h))
            x = (x + L.down.matmul(a)).astype(F32)
        x = rmsnorm(x, self.norm, self.eps)
        return self.lm_head.matmul(x)


def argmax_first(row):
    """Greedy pick of tool/smollm2_generate.dart:64-72: the first index
    holding the maximum (np.argmax returns the first occurrence)."""
    return int(np.argmax(np.asarray(row)))
