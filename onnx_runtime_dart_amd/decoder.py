"""Qwen3-shaped int4 decoder on the GPU: host side of the decoder session.

The session (``mmnb_decoder_*`` in include/mmnb.h) runs an int4 export's
per-layer node sequence -- RMSNorm, MatMulNBits q/k/v, per-head q/k RMSNorm,
GroupQueryAttention with rotary and KV cache, MatMulNBits o + residual,
RMSNorm, MatMulNBits gate/up, SiLU * up, MatMulNBits down + residual, final
RMSNorm, MatMulNBits lm_head -- and the greedy loop of
``tool/smollm2_generate.dart:48-83`` entirely in HBM.  This module builds
the weights (seeded random int4 blocks in the reference's MatMulNBits byte
format, since there are no checkpoints here) and the fused packs the session
wants:

* q, k and v concatenated along N (one MatMulNBits of N = (nh + 2 kvh) hd);
* gate and up interleaved along N (column 2j = gate j, 2j+1 = up j), so the
  GEMV that produces them can apply SiLU(gate) * up in its epilogue.

Both are plain column reorderings of the [N, K/bs, bs/2] bytes and the
[N, K/bs] scales: the arithmetic is the unfused model's.
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check
from .ops import pack_nbits


@dataclass(frozen=True)
class DecoderConfig:
    layers: int = 28
    hidden: int = 1024
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 3072
    vocab: int = 151936
    block: int = 128
    max_len: int = 320
    eps: float = 1e-6
    rope_theta: float = 1_000_000.0

    @property
    def qkv_n(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes_per_token(self):
        """MatMulNBits bytes streamed per decoded token (packed nibbles and
        fp32 scales of every projection and the lm_head)."""
        def mat(k, n):
            return k * n // 2 + n * (k // self.block) * 4
        per_layer = (mat(self.hidden, self.qkv_n) + mat(self.heads * self.head_dim, self.hidden)
                     + mat(self.hidden, 2 * self.intermediate)
                     + mat(self.intermediate, self.hidden))
        return self.layers * per_layer + mat(self.hidden, self.vocab)


# Qwen3-0.6B's shape: 28 layers, hidden 1024, 16 q / 8 kv heads of 128,
# SwiGLU 3072, vocab 151936.
QWEN3_0_6B = DecoderConfig()


@dataclass
class Matrix:
    """One MatMulNBits weight in the reference byte format (symmetric: no
    zero points, so the zero point is 8)."""
    b_q: np.ndarray     # uint8 [n, k/bs, bs/2]
    scales: np.ndarray  # fp32 [n, k/bs]
    k: int
    n: int
    block: int


def random_matrix(rng, k, n, block, scale_range=(0.002, 0.006)):
    """Random-init weight already in block-quantized form: uniform nibbles,
    scales ~U(scale_range) (w = (q - 8) * s has std ~4.6 s)."""
    nb = k // block
    b = rng.integers(0, 256, size=(n, nb, block // 2), dtype=np.uint8)
    s = rng.uniform(scale_range[0], scale_range[1], size=(n, nb)).astype(np.float32)
    return Matrix(b, s, k, n, block)


def concat_n(*ms):
    """MatMulNBits weights side by side along N."""
    return Matrix(np.concatenate([m.b_q for m in ms]), np.concatenate([m.scales for m in ms]),
                  ms[0].k, sum(m.n for m in ms), ms[0].block)


def interleave_n(a, b):
    """Columns 2j = a[j], 2j+1 = b[j]."""
    bq = np.empty((2 * a.n,) + a.b_q.shape[1:], np.uint8)
    bq[0::2], bq[1::2] = a.b_q, b.b_q
    sc = np.empty((2 * a.n, a.scales.shape[1]), np.float32)
    sc[0::2], sc[1::2] = a.scales, b.scales
    return Matrix(bq, sc, a.k, 2 * a.n, a.block)


@dataclass
class LayerWeights:
    ln1: np.ndarray
    ln2: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray
    q: Matrix
    k: Matrix
    v: Matrix
    o: Matrix
    gate: Matrix
    up: Matrix
    down: Matrix


@dataclass
class Weights:
    cfg: DecoderConfig
    embed: np.ndarray   # fp32 [vocab, hidden]
    layers: list
    norm: np.ndarray
    lm_head: Matrix


def random_weights(cfg, seed=0):
    """Seeded random-init weights of the configuration's shape."""
    rng = np.random.default_rng(seed)
    H, hd, bs = cfg.hidden, cfg.head_dim, cfg.block

    def gamma(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    layers = []
    for _ in range(cfg.layers):
        layers.append(LayerWeights(
            ln1=gamma(H), ln2=gamma(H), q_norm=gamma(hd), k_norm=gamma(hd),
            q=random_matrix(rng, H, cfg.heads * hd, bs),
            k=random_matrix(rng, H, cfg.kv_heads * hd, bs),
            v=random_matrix(rng, H, cfg.kv_heads * hd, bs),
            o=random_matrix(rng, cfg.heads * hd, H, bs),
            gate=random_matrix(rng, H, cfg.intermediate, bs),
            up=random_matrix(rng, H, cfg.intermediate, bs),
            down=random_matrix(rng, cfg.intermediate, H, bs)))
    embed = rng.standard_normal((cfg.vocab, H), dtype=np.float32)
    return Weights(cfg, embed, layers, gamma(H), random_matrix(rng, H, cfg.vocab, bs))


class GpuDecoder:
    """The decoder session on one context: packs uploaded once, KV cache and
    step state resident, a decode step replayed as a HIP graph."""

    def __init__(self, weights, ctx=None):
        self.ctx = ctx or _lib.default_context()
        self.cfg = cfg = weights.cfg
        lib = self.ctx.lib

        def pk(m):
            return pack_nbits(m.b_q, m.scales, None, k=m.k, n=m.n, bits=4, block_size=m.block,
                              ctx=self.ctx)

        self._packs = []
        self.lm = pk(weights.lm_head)
        self._packs.append(self.lm)
        c = _lib.DecoderConfig(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim,
                               cfg.intermediate, cfg.vocab, cfg.max_len, cfg.eps,
                               cfg.rope_theta)
        embed = np.ascontiguousarray(weights.embed, np.float32)
        norm = np.ascontiguousarray(weights.norm, np.float32)
        h = ctypes.c_void_p()
        check(lib.mmnb_decoder_create(self.ctx.handle, ctypes.byref(c), _lib.ptr(embed),
                                      _lib.ptr(norm), self.lm.handle, ctypes.byref(h)))
        self.handle = h
        for i, L in enumerate(weights.layers):
            qkv = pk(concat_n(L.q, L.k, L.v))
            o = pk(L.o)
            gu = pk(interleave_n(L.gate, L.up))
            down = pk(L.down)
            self._packs += [qkv, o, gu, down]
            vecs = [np.ascontiguousarray(v, np.float32) for v in (L.ln1, L.ln2, L.q_norm,
                                                                  L.k_norm)]
            check(lib.mmnb_decoder_set_layer(self.handle, i, *[_lib.ptr(v) for v in vecs],
                                             qkv.handle, o.handle, gu.handle, down.handle))

    def prefill(self, tokens):
        """Prompt through the model; returns the greedy next token."""
        t = np.ascontiguousarray(tokens, np.int64)
        nxt = ctypes.c_int32()
        check(self.ctx.lib.mmnb_decoder_prefill(self.handle, _lib.ptr(t), t.size,
                                                ctypes.byref(nxt)))
        return int(nxt.value)

    def decode(self, steps):
        """`steps` greedy steps; returns their tokens."""
        out = np.zeros(max(1, steps), np.int32)
        check(self.ctx.lib.mmnb_decoder_decode(self.handle, int(steps), _lib.ptr(out)))
        return out[:steps]

    def logits(self):
        out = np.empty(self.cfg.vocab, np.float32)
        check(self.ctx.lib.mmnb_decoder_logits(self.handle, _lib.ptr(out)))
        return out

    def position(self):
        p = ctypes.c_int64()
        check(self.ctx.lib.mmnb_decoder_position(self.handle, ctypes.byref(p)))
        return int(p.value)

    def use_graph(self, on):
        """Replay the recorded step graph (default) or launch eagerly."""
        check(self.ctx.lib.mmnb_decoder_set_graph(self.handle, int(bool(on))))

    def reset(self):
        check(self.ctx.lib.mmnb_decoder_reset(self.handle))

    def free(self):
        if self.handle:
            self.ctx.lib.mmnb_decoder_free(self.handle)
            self.handle = None
        for p in self._packs:
            p.free()
        self._packs = []
