// MatMulNBits on gfx950: weight repack, decode-shape GEMV, activation prep
// and the MFMA prefill GEMM.
//
// Reference semantics (onnx_qlinear_ops.dart:114-156): W[k, n] =
// fl32((q[n, k] - zp[n, blk]) * scale[n, blk]), y = A * W.  The kernels
// factor the scale out of each block: y = sum_blk scale * sum_{k in blk}
// a[k] * (q - zp), which differs from the reference only in rounding.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "mmnb_device.h"
#include "mmnb_internal.h"

namespace mmnb {

static int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << (r + 1)) <= v) r++;
  return r;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef float f4vec __attribute__((ext_vector_type(4)));
typedef int i4vec __attribute__((ext_vector_type(4)));
typedef unsigned u4vec __attribute__((ext_vector_type(4)));

// 16 bytes of a packed weight column for the GEMVs, which read every weight
// once per call: a non-temporal load (nt), so the stream does not displace
// the lines that are read again (activations, scales, zero points) and is
// not kept where the next call's weights would have to evict it.  Against
// plain loads, the M = 1 GEMV at K = N = 4096 (block 128, packs rotated past
// the caches) went from 4.60 to 4.40 us per call, at K = N = 16384 from 33.8
// to 32.8 us; the scales loaded the same way were slower (4.42 us).
__device__ __forceinline__ u4vec ld_weights16(const uint8_t *p) {
  return __builtin_nontemporal_load((const u4vec *)p);
}
__device__ __forceinline__ uint4 ld_weights16_u4(const uint8_t *p) {
  const u4vec v = ld_weights16(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Zero point of flat (column, block) index zi.  Z is never null: packs
// without zero points carry a buffer of 0x88 (8 in both nibbles), so the
// load is unconditional (a conditional load ends in a full vmcnt wait).
__device__ __forceinline__ int zp_of(const uint8_t *__restrict__ Z, int64_t zi) {
  const uint32_t zb = Z[zi >> 1];
  return (int)((zb >> ((zi & 1) * 4)) & 0xF);
}

// ---------------------------------------------------------------------------
// Repack: [N][src_col] bytes (reference layout) -> [N][dst_col] bytes with
// the per-32-byte dword permutation d0 d2 d4 d6 | d1 d3 d5 d7.  Nibbles with
// k >= K are written as zero: the reference never reads them (kEnd clip,
// onnx_qlinear_ops.dart:141), and zeros make padded lanes contribute exact
// zeros.  One thread per (column, 32-byte segment).
// ---------------------------------------------------------------------------
__global__ void k_repack_nbits(const uint8_t *__restrict__ src, int64_t n,
                               int64_t src_col, int64_t dst_col, int64_t K,
                               uint8_t *__restrict__ dst) {
  const int64_t segs = dst_col / kSegBytes;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * segs) return;
  const int64_t col = idx / segs, s = idx % segs;
  const uint8_t *cs = src + col * src_col;
  uint32_t d[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int64_t off = s * kSegBytes + 4 * i;
    uint32_t v = 0;
    if (off + 4 <= src_col) {
      v = (uint32_t)cs[off] | ((uint32_t)cs[off + 1] << 8) |
          ((uint32_t)cs[off + 2] << 16) | ((uint32_t)cs[off + 3] << 24);
    }
    // keep nibbles e with k = 64 s + 8 i + e < K
    const int64_t valid = K - (s * kSegK + 8 * i);
    if (valid <= 0) v = 0;
    else if (valid < 8) v &= (1u << (4 * valid)) - 1u;
    d[i] = v;
  }
  uint32_t *o = (uint32_t *)(dst + col * dst_col + s * kSegBytes);
  o[0] = d[0];
  o[1] = d[2];
  o[2] = d[4];
  o[3] = d[6];
  o[4] = d[1];
  o[5] = d[3];
  o[6] = d[5];
  o[7] = d[7];
}

int repack_nbits_weights(mmnb_ctx *ctx, const uint8_t *d_src, int64_t n, int64_t k,
                         int64_t src_col, int64_t dst_col, uint8_t *d_dst) {
  const int64_t segs = dst_col / kSegBytes;
  const int64_t total = n * segs;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  return launch(ctx, kKernRepack, k_repack_nbits, dim3((unsigned)blocks), dim3(threads), 0,
                d_src, n, src_col, dst_col, k, d_dst);
}

// ---------------------------------------------------------------------------
// Block-major copies of the scales and zero points for the prefill GEMM, in
// one buffer of rows [nb][2][ld]: row 2b holds scales[c][b], row 2b + 1 the
// zero-point nibble (c, b) as a dword, so the columns of one quantisation
// block that a GEMM tile stages are contiguous (coalesced DMA) instead of nb
// apart, and one buffer resource covers both.  One thread per (b, c).
// ---------------------------------------------------------------------------
__global__ void k_sz_block_major(const float *__restrict__ S, const uint8_t *__restrict__ Z,
                                 int64_t n, int64_t nb, int64_t ld, uint32_t *__restrict__ stz) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= ld * nb) return;
  const int64_t b = idx / ld, c = idx % ld;
  uint32_t *row = stz + 2 * b * ld;
  if (c >= n) {  // row padding
    row[c] = 0u;
    row[ld + c] = 0u;
    return;
  }
  const int64_t zi = c * nb + b;
  row[c] = __builtin_bit_cast(uint32_t, S[zi]);
  row[ld + c] = (uint32_t)(Z[zi >> 1] >> (4 * (zi & 1))) & 0xFu;
}

int build_gemm_sz(mmnb_ctx *ctx, mmnb_pack *p) {
  p->ldsz = (p->n + 3) / 4 * 4;
  const int64_t total = p->ldsz * p->n_blocks;
  int rc;
  if ((rc = device_alloc((size_t)total * 8, (void **)&p->d_st))) return rc;
  p->d_zt = (uint32_t *)(p->d_st + p->ldsz);  // inside d_st (not freed on its own)
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  return launch(ctx, kKernRepack, k_sz_block_major, dim3((unsigned)blocks), dim3(threads), 0,
                (const float *)p->d_scales, (const uint8_t *)p->d_zp, p->n, p->n_blocks,
                p->ldsz, (uint32_t *)p->d_st);
}

// (a & mask) | orv in one VALU op.  gfx9 VOP3 takes no literal, so the
// compiler splits this into v_and + v_or; with the mask in an SGPR and the
// magic in a VGPR it is one v_and_or_b32.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t orv) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(orv));
  return r;
}

// 8 nibbles of one dword -> 8 fp16 values (q - zp), exact.  (q | 0x6400)
// as fp16 is 1024 + q; (16q | 0x6400) is 1024 + 16q, so
//   lo nibble pairs: (1024 + q) - (1024 + zp)
//   hi nibble pairs: (1024 + 16q) / 16 - (64 + zp)
// Output order {n0, n4, n1, n5, n2, n6, n3, n7}; the prepared activations
// use the same k permutation.
__device__ __forceinline__ half8_t dequant8(uint32_t w, int zp, uint32_t magic) {
  const uint32_t t0 = and_or(w, 0x000F000Fu, magic);
  const uint32_t t1 = and_or(w, 0x00F000F0u, magic);
  const uint32_t w8 = w >> 8;
  const uint32_t t2 = and_or(w8, 0x000F000Fu, magic);
  const uint32_t t3 = and_or(w8, 0x00F000F0u, magic);
  // 1024 + zp and 64 + zp (zp <= 15) as fp16 bits: ulp 1 at 1024, 1/16 at 64
  const half2_t zz = __builtin_bit_cast(half2_t, (uint32_t)(0x6400 + zp) * 0x10001u);
  const half2_t zs = __builtin_bit_cast(half2_t, (uint32_t)(0x5400 + (zp << 4)) * 0x10001u);
  const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2_t h0 = __builtin_bit_cast(half2_t, t0) - zz;
  const half2_t h1 = __builtin_bit_cast(half2_t, t1) * sixteenth - zs;
  const half2_t h2 = __builtin_bit_cast(half2_t, t2) - zz;
  const half2_t h3 = __builtin_bit_cast(half2_t, t3) * sixteenth - zs;
  half8_t r = {h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
  return r;
}

// ---------------------------------------------------------------------------
// Decode-shape GEMV on the vector ALUs (fp32 FMA), M = 1.
//
// A column's K extent is cut into 16-byte chunks (32 nibbles); chunk c =
// (segment s = c/2, half g = c%2) holds k = 64s + 16j + 8g + e for dword
// j = 0..3, nibble e = 0..7.  A workgroup owns 2R columns and all of K:
//   wave w, lane l: half h = l/32 picks one column of each pair, t = l%32;
//   the lane owns chunk c = 32w + t (+ 32 nw per extra iteration) of the R
//   columns 2r + h, r = 0..R-1.  Both halves need the same activations: each
//   loads half of them and a lane swap completes the other half
//   (load_chunk32_paired; against every lane loading all 32, the headline
//   K = N = 4096 call went from 4.69 to 4.59 us).
// Up to 4 waves split K (one pass covers K <= 4096; longer K iterates:
// 16-wave workgroups covering K = 16384 in one pass measured 20% slower).
// Per iteration a lane issues all of its loads -- its 32 activations, the scales (and zero
// points), then the R weight chunks in column order -- before any
// arithmetic, pinned there by a scheduling barrier: left to itself the
// compiler sinks loads next to their first use, which splits them into
// several dependent round trips.  Column r's arithmetic then waits only for
// loads up to its own chunk.  The activations of a chunk are reused for R
// columns.  Each nibble becomes the exact (q - zp), scaled by a power of two
// (dq_nibbles), before the fp32 FMAs: acc += scale * sum a * (q - zp), as
// the reference's per-weight (q - zp) * scale (a block whose nibbles all
// equal the zero point adds exactly zero).  The 32 lanes of a column
// half-wave reduce with DPP/swizzle, the waves through LDS.
// ---------------------------------------------------------------------------

constexpr int kGemvMaxWaves = 4;   // M = 1 GEMV
constexpr int kDecMaxWaves = 4;    // decoder-step GEMV (K <= 4096)

template <int R, int NBPC, bool HAS_ZP, bool FAST>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void k_gemv_valu(
    const float *__restrict__ A, const uint8_t *__restrict__ W, int64_t col_bytes,
    const float *__restrict__ S, const uint8_t *__restrict__ Z, int nb, int bs_log2, int K,
    int N, float *__restrict__ Y, int C, int iters) {
  __shared__ float red[kGemvMaxWaves][2 * R];
  // every kernel argument (and the block size) in SGPRs before anything
  // else: left to itself the compiler fetched them in two dependent rounds
  // of scalar loads ahead of the first weight load
  kernarg_fence(A, W, col_bytes, S, Z, nb, bs_log2, K, N, Y, C, iters, blockDim.x);
  const int nw = blockDim.x >> 6;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int h = l >> 5, t = l & 31;
  const int col0 = blockIdx.x * (2 * R);

  int colr[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int c = col0 + 2 * r + h;
    colr[r] = c < N ? c : N - 1;
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;

  for (int it = 0; it < iters; it++) {
    const int c = 32 * w + t + it * 32 * nw;
    const bool cv = c < C;
    const int cc = cv ? c : 0;
    const int s = cc >> 1, g = cc & 1;
    // ---- every load of this iteration.  A lane past the last chunk reads
    // chunk 0 (cc) with zero scales, so it adds exactly nothing.
    float av[32];
    const float *ar = A + s * kSegK + 8 * g;
    if constexpr (FAST) {
      // rows hold k64 values: every 8-float run of a chunk is inside the row
      load_chunk32_paired(ar, h, av);
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int k0 = s * kSegK + 8 * g + 16 * j;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int k = k0 + e < K ? k0 + e : K - 1;
          const float x = A[k];
          av[8 * j + e] = (cv && k0 + e < K) ? x : 0.0f;
        }
      }
    }
    float sraw[R][NBPC];
    uint32_t zraw[R][NBPC];
    bool inbq[NBPC];
    int zsh[R][NBPC];
#pragma unroll
    for (int q = 0; q < NBPC; q++) {
      // block of dwords j in [q*4/NBPC, (q+1)*4/NBPC)
      const int kq = s * kSegK + 16 * (q * (4 / NBPC)) + (NBPC == 4 ? 8 * g : 0);
      int blk = kq >> bs_log2;
      inbq[q] = cv && blk < nb;
      blk = blk < nb ? blk : nb - 1;
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int zi = colr[r] * nb + blk;
        sraw[r][q] = S[zi];
        if (HAS_ZP) zraw[r][q] = Z[zi >> 1];
        zsh[r][q] = (zi & 1) * 4;
      }
    }
    uint4 wv[R];
#pragma unroll
    for (int r = 0; r < R; r++)
      wv[r] = ld_weights16_u4(W + (int64_t)colr[r] * col_bytes + (int64_t)cc * 16);
    __builtin_amdgcn_sched_barrier(0);
    // ---- arithmetic: exact S * (q - zp) per weight (dq_nibbles); the block's
    // scale carries the 1 / S (dq_unscale, exact for normal scales), so the
    // sums range like the reference's (q - zp) * scale terms
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
#pragma unroll
      for (int q = 0; q < NBPC; q++) {
        const uint32_t zc =
            HAS_ZP ? dq8_const((int)((zraw[r][q] >> zsh[r][q]) & 0xF)) : 0u;
        float d = 0.0f;
#pragma unroll
        for (int jj = 0; jj < 4 / NBPC; jj++) {
          const int j = q * (4 / NBPC) + jj;
          float qv[8];
          dq_nibbles<HAS_ZP>(wd[j], zc, qv);
#pragma unroll
          for (int e = 0; e < 8; e++) d = fmaf(av[8 * j + e], qv[e], d);
        }
        // a lane past the last chunk (or a block past the last one) drops
        // its d: its activations may be chunk 0's, and 0 * inf would be NaN
        const float sc = sraw[r][q] * dq_unscale<HAS_ZP>();
        acc[r] = inbq[q] ? fmaf(sc, d, acc[r]) : acc[r];
      }
      // column by column: the scheduler would otherwise hoist later
      // columns' dequantisation and so wait for every weight load first
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // ---- reductions: 32 lanes of a half-wave, then the waves
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float v = half_wave_sum(acc[r]);
    if (t == 0) red[w][2 * r + h] = v;
  }
  __syncthreads();
  if ((int)threadIdx.x < 2 * R) {
    float v = 0.0f;
    for (int ww = 0; ww < nw; ww++) v += red[ww][threadIdx.x];
    const int col = col0 + threadIdx.x;
    if (col < N) Y[col] = v;
  }
}

template <int R>
static int launch_gemv_r(mmnb_ctx *ctx, int nbpc, dim3 grid, dim3 block, const float *A,
                         const mmnb_pack *p, float *Y, int C, int iters, bool fast,
                         int bs_log2) {
  const int nb = (int)p->n_blocks, K = (int)p->k, N = (int)p->n;
#define MMNB_GEMV_LAUNCH(Q, ZP, F)                                                           \
  return launch(ctx, kKernGemv, k_gemv_valu<R, Q, ZP, F>, grid, block, 0, A, p->d_w,         \
                p->col_bytes, p->d_scales, p->d_zp, nb, bs_log2, K, N, Y, C, iters)
#define MMNB_GEMV_LAUNCH_Q(ZP, F)             \
  {                                          \
    if (nbpc == 4) MMNB_GEMV_LAUNCH(4, ZP, F); \
    if (nbpc == 2) MMNB_GEMV_LAUNCH(2, ZP, F); \
    MMNB_GEMV_LAUNCH(1, ZP, F);                \
  }
  if (p->has_zp) {
    if (fast) MMNB_GEMV_LAUNCH_Q(true, true);
    MMNB_GEMV_LAUNCH_Q(true, false);
  }
  if (fast) MMNB_GEMV_LAUNCH_Q(false, true);
  MMNB_GEMV_LAUNCH_Q(false, false);
#undef MMNB_GEMV_LAUNCH_Q
#undef MMNB_GEMV_LAUNCH
}

// ---------------------------------------------------------------------------
// Decoder-step MatMulNBits (M = 1, no zero points, block >= 64) with the
// neighbouring graph nodes folded in, so one decoder layer needs five
// launches instead of a dozen:
//   NORM   RMSNorm prologue (SimplifiedLayerNormalization before q/k/v,
//          gate/up and lm_head): every workgroup sums x^2 over its chunks
//          (the 32 lanes of half 0 of each wave cover K once), then scales
//          its activations by rsqrt(mean + eps) * gamma;
//   EPI    kDecResidual (the residual Add after o and down),
//          kDecSwiglu (gate/up columns interleaved 2j/2j+1 in the pack, so a
//          workgroup holds both halves of its outputs: silu(g) * u),
//          kDecArgmax (lm_head: each workgroup stores the best key
//          (orderable value << 32 | ~index) of its columns; the greedy
//          token is the maximum key, ties going to the lowest index).
//   ATTN   the activations are the decode attention's output, merged here
//          from its split partials (DecAttnPartials): every workgroup
//          merges all K of them into LDS, so the attention launch needs no
//          cross-workgroup count and merge of its own.
// Lane layout and arithmetic (exact q - 8 per weight) follow k_gemv_valu
// with M = 1 and one quantisation block per chunk; K is at most 4096 (one chunk per lane).
// ---------------------------------------------------------------------------

// a = the merged attention output, into sx[K] (K <= kDecAttnMaxK, whole
// workgroup of kDecAttnMergeThreads).  Per query head the splits' maxima
// give M, and a = sum_s w_s o_s with w_s = e^(m_s - M) / sum_u e^(m_u - M) l_u
// over all nsmax splits (at most NS, a static bound): a split past the
// position holds an empty partial (max -inf, sum 0, o 0) that weighs 0, so
// the merge needs no position.  load() issues every load at once: thread t
// holds the (max, sum) pair of (head t / G, split t % G) -- a head's splits
// in one aligned group of G lanes -- and the o parts of the float4 quads t
// and t + 256 of a.  finish(), after the caller
// has issued its own loads: each head's maximum and denominator by DPP
// within its lane group, the weights through LDS (one exponential per
// pair), then each quad's weighted sum; it ends in a barrier.  Measured on
// the Qwen3-0.6B-shape decode step (ms per token): two quads per thread on
// the GEMV's four waves 0.577-0.580; one quad on eight waves 0.584; four
// quads on two waves 0.592; each lane merging only its own chunk's 32
// values (no LDS copy, no second barrier; four quads per lane) 0.615.
static_assert(kDecAttnMergeThreads == 64 * kDecMaxWaves, "the merge runs on the GEMV's block");

template <int NS>
struct DecAttnMerge {
  static constexpr int G = NS <= 8 ? 8 : 16;  // lanes per head's pairs
  static constexpr int QP = kDecAttnMaxK / 4 / kDecAttnMergeThreads;  // quads per thread
  float4 ov[QP][NS];
  float2 ml;
  int qi[QP], qh[QP];

  __device__ __forceinline__ void load(const DecAttnPartials &pa, int K) {
    const int t = threadIdx.x, nq = K >> 2, nh = K / pa.hd;
    ml = *(const float2 *)(pa.ml + 2 * (min(t / G, nh - 1) * pa.nsmax +
                                        min(t % G, pa.nsmax - 1)));
    // floor(4q / hd) as (4q + 1/2) / hd in float: the quotient lies at least
    // 1/(2 hd) from an integer, far beyond the product's rounding error
    const float rhd = 1.0f / (float)pa.hd;
#pragma unroll
    for (int i = 0; i < QP; i++) {
      qi[i] = min(t + kDecAttnMergeThreads * i, nq - 1);
      qh[i] = (int)(((float)(4 * qi[i]) + 0.5f) * rhd);
      const int d = 4 * qi[i] - qh[i] * pa.hd;
      const int64_t p0 = (int64_t)qh[i] * pa.nsmax;
#pragma unroll
      for (int s = 0; s < NS; s++)
        ov[i][s] = *(const float4 *)(pa.o + (p0 + min(s, pa.nsmax - 1)) * pa.hd + d);
    }
  }

  __device__ __forceinline__ void finish(const DecAttnPartials &pa, float *sx) {
    __shared__ float sw[kDecAttnMergeThreads];
    const int t = threadIdx.x, nsplit = pa.nsmax;
    // pair (head t / G, split t % G); lanes past nsmax and empty partials
    // weigh 0.  Every lane takes part in the group reductions.
    const bool live = t % G < nsplit && ml.x != -INFINITY;
    const float M = group_max<G>(live ? ml.x : -INFINITY);
    const float e = live ? expf(ml.x - M) : 0.0f;
    const float den = group_sum<G>(e * (live ? ml.y : 0.0f));
    sw[t] = e / den;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < QP; i++) {
      float n0 = 0.0f, n1 = 0.0f, n2 = 0.0f, n3 = 0.0f;
#pragma unroll
      for (int s = 0; s < NS; s++) {
        if (s < nsplit) {  // uniform: lanes past nsmax are skipped, not weighted
          const float w = sw[qh[i] * G + s];
          n0 = fmaf(w, ov[i][s].x, n0);
          n1 = fmaf(w, ov[i][s].y, n1);
          n2 = fmaf(w, ov[i][s].z, n2);
          n3 = fmaf(w, ov[i][s].w, n3);
        }
      }
      if (qi[i] == t + kDecAttnMergeThreads * i)
        *(float4 *)(sx + 4 * qi[i]) = make_float4(n0, n1, n2, n3);
    }
    __syncthreads();
  }
};

template <int R, bool NORM, int EPI, int ATTN = 0>
__global__ __launch_bounds__(64 * kDecMaxWaves) void k_dec_gemv(
    const float *__restrict__ X, const float *__restrict__ gamma, float eps,
    const uint8_t *__restrict__ W, int64_t col_bytes, const float *__restrict__ S, int nb,
    int bs_log2, int K, int N, const float *resid, float *Y,
    unsigned long long *__restrict__ argmax, int C, DecAttnPartials pa) {
  __shared__ float red[kDecMaxWaves][2 * R];
  __shared__ float nrm[kDecMaxWaves];
  __shared__ float outv[2 * R];
  __shared__ __align__(16) float sx[ATTN ? kDecAttnMaxK : 4];
  kernarg_fence(X, gamma, eps, W, col_bytes, S, nb, bs_log2, K, N, resid, Y, argmax, C,
                blockDim.x);
  if constexpr (ATTN) kernarg_fence(pa.o, pa.ml, pa.nsmax, pa.hd);
  const int nw = blockDim.x >> 6;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int h = l >> 5, t = l & 31;
  const int col0 = blockIdx.x * (2 * R);
  int colr[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int c = col0 + 2 * r + h;
    colr[r] = c < N ? c : N - 1;
  }
  const int c = 32 * w + t;
  const bool cv = c < C;
  const int cc = cv ? c : 0;
  const int s = cc >> 1, g = cc & 1;
  // ---- loads: activations (and gamma; with ATTN the attention partials),
  // scales, then weights
  float av[32], gv[32];
  [[maybe_unused]] DecAttnMerge<ATTN ? ATTN : 1> mg;
  if constexpr (ATTN)
    mg.load(pa, K);
  else
    load_chunk32_paired(X + s * kSegK + 8 * g, h, av);
  if constexpr (NORM) load_chunk32_paired(gamma + s * kSegK + 8 * g, h, gv);
  const int blk = (s * kSegK) >> bs_log2;
  float sraw[R];
#pragma unroll
  for (int r = 0; r < R; r++) sraw[r] = S[colr[r] * nb + blk];
  // the residual of output column col0 + thread, loaded with the rest (a
  // load under the epilogue's column test would be a round trip of its own);
  // only this workgroup writes those columns
  float rres = 0.0f;
  if constexpr (EPI == kDecResidual) rres = resid[min(col0 + (int)threadIdx.x, N - 1)];
  uint4 wv[R];
#pragma unroll
  for (int r = 0; r < R; r++)
    wv[r] = ld_weights16_u4(W + (int64_t)colr[r] * col_bytes + (int64_t)cc * 16);
  // every load above is in flight before any arithmetic (see k_gemv_valu)
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ATTN) {  // merge, then the chunk's runs k = base + 16 j + e out of LDS
    mg.finish(pa, sx);
    const float *xr = sx + s * kSegK + 8 * g;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 a0 = *(const float4 *)(xr + 16 * j);
      const float4 a1 = *(const float4 *)(xr + 16 * j + 4);
      av[8 * j + 0] = a0.x; av[8 * j + 1] = a0.y; av[8 * j + 2] = a0.z; av[8 * j + 3] = a0.w;
      av[8 * j + 4] = a1.x; av[8 * j + 5] = a1.y; av[8 * j + 6] = a1.z; av[8 * j + 7] = a1.w;
    }
  }
  if constexpr (NORM) {
    float ss = 0.0f;
    if (h == 0 && cv) {
#pragma unroll
      for (int e = 0; e < 32; e++) ss = fmaf(av[e], av[e], ss);
    }
    ss = half_wave_sum(ss);
    if (l == 0) nrm[w] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int ww = 0; ww < nw; ww++) tot += nrm[ww];
    const float inv = (float)(1.0 / sqrt((double)tot / (double)K + (double)eps));
#pragma unroll
    for (int e = 0; e < 32; e++) av[e] = av[e] * inv * gv[e];
  }
  // ---- arithmetic: exact (q - 8) / 16 per weight (dq_nibbles), the 16
  // folded into the block's scale; column by column, so that column r waits only for its own
  // weights.  The empty asm pins each column's sum in its place: without it
  // the compiler sinks the FMAs of every column but the first to the end,
  // keeping all 8R dequantised values live (270 VGPRs at R = 8).
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float qv[8];
      dq_nibbles<false>(wd[j], 0u, qv);
#pragma unroll
      for (int e = 0; e < 8; e++) d = fmaf(av[8 * j + e], qv[e], d);
    }
    const float sc = cv ? sraw[r] * dq_unscale<false>() : 0.0f;
    acc[r] = sc * d;
    asm volatile("" : "+v"(acc[r]));
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- reductions: 32 lanes of a half-wave, then the waves
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float v = half_wave_sum(acc[r]);
    if (t == 0) red[w][2 * r + h] = v;
  }
  __syncthreads();
  float v = 0.0f;
  const int i = threadIdx.x;
  if (i < 2 * R) {
    for (int ww = 0; ww < nw; ww++) v += red[ww][i];
  }
  const int col = col0 + i;
  if constexpr (EPI == kDecPlain) {
    if (i < 2 * R && col < N) Y[col] = v;
  } else if constexpr (EPI == kDecResidual) {
    if (i < 2 * R && col < N) Y[col] = rres + v;
  } else if constexpr (EPI == kDecSwiglu) {
    if (i < 2 * R) outv[i] = v;
    __syncthreads();
    if (i < R && col0 + 2 * i + 1 < N) {
      const float gg = outv[2 * i], uu = outv[2 * i + 1];
      const float sig = 1.0f / (1.0f + expf(-gg));
      Y[col0 / 2 + i] = (gg * sig) * uu;
    }
  } else {  // kDecArgmax: this workgroup's best key, reduced by the caller
    __shared__ unsigned long long keys[2 * R];
    if (i < 2 * R) {
      if (col < N) Y[col] = v;
      keys[i] = col < N ? argmax_key(v, col) : 0ull;
    }
    __syncthreads();
    if (i == 0) {
      unsigned long long best = keys[0];
      for (int q = 1; q < 2 * R; q++) best = keys[q] > best ? keys[q] : best;
      argmax[blockIdx.x] = best;
    }
  }
}

// Columns per wave half R: the largest that keeps two waves per SIMD slot
// of the chip (workgroups x waves >= 2 x CUs; nw waves split K).  Measured
// on the Qwen3-0.6B decode step: o and down (N = 1024, 2-3 waves) at R = 2
// and q|k|v, gate/up (N = 4096, 6144, one wave) at R = 4 beat every other
// pairing by 0.8-4%.
static int dec_gemv_r(const mmnb_ctx *ctx, int64_t n, int nw) {
  int R = 8;
  while (R > 1 && (n + 2 * R - 1) / (2 * R) * nw < 2 * (int64_t)ctx->cu_count) R >>= 1;
  return R;
}

static int dec_gemv_waves(int64_t k) { return (int)((k / 32 + 31) / 32); }

int64_t dec_gemv_blocks(const mmnb_ctx *ctx, int64_t n, int64_t k) {
  const int R = dec_gemv_r(ctx, n, dec_gemv_waves(k));
  return (n + 2 * R - 1) / (2 * R);
}

int launch_dec_gemv(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_x,
                    const float *norm_gamma, float eps, int epi, const float *resid,
                    float *d_y, unsigned long long *d_argmax) {
  if (p->has_zp || p->block < 64 || p->generic)
    return fail(MMNB_ERR_UNSUPPORTED,
                "decoder GEMV: needs a power-of-two block >= 64 and no zero points");
  if (p->k % kSegK != 0 || p->k > 4096)
    return fail(MMNB_ERR_UNSUPPORTED, "decoder GEMV: K must be a multiple of 64, <= 4096");
  const int C = (int)(p->col_bytes / 16);
  const int nw = (C + 31) / 32;
  const int64_t n = p->n;
  const int R = dec_gemv_r(ctx, n, dec_gemv_waves(p->k));
  const dim3 grid((unsigned)((n + 2 * R - 1) / (2 * R)));
  const dim3 block((unsigned)(64 * nw));
  const int bs_log2 = ilog2(p->block);
  const bool norm = norm_gamma != nullptr;
  const int kid = epi == kDecResidual ? kKernDecGemvRes
                  : epi == kDecSwiglu ? kKernDecGemvGlu
                  : epi == kDecArgmax ? kKernDecGemvLm : kKernDecGemv;
#define MMNB_DEC(RR, NN, EE)                                                                   \
  return launch(ctx, kid, k_dec_gemv<RR, NN, EE>, grid, block, 0, d_x, norm_gamma, eps,         \
                p->d_w, p->col_bytes, p->d_scales, (int)p->n_blocks, bs_log2, (int)p->k,     \
                (int)n, resid, d_y, d_argmax, C, DecAttnPartials{})
#define MMNB_DEC_R(NN, EE)              \
  {                                     \
    if (R == 8) MMNB_DEC(8, NN, EE);    \
    if (R == 4) MMNB_DEC(4, NN, EE);    \
    if (R == 2) MMNB_DEC(2, NN, EE);    \
    MMNB_DEC(1, NN, EE);                \
  }
  if (epi == kDecResidual && !norm) MMNB_DEC_R(false, kDecResidual);
  if (epi == kDecSwiglu && norm) MMNB_DEC_R(true, kDecSwiglu);
  if (epi == kDecArgmax && norm) MMNB_DEC_R(true, kDecArgmax);
  if (epi == kDecPlain && norm) MMNB_DEC_R(true, kDecPlain);
  if (epi == kDecPlain && !norm) MMNB_DEC_R(false, kDecPlain);
#undef MMNB_DEC_R
#undef MMNB_DEC
  return fail(MMNB_ERR_UNSUPPORTED, "decoder GEMV: unsupported prologue/epilogue pair");
}

int launch_dec_gemv_attn(mmnb_ctx *ctx, const mmnb_pack *p, const DecAttnPartials &pa,
                         const float *resid, float *d_y) {
  if (p->has_zp || p->block < 64 || p->generic)
    return fail(MMNB_ERR_UNSUPPORTED,
                "decoder GEMV: needs a power-of-two block >= 64 and no zero points");
  if (p->k % kSegK != 0 || p->k > kDecAttnMaxK)
    return fail(MMNB_ERR_UNSUPPORTED, "decoder GEMV (attention merge): K must be a multiple "
                                      "of 64, <= 2048");
  if (!pa.o || !pa.ml || pa.nsmax < 1 || pa.nsmax > kDecAttnMaxSplits ||
      pa.hd < 4 || pa.hd % 4 != 0 || p->k % pa.hd != 0 ||
      p->k / pa.hd * (pa.nsmax <= 8 ? 8 : 16) > kDecAttnMergeThreads)
    return fail(MMNB_ERR_ARG, "decoder GEMV (attention merge): bad partials");
  const int C = (int)(p->col_bytes / 16);
  const int64_t n = p->n;
  const int R = dec_gemv_r(ctx, n, dec_gemv_waves(p->k));
  const dim3 grid((unsigned)((n + 2 * R - 1) / (2 * R)));
  const dim3 block((unsigned)kDecAttnMergeThreads);  // = 64 * kDecMaxWaves
  const int bs_log2 = ilog2(p->block);
#define MMNB_DEC(RR, NS)                                                                      \
  return launch(ctx, kKernDecGemvRes, k_dec_gemv<RR, false, kDecResidual, NS>, grid, block,   \
                0, pa.o, nullptr, 0.0f, p->d_w, p->col_bytes, p->d_scales, (int)p->n_blocks,  \
                bs_log2, (int)p->k, (int)n, resid, d_y, nullptr, C, pa)
#define MMNB_DEC_NS(RR)                   \
  {                                       \
    if (pa.nsmax <= 2) MMNB_DEC(RR, 2);   \
    if (pa.nsmax <= 4) MMNB_DEC(RR, 4);   \
    if (pa.nsmax <= 6) MMNB_DEC(RR, 6);   \
    if (pa.nsmax <= 8) MMNB_DEC(RR, 8);   \
    if (pa.nsmax <= 12) MMNB_DEC(RR, 12); \
    MMNB_DEC(RR, 16);                     \
  }
  if (R == 8) MMNB_DEC_NS(8);
  if (R == 4) MMNB_DEC_NS(4);
  if (R == 2) MMNB_DEC_NS(2);
  MMNB_DEC_NS(1);
#undef MMNB_DEC_NS
#undef MMNB_DEC
}

// ---------------------------------------------------------------------------
// Decode-shape GEMV for 2 <= M <= 8, activations staged in LDS.
//
// Holding a chunk's 32 activations per row in registers (the M = 1 kernel)
// costs 32*M VGPRs and re-reads A through L1 for every pair of columns; at
// M = 8 that spills.  Here the workgroup first copies A (all rows, K padded
// to the staged chunk range, zeros past K) into LDS in chunk-major order,
//     slot((m, j, h4), c) = ((m*4 + j)*2 + h4) * P + c    (float4 slots)
// holding k = 64(c/2) + 16j + 8(c%2) + 4*h4 .. +3, so the 32 lanes of a
// half-wave (consecutive chunks c) read consecutive 16-byte slots (no bank
// conflicts; P = slots + 1 spreads the staging writes over banks).
//
// Work split: a "column group" is 2R columns; kw waves split its K (lane
// (w, h, t) owns chunk 32w + t (+ 32*kw per iteration) of columns 2r + h,
// r < R).  A workgroup runs cg column groups side by side (cg*kw waves)
// and walks the groups grid-stride, reusing the staged activations.  Per
// dword j of a chunk a lane reads its 8*M activations once and applies them
// to its R columns.  Each nibble becomes the exact (q - zp), scaled by a
// power of two (dq_nibbles), before the fp32 FMAs.
// ---------------------------------------------------------------------------
// Weight, scale and zero-point loads of one chunk (lane's chunk c of its R
// columns); kept separate so the first group's loads can be issued before
// the activations are staged.
template <int R, int NBPC, bool HAS_ZP>
struct GemvChunk {
  u4vec wv[R];
  float sraw[R][NBPC];
  uint32_t zraw[R][NBPC];
  int zsh[R][NBPC];
  bool inbq[NBPC];

  __device__ __forceinline__ void load(const uint8_t *__restrict__ W, int64_t col_bytes,
                                       const float *__restrict__ S,
                                       const uint8_t *__restrict__ Z, int nb, int bs_log2,
                                       const int (&colr)[R], int c, int C) {
    const bool cv = c < C;
    const int cc = cv ? c : 0;
    const int s = cc >> 1, gg = cc & 1;
#pragma unroll
    for (int r = 0; r < R; r++)
      wv[r] = ld_weights16(W + (int64_t)colr[r] * col_bytes + (int64_t)cc * 16);
#pragma unroll
    for (int q = 0; q < NBPC; q++) {
      const int kq = s * kSegK + 16 * (q * (4 / NBPC)) + (NBPC == 4 ? 8 * gg : 0);
      int blk = kq >> bs_log2;
      inbq[q] = cv && blk < nb;
      blk = blk < nb ? blk : nb - 1;
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int zi = colr[r] * nb + blk;
        sraw[r][q] = S[zi];
        if (HAS_ZP) zraw[r][q] = Z[zi >> 1];
        zsh[r][q] = (zi & 1) * 4;
      }
    }
  }
};

template <int M, int R, int NBPC, bool HAS_ZP>
__global__ __launch_bounds__(512) void k_gemv_lds(
    const float *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W,
    int64_t col_bytes, const float *__restrict__ S, const uint8_t *__restrict__ Z, int nb,
    int bs_log2, int K, int N, float *__restrict__ Y, int C, int kw, int iters, int groups,
    int vec) {
  extern __shared__ float4 sact[];
  __shared__ float red[8][M][2 * R];
  kernarg_fence(A, lda, W, col_bytes, S, Z, nb, bs_log2, K, N, Y, C, kw, iters, groups, vec,
                blockDim.x, gridDim.x);
  const int cs = 32 * kw * iters;  // staged chunk slots
  const int P = cs + 1;            // slot pitch (float4)
  const int nthr = blockDim.x;
  const int cg = nthr / (64 * kw);  // column groups side by side
  const int wg = threadIdx.x >> 6;        // wave in workgroup
  const int sub = wg / kw, w = wg % kw;   // column group slot, K part
  const int l = threadIdx.x & 63, h = l >> 5, t = l & 31;

  int g0 = blockIdx.x * cg;
  int colr[R];
  auto set_cols = [&](int gbase) {
    const int g = gbase + sub;
    const int col0 = (g < groups ? g : 0) * (2 * R);
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int c = col0 + 2 * r + h;
      colr[r] = c < N ? c : N - 1;
    }
  };
  // first group's weights in flight before the activations are staged
  GemvChunk<R, NBPC, HAS_ZP> ch;
  set_cols(g0);
  ch.load(W, col_bytes, S, Z, nb, bs_log2, colr, 32 * w + t, C);

  // ---- stage A -> LDS: up to 8 independent 16-byte loads per thread in flight
  const int k4n = cs * 8;  // float4 per row
  const int total = M * k4n;
  for (int base = threadIdx.x; base < total; base += 8 * nthr) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = base + u * nthr;
      const int m = i / k4n, k = 4 * (i - m * k4n);
      const float *ar = A + (int64_t)m * lda + k;
      if (i >= total) {
        v[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      } else if (vec && k + 4 <= K) {
        v[u] = *(const float4 *)ar;
      } else {
        v[u].x = k + 0 < K ? ar[0] : 0.0f;
        v[u].y = k + 1 < K ? ar[1] : 0.0f;
        v[u].z = k + 2 < K ? ar[2] : 0.0f;
        v[u].w = k + 3 < K ? ar[3] : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = base + u * nthr;
      if (i < total) {
        const int m = i / k4n, k = 4 * (i - m * k4n);
        const int c = 2 * (k >> 6) + ((k >> 3) & 1);
        const int j = (k >> 4) & 3, h4 = (k >> 2) & 1;
        sact[((m * 4 + j) * 2 + h4) * P + c] = v[u];
      }
    }
  }
  __syncthreads();

  for (; g0 < groups; g0 += gridDim.x * cg) {
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
      for (int r = 0; r < R; r++) acc[m][r] = 0.0f;

    for (int it = 0; it < iters; it++) {
      const int c = 32 * w + t + it * 32 * kw;  // < cs: a staged slot
      if (it > 0) ch.load(W, col_bytes, S, Z, nb, bs_log2, colr, c, C);
      float d[M][R];
#pragma unroll
      for (int m = 0; m < M; m++)
#pragma unroll
        for (int r = 0; r < R; r++) d[m][r] = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int q = j / (4 / NBPC);
        float av[M][8];
#pragma unroll
        for (int m = 0; m < M; m++) {
          const float4 x0 = sact[((m * 4 + j) * 2 + 0) * P + c];
          const float4 x1 = sact[((m * 4 + j) * 2 + 1) * P + c];
          av[m][0] = x0.x; av[m][1] = x0.y; av[m][2] = x0.z; av[m][3] = x0.w;
          av[m][4] = x1.x; av[m][5] = x1.y; av[m][6] = x1.z; av[m][7] = x1.w;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t zc =
              HAS_ZP ? dq8_const((int)((ch.zraw[r][q] >> ch.zsh[r][q]) & 0xF)) : 0u;
          // exact scaled (q - zp), one SDWA convert per nibble (dq_nibbles)
          float qv[8];
          dq_nibbles<HAS_ZP>(ch.wv[r][j], zc, qv);
#pragma unroll
          for (int m = 0; m < M; m++) {
            float x = d[m][r];
#pragma unroll
            for (int e = 0; e < 8; e++) x = fmaf(av[m][e], qv[e], x);
            d[m][r] = x;
          }
        }
        if (((j + 1) % (4 / NBPC)) == 0) {
#pragma unroll
          for (int r = 0; r < R; r++) {
            const float sc = ch.inbq[q] ? ch.sraw[r][q] * dq_unscale<HAS_ZP>() : 0.0f;
#pragma unroll
            for (int m = 0; m < M; m++) {
              acc[m][r] = fmaf(sc, d[m][r], acc[m][r]);
              d[m][r] = 0.0f;
            }
          }
        }
      }
    }
    // next group's first chunk in flight during the reductions
    const int g1 = g0 + gridDim.x * cg;
    if (g1 < groups) {
      set_cols(g1);
      ch.load(W, col_bytes, S, Z, nb, bs_log2, colr, 32 * w + t, C);
    }
    // ---- reductions: 32 lanes of a half-wave, then the kw waves of the group
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
      for (int r = 0; r < R; r++) {
        const float v = half_wave_sum(acc[m][r]);
        if (t == 0) red[wg][m][2 * r + h] = v;
      }
    __syncthreads();
    for (int i = threadIdx.x; i < cg * M * 2 * R; i += nthr) {
      const int sg = i / (M * 2 * R), rem = i % (M * 2 * R);
      const int m = rem / (2 * R), cl = rem % (2 * R);
      const int gi = g0 + sg;
      float v = 0.0f;
      for (int ww = 0; ww < kw; ww++) v += red[sg * kw + ww][m][cl];
      const int col = gi * (2 * R) + cl;
      if (gi < groups && col < N) Y[(int64_t)m * N + col] = v;
    }
    __syncthreads();
  }
}

template <int M, int R>
static int launch_gemv_lds_mr(mmnb_ctx *ctx, int nbpc, dim3 grid, dim3 block, size_t shmem,
                              const float *A, int64_t lda, const mmnb_pack *p, float *Y,
                              int C, int kw, int iters, int groups, int vec, int bs_log2) {
  const int nb = (int)p->n_blocks, K = (int)p->k, N = (int)p->n;
#define MMNB_GEMV_LDS_LAUNCH(Q, ZP)                                                          \
  {                                                                                          \
    auto kern = k_gemv_lds<M, R, Q, ZP>;                                                     \
    if (shmem > 65536) {                                                                     \
      hipError_t e_ = hipFuncSetAttribute((const void *)kern,                               \
                                          hipFuncAttributeMaxDynamicSharedMemorySize,        \
                                          (int)shmem);                                       \
      if (e_ != hipSuccess) return check_hip(e_, "hipFuncSetAttribute");                     \
    }                                                                                        \
    return launch(ctx, kKernGemv, kern, grid, block, shmem, A, lda, p->d_w, p->col_bytes,   \
                  p->d_scales, p->d_zp, nb, bs_log2, K, N, Y, C, kw, iters, groups, vec);   \
  }
  if (p->has_zp) {
    if (nbpc == 4) MMNB_GEMV_LDS_LAUNCH(4, true);
    if (nbpc == 2) MMNB_GEMV_LDS_LAUNCH(2, true);
    MMNB_GEMV_LDS_LAUNCH(1, true);
  }
  if (nbpc == 4) MMNB_GEMV_LDS_LAUNCH(4, false);
  if (nbpc == 2) MMNB_GEMV_LDS_LAUNCH(2, false);
  MMNB_GEMV_LDS_LAUNCH(1, false);
#undef MMNB_GEMV_LDS_LAUNCH
}

template <int M>
static int launch_gemv_lds_m(mmnb_ctx *ctx, int R, int nbpc, dim3 grid, dim3 block,
                             size_t shmem, const float *A, int64_t lda, const mmnb_pack *p,
                             float *Y, int C, int kw, int iters, int groups, int vec,
                             int bs_log2) {
  if (R == 4)
    return launch_gemv_lds_mr<M, 4>(ctx, nbpc, grid, block, shmem, A, lda, p, Y, C, kw, iters,
                                    groups, vec, bs_log2);
  if (R == 2)
    return launch_gemv_lds_mr<M, 2>(ctx, nbpc, grid, block, shmem, A, lda, p, Y, C, kw, iters,
                                    groups, vec, bs_log2);
  return launch_gemv_lds_mr<M, 1>(ctx, nbpc, grid, block, shmem, A, lda, p, Y, C, kw, iters,
                                  groups, vec, bs_log2);
}


static int launch_gemm(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                       int64_t m, float *d_y);

// Waves splitting K (kw), chunk iterations and staged-activation LDS bytes
// of the multi-row GEMV for M rows.
static size_t gemv_multi_lds(const mmnb_pack *p, int64_t m, int *kw_out, int *iters_out) {
  const int C = (int)(p->col_bytes / 16);
  int kw = (C + 31) / 32, iters = 1;
  if (kw > 4) {
    iters = (kw + 3) / 4;
    kw = (C + 32 * iters - 1) / (32 * iters);
  }
  if (kw_out) *kw_out = kw;
  if (iters_out) *iters_out = iters;
  const int cs = 32 * kw * iters;
  return (size_t)m * 8 * (cs + 1) * 16;
}

// Whether 2 <= M <= 8 rows of A fit the multi-row GEMV's LDS (the kernel
// also holds a static 8 x M x 8 float reduction buffer).
static bool gemv_multi_fits(const mmnb_ctx *ctx, const mmnb_pack *p, int64_t m) {
  return gemv_multi_lds(p, m, nullptr, nullptr) + 8 * 8 * 8 * 4 <= (size_t)ctx->lds_max;
}

// 2 <= M <= 8: the LDS-staged kernel, or the MFMA GEMM when A does not fit
// the workgroup's LDS.
static int launch_gemv_multi(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a,
                             int64_t lda, int64_t m, float *d_y) {
  const int C = (int)(p->col_bytes / 16);
  int kw, iters;
  const size_t shmem = gemv_multi_lds(p, m, &kw, &iters);
  if (!gemv_multi_fits(ctx, p, m)) return launch_gemm(ctx, p, d_a, lda, m, d_y);
  const int64_t n = p->n;
  // Every workgroup stages all of A, so fewer, wider workgroups win: up to
  // 8 waves (cg column groups of kw waves), then the most columns per lane
  // (R) that still leaves a workgroup on three quarters of the CUs.
  int cg = 8 / kw;
  if (ctx->gemv_cg > 0 && ctx->gemv_cg * kw <= 8) cg = ctx->gemv_cg;  // tuning override
  int R = 4;
  while (R > 1 && (n + 2 * R * cg - 1) / (2 * R * cg) < 3 * ctx->cu_count / 4) R >>= 1;
  if (ctx->gemv_r > 0 && ctx->gemv_r <= 4) R = ctx->gemv_r;  // tuning override
  const int groups = (int)((n + 2 * R - 1) / (2 * R));
  const dim3 grid((unsigned)((groups + cg - 1) / cg));
  const dim3 block((unsigned)(64 * kw * cg));
  const int vec = ((lda % 4 == 0) && (((uintptr_t)d_a & 15) == 0)) ? 1 : 0;
  const int bs_log2 = ilog2(p->block);
  const int nbpc = p->block >= 64 ? 1 : (p->block == 32 ? 2 : 4);
  switch (m) {
#define MMNB_CASE(MM)                                                                        \
  case MM:                                                                                   \
    return launch_gemv_lds_m<MM>(ctx, R, nbpc, grid, block, shmem, d_a, lda, p, d_y, C, kw, \
                                 iters, groups, vec, bs_log2);
    MMNB_CASE(2)
    MMNB_CASE(3)
    MMNB_CASE(4)
    MMNB_CASE(5)
    MMNB_CASE(6)
    MMNB_CASE(7)
    MMNB_CASE(8)
#undef MMNB_CASE
    default:
      return fail(MMNB_ERR_ARG, "GEMV: M out of range");
  }
}

static int launch_gemv(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                       int64_t m, float *d_y) {
  if (m > 1) return launch_gemv_multi(ctx, p, d_a, lda, m, d_y);
  const int C = (int)(p->col_bytes / 16);  // chunks per column
  // waves splitting K: one chunk per lane up to 4 waves, then iterate
  int nw = (C + 31) / 32;
  int iters = 1;
  if (nw > kGemvMaxWaves) {
    iters = (nw + kGemvMaxWaves - 1) / kGemvMaxWaves;
    nw = (C + 32 * iters - 1) / (32 * iters);
  }
  // columns per workgroup 2R.  Timed over R = 1, 2, 4, 8 at (K, N) =
  // (1024, 1024 / 2048 / 6144), (2048, 2048), (3072, 1024), (4096, 4096),
  // (4096, 14336), (14336, 4096), (8192, 8192), (16384, 16384) and
  // (1024, 151936): R = 2 was best up to 8.4 MB of packed weights (within 3%
  // of R = 1 at (2048, 2048)), R = 4 from 29 MB up (every workgroup reads the
  // whole activation row from L2, so more workgroups cost more there)
  const int64_t n = p->n;
  int R = p->col_bytes * n > ((int64_t)16 << 20) ? 4 : 2;
  if (ctx->gemv_r > 0) R = ctx->gemv_r;  // tuning override
  const dim3 grid((unsigned)((n + 2 * R - 1) / (2 * R)));
  const dim3 block((unsigned)(64 * nw));
  // Aligned float4 path: every 8-float run of a chunk lies inside the row,
  // i.e. rows hold k64 values (zero padded past K by the host entry point, or
  // K itself is a multiple of 64).
  const bool f = (lda % 4 == 0) && (((uintptr_t)d_a & 15) == 0) && (lda >= p->k64);
  const int bs_log2 = ilog2(p->block);
  const int nbpc = p->block >= 64 ? 1 : (p->block == 32 ? 2 : 4);
  if (R == 8) return launch_gemv_r<8>(ctx, nbpc, grid, block, d_a, p, d_y, C, iters, f, bs_log2);
  if (R == 4) return launch_gemv_r<4>(ctx, nbpc, grid, block, d_a, p, d_y, C, iters, f, bs_log2);
  if (R == 2) return launch_gemv_r<2>(ctx, nbpc, grid, block, d_a, p, d_y, C, iters, f, bs_log2);
  return launch_gemv_r<1>(ctx, nbpc, grid, block, d_a, p, d_y, C, iters, f, bs_log2);
}

// ---------------------------------------------------------------------------
// Activation prep for the MFMA GEMM.
//
// Each row m of A is scaled by 2^e_m (e_m chosen so max|a| * 2^e_m lies in
// [2^13, 2^14)) and split into two fp16 terms, hi = fp16(a'), lo = fp16(a' -
// hi); |a' - hi - lo| <= 2^-22 |a'| (or 2^-25 absolute in fp16's subnormal
// range).  The weights (q - zp) are exact small integers in fp16, so both
// MFMA passes form exact products and accumulate in fp32.
//
// Output layout: one 1 KB unit per (32-row block rb, 64-k segment s, 16-k
// step j, part p) holding the 32x16 A operand of v_mfma_f32_32x32x16_f16 in
// lane order: lane l -> row rb*32 + l%32, k = 64s + 16j + 8(l/32) + perm[e],
// perm = {0,4,1,5,2,6,3,7} (the order the weight dequantisation produces).
// Rows >= M and k >= K are zero.
//
// One launch.  A 128-byte line of a unit holds one half (16 B) of 8
// consecutive rows, so rows go in groups of 8 whose lines one XCD writes,
// and its L2 merges the 16-byte pieces of a line before write-back: a
// workgroup owns one row, and the 8 workgroups of a group are b, b + 8, ...,
// b + 56 of each 64 (workgroups are dealt to the 8 XCDs round robin, so all
// 8 land on one XCD; the mapping only matters for speed).  Eight waves per
// row, each covering 512 k of every 4096-k chunk; lane l reads 8 consecutive
// k (two float4) at 8 l.  The row's maximum over K (first chunk kept in
// registers, so K <= 4096 reads A once), then the conversion.  Measured
// against 4 rows per workgroup with two waves per row (K = N = 4096, bs32 +
// zp, prep per call 6.8 / 7.3 / 8.7 / 18.6 us at M = 128 / 256 / 512 / 2048,
// against 5.0 / 5.7 / 7.2 / 16.6 us here; 2 rows with four waves per row
// fell in between), one workgroup of 8 rows (11.3 against 8.2 us at M = 512)
// and 2-row workgroups with 16-k lanes (21.5 against 17.5 us at M = 2048).
// ---------------------------------------------------------------------------
constexpr int kPrepWaves = 8;     // waves per row (one row per workgroup)
constexpr int kPrepChunk = 4096;  // k per pass of a row's waves

__global__ __launch_bounds__(64 * kPrepWaves) void k_prep_a(
    const float *__restrict__ A, int64_t lda, int64_t M, int64_t K, int64_t segsp,
    int *__restrict__ row_exp, uint4 *__restrict__ out, int *__restrict__ clear, int nclear,
    int nblocks) {
  // every argument in SGPRs up front (one round of scalar loads); the grid
  // size comes as an argument: gridDim.x was a vector load of the hidden
  // arguments, waited for (vmcnt(0)) before the first load of A
  kernarg_fence(A, lda, M, K, segsp, row_exp, out, clear, nclear, nblocks);
  // the GEMM's K-slice counters when they live in a caller's workspace:
  // zeroed here, before the GEMM (the next launch on the stream) counts in
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < nclear; i += 64 * kPrepWaves) clear[i] = 0;
  __shared__ float wmax[kPrepWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int b = blockIdx.x;
  const int64_t row = b / 64 < nblocks / 64
                          ? (int64_t)(b / 64 * 8 + b % 8) * 8 + (b % 64) / 8
                          : (int64_t)b;
  const int64_t kp = segsp * kSegK;  // padded K
  const bool vec = ((lda & 3) == 0) && ((((uintptr_t)A) & 15) == 0);
  auto load8 = [&](int64_t k0, float *v) {
    const float *ar = A + row * lda + k0;
    if (row < M && vec && k0 + 8 <= K) {
      const float4 x0 = *(const float4 *)ar;
      const float4 x1 = *(const float4 *)(ar + 4);
      v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
      v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (row < M && k0 + e < K) ? ar[e] : 0.0f;
    }
  };
  const int kl = (kPrepChunk / kPrepWaves) * wave + 8 * lane;
  // ---- the row's maximum (first chunk kept)
  float keep[8];
  load8(kl, keep);
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) mx = fmaxf(mx, finite_abs(keep[e]));
  int64_t k0 = kPrepChunk;
  for (; k0 + 3 * kPrepChunk < K; k0 += 4 * kPrepChunk) {  // four loads in flight
    float v[4][8];
#pragma unroll
    for (int u = 0; u < 4; u++) load8(k0 + u * kPrepChunk + kl, v[u]);
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int e = 0; e < 8; e++) mx = fmaxf(mx, finite_abs(v[u][e]));
  }
  for (; k0 < K; k0 += kPrepChunk) {
    float v[8];
    load8(k0 + kl, v);
#pragma unroll
    for (int e = 0; e < 8; e++) mx = fmaxf(mx, finite_abs(v[e]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  float rm = wmax[0];
#pragma unroll
  for (int w = 1; w < kPrepWaves; w++) rm = fmaxf(rm, wmax[w]);
  const int ex = prep_a_exponent(rm);
  if (t == 0 && row < M) row_exp[row] = ex;
  // ---- convert: 8 k (one half of a 16-k step) per lane and chunk
  for (int64_t k0 = 0; k0 < kp; k0 += kPrepChunk) {
    const int64_t kk = k0 + kl;
    if (kk < kp) {  // kp is a multiple of 64: the 8 k lie inside
      float v[8];
      if (k0 == 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = keep[e];
      } else {
        load8(kk, v);
      }
      prep_a_store8(out, segsp, row, kk & ~(int64_t)15, (int)((kk >> 3) & 1), v, ex);
    }
  }
}

static int launch_prep_a(mmnb_ctx *ctx, const float *d_a, int64_t lda, int64_t m, int64_t k,
                         int64_t mpad, int64_t segsp, int *d_exp, uint4 *d_ap, int *clear,
                         int nclear) {
  return launch(ctx, kKernPrep, k_prep_a, dim3((unsigned)mpad), dim3(64 * kPrepWaves), 0, d_a,
                lda, m, k, segsp, d_exp, d_ap, clear, nclear, (int)mpad);
}

// ---------------------------------------------------------------------------
// Prefill GEMM, fed by direct global->LDS DMA.
//
// Workgroup tile 64 (M) x 128*CB (N).  A group of 4 waves in 1 x 4 owns the
// tile over a range of K: wave tile 64 x 32*CB (both 32-row A blocks, CB
// 32-column weight blocks, so every weight is dequantised once per group and
// every A fragment read from LDS feeds CB column blocks).  GROUPS = 2 splits
// K between two such groups (8 waves, two per SIMD) when the tiles alone
// leave a single wave per SIMD; the partial tiles are summed through LDS at
// the end.
//
// Every operand of a 64-k segment -- the prepared activations (16 KB), the
// packed weights (128*CB columns x 32 B), the tile's scales and zero points
// (from block-major copies, so one block's columns are contiguous and move
// as 16 B per lane) -- is copied by buffer_load_dwordx4 ... lds into one of
// NST LDS stages, so NST-1 segments are in flight without a register round
// trip.  (The buffer form rather than global_load_lds: after a pending FLAT
// DMA the compiler waits for every outstanding LDS read before the first
// MFMA of a matrix phase; with buffer loads it waits per fragment.  M = 512,
// K = N = 4096 kernel, one device: block 128 39.7 -> 36.5 us, block 32
// 41.0 -> 40.8 us.)
// Every thread issues the same number of DMA loads per stage (kL), so "stage
// s has landed" is vmcnt <= (NST-2)*kL once the next stages are issued; a
// barrier then publishes the stage to all waves.
//
// Each 16-k step issues 2 (row blocks) x CB x 2 (hi, lo)
// v_mfma_f32_32x32x16_f16 into the partial set of its quantisation block
// (zero accumulator input at the block's first step); acc += scale[n, blk]
// * partials is applied while the next block's MFMAs run (two sets).
// ---------------------------------------------------------------------------
constexpr int kGemmBM = 64;   // two 32-row blocks
constexpr int kGemmBN = 128;  // four 32-column blocks
constexpr int kGemmGroup = 2; // row bands per tile group (L2 reuse of A)


template <int NBPS, int NST, int GROUPS, int CB>
__global__ __launch_bounds__(256 * GROUPS) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_mfma(
    const uint4 *__restrict__ Ap, const int *__restrict__ row_exp, int segs, int segsp,
    const uint8_t *__restrict__ W, int64_t col_bytes, const float *__restrict__ ST,
    const uint32_t *__restrict__ ZT, int ldsz, int nb, int bs_log2, int M, int N, int grid_x,
    int grid_y, float *__restrict__ Y, int ksplit, float *__restrict__ part,
    int *__restrict__ tile_cnt) {
  constexpr int kBN = kGemmBN * CB;                    // columns per workgroup tile
  constexpr int kSz = kBN * NBPS;                       // scale (and zero-point) dwords per stage
  constexpr int kStageU4 = 1024 + 256 * CB + kSz / 2;   // uint4 per stage: A, W, scales + zp
  constexpr int kSzI = CB * NBPS / 4 > 0 ? CB * NBPS / 4 : 1;  // 1 KB scale/zp loads per wave
  constexpr int kL = 4 + CB + kSzI;                     // DMA loads per thread per stage
  constexpr int kSOff = 1024 + 256 * CB;                // scales / zero points in a stage
  constexpr bool kPingPong = GROUPS == 2 && CB == 1;
  extern __shared__ uint4 smem_all[];
  // wave-uniform indices in scalar registers
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wid >> 2, wave = wid & 3;
  const int tid = threadIdx.x & 255, lane = tid & 63;
  const int cl = lane & 31, g = lane >> 5;
  const uint32_t magic = 0x64006400u;
  uint4 *smem = smem_all + grp * NST * kStageU4;
  kernarg_fence(Ap, row_exp, segs, segsp, W, col_bytes, ST, ldsz, nb, bs_log2, M, N, grid_x,
                grid_y, Y, ksplit, part, tile_cnt);

  // XCD-aware tile order: consecutive workgroup ids go to different XCDs
  // (round robin), so regroup them into contiguous chunks per XCD, then walk
  // the chunk kGemmGroup row bands at a time.  With ksplit > 1 the ksplit
  // consecutive ids of a chunk are one tile's K slices.
  const int Gt = grid_x * grid_y * ksplit;
  int L = blockIdx.x;
  if ((Gt & 7) == 0) L = (L & 7) * (Gt >> 3) + (L >> 3);
  const int split = L % ksplit;
  L /= ksplit;
  const int tile = L;
  // this group's contiguous segment range [sbeg, sbeg + nseg) of the slice
  const int nseg = segsp / (GROUPS * ksplit);
  const int sbeg = (split * GROUPS + grp) * nseg;
  const int per_group = kGemmGroup * grid_x;
  const int first_y = (L / per_group) * kGemmGroup;
  const int rows_in_group = min(grid_y - first_y, kGemmGroup);
  const int ty = first_y + (L % per_group) % rows_in_group;
  const int tx = (L % per_group) / rows_in_group;
  const int rb0 = ty * 2;
  const int n0 = tx * kBN;
  // the exponent of tile row `lane`, loaded now (it is ready long before the
  // epilogue, which takes it from this lane by a shuffle instead of a memory
  // round trip after the K loop)
  const int rexp = row_exp[min(rb0 * 32 + lane, M - 1)];

  // DMA sources, as buffer resources of the tile's operands with per-lane
  // byte offsets (the stage's part in the scalar offset).  Activations:
  // thread's unit pieces idx = tid + 256 i (unit idx/64 = row block
  // (idx/64)/8, step*2+part (idx/64)%8); the prepared buffer holds segsp
  // segments of 8 KB per row block, zero past K.
  const __amdgpu_buffer_rsrc_t a_rs = buf_rsrc(Ap + (size_t)rb0 * segsp * 8 * 64);
  uint32_t a_off[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int idx = tid + 256 * i;
    const int u = idx >> 6;
    a_off[i] = (uint32_t)(((u >> 3) * segsp * 8 + (u & 7)) * 64 + (idx & 63)) * 16u;
  }
  // nibbles: columns n0 .. (clamped to N - 1), 32 bytes per segment
  const __amdgpu_buffer_rsrc_t w_rs = buf_rsrc(W + (size_t)n0 * col_bytes);
  uint32_t w_off[CB];
#pragma unroll
  for (int i = 0; i < CB; i++) {
    const int wcol = min(n0 + 128 * i + (tid >> 1), N - 1);
    w_off[i] = (uint32_t)((wcol - n0) * col_bytes) + (tid & 1) * 16u;
  }
  // Scale / zero-point dword slots of a stage: [0, kSz) scales, [kSz, 2 kSz)
  // zero points, each indexed (block q, column c) as q * kBN + c.  They move
  // in 1 KB chunks (256 slots, 4 consecutive columns per lane, 16 B loads
  // from the block-major copies, whose rows are ldsz = N rounded up to 4
  // apart): wave w loads chunks w, w + 4, ... of the 2 kSz / 256; with fewer
  // chunks than waves the extra waves repeat one (same data, same place).
  // Both copies live in one buffer of rows [nb][2][ldsz] (ST = its start,
  // ZT = ST + ldsz): a lane's 16 bytes of block b2 sit at dword
  // (2 b2 + zp) ldsz + column.
  constexpr int kSzChunks = 2 * kSz / 256;
  int sz_col[kSzI], sz_q[kSzI], sz_chunk[kSzI];
  bool sz_isz[kSzI];
#pragma unroll
  for (int i = 0; i < kSzI; i++) {
    sz_chunk[i] = (wave + 4 * i) % kSzChunks;
    int slot = sz_chunk[i] * 256 + 4 * lane;
    sz_isz[i] = slot >= kSz;
    if (sz_isz[i]) slot -= kSz;
    sz_col[i] = min(n0 + slot % kBN, ldsz - 4) + (sz_isz[i] ? ldsz : 0);
    sz_q[i] = slot / kBN;
  }

  // this lane's output columns (CB 32-column blocks of the wave)
  int col[CB], my_c[CB];
  bool colok[CB];
#pragma unroll
  for (int cb = 0; cb < CB; cb++) {
    const int ccol = n0 + (wave * CB + cb) * 32 + cl;
    colok[cb] = ccol < N;
    col[cb] = colok[cb] ? ccol : N - 1;
    my_c[cb] = (wave * CB + cb) * 32 + cl;
  }

  auto issue = [&](int seg, int buf) {
    const int sa_ = min(seg, segsp - 1);
    const int sg = min(seg, segs - 1);
    uint4 *st = smem + buf * kStageU4;
#pragma unroll
    for (int i = 0; i < 4; i++)
      dma16_buf(a_rs, a_off[i], (uint32_t)sa_ * 8192u, st + 256 * i + 64 * wave);
#pragma unroll
    for (int i = 0; i < CB; i++)
      dma16_buf(w_rs, w_off[i], (uint32_t)sg * kSegBytes, st + 1024 + 256 * i + 64 * wave);
    // the stage's first block (clamped; a lane's block lies 0 .. NBPS - 1
    // rows below it) rides in the resource, so offsets stay within a few rows
    const int blk0 = min((sa_ * kSegK) >> bs_log2, nb - 1);
    const __amdgpu_buffer_rsrc_t sz_rs = buf_rsrc(ST + (size_t)blk0 * 2 * ldsz);
    uint32_t *sz = (uint32_t *)(st + kSOff);
#pragma unroll
    for (int i = 0; i < kSzI; i++) {
      const int blk = (sa_ * kSegK + sz_q[i] * (kSegK / NBPS)) >> bs_log2;
      const int b2 = blk < nb ? blk : nb - 1;
      dma16_buf(sz_rs, (uint32_t)((b2 - blk0) * 2 * ldsz + sz_col[i]) * 4u, 0u,
                sz + 256 * sz_chunk[i]);
    }
  };

  float16_t acc[2][CB];
  const float16_t zero16 = {};
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int cb = 0; cb < CB; cb++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[t][cb][r] = 0.0f;
  // the DMA ring slot of stage seg + NST - 1 (the one computed before seg)
  auto next_buf = [](int b) { return b == 0 ? NST - 1 : b - 1; };

  if constexpr (kPingPong) {
    // Ping-pong: each stage is a vector phase (scale / zero-point reads,
    // dequantisation of the stage's weights, the previous stage's block
    // epilogues) and a matrix phase (A fragment reads and the MFMAs).  The
    // two K groups run them half a stage apart, separated by workgroup
    // barriers, so on every SIMD one group's wave issues MFMAs while the
    // other group's wave runs its vector phase:
    //   group 0: wait(s)  B  issue(s+1) V(s)  B  M(s)
    //   group 1:          B  M(s-1) wait(s)  B  issue(s+1) V(s)
    // Both run the same number of barriers (two per stage and one after the
    // loop).  A stage slot is refilled only after the barrier that follows
    // the group's last read of it; a stage is read only after the barrier
    // that follows every wave's wait for its own DMA of it.
    constexpr int kJB = 4 / NBPS;   // k steps per quantisation block
    float16_t P[NBPS][2][CB];       // partials of the stage's blocks
    float psc[CB][NBPS];            // their scales (0 before the first stage)
    half8_t bq[4][CB];              // the stage's dequantised weights
#pragma unroll
    for (int q = 0; q < NBPS; q++)
#pragma unroll
      for (int cb = 0; cb < CB; cb++) {
        psc[cb][q] = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int r = 0; r < 16; r++) P[q][t][cb][r] = 0.0f;
      }
    auto vphase = [&](const int seg, const int b) __attribute__((always_inline)) {
      const uint4 *st = smem + b * kStageU4;
      const uint32_t *sS = (const uint32_t *)(st + kSOff);
      u4vec wv[CB];
      int zpv[CB][NBPS];
      float scv[CB][NBPS];
#pragma unroll
      for (int cb = 0; cb < CB; cb++) {
        wv[cb] = ((const u4vec *)(st + 1024))[((wave * CB + cb) * 32 + cl) * 2 + g];
#pragma unroll
        for (int q = 0; q < NBPS; q++) {
          const int blk = (seg * kSegK + q * (kSegK / NBPS)) >> bs_log2;
          const float sv = __builtin_bit_cast(float, sS[q * kBN + my_c[cb]]);
          zpv[cb][q] = (int)sS[kSz + q * kBN + my_c[cb]];
          scv[cb][q] = blk < nb ? sv : 0.0f;
        }
      }
#pragma unroll
      for (int q = 0; q < NBPS; q++)
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
          for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int r = 0; r < 16; r++)
              acc[rb][cb][r] = fmaf(psc[cb][q], P[q][rb][cb][r], acc[rb][cb][r]);
#pragma unroll
      for (int cb = 0; cb < CB; cb++)
#pragma unroll
        for (int q = 0; q < NBPS; q++) psc[cb][q] = scv[cb][q];
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) bq[j][cb] = dequant8(wv[cb][j], zpv[cb][j / kJB], magic);
    };
    auto mphase = [&](const int b) __attribute__((always_inline)) {
      const u4vec *sAv = (const u4vec *)(smem + b * kStageU4);
      // The 16 MFMAs in a fixed order, and the A fragments read in that same
      // order, so each MFMA waits only for its own read (LDS reads return in
      // order; the DMA goes through buffer loads, which the compiler counts
      // on vmcnt, so it keeps the waits incremental).  MFMA i takes step
      // J(i), row block RB(i), part H(i): with two or more blocks per stage
      // steps j and j + 2 (different blocks) go together, so four
      // accumulators alternate and a dependent MFMA issues four after its
      // predecessor; with one block, the two row blocks alternate.
      auto J = [](int i) { return NBPS >= 2 ? i / 8 + 2 * ((i >> 1) & 1) : i / 4; };
      auto H = [](int i) { return NBPS >= 2 ? (i >> 2) & 1 : (i >> 1) & 1; };
      half8_t af[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        af[i] = __builtin_bit_cast(half8_t, sAv[((i & 1) * 8 + J(i) * 2 + H(i)) * 64 + lane]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int j = J(i), rb = i & 1, q = j / kJB;
        const bool first = (j % kJB) == 0 && H(i) == 0;
        P[q][rb][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bq[j][0],
                                                             first ? zero16 : P[q][rb][0], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // the scheduler may not move any instruction across a phase boundary
    // (s_barrier alone orders only memory operations)
    auto phase_barrier = []() __attribute__((always_inline)) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int p = 0; p < NST - 1; p++) issue(sbeg + p, p);
    int buf = 0;
    if (grp == 0) {
      for (int seg = sbeg; seg < sbeg + nseg; seg++) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * kL));
        phase_barrier();
        issue(seg + NST - 1, next_buf(buf));
        vphase(seg, buf);
        phase_barrier();
        mphase(buf);
        if (++buf == NST) buf = 0;
      }
      phase_barrier();
    } else {
      int prev = 0;
      for (int seg = sbeg; seg < sbeg + nseg; seg++) {
        __builtin_amdgcn_s_barrier();
        if (seg > sbeg) mphase(prev);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * kL));
        __builtin_amdgcn_s_barrier();
        issue(seg + NST - 1, next_buf(buf));
        vphase(seg, buf);
        prev = buf;
        if (++buf == NST) buf = 0;
      }
      __builtin_amdgcn_s_barrier();
      mphase(prev);
    }
    // the last stage's blocks
#pragma unroll
    for (int q = 0; q < NBPS; q++)
#pragma unroll
      for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            acc[rb][cb][r] = fmaf(psc[cb][q], P[q][rb][cb][r], acc[rb][cb][r]);
  } else {
    // Two partial sets D[0], D[1].  A quantisation block's MFMAs accumulate
    // into one set while the previous block's partials (the other set) are
    // scaled into acc, so the epilogue FMAs overlap MFMAs instead of waiting
    // for them.  With NBPS blocks per stage the sets alternate by block; with
    // one block or less per stage (NBPS == 1) every stage is its own partial,
    // scaled by its block's scale, and the sets alternate by stage parity.
    float16_t D[2][2][CB];
    float pend[CB];  // scale of the set awaiting its epilogue (0 before the first)
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int cb = 0; cb < CB; cb++) {
        pend[cb] = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          D[0][t][cb][r] = 0.0f;
          D[1][t][cb][r] = 0.0f;
        }
      }

#pragma unroll
    for (int p = 0; p < NST - 1; p++) issue(sbeg + p, p);
    int buf = 0;
    auto stage = [&](const int seg, auto parity) __attribute__((always_inline)) {
      constexpr int P = decltype(parity)::value;
      // this thread's DMA for stage `seg` has landed; the barrier (without a
      // fence, which would wait for every outstanding load) makes all of it
      // visible, and frees the stage computed in the previous iteration
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * kL));
      __builtin_amdgcn_s_barrier();
      issue(seg + NST - 1, buf == 0 ? NST - 1 : buf - 1);
      const uint4 *st = smem + buf * kStageU4;
      const u4vec *sAv = (const u4vec *)st;
      const uint32_t *sS = (const uint32_t *)(st + kSOff);
      u4vec wv[CB];
      int zpv[CB][NBPS];
      float scv[CB][NBPS];
#pragma unroll
      for (int cb = 0; cb < CB; cb++) {
        wv[cb] = ((const u4vec *)(st + 1024))[((wave * CB + cb) * 32 + cl) * 2 + g];
#pragma unroll
        for (int q = 0; q < NBPS; q++) {
          const int blk = (seg * kSegK + q * (kSegK / NBPS)) >> bs_log2;
          const float sv = __builtin_bit_cast(float, sS[q * kBN + my_c[cb]]);
          zpv[cb][q] = (int)sS[kSz + q * kBN + my_c[cb]];
          scv[cb][q] = blk < nb ? sv : 0.0f;
        }
      }
      // with one column block per wave every A fragment of the stage is read
      // up front (16 x 16 B per lane), so the MFMAs wait on in-order LDS
      // returns instead of one read each; two blocks read them per k step
      constexpr int kPre = CB == 1 ? 4 : 1;
      half8_t af[kPre][2][2];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (CB == 1 ? j == 0 : true) {
#pragma unroll
          for (int jj = 0; jj < kPre; jj++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
              for (int h = 0; h < 2; h++)
                af[jj][rb][h] = __builtin_bit_cast(
                    half8_t, sAv[(rb * 8 + (j + jj) * 2 + h) * 64 + lane]);
        }
        const int jf = CB == 1 ? j : 0;
        constexpr int kJB = 4 / NBPS;  // k steps per block (NBPS > 1)
        const int q = j / kJB;
        const bool first = (j % kJB) == 0;
        half8_t b[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) b[cb] = dequant8(wv[cb][j], zpv[cb][q], magic);
        // set S takes this block; the other set holds the block before it
        auto mma = [&](auto set) __attribute__((always_inline)) {
          constexpr int S = decltype(set)::value;
#pragma unroll
          for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
              D[S][rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  af[jf][rb][0], b[cb], first ? zero16 : D[S][rb][cb], 0, 0, 0);
              D[S][rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[jf][rb][1], b[cb],
                                                                    D[S][rb][cb], 0, 0, 0);
            }
          if (first) {
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
              for (int cb = 0; cb < CB; cb++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                  acc[rb][cb][r] = fmaf(pend[cb], D[1 - S][rb][cb][r], acc[rb][cb][r]);
          }
        };
        if (NBPS > 1 ? (q & 1) : P)
          mma(std::integral_constant<int, 1>());
        else
          mma(std::integral_constant<int, 0>());
        if ((j + 1) % kJB == 0) {
#pragma unroll
          for (int cb = 0; cb < CB; cb++) pend[cb] = scv[cb][q];
        }
      }
      if (++buf == NST) buf = 0;
    };
    if constexpr (NBPS > 1) {
      for (int seg = sbeg; seg < sbeg + nseg; seg++) stage(seg, std::integral_constant<int, 0>());
    } else {
      for (int seg = sbeg; seg < sbeg + nseg; seg += 2) {
        stage(seg, std::integral_constant<int, 0>());
        if (seg + 1 < sbeg + nseg) stage(seg + 1, std::integral_constant<int, 1>());
      }
    }
    // the last block's partials: set 1 unless NBPS == 1 and the stage count is odd
    const bool last1 = NBPS > 1 || (nseg & 1) == 0;
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
      for (int cb = 0; cb < CB; cb++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          acc[rb][cb][r] = fmaf(pend[cb], last1 ? D[1][rb][cb][r] : D[0][rb][cb][r],
                                acc[rb][cb][r]);
  }
  // drain the DMA still in flight (clamped stages past the end) before the
  // LDS is reused or the workgroup exits
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if constexpr (GROUPS > 1) {
    // partial tiles of groups 1.. -> LDS, summed by group 0
    __syncthreads();
    float *red = (float *)smem_all;  // (GROUPS-1) x 32*CB x 256 floats
    if (grp > 0) {
#pragma unroll
      for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            red[((grp - 1) * 32 * CB + (rb * CB + cb) * 16 + r) * 256 + tid] = acc[rb][cb][r];
    }
    __syncthreads();
    if (grp == 0) {
      for (int gg = 1; gg < GROUPS; gg++)
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
          for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int r = 0; r < 16; r++)
              acc[rb][cb][r] += red[((gg - 1) * 32 * CB + (rb * CB + cb) * 16 + r) * 256 + tid];
    }
  }
  if (ksplit > 1) {
    // K slices: every slice stores its tile partial (agent scope, so the
    // last slice reads it from any XCD), then counts in; the last one to
    // arrive sums the ksplit partials in slice order (the same bits whatever
    // the arrival order), resets the counter and stores the tile.  Every
    // wave takes part in the barriers.
    __shared__ int s_last;
    constexpr int kPart = 32 * CB * 256;  // floats per tile partial
    float *pt = part + (size_t)tile * ksplit * kPart;
    if (grp == 0) {
#pragma unroll
      for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            st_act<true>(pt + (size_t)split * kPart + ((rb * CB + cb) * 16 + r) * 256 + tid,
                         acc[rb][cb][r]);
    }
    // Ordering: the workgroup barrier orders every thread's partial stores
    // before thread 0's count, whose release (agent scope) pairs with the
    // acquire fence of the last slice (which read the count the others'
    // releases wrote); the barrier below extends it to that workgroup's
    // loads.  Only the last slice acquires (an agent-scope acquire
    // invalidates this XCD's L2).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev =
          __hip_atomic_fetch_add(&tile_cnt[tile], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == ksplit - 1;
      if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!s_last) return;  // whole workgroup
    if (grp == 0) {
      // one round trip per two slices (ksplit is even): both slices' values,
      // then the adds in slice order
      for (int sl = 0; sl < ksplit; sl += 2) {
        float t[2][2][CB][16];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const float *q = pt + (size_t)(sl + h) * kPart + tid;
#pragma unroll
          for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
#pragma unroll
              for (int r = 0; r < 16; r++)
                t[h][rb][cb][r] = ld_act<true>(q + ((rb * CB + cb) * 16 + r) * 256);
        }
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
          for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const float a = sl == 0 ? t[0][rb][cb][r] : acc[rb][cb][r] + t[0][rb][cb][r];
              acc[rb][cb][r] = a + t[1][rb][cb][r];
            }
      }
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(&tile_cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (grp > 0) return;
  // 32x32 f32 accumulator layout: lane l holds column l%32, rows
  // (r/4)*8 + (l/32)*4 + r%4 for r = 0..15.
  // (every lane takes part in the shuffles: the column test is on the store)
#pragma unroll
  for (int cb = 0; cb < CB; cb++) {
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int tr = rb * 32 + (r >> 2) * 8 + g * 4 + (r & 3);  // row in the tile
        const int row = rb0 * 32 + tr;
        const int ex = __shfl(rexp, tr, 64);
        if (colok[cb] && row < M) Y[(size_t)row * N + col[cb]] = ldexpf(acc[rb][cb][r], -ex);
      }
    }
  }
}

// Launch shape of the prefill GEMM for a pack and M (tile width, K groups,
// LDS stages, K slices) and the padded segment count of the prepared A.
struct GemmPlan {
  int64_t segs, mpad, segsp, tiles;
  int gx, gy, cb, nbps, groups, nst, ksplit;
  size_t ap_bytes, shmem;
};

static int gemm_plan(const mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, GemmPlan &pl) {
  const int64_t segs = p->k64 / kSegK;
  const int64_t mpad = (m + kGemmBM - 1) / kGemmBM * kGemmBM;
  const int gy = (int)(mpad / kGemmBM);
  // 256-column tiles (each wave two 32-column blocks, so every A fragment
  // read from LDS feeds twice the MFMAs and A streams half as often) when
  // there is at least one such tile per CU (measured on 256 CUs: 256 tiles
  // gain 7%, 448 tiles 8%; 128 tiles lose 40%); 128 otherwise.
  int cb = ((p->n + 2 * kGemmBN - 1) / (2 * kGemmBN)) * gy >= ctx->cu_count ? 2 : 1;
  if (ctx->gemm_cb) cb = ctx->gemm_cb;
  const int gx = (int)((p->n + cb * kGemmBN - 1) / (cb * kGemmBN));
  const int nbps = p->block >= 64 ? 1 : (p->block == 32 ? 2 : 4);
  // K split over two wave groups when the tiles alone leave CUs with one
  // wave per SIMD; each group's range covers whole quantisation blocks.
  const int groups = ((int64_t)gx * gy < 2 * (int64_t)ctx->cu_count && segs >= 16) ? 2 : 1;
  const int nst = cb == 2 ? 2 : ctx->gemm_stages;
  // K slices across workgroups when the tiles (with the K groups) still
  // leave CUs idle: the largest power of two <= 8 that fits the CUs, keeps
  // at least 4 stages per group and splits K without padding; each slice
  // covers whole quantisation blocks.
  const int64_t bstages = std::max<int64_t>(1, p->block / kSegK);
  const int64_t tiles = (int64_t)gx * gy;
  int ksplit = 1;
  if (tiles <= kGemmMaxSplitTiles) {
    if (ctx->gemm_ksplit) {
      ksplit = ctx->gemm_ksplit;
    } else {
      for (int ks = 8; ks > 1; ks >>= 1) {
        const int64_t unit = groups * ks * bstages;
        if (tiles * ks <= ctx->cu_count && segs % unit == 0 && segs / (groups * ks) >= 4) {
          ksplit = ks;
          break;
        }
      }
    }
  }
  const int64_t align = groups * ksplit * bstages;
  const int64_t segsp = (segs + align - 1) / align * align;
  const int64_t rblocks = mpad / 32;
  const size_t ap_bytes = (size_t)(rblocks * segsp * 4 * 2 * 64) * 16;
  const size_t shmem = (size_t)groups * nst * (1024 + 256 * cb + 64 * cb * nbps) * 16;
  if (shmem > (size_t)ctx->lds_max)
    return fail(MMNB_ERR_UNSUPPORTED, "GEMM: LDS stages exceed the device limit");
  pl = GemmPlan{segs, mpad, segsp, tiles, gx, gy, cb, nbps, groups, nst, ksplit, ap_bytes, shmem};
  return MMNB_OK;
}

// The GEMM proper on a prepared A (d_ap, d_exp laid out for `pl`).
// K-slice partial tiles of a plan (bytes; 0 without K slices).
static size_t gemm_part_bytes(const GemmPlan &pl) {
  return pl.ksplit > 1 ? (size_t)pl.tiles * pl.ksplit * 32 * pl.cb * 256 * 4 : 0;
}

// d_part: the K-slice partial tiles (gemm_part_bytes), d_cnt: the per-tile
// arrival counters (zero at rest); both unused without K slices.
static int gemm_run(mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, const GemmPlan &pl,
                    const void *d_ap, const void *d_exp, float *d_y, void *d_part, int *d_cnt) {
  const int64_t segs = pl.segs, segsp = pl.segsp;
  const int gx = pl.gx, gy = pl.gy, cb = pl.cb, nbps = pl.nbps, groups = pl.groups,
            nst = pl.nst, ksplit = pl.ksplit;
  const size_t shmem = pl.shmem;
  const int bs_log2 = ilog2(p->block);
  const dim3 grid((unsigned)(gx * gy * ksplit));
#define MMNB_GEMM_LAUNCH(Q, NS, GR, CB)                                                      \
  {                                                                                          \
    auto kern = k_gemm_mfma<Q, NS, GR, CB>;                                                  \
    if (shmem > 65536) {                                                                     \
      hipError_t e_ = hipFuncSetAttribute(                                                   \
          (const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);       \
      if (e_ != hipSuccess) return check_hip(e_, "hipFuncSetAttribute");                     \
    }                                                                                        \
    return launch(ctx, kKernGemm, kern, grid, dim3(256 * GR), shmem, (const uint4 *)d_ap,   \
                  (const int *)d_exp, (int)segs, (int)segsp, p->d_w, p->col_bytes,          \
                  p->d_st, p->d_zt, (int)p->ldsz, (int)p->n_blocks, bs_log2, (int)m,        \
                  (int)p->n, gx, gy, d_y, ksplit, (float *)d_part, d_cnt);                  \
  }
#define MMNB_GEMM_NB(NS, GR, CB)                     \
  {                                                  \
    if (nbps == 1) MMNB_GEMM_LAUNCH(1, NS, GR, CB);  \
    if (nbps == 2) MMNB_GEMM_LAUNCH(2, NS, GR, CB);  \
    MMNB_GEMM_LAUNCH(4, NS, GR, CB);                 \
  }
  if (cb == 2) {
    if (groups == 2) MMNB_GEMM_NB(2, 2, 2);
    MMNB_GEMM_NB(2, 1, 2);
  }
  if (groups == 2) {
    if (nst == 3) MMNB_GEMM_NB(3, 2, 1);
    MMNB_GEMM_NB(2, 2, 1);
  }
  if (nst == 3) MMNB_GEMM_NB(3, 1, 1);
  MMNB_GEMM_NB(2, 1, 1);
#undef MMNB_GEMM_NB
#undef MMNB_GEMM_LAUNCH
}


// The context's K-slice partials (grow-only scratch) for a plan.
static int gemm_ctx_part(mmnb_ctx *ctx, const GemmPlan &pl, void **d_part) {
  *d_part = nullptr;
  const size_t pb = gemm_part_bytes(pl);
  return pb ? scratch_get(ctx, 10, pb, d_part) : MMNB_OK;
}

static int launch_gemm(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                       int64_t m, float *d_y) {
  GemmPlan pl;
  int rc;
  if ((rc = gemm_plan(ctx, p, m, pl))) return rc;
  void *d_ap = nullptr, *d_exp = nullptr, *d_part = nullptr;
  if ((rc = scratch_get(ctx, 2, pl.ap_bytes, &d_ap))) return rc;
  if ((rc = scratch_get(ctx, 3, (size_t)pl.mpad * 4, &d_exp))) return rc;
  if ((rc = gemm_ctx_part(ctx, pl, &d_part))) return rc;
  if ((rc = launch_prep_a(ctx, d_a, lda, m, p->k, pl.mpad, pl.segsp, (int *)d_exp,
                           (uint4 *)d_ap, nullptr, 0)))
    return rc;
  return gemm_run(ctx, p, m, pl, d_ap, d_exp, d_y, d_part, ctx->d_gemm_cnt);
}

int gemm_prepared_a(mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, int64_t *segsp,
                    int64_t *mpad, void **d_ap, int **d_exp) {
  if (m <= 8) return fail(MMNB_ERR_ARG, "prepared A: M <= 8 takes the GEMV");
  GemmPlan pl;
  int rc;
  if ((rc = gemm_plan(ctx, p, m, pl))) return rc;
  if ((rc = scratch_get(ctx, 2, pl.ap_bytes, d_ap))) return rc;
  if ((rc = scratch_get(ctx, 3, (size_t)pl.mpad * 4, (void **)d_exp))) return rc;
  *segsp = pl.segsp;
  *mpad = pl.mpad;
  return MMNB_OK;
}

int launch_matmul_nbits_prepared(mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, float *d_y) {
  GemmPlan pl;
  int rc;
  if ((rc = gemm_plan(ctx, p, m, pl))) return rc;
  void *d_ap = nullptr, *d_exp = nullptr, *d_part = nullptr;
  if ((rc = scratch_get(ctx, 2, pl.ap_bytes, &d_ap))) return rc;
  if ((rc = scratch_get(ctx, 3, (size_t)pl.mpad * 4, &d_exp))) return rc;
  if ((rc = gemm_ctx_part(ctx, pl, &d_part))) return rc;
  return gemm_run(ctx, p, m, pl, d_ap, d_exp, d_y, d_part, ctx->d_gemm_cnt);
}

// MatMulNBits with every scratch buffer carved from a caller's workspace
// (ws, ws_bytes; 256-byte aligned): the GEMM's K-slice counters, row
// exponents, prepared activations and K-slice partials, each followed by
// kTailPad bytes of slack.  Allocates nothing.
int launch_matmul_nbits_ws(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                           int64_t m, float *d_y, void *ws, size_t ws_bytes) {
  if (p->generic) return launch_nbits_generic(ctx, p, d_a, lda, m, d_y);  // no scratch
  // the GEMVs use no scratch (the multi-row one falls back to the GEMM when A
  // does not fit its LDS: that GEMM takes the workspace below)
  if (m == 1 || (m <= 8 && gemv_multi_fits(ctx, p, m)))
    return launch_gemv(ctx, p, d_a, lda, m, d_y);
  GemmPlan pl;
  int rc;
  if ((rc = gemm_plan(ctx, p, m, pl))) return rc;
  auto up = [](size_t b) { return (b + kTailPad + 255) / 256 * 256; };
  const size_t o_cnt = 0;
  const size_t o_exp = o_cnt + up((size_t)kGemmMaxSplitTiles * 4);
  const size_t o_ap = o_exp + up((size_t)pl.mpad * 4);
  const size_t o_part = o_ap + up(pl.ap_bytes);
  const size_t need = o_part + up(gemm_part_bytes(pl));
  if (need > ws_bytes)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: this M x K needs " + std::to_string(need) +
                    " bytes of scratch, more than the " + std::to_string(ws_bytes) +
                    "-byte fixed workspace");
  char *b = (char *)ws;
  int *d_cnt = (int *)(b + o_cnt);
  const int nclear = pl.ksplit > 1 ? (int)pl.tiles : 0;
  if ((rc = launch_prep_a(ctx, d_a, lda, m, p->k, pl.mpad, pl.segsp, (int *)(b + o_exp),
                           (uint4 *)(b + o_ap), d_cnt, nclear)))
    return rc;
  return gemm_run(ctx, p, m, pl, b + o_ap, b + o_exp, d_y,
                  pl.ksplit > 1 ? (void *)(b + o_part) : nullptr, d_cnt);
}

int launch_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                        int64_t m, float *d_y) {
  if (p->generic) return launch_nbits_generic(ctx, p, d_a, lda, m, d_y);
  if (m <= 8) return launch_gemv(ctx, p, d_a, lda, m, d_y);
  return launch_gemm(ctx, p, d_a, lda, m, d_y);
}

}  // namespace mmnb
