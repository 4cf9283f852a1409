// Decoder ops around MatMulNBits on gfx950, and a Qwen3-shaped int4 decoder
// session built from them.
//
//   RMSNorm              opRMSNorm (lib/src/onnx_ops.dart:1436-1490)
//   RotaryEmbedding      opRotaryEmbedding (:2121-2181)
//   GroupQueryAttention  opGroupQueryAttention (:1508-1640)
//
// The op kernels keep the reference's arithmetic where it is cheap to do so
// (sums of squares, rotations and the softmax normaliser in double, one
// binary32 rounding per stored value); the attention products run in fp32.
//
// The decoder session keeps every weight pack, the KV cache and the step
// state in HBM.  Prefill runs the general kernels over all prompt rows; a
// decode step is five launches per layer (fused RMSNorm + MatMulNBits
// prologues, residual / SwiGLU / greedy-argmax epilogues, one attention
// kernel) and is captured once as a HIP graph whose kernels read the
// position and token from device memory, so replaying it advances the
// sequence with no host work.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "mmnb_device.h"
#include "mmnb_internal.h"

namespace mmnb {

// ---------------------------------------------------------------------------
// Block-wide sums (256 threads).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double block_sum_d(double v, double *sh) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
  const int nw = (blockDim.x + 63) >> 6;
  for (int i = 0; i < nw; i++) t += sh[i];
  return t;
}

// ---------------------------------------------------------------------------
// RMSNorm over the last axis, one workgroup per row.  With `add` non-null
// the row is first replaced by x + add (the residual Add node before the
// norm), written back to `xsum`.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const float *X, int64_t dim,
                                                 const float *__restrict__ G, float eps,
                                                 float *__restrict__ Y, const float *add,
                                                 float *xsum) {
  __shared__ double sh[4];
  const int64_t r = blockIdx.x;
  const float *x = X + r * dim;
  double ss = 0.0;
  for (int64_t k = threadIdx.x; k < dim; k += blockDim.x) {
    float v = x[k];
    if (add) {
      v = v + add[r * dim + k];
      xsum[r * dim + k] = v;
    }
    ss += (double)v * (double)v;
  }
  ss = block_sum_d(ss, sh);
  const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
  const float *xs = add ? xsum + r * dim : x;
  for (int64_t k = threadIdx.x; k < dim; k += blockDim.x)
    Y[r * dim + k] = (float)((double)xs[k] * inv * (double)G[k]);
}

// ---------------------------------------------------------------------------
// k_rmsnorm (same sums, same products, so the same fp32 values) written
// straight into the prefill GEMM's prepared activations (prep_a_store16), so
// the GEMM that consumes the norm needs no k_prep_a launch.  One workgroup
// per row of the padded row count; rows >= M and k >= dim are written as
// zeros.  dim <= 4096: the row sits in LDS between the sum of squares
// (thread t sums k = t, t+256, ..., as in k_rmsnorm) and the conversion
// (thread t owns k = 16t .. 16t+15).  With `add` the row is x + add, also
// written back to xsum.
// ---------------------------------------------------------------------------
constexpr int kPrepMaxDim = 4096;

__device__ __forceinline__ int prep_row_exponent(float mx, float *wmx) {
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) wmx[threadIdx.x >> 6] = mx;
  __syncthreads();
  return prep_a_exponent(fmaxf(fmaxf(wmx[0], wmx[1]), fmaxf(wmx[2], wmx[3])));
}

__global__ __launch_bounds__(256) void k_rmsnorm_prep(const float *X, int64_t M, int64_t dim,
                                                      const float *__restrict__ G, float eps,
                                                      const float *add, float *xsum,
                                                      int64_t segsp, int64_t kp,
                                                      int *__restrict__ row_exp,
                                                      uint4 *__restrict__ out) {
  __shared__ double sh[4];
  __shared__ float srow[kPrepMaxDim];
  __shared__ float wmx[4];
  const int64_t r = blockIdx.x;
  const bool live = r < M;  // whole workgroup
  const int t = threadIdx.x;
  const int64_t k0 = 16 * t;
  // every load first (clamped indices): the row (thread t: k = t + 256 j),
  // the residual, and the gammas of the conversion's k = 16t .. 16t+15
  float xr[kPrepMaxDim / 256], ar[kPrepMaxDim / 256], gv[16];
  const int64_t rr = live ? r : 0;
#pragma unroll
  for (int j = 0; j < kPrepMaxDim / 256; j++) {
    const int64_t k = t + 256 * j;
    const int64_t kc = k < dim ? k : dim - 1;
    xr[j] = X[rr * dim + kc];
    ar[j] = add ? add[rr * dim + kc] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 16; e++) gv[e] = G[k0 + e < dim ? k0 + e : dim - 1];
  double inv = 0.0;
  if (live) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < kPrepMaxDim / 256; j++) {
      const int64_t k = t + 256 * j;
      if (k < dim) {
        float v = xr[j];
        if (add) {
          v = v + ar[j];
          xsum[r * dim + k] = v;
        }
        srow[k] = v;
        ss += (double)v * (double)v;
      }
    }
    ss = block_sum_d(ss, sh);  // its barriers also publish srow
    inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
  }
  float v[16];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const int64_t k = k0 + e;
    const bool ok = live && k < dim;
    const float gk = gv[e];
    const float y = (float)((double)srow[k] * inv * (double)gk);
    v[e] = ok ? y : 0.0f;
    mx = fmaxf(mx, finite_abs(v[e]));
  }
  const int ex = prep_row_exponent(mx, wmx);
  if (t == 0 && live) row_exp[r] = ex;
  if (k0 < kp) prep_a_store16(out, segsp, r, k0, v, ex);  // kp may be below 4096
#pragma unroll
  for (int e = 0; e < 16; e++) v[e] = 0.0f;
  for (int64_t kz = k0 + kPrepMaxDim; kz < kp; kz += kPrepMaxDim)
    prep_a_store16(out, segsp, r, kz, v, 0);
}

// k_swiglu_rows into the prepared activations of the down projection (one
// workgroup per padded row, I <= 4096, thread t owns k = 16t .. 16t+15).
__global__ __launch_bounds__(256) void k_swiglu_prep(const float *__restrict__ gu, int64_t M,
                                                     int64_t I, int64_t segsp, int64_t kp,
                                                     int *__restrict__ row_exp,
                                                     uint4 *__restrict__ out) {
  __shared__ float wmx[4];
  const int64_t r = blockIdx.x;
  const bool live = r < M;
  const int t = threadIdx.x;
  const int64_t k0 = 16 * t;
  float v[16];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const int64_t k = k0 + e;
    const bool ok = live && k < I;
    const int64_t i = ok ? r * 2 * I + 2 * k : 0;
    const float g = gu[i], u = gu[i + 1];
    const float sig = (float)(1.0 / (1.0 + exp(-(double)g)));
    v[e] = ok ? (g * sig) * u : 0.0f;
    mx = fmaxf(mx, finite_abs(v[e]));
  }
  const int ex = prep_row_exponent(mx, wmx);
  if (t == 0 && live) row_exp[r] = ex;
  if (k0 < kp) prep_a_store16(out, segsp, r, k0, v, ex);  // kp may be below 4096
#pragma unroll
  for (int e = 0; e < 16; e++) v[e] = 0.0f;
  for (int64_t kz = k0 + kPrepMaxDim; kz < kp; kz += kPrepMaxDim)
    prep_a_store16(out, segsp, r, kz, v, 0);
}

// ---------------------------------------------------------------------------
// Rotary embedding of one [heads, head] row block at position p (3-D layout
// [b, s, heads * head]).  Rotated pairs in double, as the reference.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rotate_row(const float *x, float *y, int heads, int head,
                                           int half_rot, int interleaved, const float *cos,
                                           const float *sin, int64_t p) {
  const int rot = 2 * half_rot;
  for (int e = threadIdx.x; e < heads * head; e += blockDim.x) {
    const int h = e / head, i = e % head;
    const float *xh = x + (int64_t)h * head;
    float out;
    if (i >= rot) {
      out = xh[i];
    } else if (interleaved) {
      const int pi = i >> 1;
      const double c = cos[p * half_rot + pi], sn = sin[p * half_rot + pi];
      const double x0 = xh[2 * pi], x1 = xh[2 * pi + 1];
      out = (float)((i & 1) ? x1 * c + x0 * sn : x0 * c - x1 * sn);
    } else {
      const int hr = half_rot;
      const int pi = i < hr ? i : i - hr;
      const double c = cos[p * half_rot + pi], sn = sin[p * half_rot + pi];
      const double x0 = xh[pi], x1 = xh[pi + hr];
      out = (float)(i < hr ? x0 * c - x1 * sn : x1 * c + x0 * sn);
    }
    y[(int64_t)h * head + i] = out;
  }
}

// One workgroup per (b, s) row.  pos: int64 [s] (rank 1) or [b, s].
__global__ __launch_bounds__(256) void k_rotary(const float *__restrict__ X, int64_t seq,
                                                int heads, int head,
                                                const int64_t *__restrict__ pos, int pos_rank,
                                                int64_t pos_const, const float *__restrict__ cos,
                                                const float *__restrict__ sin, int half_rot,
                                                int interleaved, float *__restrict__ Y) {
  const int64_t row = blockIdx.x;  // b * seq + s
  const int64_t s = row % seq;
  const int64_t p = pos ? (pos_rank == 1 ? pos[s] : pos[row]) : pos_const + s;
  const int64_t hid = (int64_t)heads * head;
  rotate_row(X + row * hid, Y + row * hid, heads, head, half_rot, interleaved, cos, sin, p);
}

// ---------------------------------------------------------------------------
// present[b, kvh, cap] = past[b, kvh, 0:P] ++ new[b, s, kvh] (k and v)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gqa_present(
    const float *__restrict__ past_k, const float *__restrict__ past_v, int64_t P,
    const float *__restrict__ k, const float *__restrict__ v, int64_t seq, int kvh, int hd,
    int64_t cap, float *__restrict__ pk, float *__restrict__ pv) {
  const int64_t b = blockIdx.y, hh = blockIdx.x % kvh, j = blockIdx.x / kvh;  // j < P + seq
  const int64_t dst = ((b * kvh + hh) * cap + j) * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float kv, vv;
    if (j < P) {
      const int64_t src = ((b * kvh + hh) * P + j) * hd + d;
      kv = past_k[src];
      vv = past_v[src];
    } else {
      const int64_t src = ((b * seq + (j - P)) * kvh + hh) * hd + d;
      kv = k[src];
      vv = v[src];
    }
    pk[dst + d] = kv;
    pv[dst + d] = vv;
  }
}

// ---------------------------------------------------------------------------
// Attention rows: query i (absolute position P + i) of head h attends
// causally to keys 0..P+i of the present cache [b, kvh, cap, hd], plus an
// optional additive bias [b, bias_heads, seq, total].  A workgroup takes
// 16 queries of one head; key tiles of 32 are staged in LDS; thread
// (query qi, lane kl of 16) scores keys kl and kl+16 of a tile and owns
// output dims d = kl (mod 16); online softmax per query.  hd <= 128.
// ---------------------------------------------------------------------------
constexpr int kAttnQ = 16, kAttnKT = 32, kAttnMaxHd = 128;

__global__ __launch_bounds__(256) void k_attn_rows(
    const float *__restrict__ Q, int64_t q_row_stride, int64_t seq, int nh, int kvh, int hd,
    const float *__restrict__ pk, const float *__restrict__ pv, int64_t cap, int64_t P,
    float scale, const float *__restrict__ bias, int bias_heads, float *__restrict__ out,
    int64_t out_row_stride) {
  __shared__ float sK[kAttnKT][kAttnMaxHd + 1];
  __shared__ float sV[kAttnKT][kAttnMaxHd];
  __shared__ float sQ[kAttnQ][kAttnMaxHd];
  __shared__ float sP[kAttnQ][kAttnKT];
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int kv = h / (nh / kvh);
  const int qi = threadIdx.x >> 4, kl = threadIdx.x & 15;
  const int64_t i = (int64_t)blockIdx.x * kAttnQ + qi;  // query row
  const bool qok = i < seq;
  const int64_t T = P + seq;
  for (int e = threadIdx.x; e < kAttnQ * hd; e += blockDim.x) {
    const int r = e / hd, d = e % hd;
    const int64_t ii = (int64_t)blockIdx.x * kAttnQ + r;
    sQ[r][d] = ii < seq ? Q[(b * seq + ii) * q_row_stride + (int64_t)h * hd + d] : 0.0f;
  }
  const float *Kb = pk + (b * kvh + kv) * cap * hd;
  const float *Vb = pv + (b * kvh + kv) * cap * hd;
  const int64_t last = qok ? P + i : -1;  // last key this query sees
  const int64_t q0 = (int64_t)blockIdx.x * kAttnQ;
  const int64_t qmax = std::min<int64_t>(q0 + kAttnQ, seq) - 1;
  const int64_t kend = P + qmax + 1;  // keys any query of the block sees
  float m = -INFINITY, l = 0.0f;
  float o[kAttnMaxHd / 16];
#pragma unroll
  for (int e = 0; e < kAttnMaxHd / 16; e++) o[e] = 0.0f;
  for (int64_t k0 = 0; k0 < kend; k0 += kAttnKT) {
    __syncthreads();
    {
      // all of this thread's tile elements in flight before any store
      constexpr int kPer = kAttnKT * kAttnMaxHd / 256;
      float kk[kPer], vv[kPer];
#pragma unroll
      for (int u = 0; u < kPer; u++) {
        const int e = threadIdx.x + 256 * u;
        const int j = e / hd, d = e % hd;
        const bool ok = e < kAttnKT * hd && k0 + j < T;
        const int64_t idx = ok ? (k0 + j) * hd + d : 0;  // unconditional load
        const float k_ = Kb[idx], v_ = Vb[idx];
        kk[u] = ok ? k_ : 0.0f;
        vv[u] = ok ? v_ : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kPer; u++) {
        const int e = threadIdx.x + 256 * u;
        if (e < kAttnKT * hd) {
          const int j = e / hd, d = e % hd;
          sK[j][d] = kk[u];
          sV[j][d] = vv[u];
        }
      }
    }
    __syncthreads();
    float sc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int j = kl + 16 * u;
      const int64_t kj = k0 + j;
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot = fmaf(sQ[qi][d], sK[j][d], dot);
      float v = dot * scale;
      if (bias && qok && kj <= last)
        v += bias[((b * bias_heads + (h % bias_heads)) * seq + i) * T + kj];
      sc[u] = (qok && kj <= last) ? v : -INFINITY;
    }
    // tile max over the 16 lanes of this query
    float tm = fmaxf(sc[0], sc[1]);
    for (int off = 8; off > 0; off >>= 1) tm = fmaxf(tm, __shfl_xor(tm, off, 16));
    const float mn = fmaxf(m, tm);
    float p0 = 0.0f, p1 = 0.0f, corr = 1.0f;
    if (mn != -INFINITY) {
      p0 = sc[0] == -INFINITY ? 0.0f : expf(sc[0] - mn);
      p1 = sc[1] == -INFINITY ? 0.0f : expf(sc[1] - mn);
      corr = m == -INFINITY ? 0.0f : expf(m - mn);
    }
    float ps = p0 + p1;
    for (int off = 8; off > 0; off >>= 1) ps += __shfl_xor(ps, off, 16);
    l = l * corr + ps;
    m = mn;
    sP[qi][kl] = p0;
    sP[qi][kl + 16] = p1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kAttnMaxHd / 16; e++) {
      const int d = kl + 16 * e;
      if (d < hd) {
        float acc = o[e] * corr;
        for (int j = 0; j < kAttnKT; j++) acc = fmaf(sP[qi][j], sV[j][d], acc);
        o[e] = acc;
      }
    }
  }
  if (qok) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int e = 0; e < kAttnMaxHd / 16; e++) {
      const int d = kl + 16 * e;
      if (d < hd) out[(b * seq + i) * out_row_stride + (int64_t)h * hd + d] = o[e] * inv;
    }
  }
}

// ---------------------------------------------------------------------------
// Attention rows on the matrix cores: v_mfma_f32_16x16x4_f32 (fp32 products
// and sums, as in k_attn_rows, in another order).  A workgroup takes 16
// queries of one head; its 8 waves take the key blocks (16 keys) round robin
// and merge their (max, sum, o) through LDS at the end, pairwise in a fixed
// order.  Per key block a wave forms S^T = K Q^T (16 keys x 16 queries,
// HD/4 MFMAs), runs the online softmax on it and accumulates O^T += V^T P^T
// (HD/4 MFMAs).  16x16x4 operand layouts: A lane l = row l%16, k slot l/16;
// B lane l = column l%16, k slot l/16; D lane l = column l%16, rows
// 4(l/16) + r.  For lane (c = l%16, g = l/16):
//   S^T step t: A = K[key c][d], B = Q[query c][d], d = g*HD/4 + t;
//     D = the scores of query c for keys 4g + r.
//   O^T step t: k slot g' carries key 4g' + t, so B is the lane's own p[t];
//     A = V[key 4g + t][c*HD/16 + db] for d block db;
//     D = o of query c at d = (4g + r)*HD/16 + db.
// K and V go straight to registers (float4 / float2 loads); the two key
// blocks of an iteration have all their loads in flight before the first
// block's arithmetic.
// ---------------------------------------------------------------------------
constexpr int kAttnMfWaves = 8;
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int N>
__device__ __forceinline__ void ld_run(const float *__restrict__ p, float *v) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
      const float4 x = *(const float4 *)(p + e);
      v[e] = x.x; v[e + 1] = x.y; v[e + 2] = x.z; v[e + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; e += 2) {
      const float2 x = *(const float2 *)(p + e);
      v[e] = x.x; v[e + 1] = x.y;
    }
  }
}

template <int HD>
__global__ __launch_bounds__(64 * kAttnMfWaves) void k_attn_mfma(
    const float *__restrict__ Q, int64_t q_row_stride, int64_t seq, int nh, int kvh,
    const float *__restrict__ pk, const float *__restrict__ pv, int64_t cap, int64_t P,
    float scale, const float *__restrict__ bias, int bias_heads, float *__restrict__ out,
    int64_t out_row_stride) {
  constexpr int kQd = HD / 4;   // d values per lane of an S^T operand
  constexpr int kVd = HD / 16;  // d blocks of O^T (d values per lane per key)
  __shared__ float s_slot[kAttnMfWaves / 2][kQd + 2][64];
  const int w = threadIdx.x >> 6, ln = threadIdx.x & 63, c = ln & 15, g = ln >> 4;
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int kv = h / (nh / kvh);
  const int64_t q0 = (int64_t)blockIdx.x * 16;
  const int64_t qi = q0 + c;
  const bool qok = qi < seq;
  const int64_t T = P + seq;
  const int64_t last = qok ? P + qi : -1;  // last key query c sees
  const int64_t qmax = (q0 + 16 < seq ? q0 + 16 : seq) - 1;
  const int nkb = (int)((P + qmax + 1 + 15) / 16);  // key blocks any query here sees
  const float *Kb = pk + (b * kvh + kv) * cap * HD;
  const float *Vb = pv + (b * kvh + kv) * cap * HD;
  const float *brow = bias ? bias + ((b * bias_heads + (h % bias_heads)) * seq +
                                     (qok ? qi : 0)) * T
                           : nullptr;

  float qf[kQd];
  ld_run<kQd>(Q + (b * seq + (qok ? qi : seq - 1)) * q_row_stride + (int64_t)h * HD + g * kQd,
              qf);
#pragma unroll
  for (int t = 0; t < kQd; t++) qf[t] = qok ? qf[t] : 0.0f;

  float m = -INFINITY, l = 0.0f;
  f32x4 o[kVd];
#pragma unroll
  for (int db = 0; db < kVd; db++) o[db] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  auto load_block = [&](int kb, float (&kf)[kQd], float (&vf)[4][kVd]) {
    int64_t key = (int64_t)kb * 16 + c;
    key = key < T ? key : T - 1;
    ld_run<kQd>(Kb + key * HD + g * kQd, kf);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int64_t kt = (int64_t)kb * 16 + 4 * g + t;
      kt = kt < T ? kt : T - 1;
      ld_run<kVd>(Vb + kt * HD + c * kVd, vf[t]);
    }
  };
  auto block = [&](int kb, const float (&kf)[kQd], const float (&vf)[4][kVd]) {
    f32x4 s4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < kQd; t++) s4 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t], qf[t], s4, 0, 0, 0);
    float sv[4];
    float bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t key = (int64_t)kb * 16 + 4 * g + r;
      const bool ok = key <= last;
      float v = s4[r] * scale;
      if (bias) v += brow[ok ? key : 0];
      sv[r] = ok ? v : -INFINITY;
      bm = fmaxf(bm, sv[r]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    float p[4], corr = 1.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = 0.0f;
    if (mn != -INFINITY) {
#pragma unroll
      for (int r = 0; r < 4; r++) p[r] = sv[r] == -INFINITY ? 0.0f : expf(sv[r] - mn);
      corr = m == -INFINITY ? 0.0f : expf(m - mn);
    }
    float ps = (p[0] + p[1]) + (p[2] + p[3]);
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * corr + ps;
    m = mn;
#pragma unroll
    for (int db = 0; db < kVd; db++) o[db] *= corr;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int db = 0; db < kVd; db++)
        o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[t][db], p[t], o[db], 0, 0, 0);
  };

  for (int kb0 = w; kb0 < nkb; kb0 += 2 * kAttnMfWaves) {
    const int kb1 = kb0 + kAttnMfWaves;
    float kf0[kQd], kf1[kQd], vf0[4][kVd], vf1[4][kVd];
    load_block(kb0, kf0, vf0);
    load_block(kb1 < nkb ? kb1 : kb0, kf1, vf1);  // unconditional (clamped)
    block(kb0, kf0, vf0);
    if (kb1 < nkb) block(kb1, kf1, vf1);
  }

  // ---- merge the waves' partials: (0,4) (1,5) (2,6) (3,7), then (0,2)
  // (1,3), then (0,1); each wave stores its lanes' state in lane order
#pragma unroll
  for (int half = kAttnMfWaves / 2; half >= 1; half >>= 1) {
    __syncthreads();
    if (w >= half && w < 2 * half) {
      float *sl = &s_slot[w - half][0][0];
#pragma unroll
      for (int db = 0; db < kVd; db++)
#pragma unroll
        for (int r = 0; r < 4; r++) sl[(db * 4 + r) * 64 + ln] = o[db][r];
      sl[kQd * 64 + ln] = m;
      sl[(kQd + 1) * 64 + ln] = l;
    }
    __syncthreads();
    if (w < half) {
      const float *sl = &s_slot[w][0][0];
      const float m2 = sl[kQd * 64 + ln], l2 = sl[(kQd + 1) * 64 + ln];
      const float M = fmaxf(m, m2);
      if (M != -INFINITY) {
        const float a1 = m == -INFINITY ? 0.0f : expf(m - M);
        const float a2 = m2 == -INFINITY ? 0.0f : expf(m2 - M);
        l = a1 * l + a2 * l2;
#pragma unroll
        for (int db = 0; db < kVd; db++)
#pragma unroll
          for (int r = 0; r < 4; r++) o[db][r] = a1 * o[db][r] + a2 * sl[(db * 4 + r) * 64 + ln];
        m = M;
      }
    }
  }
  if (w == 0 && qok) {
    const float inv = 1.0f / l;
    float *orow = out + (b * seq + qi) * out_row_stride + (int64_t)h * HD;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int db = 0; db < kVd; db += 2) {
        const float2 v2 = {o[db][r] * inv, o[db + 1][r] * inv};
        *(float2 *)(orow + (4 * g + r) * kVd + db) = v2;
      }
  }
}

// ---------------------------------------------------------------------------
// Decoder prefill helpers.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed_rows(const int64_t *__restrict__ tok,
                                                    const float *__restrict__ table, int64_t H,
                                                    float *__restrict__ x) {
  const int64_t r = blockIdx.x;
  const float *src = table + tok[r] * H;
  for (int64_t k = threadIdx.x; k < H; k += blockDim.x) x[r * H + k] = src[k];
}

// Per-head RMSNorm of q / k then rotary, one workgroup (hd threads) per
// (row, head); k and v land in the cache at position P + row.
__device__ __forceinline__ float head_norm_rope(float x, const float *__restrict__ g, float eps,
                                                int hd, const float *__restrict__ cos,
                                                const float *__restrict__ sin, int64_t p,
                                                float *sh, double *shd) {
  const int d = threadIdx.x;
  const double ss = block_sum_d((double)x * (double)x, shd);
  const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
  const float xn = (float)((double)x * inv * (double)g[d]);
  sh[d] = xn;
  __syncthreads();
  const int hr = hd / 2;
  const int pi = d < hr ? d : d - hr;
  const double c = cos[p * hr + pi], sn = sin[p * hr + pi];
  const double x0 = sh[pi], x1 = sh[pi + hr];
  const float r = (float)(d < hr ? x0 * c - x1 * sn : x1 * c + x0 * sn);
  __syncthreads();
  return r;
}

__global__ void k_qk_prep_rows(const float *__restrict__ qkv, int64_t qkv_stride, int nh,
                               int kvh, int hd, const float *__restrict__ qn,
                               const float *__restrict__ kn, float eps,
                               const float *__restrict__ cos, const float *__restrict__ sin,
                               int64_t P, float *__restrict__ qout, float *__restrict__ ck,
                               float *__restrict__ cv, int64_t cap) {
  __shared__ float sh[kAttnMaxHd];
  __shared__ double shd[4];
  const int64_t r = blockIdx.x;
  const int hi = blockIdx.y;
  const int d = threadIdx.x;
  const float *row = qkv + r * qkv_stride;
  const int64_t p = P + r;
  if (hi < nh) {
    const float y = head_norm_rope(row[hi * hd + d], qn, eps, hd, cos, sin, p, sh, shd);
    qout[r * (int64_t)nh * hd + hi * hd + d] = y;
  } else {
    const int kh = hi - nh;
    const float y = head_norm_rope(row[(nh + kh) * hd + d], kn, eps, hd, cos, sin, p, sh, shd);
    ck[((int64_t)kh * cap + p) * hd + d] = y;
    cv[((int64_t)kh * cap + p) * hd + d] = row[(nh + kvh + kh) * hd + d];
  }
}

// a[r, j] = silu(gu[r, 2j]) * gu[r, 2j+1]: sigmoid in double stored as
// binary32, then two binary32 products (the Sigmoid, Mul, Mul nodes).
__global__ __launch_bounds__(256) void k_swiglu_rows(const float *__restrict__ gu, int64_t I,
                                                     float *__restrict__ a) {
  const int64_t r = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= I) return;
  const float g = gu[r * 2 * I + 2 * j], u = gu[r * 2 * I + 2 * j + 1];
  const float sig = (float)(1.0 / (1.0 + exp(-(double)g)));
  a[r * I + j] = (g * sig) * u;
}

// ---------------------------------------------------------------------------
// Decode step.  State lives in device memory so a captured graph advances
// the sequence by itself.
// ---------------------------------------------------------------------------
struct DecState {
  int pos;    // position of the token being fed
  int token;  // token being fed
  int step;   // decode steps taken (index into the output list)
  int pad;
  unsigned long long argmax;  // (orderable logit << 32 | ~index) of the best logit
};

__global__ __launch_bounds__(256) void k_dec_begin(DecState *__restrict__ st,
                                                   const float *__restrict__ table, int64_t H,
                                                   int64_t vocab, float *__restrict__ x,
                                                   const float *__restrict__ cos,
                                                   const float *__restrict__ sin, int half,
                                                   int rows, float *__restrict__ rot) {
  // every argument in SGPRs up front (one round of scalar loads)
  kernarg_fence(st, table, H, vocab, x, cos, sin, half, rows, rot, blockDim.x);
  // the token comes from the previous step's argmax, always in range; the
  // clamp only keeps a corrupted state from reading outside the table
  int64_t tok = st->token;
  tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
  // the step's rotary row (cos | sin at pos; half <= 64 < blockDim), so that
  // the attention's loads do not wait for the position; loaded first
  int pos = st->pos;
  pos = pos < 0 ? 0 : (pos >= rows ? rows - 1 : pos);
  const int ic = (int)threadIdx.x < half ? (int)threadIdx.x : 0;
  const float cv = cos[(int64_t)pos * half + ic], sv = sin[(int64_t)pos * half + ic];
  // four loads in flight per thread (a plain loop waited for each in turn)
  for (int64_t k0 = threadIdx.x; k0 < H; k0 += 4 * (int64_t)blockDim.x) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int64_t k = k0 + u * (int64_t)blockDim.x;
      v[u] = table[tok * H + (k < H ? k : H - 1)];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int64_t k = k0 + u * (int64_t)blockDim.x;
      if (k < H) x[k] = v[u];
    }
  }
  if ((int)threadIdx.x < half) {
    rot[threadIdx.x] = cv;
    rot[half + threadIdx.x] = sv;
  }
}

// Greedy token: the maximum of the lm_head workgroups' keys (one workgroup).
__global__ __launch_bounds__(1024) void k_dec_end(DecState *__restrict__ st,
                                                  const unsigned long long *__restrict__ keys,
                                                  int nkeys, int32_t *__restrict__ out_tokens,
                                                  int out_cap) {
  __shared__ unsigned long long sk[16];
  kernarg_fence(st, keys, nkeys, out_tokens, out_cap, blockDim.x);
  const int step = st->step, pos = st->pos;  // read now, not after the reduction
  unsigned long long best = 0ull;
  // eight keys in flight per thread (clamped: a repeated key leaves the
  // maximum alone); a plain loop waited for every key in turn
  for (int i0 = threadIdx.x; i0 < nkeys; i0 += 8 * (int)blockDim.x) {
    unsigned long long k8[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = i0 + u * (int)blockDim.x;
      k8[u] = keys[i < nkeys ? i : nkeys - 1];
    }
#pragma unroll
    for (int u = 0; u < 8; u++) best = k8[u] > best ? k8[u] : best;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long key = sk[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) key = sk[w] > key ? sk[w] : key;
    st->argmax = key;
    const int tok = (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    st->token = tok;
    if (step >= 0 && step < out_cap) out_tokens[step] = tok;
    st->step = step + 1;
    st->pos = pos + 1;
  }
}

// Decode attention for one token, spread over the GPU: one workgroup per
// (split of KS keys, KV head), serving every query head of that KV
// group, so each cached key and value is read once per layer and the read
// is shared by many CUs (one CU alone streams only a few tens of GB/s of
// dependent loads).  The workgroup first issues the loads its per-head
// RMSNorm needs (q heads, new k and v, gammas, rotary row), then its K / V
// tile (unconditional loads: a conditional load would end in a full vmcnt
// wait), so the norms run while the tile is in flight.  Each wave then owns
// 8 keys: scores (8 lanes per key, DPP reduction), a softmax over its keys
// (the 8 scores read out with readlane, so wave-uniform) and p.v with no
// LDS round trip; one barrier later the KS / 8 waves' (max, sum, o) are merged
// into the split's partial per query head.  Where the o projection can
// take them (caches of up to kDecAttnMaxSplits splits, heads * head_dim <=
// kDecAttnMaxK) the partials are left for its prologue to merge
// (launch_dec_gemv_attn), so this launch ends with its partial stores.
// Otherwise the last split of a KV head to finish (counter, reset by it)
// merges them, partials and counters going through agent-scope atomics.
// At the Qwen3-0.6B shape (position ~300, decode step as a graph) leaving
// the merge to the o projection takes 0.611 -> 0.577 ms per token: the
// count and last-arriver merge are three memory round trips after the
// partial, the prologue's merge overlaps the projection's weight loads.  The
// split holding position pos uses the new k / v directly and also writes
// them into the cache; no workgroup reads an entry written in the same
// launch.
// Keys per split kDecKS = 64 (8 waves).  At the Qwen3-0.6B shape (cache 320,
// position ~300, decode step as a graph): 32-key splits 0.568 ms per token,
// 64 0.559-0.561, 128 0.612; the o projection merges half the partials of
// 32-key splits, and 64-key splits keep that merge (<= 16 splits) up to
// 1024 rows.
constexpr int kDecKW = 8;  // keys per wave
constexpr int kDecKS = 64;
template <int KS>
constexpr int dec_attn_threads() { return 64 * (KS / kDecKW); }
constexpr int kDecMaxGroup = 4;     // query heads per KV head
constexpr int kDecMaxLen = 8192;    // longest cache of a decoder session

// Sum over each aligned group of 8 lanes (DPP within a row).
__device__ __forceinline__ float lane8_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror: lanes 0-7 <-> 7-0 of each half row
  return v;
}

// v + (v moved by the DPP control CTRL) for a double (both halves move).
template <int CTRL>
__device__ __forceinline__ double dpp_add_d(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF,
                                                            false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL,
                                                            0xF, 0xF, false);
  return v + __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum over the whole wave, wave-uniform: 16-lane sums by DPP, then the four
// rows read out with readlane.
__device__ __forceinline__ double wave_sum_d(double v) {
  v = dpp_add_d<0xB1>(v);
  v = dpp_add_d<0x4E>(v);
  v = dpp_add_d<0x141>(v);
  v = dpp_add_d<0x140>(v);  // row_mirror
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// Operands of one layer's decode attention.  The partial of query head
// qh = kh * group + g over split s: o[HD] at po + (qh * nsmax + s) * HD and
// (max, sum) at pml + 2 * (qh * nsmax + s).
struct DecAttnArgs {
  const float *qkv;
  int nh, kvh;
  const float *qn, *kn;
  float eps;
  const float *rot;  // cos | sin of the step's position (HD/2 each)
  float *ck, *cv;
  int64_t cap;
  float scale;
  float *po, *pml;
  int nsmax;
  float *out;
};

// One split of KS keys of KV head kh at position pos: the group's q
// heads and the new k (per-head RMSNorm in double, rotary at pos), scores,
// a softmax and o = sum p v per wave of kDecKW keys, then the split's
// partial (max, sum, o) of every query head of the group.  The split
// holding pos also writes the new k / v into the cache.  Whole workgroup,
// KS / 8 waves.
template <int HD, bool COH, int KS>
__device__ bool dec_attn_partial(const DecAttnArgs &a, int pos_in, int split, int kh) {
  constexpr int kDecAttnWaves = KS / kDecKW;
  constexpr int kDpk = HD / 8;  // K dims per lane (a multiple of 4)
  constexpr int kHr = HD / 2;   // rotary half; norm lanes hold dims l, l + kHr
  __shared__ __align__(16) float sq[kDecMaxGroup][HD];
  __shared__ __align__(16) float skn[HD];
  __shared__ __align__(16) float svn[HD];
  __shared__ __align__(16) float so[kDecAttnWaves][kDecMaxGroup][HD];
  __shared__ float sm[kDecAttnWaves][kDecMaxGroup], sl[kDecAttnWaves][kDecMaxGroup];
  const int nh = a.nh, kvh = a.kvh, group = nh / kvh;
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int jk = t >> 3, p8 = t & 7;  // K layout: key, dim slice
  const int j0 = split * KS;
  const float *Kb = a.ck + (int64_t)kh * a.cap * HD;
  const float *Vb = a.cv + (int64_t)kh * a.cap * HD;
  // ---- loads, in the order they are used.  Norm rows: wave w takes q head
  // min(w, group - 1) of the group (kept if w < group) and every wave the
  // new k (kept by wave 0), so that no load or norm sits behind a branch;
  // lane l < kHr holds dims l and l + kHr, so the rotary pair is in one lane.
  const int lc = l < kHr ? l : 0;
  float x0[2], x1[2], g0[2], g1[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const float *xr = a.qkv + (i == 0 ? kh * group + min(w, group - 1) : nh + kh) * HD;
    const float *gr = i == 0 ? a.qn : a.kn;
    x0[i] = xr[lc];
    x1[i] = xr[lc + kHr];
    g0[i] = gr[lc];
    g1[i] = gr[lc + kHr];
  }
  const int lv = 2 * l < HD ? l : 0;  // V layout: dims 2 lv, 2 lv + 1
  const float2 xv = *(const float2 *)(a.qkv + (nh + kvh + kh) * HD + 2 * lv);
  const double cs = (double)a.rot[lc];
  const double sn = (double)a.rot[kHr + lc];
  // the norm's loads go out first (a wait for one of them waits for every
  // load issued before it)
  __builtin_amdgcn_sched_barrier(0);
  // K / V tile: addresses independent of pos (rows are clamped to the
  // cache; rows >= pos are replaced or dropped below)
  float kreg[kDpk];
  {
    const int j = j0 + jk;
    const float *kr = Kb + (int64_t)(j < a.cap ? j : a.cap - 1) * HD + p8 * kDpk;
#pragma unroll
    for (int e = 0; e < kDpk; e += 4) {
      const float4 v4 = *(const float4 *)(kr + e);
      kreg[e] = v4.x;
      kreg[e + 1] = v4.y;
      kreg[e + 2] = v4.z;
      kreg[e + 3] = v4.w;
    }
  }
  float2 vreg[kDecKW];
#pragma unroll
  for (int u = 0; u < kDecKW; u++) {
    const int j = j0 + w * kDecKW + u;
    vreg[u] = *(const float2 *)(Vb + (int64_t)(j < a.cap ? j : a.cap - 1) * HD + 2 * lv);
  }
  // the position is first used here, after every load is out (a use
  // before them would hold them until it arrives); splits past it leave
  int pos = pos_in;
  asm volatile("" : "+v"(pos));
  const int L = pos + 1;
  const int nsplit = (L + KS - 1) / KS;
  if (split >= nsplit) {
    asm volatile("" ::"v"(kreg[0]), "v"(vreg[0].x), "v"(x0[0]), "v"(xv.x));
    if constexpr (!COH) {
      // a split past pos leaves an empty partial (max -inf, sum 0, o 0) for
      // the o projection's merge, which so needs no position of its own
      const int t = threadIdx.x;
      for (int i = t; i < group * HD; i += KS / kDecKW * 64)
        a.po[((int64_t)(kh * group) * a.nsmax + (int64_t)(i / HD) * a.nsmax + split) * HD +
             i % HD] = 0.0f;
      if (t < group) {
        const int64_t ps = (int64_t)(kh * group + t) * a.nsmax + split;
        a.pml[2 * ps] = -INFINITY;
        a.pml[2 * ps + 1] = 0.0f;
      }
    }
    return false;
  }
  // ---- per-head RMSNorm (double sums, wave-local) and rotary at pos
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const double ss = l < kHr ? (double)x0[i] * x0[i] + (double)x1[i] * x1[i] : 0.0;
    const double inv = 1.0 / sqrt(wave_sum_d(ss) / (double)HD + (double)a.eps);
    const float y0 = (float)((double)x0[i] * inv * (double)g0[i]);
    const float y1 = (float)((double)x1[i] * inv * (double)g1[i]);
    const float r0 = (float)((double)y0 * cs - (double)y1 * sn);
    const float r1 = (float)((double)y1 * cs + (double)y0 * sn);
    if (l < kHr && (i == 0 ? w < group : w == 0)) {
      float *dst = i == 0 ? sq[w] : skn;
      dst[l] = r0;
      dst[l + kHr] = r1;
    }
  }
  if (w == 3 && 2 * l < HD) *(float2 *)(svn + 2 * l) = xv;
  __syncthreads();
  // ---- scores of this wave's keys, for each query head of the group
  const int j = j0 + jk;
  if (j == pos) {
#pragma unroll
    for (int e = 0; e < kDpk; e++) kreg[e] = skn[p8 * kDpk + e];
  }
  float sc[kDecMaxGroup];
#pragma unroll
  for (int g = 0; g < kDecMaxGroup; g++) {
    sc[g] = -INFINITY;
    if (g < group) {
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < kDpk; e += 4) {
        const float4 q4 = *(const float4 *)(&sq[g][p8 * kDpk + e]);
        dot = fmaf(q4.x, kreg[e], dot);
        dot = fmaf(q4.y, kreg[e + 1], dot);
        dot = fmaf(q4.z, kreg[e + 2], dot);
        dot = fmaf(q4.w, kreg[e + 3], dot);
      }
      dot = lane8_sum(dot);
      sc[g] = j < L ? dot * a.scale : -INFINITY;
    }
  }
  // values of keys past pos are dropped here (their probability is 0, but
  // the row they were read from may hold anything)
  {
    const float2 vnew = *(const float2 *)(svn + 2 * lv);
#pragma unroll
    for (int u = 0; u < kDecKW; u++) {
      const int jv = j0 + w * kDecKW + u;
      if (jv >= pos) vreg[u] = jv == pos ? vnew : make_float2(0.0f, 0.0f);
    }
  }
  // ---- softmax over the wave's keys and o = sum_u p_u v_u.  The maximum
  // from the scores read out of lanes 8u (wave-uniform); each lane then
  // forms the probability of its own key, one exponential per lane in
  // parallel, and the 8 probabilities are read out of lanes 8u in turn (the
  // wave-uniform scores fed 8 dependent exponentials per lane: ~2 us per
  // layer of the decode step).  A wave whose keys are all past pos
  // contributes max -inf and nothing else.
#pragma unroll
  for (int g = 0; g < kDecMaxGroup; g++) {
    if (g < group) {
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < kDecKW; u++)
        mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                     __builtin_bit_cast(int, sc[g]), 8 * u)));
      const float pl = mx != -INFINITY ? expf(sc[g] - mx) : 0.0f;  // 0 past pos
      float ls = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
      for (int u = 0; u < kDecKW; u++) {
        const float pu = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pl), 8 * u));
        ls += pu;
        o0 = fmaf(pu, vreg[u].x, o0);
        o1 = fmaf(pu, vreg[u].y, o1);
      }
      if (2 * l < HD) *(float2 *)(&so[w][g][2 * l]) = make_float2(o0, o1);
      if (l == 0) {
        sm[w][g] = mx;
        sl[w][g] = ls;
      }
    }
  }
  __syncthreads();
  // ---- the split's partial: thread (head g, dim pair dp) merges the waves
  {
    const int g = t / kHr, dp = t % kHr;
    // the waves' weights e^(m_w - M): lane dp forms that of wave dp % NW
    // (one exponential per lane) and takes the others from the lanes of its
    // aligned group of NW, which share g (NW divides kHr)
    static_assert(kHr % kDecAttnWaves == 0, "wave weights by lane groups");
    float M = sm[0][g < group ? g : 0];
#pragma unroll
    for (int ww = 1; ww < kDecAttnWaves; ww++) M = fmaxf(M, sm[ww][g < group ? g : 0]);
    const float mine = expf(sm[dp % kDecAttnWaves][g < group ? g : 0] - M);  // 0: max -inf
    const int base = (threadIdx.x & 63) & ~(kDecAttnWaves - 1);
    if (g < group) {
      float ls = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
      for (int ww = 0; ww < kDecAttnWaves; ww++) {
        const float wt = __shfl(mine, base + ww, 64);
        const float2 ov = *(const float2 *)(&so[ww][g][2 * dp]);
        ls = fmaf(wt, sl[ww][g], ls);
        o0 = fmaf(wt, ov.x, o0);
        o1 = fmaf(wt, ov.y, o1);
      }
      const int64_t ps = (int64_t)(kh * group + g) * a.nsmax + split;
      float *pp = a.po + ps * HD;
      if (dp == 0) {
        st_act<COH>(a.pml + 2 * ps, M);
        st_act<COH>(a.pml + 2 * ps + 1, ls);
      }
      st_act<COH>(pp + 2 * dp, o0);
      st_act<COH>(pp + 1 + 2 * dp, o1);
    }
  }
  // the split holding position pos writes the new k / v into the cache
  // (issued late: an outstanding store would hold up every vmcnt wait above)
  if (split == nsplit - 1 && t < HD) {
    a.ck[((int64_t)kh * a.cap + pos) * HD + t] = skn[t];
    a.cv[((int64_t)kh * a.cap + pos) * HD + t] = svn[t];
  }
  return true;
}

// Merges the nsplit partials of KV head kh into out (every query head of the
// group).  Each thread (head g, dim) loads the (max, sum, o[dim]) of 16
// splits at once (one memory round trip for caches up to 16 * KS; the
// (max, sum) addresses are the same across the head's threads) and forms
// the weights exp(m_s - M) itself, so no barrier is needed; longer caches
// take further batches of 16, rescaling what is summed so far to the new
// maximum.  Whole workgroup.
template <int HD, int KS>
__device__ void dec_attn_merge(const DecAttnArgs &a, int pos, int kh) {
  const int group = a.nh / a.kvh, t = threadIdx.x;
  const int nsplit = (pos + 1 + KS - 1) / KS;
  for (int i = t; i < group * HD; i += dec_attn_threads<KS>()) {
    const int gi = i / HD, di = i % HD;
    const int64_t p0 = (int64_t)(kh * group + gi) * a.nsmax;
    float M = -INFINITY, den = 0.0f, num = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += 16) {
      float mv[16], lv[16], ov[16];
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const int64_t ps = p0 + min(s0 + u, nsplit - 1);
        mv[u] = ld_act<true>(a.pml + 2 * ps);
        lv[u] = ld_act<true>(a.pml + 2 * ps + 1);
        ov[u] = ld_act<true>(a.po + ps * HD + di);
      }
      // every split has a key at or before pos, so its max is finite
      float Mb = M;
#pragma unroll
      for (int u = 0; u < 16; u++)
        if (s0 + u < nsplit) Mb = fmaxf(Mb, mv[u]);
      const float c = expf(M - Mb);  // 0 on the first batch
      den *= c;
      num *= c;
#pragma unroll
      for (int u = 0; u < 16; u++) {
        if (s0 + u < nsplit) {
          const float wgt = expf(mv[u] - Mb);
          den = fmaf(wgt, lv[u], den);
          num = fmaf(wgt, ov[u], num);
        }
      }
      M = Mb;
    }
    a.out[(kh * group + gi) * HD + di] = num / den;
  }
}

// Launch form: grid (splits, KV heads).  MERGE: the last split of a KV
// head to finish (counter, reset by it) merges the partials into out;
// otherwise every split leaves its partial for the next launch (the o
// projection's prologue, launch_dec_gemv_attn), whose start orders it.
template <int HD, bool MERGE, int KS>
__global__ __launch_bounds__(dec_attn_threads<KS>()) void k_dec_attn(const DecState *__restrict__ st,
                                                  DecAttnArgs a, int *counters) {
  __shared__ int s_last;
  const int split = blockIdx.x, kh = blockIdx.y;
  // every argument the loads need in SGPRs up front (one round of scalar
  // loads instead of dependent rounds ahead of the first load)
  kernarg_fence(st, a.qkv, a.nh, a.kvh, a.qn, a.kn, a.eps, a.rot, a.ck, a.cv, a.cap, a.scale,
                a.po, a.pml, a.nsmax);
  if constexpr (MERGE) kernarg_fence(counters, a.out);
  // the position through the vector memory path, used only once the
  // partial's loads are out: a scalar load would join the kernel-argument
  // loads' wait, in front of every other load
  const int pos_v = __hip_atomic_load(const_cast<int *>(&st->pos), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
  if (!dec_attn_partial<HD, MERGE, KS>(a, pos_v, split, kh)) return;  // whole workgroup
  if constexpr (!MERGE) return;
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);
  const int nsplit = (pos + 1 + KS - 1) / KS;
  // ---- publish: the barrier orders every thread's partial stores before
  // thread 0's count; its release (agent scope) pairs with the acquire fence
  // of the last split, which reads the count the others' releases wrote, and
  // that workgroup's barrier extends it to the merge's loads.  Only the last
  // split acquires (an agent-scope acquire invalidates this XCD's L2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev =
        __hip_atomic_fetch_add(&counters[kh], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == nsplit - 1;
    if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!s_last) return;
  dec_attn_merge<HD, KS>(a, pos, kh);
  if (threadIdx.x == 0)
    __hip_atomic_store(&counters[kh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Op launchers
// ---------------------------------------------------------------------------
static int launch_rmsnorm(mmnb_ctx *ctx, const float *x, int64_t rows, int64_t dim,
                          const float *g, float eps, float *y, const float *add, float *xsum) {
  if (rows == 0) return MMNB_OK;
  return launch(ctx, kKernDecOps, k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, x, dim, g, eps,
                y, add, xsum);
}

static int launch_attn_rows(mmnb_ctx *ctx, const float *q, int64_t q_stride, int64_t batch,
                            int64_t seq, int nh, int kvh, int hd, const float *pk,
                            const float *pv, int64_t cap, int64_t P, float scale,
                            const float *bias, int bias_heads, float *out, int64_t out_stride) {
  const dim3 grid((unsigned)((seq + kAttnQ - 1) / kAttnQ), (unsigned)nh, (unsigned)batch);
  // matrix-core kernel: head size a multiple of 32, float4-aligned rows
  const bool al = ((((uintptr_t)q | (uintptr_t)pk | (uintptr_t)pv | (uintptr_t)out) & 15) == 0) &&
                  q_stride % 4 == 0 && out_stride % 4 == 0;
  if (al && ctx->attn_mfma) {
#define MMNB_ATTN_MF(HD)                                                                      \
  launch(ctx, kKernDecAttn, k_attn_mfma<HD>, grid, dim3(64 * kAttnMfWaves), 0, q, q_stride,  \
         seq, nh, kvh, pk, pv, cap, P, scale, bias, bias_heads, out, out_stride)
    switch (hd) {
      case 32: return MMNB_ATTN_MF(32);
      case 64: return MMNB_ATTN_MF(64);
      case 96: return MMNB_ATTN_MF(96);
      case 128: return MMNB_ATTN_MF(128);
      default: break;
    }
#undef MMNB_ATTN_MF
  }
  return launch(ctx, kKernDecAttn, k_attn_rows, grid, dim3(256), 0, q, q_stride, seq, nh, kvh,
                hd, pk, pv, cap, P, scale, bias, bias_heads, out, out_stride);
}

}  // namespace mmnb

using namespace mmnb;

// ---------------------------------------------------------------------------
// C ABI: ops
// ---------------------------------------------------------------------------
int mmnb_rmsnorm_dev(mmnb_ctx *ctx, const float *d_x, int64_t rows, int64_t dim,
                     const float *d_gamma, float eps, float *d_y) {
  MMNB_GUARD_CTX(ctx);
  if (rows < 0 || dim <= 0) return fail(MMNB_ERR_ARG, "RMSNorm: bad shape");
  if (rows == 0) return MMNB_OK;
  if (!d_x || !d_gamma || !d_y) return fail(MMNB_ERR_ARG, "RMSNorm: null buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch_rmsnorm(ctx, d_x, rows, dim, d_gamma, eps, d_y, nullptr, nullptr);
}

int mmnb_rotary_dev(mmnb_ctx *ctx, const float *d_x, int64_t batch, int64_t seq,
                    int64_t hidden, int64_t num_heads, const int64_t *d_pos, int64_t pos_rank,
                    const float *d_cos, const float *d_sin, int64_t half_rot, int interleaved,
                    float *d_y) {
  MMNB_GUARD_CTX(ctx);
  if (batch < 0 || seq < 0 || hidden <= 0 || half_rot <= 0 || num_heads < 0)
    return fail(MMNB_ERR_ARG, "RotaryEmbedding: bad shape");
  const int64_t head = num_heads > 0 ? hidden / num_heads : 2 * half_rot;
  if (head <= 0 || hidden % head != 0 || 2 * half_rot > head)
    return fail(MMNB_ERR_ARG, "RotaryEmbedding: hidden, num_heads and rotary dim disagree");
  if (pos_rank != 1 && pos_rank != 2) return fail(MMNB_ERR_ARG, "RotaryEmbedding: pos rank");
  if (batch * seq == 0) return MMNB_OK;
  if (!d_x || !d_pos || !d_cos || !d_sin || !d_y)
    return fail(MMNB_ERR_ARG, "RotaryEmbedding: null buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch(ctx, kKernDecOps, k_rotary, dim3((unsigned)(batch * seq)), dim3(256), 0, d_x,
                seq, (int)(hidden / head), (int)head, d_pos, (int)pos_rank, (int64_t)0, d_cos,
                d_sin, (int)half_rot, interleaved, d_y);
}

int mmnb_gqa_dev(mmnb_ctx *ctx, const float *d_q, const float *d_k, const float *d_v,
                 int64_t batch, int64_t seq, int64_t num_heads, int64_t kv_heads,
                 int64_t head_size, float scale, const float *d_past_k, const float *d_past_v,
                 int64_t past_len, const float *d_cos, const float *d_sin, int64_t half_rot,
                 int do_rotary, int interleaved, const float *d_bias, int64_t bias_heads,
                 float *d_out, float *d_present_k, float *d_present_v) {
  MMNB_GUARD_CTX(ctx);
  if (batch < 0 || seq < 0 || num_heads <= 0 || kv_heads <= 0 || head_size <= 0 ||
      past_len < 0)
    return fail(MMNB_ERR_ARG, "GroupQueryAttention: bad shape");
  if (num_heads % kv_heads != 0)
    return fail(MMNB_ERR_ARG, "GroupQueryAttention: num_heads % kv_num_heads != 0");
  if (head_size > kAttnMaxHd)
    return fail(MMNB_ERR_UNSUPPORTED, "GroupQueryAttention: head size above 128");
  if (do_rotary && (!d_cos || !d_sin || 2 * half_rot > head_size || half_rot <= 0))
    return fail(MMNB_ERR_ARG, "GroupQueryAttention: rotary caches");
  if (d_bias && bias_heads <= 0) return fail(MMNB_ERR_ARG, "GroupQueryAttention: bias heads");
  // The reference builds rotary positions as [1, seq] and indexes them by
  // batch (onnx_ops.dart:1537-1541, :2150): batch > 1 with rotary throws.
  if (do_rotary && batch > 1)
    return fail(MMNB_ERR_ARG, "GroupQueryAttention: rotary with batch > 1 (position ids are [1, seq])");
  if (batch * seq == 0) return MMNB_OK;
  if (!d_q || !d_k || !d_v || !d_out || !d_present_k || !d_present_v ||
      (past_len > 0 && (!d_past_k || !d_past_v)))
    return fail(MMNB_ERR_ARG, "GroupQueryAttention: null buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  const int nh = (int)num_heads, kvh = (int)kv_heads, hd = (int)head_size;
  const int64_t T = past_len + seq;
  const float *q = d_q, *k = d_k;
  if (do_rotary) {
    void *tmp = nullptr;
    const size_t qn = (size_t)(batch * seq * nh * hd), kn = (size_t)(batch * seq * kvh * hd);
    if ((rc = scratch_get(ctx, 4, (qn + kn) * 4, &tmp))) return rc;
    float *qr = (float *)tmp, *kr = qr + qn;
    if ((rc = launch(ctx, kKernDecOps, k_rotary, dim3((unsigned)(batch * seq)), dim3(256), 0,
                     d_q, seq, nh, hd, (const int64_t *)nullptr, 1, past_len, d_cos, d_sin,
                     (int)half_rot, interleaved, qr)))
      return rc;
    if ((rc = launch(ctx, kKernDecOps, k_rotary, dim3((unsigned)(batch * seq)), dim3(256), 0,
                     d_k, seq, kvh, hd, (const int64_t *)nullptr, 1, past_len, d_cos, d_sin,
                     (int)half_rot, interleaved, kr)))
      return rc;
    q = qr;
    k = kr;
  }
  if ((rc = launch(ctx, kKernDecOps, k_gqa_present, dim3((unsigned)(kvh * T), (unsigned)batch),
                   dim3(128), 0, d_past_k, d_past_v, past_len, k, d_v, seq, kvh, hd, T,
                   d_present_k, d_present_v)))
    return rc;
  const float sc = scale > 0.0f ? scale : (float)(1.0 / std::sqrt((double)hd));
  return launch_attn_rows(ctx, q, (int64_t)nh * hd, batch, seq, nh, kvh, hd, d_present_k,
                          d_present_v, T, past_len, sc, d_bias, (int)bias_heads, d_out,
                          (int64_t)nh * hd);
}

// ---------------------------------------------------------------------------
// Decoder session
// ---------------------------------------------------------------------------
struct mmnb_decoder {
  mmnb_ctx *ctx = nullptr;
  mmnb_decoder_config cfg{};
  struct Layer {
    float *ln1 = nullptr, *ln2 = nullptr, *qn = nullptr, *kn = nullptr;
    const mmnb_pack *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
  };
  std::vector<Layer> layers;
  const mmnb_pack *lm = nullptr;
  float *embed = nullptr, *final_norm = nullptr;
  float *x = nullptr, *h = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr,
        *gu = nullptr, *act = nullptr, *tmp = nullptr, *logits = nullptr;
  float *cache_k = nullptr, *cache_v = nullptr, *cos = nullptr, *sin = nullptr;
  float *rot = nullptr;     // the decode step's rotary row: cos | sin, hd/2 each
  float *part = nullptr;    // attention partials: o [heads, splits, hd], then (max, sum)
  bool attn_defer = false;  // the o projection merges them (else the attention launch)
  int ks = kDecKS;          // keys per attention split
  int *counters = nullptr;  // per KV head: attention splits finished
  DecState *state = nullptr;
  unsigned long long *keys = nullptr;  // lm_head workgroups' best (value, ~index)
  int64_t nkeys = 0;
  int32_t *out_tokens = nullptr;
  int64_t *tok = nullptr;
  int64_t pos = 0;        // host mirror of the sequence length
  int64_t steps_done = 0; // host mirror of DecState::step
  bool primed = false;    // a token is waiting in DecState::token
  hipGraphExec_t graph = nullptr;
  bool use_graph = true;  // replay the recorded step (else launch it eagerly)
  std::vector<void *> allocs;
};

static int dec_alloc(mmnb_decoder *d, size_t bytes, void **p) {
  int rc = device_alloc(bytes, p);
  if (rc) return rc;
  d->allocs.push_back(*p);
  return MMNB_OK;
}

static int dec_upload(mmnb_decoder *d, const float *host, size_t n, float **out) {
  int rc = dec_alloc(d, n * 4, (void **)out);
  if (rc) return rc;
  MMNB_HIP(hipMemcpy(*out, host, n * 4, hipMemcpyHostToDevice));
  return MMNB_OK;
}

int mmnb_decoder_free(mmnb_decoder *d) {
  if (!d) return MMNB_OK;
  if (d->ctx) (void)hipSetDevice(d->ctx->device);
  if (d->ctx) (void)hipStreamSynchronize(d->ctx->stream);
  if (d->graph) (void)hipGraphExecDestroy(d->graph);
  for (void *p : d->allocs) (void)hipFree(p);
  delete d;
  return MMNB_OK;
}

int mmnb_decoder_create(mmnb_ctx *ctx, const mmnb_decoder_config *cfg, const float *embed,
                        const float *final_norm, const mmnb_pack *lm_head,
                        mmnb_decoder **out) {
  MMNB_GUARD_CTX(ctx);
  if (!cfg || !embed || !final_norm || !lm_head || !out)
    return fail(MMNB_ERR_ARG, "decoder: null argument");
  const mmnb_decoder_config &c = *cfg;
  if (c.layers <= 0 || c.hidden <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.head_dim <= 0 ||
      c.intermediate <= 0 || c.vocab <= 0 || c.max_len <= 0 || c.max_len > kDecMaxLen ||
      c.heads % c.kv_heads != 0 || c.heads / c.kv_heads > kDecMaxGroup)
    return fail(MMNB_ERR_ARG, "decoder: bad configuration");
  if (c.head_dim > kAttnMaxHd || (c.head_dim % 32) || c.hidden % 64 || (c.heads * c.head_dim) % 64 ||
      c.intermediate % 64 || c.hidden > 4096 || c.intermediate > 4096 ||
      c.heads * c.head_dim > 4096)
    return fail(MMNB_ERR_UNSUPPORTED,
                "decoder: needs head_dim <= 128 (a multiple of 32) and hidden, heads*head_dim, "
                "intermediate multiples of 64 and <= 4096");
  if (lm_head->kind != kPackNBits || lm_head->ext || lm_head->generic || lm_head->k != c.hidden ||
      lm_head->n != c.vocab ||
      lm_head->ctx != ctx)
    return fail(MMNB_ERR_ARG, "decoder: lm_head pack shape");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  mmnb_decoder *d = new (std::nothrow) mmnb_decoder();
  if (!d) return fail(MMNB_ERR_OOM, "decoder: out of host memory");
  d->ctx = ctx;
  d->cfg = c;
  d->layers.resize((size_t)c.layers);
  d->lm = lm_head;
  d->nkeys = dec_gemv_blocks(ctx, c.vocab, c.hidden);
  const int64_t H = c.hidden, nh = c.heads, kvh = c.kv_heads, hd = c.head_dim,
                I = c.intermediate, Lmax = c.max_len;
  const int64_t QKV = (nh + 2 * kvh) * hd;
  d->ks = kDecKS;
  const int64_t nsplit = (Lmax + d->ks - 1) / d->ks;
  auto A = [&](size_t bytes, void **p) { return dec_alloc(d, bytes, p); };
  if ((rc = dec_upload(d, embed, (size_t)(c.vocab * H), &d->embed)) ||
      (rc = dec_upload(d, final_norm, (size_t)H, &d->final_norm)) ||
      (rc = A((size_t)(Lmax * H) * 4, (void **)&d->x)) ||
      (rc = A((size_t)(Lmax * H) * 4, (void **)&d->h)) ||
      (rc = A((size_t)(Lmax * QKV) * 4, (void **)&d->qkv)) ||
      (rc = A((size_t)(Lmax * nh * hd) * 4, (void **)&d->q)) ||
      (rc = A((size_t)(Lmax * nh * hd) * 4, (void **)&d->attn)) ||
      (rc = A((size_t)(Lmax * 2 * I) * 4, (void **)&d->gu)) ||
      (rc = A((size_t)(Lmax * I) * 4, (void **)&d->act)) ||
      (rc = A((size_t)(Lmax * H) * 4, (void **)&d->tmp)) ||
      (rc = A((size_t)c.vocab * 4, (void **)&d->logits)) ||
      (rc = A((size_t)(c.layers * kvh * Lmax * hd) * 4, (void **)&d->cache_k)) ||
      (rc = A((size_t)(c.layers * kvh * Lmax * hd) * 4, (void **)&d->cache_v)) ||
      (rc = A((size_t)(nh * nsplit * (hd + 2)) * 4, (void **)&d->part)) ||
      (rc = A((size_t)hd * 4, (void **)&d->rot)) ||
      (rc = A((size_t)kvh * 4, (void **)&d->counters)) ||
      (rc = A(sizeof(DecState), (void **)&d->state)) ||
      (rc = A((size_t)dec_gemv_blocks(ctx, c.vocab, c.hidden) * 8, (void **)&d->keys)) ||
      (rc = A((size_t)Lmax * 4, (void **)&d->out_tokens)) ||
      (rc = A((size_t)Lmax * 8, (void **)&d->tok))) {
    mmnb_decoder_free(d);
    return rc;
  }
  // rotary caches [Lmax, hd/2]: angle = pos * theta^(-2i/hd), in double
  std::vector<float> cs((size_t)(Lmax * hd / 2)), sn((size_t)(Lmax * hd / 2));
  for (int64_t p = 0; p < Lmax; p++)
    for (int64_t i = 0; i < hd / 2; i++) {
      const double inv = 1.0 / std::pow((double)c.rope_theta, (double)(2 * i) / (double)hd);
      const double ang = (double)p * inv;
      cs[(size_t)(p * hd / 2 + i)] = (float)std::cos(ang);
      sn[(size_t)(p * hd / 2 + i)] = (float)std::sin(ang);
    }
  if ((rc = dec_upload(d, cs.data(), cs.size(), &d->cos)) ||
      (rc = dec_upload(d, sn.data(), sn.size(), &d->sin))) {
    mmnb_decoder_free(d);
    return rc;
  }
  hipError_t e = hipMemset(d->state, 0, sizeof(DecState));
  if (e == hipSuccess) e = hipMemset(d->counters, 0, (size_t)kvh * 4);
  d->attn_defer = ctx->dec_attn_defer && nsplit <= kDecAttnMaxSplits &&
                  nh * hd <= kDecAttnMaxK &&
                  nh * (nsplit <= 8 ? 8 : 16) <= kDecAttnMergeThreads;
  if (e != hipSuccess) {
    mmnb_decoder_free(d);
    return check_hip(e, "hipMemset");
  }
  *out = d;
  return MMNB_OK;
}

int mmnb_decoder_set_layer(mmnb_decoder *d, int64_t layer, const float *ln1, const float *ln2,
                           const float *q_norm, const float *k_norm, const mmnb_pack *qkv,
                           const mmnb_pack *o, const mmnb_pack *gate_up,
                           const mmnb_pack *down) {
  if (!d) return fail(MMNB_ERR_ARG, "decoder: null handle");
  const mmnb_decoder_config &c = d->cfg;
  if (layer < 0 || layer >= c.layers) return fail(MMNB_ERR_ARG, "decoder: layer index");
  if (!ln1 || !ln2 || !q_norm || !k_norm || !qkv || !o || !gate_up || !down)
    return fail(MMNB_ERR_ARG, "decoder: null argument");
  const int64_t H = c.hidden, hd = c.head_dim, nh = c.heads, kvh = c.kv_heads,
                I = c.intermediate;
  auto ok = [&](const mmnb_pack *p, int64_t k, int64_t n) {
    return p->kind == kPackNBits && !p->ext && !p->generic && p->ctx == d->ctx && p->k == k &&
           p->n == n;
  };
  if (!ok(qkv, H, (nh + 2 * kvh) * hd) || !ok(o, nh * hd, H) || !ok(gate_up, H, 2 * I) ||
      !ok(down, I, H))
    return fail(MMNB_ERR_ARG, "decoder: layer pack shapes do not match the configuration");
  CtxLock lk(d->ctx);
  int rc = set_device(d->ctx);
  if (rc) return rc;
  mmnb_decoder::Layer &L = d->layers[(size_t)layer];
  if (L.ln1) return fail(MMNB_ERR_ARG, "decoder: layer already set");
  if ((rc = dec_upload(d, ln1, (size_t)H, &L.ln1)) || (rc = dec_upload(d, ln2, (size_t)H, &L.ln2)) ||
      (rc = dec_upload(d, q_norm, (size_t)hd, &L.qn)) ||
      (rc = dec_upload(d, k_norm, (size_t)hd, &L.kn)))
    return rc;
  L.qkv = qkv;
  L.o = o;
  L.gu = gate_up;
  L.down = down;
  return MMNB_OK;
}

static int dec_check_ready(mmnb_decoder *d) {
  for (auto &L : d->layers)
    if (!L.ln1) return fail(MMNB_ERR_ARG, "decoder: a layer is not set");
  return MMNB_OK;
}

int mmnb_decoder_reset(mmnb_decoder *d) {
  if (!d) return fail(MMNB_ERR_ARG, "decoder: null handle");
  CtxLock lk(d->ctx);
  int rc = set_device(d->ctx);
  if (rc) return rc;
  MMNB_HIP(hipStreamSynchronize(d->ctx->stream));
  MMNB_HIP(hipMemset(d->state, 0, sizeof(DecState)));
  MMNB_HIP(hipMemset(d->counters, 0, (size_t)d->cfg.kv_heads * 4));
  d->pos = 0;
  d->steps_done = 0;
  d->primed = false;
  return MMNB_OK;
}

// Prompt rows through every layer (the general kernels), then the greedy
// token of the last row.  The KV cache grows by n.
int mmnb_decoder_prefill(mmnb_decoder *d, const int64_t *tokens, int64_t n,
                         int32_t *next_token) {
  if (!d) return fail(MMNB_ERR_ARG, "decoder: null handle");
  mmnb_ctx *ctx = d->ctx;
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "decoder: prefill during graph capture");
  const mmnb_decoder_config &c = d->cfg;
  if (n <= 0 || !tokens) return fail(MMNB_ERR_ARG, "decoder: empty prompt");
  if (d->pos + n > c.max_len) return fail(MMNB_ERR_ARG, "decoder: prompt exceeds max_len");
  for (int64_t i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= c.vocab) return fail(MMNB_ERR_ARG, "decoder: token id");
  int rc = dec_check_ready(d);
  if (rc) return rc;
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  hipStream_t s = ctx->stream;
  const int64_t H = c.hidden, nh = c.heads, kvh = c.kv_heads, hd = c.head_dim,
                I = c.intermediate, Lmax = c.max_len;
  const int64_t QKV = (nh + 2 * kvh) * hd;
  const int64_t P = d->pos;
  const float eps = c.eps;
  const float scale = (float)(1.0 / std::sqrt((double)hd));
  MMNB_HIP(hipMemcpyAsync(d->tok, tokens, (size_t)n * 8, hipMemcpyHostToDevice, s));
  if ((rc = launch(ctx, kKernDecOps, k_embed_rows, dim3((unsigned)n), dim3(256), 0,
                   (const int64_t *)d->tok, (const float *)d->embed, H, d->x)))
    return rc;
  // With more than 8 rows the projections take the MFMA GEMM; the norms and
  // SwiGLU that feed them then write its prepared activations themselves
  // (k_rmsnorm_prep, k_swiglu_prep) instead of fp32 rows for k_prep_a.
  const bool fuse = ctx->prep_fuse && n > 8 && H <= kPrepMaxDim && I <= kPrepMaxDim;
  // x (+= add) normalised with gamma, as the input of the projection `next`
  auto norm_into = [&](const float *gamma, const float *add, const mmnb_pack *next) -> int {
    if (!fuse) return launch_rmsnorm(ctx, d->x, n, H, gamma, eps, d->h, add, add ? d->x : nullptr);
    int64_t segsp = 0, mpad = 0;
    void *ap = nullptr;
    int *ex = nullptr;
    int e = gemm_prepared_a(ctx, next, n, &segsp, &mpad, &ap, &ex);
    if (e) return e;
    return launch(ctx, kKernDecOps, k_rmsnorm_prep, dim3((unsigned)mpad), dim3(256), 0,
                  (const float *)d->x, n, H, gamma, eps, add, add ? d->x : nullptr, segsp,
                  segsp * kSegK, ex, (uint4 *)ap);
  };
  auto gemm_from_norm = [&](const mmnb_pack *pk, float *y) -> int {
    return fuse ? launch_matmul_nbits_prepared(ctx, pk, n, y)
                : launch_matmul_nbits(ctx, pk, d->h, H, n, y);
  };
  if ((rc = norm_into(d->layers[0].ln1, nullptr, d->layers[0].qkv))) return rc;
  for (int64_t li = 0; li < c.layers; li++) {
    const mmnb_decoder::Layer &L = d->layers[(size_t)li];
    float *ck = d->cache_k + li * kvh * Lmax * hd, *cv = d->cache_v + li * kvh * Lmax * hd;
    if ((rc = gemm_from_norm(L.qkv, d->qkv))) return rc;
    if ((rc = launch(ctx, kKernDecOps, k_qk_prep_rows, dim3((unsigned)n, (unsigned)(nh + kvh)),
                     dim3((unsigned)hd), 0, (const float *)d->qkv, QKV, (int)nh, (int)kvh,
                     (int)hd, (const float *)L.qn, (const float *)L.kn, eps,
                     (const float *)d->cos, (const float *)d->sin, P, d->q, ck, cv, Lmax)))
      return rc;
    if ((rc = launch_attn_rows(ctx, d->q, nh * hd, 1, n, (int)nh, (int)kvh, (int)hd, ck, cv,
                               Lmax, P, scale, nullptr, 1, d->attn, nh * hd)))
      return rc;
    if ((rc = launch_matmul_nbits(ctx, L.o, d->attn, nh * hd, n, d->tmp))) return rc;
    // x += o; h = rmsnorm(x)
    if ((rc = norm_into(L.ln2, d->tmp, L.gu))) return rc;
    if ((rc = gemm_from_norm(L.gu, d->gu))) return rc;
    if (fuse) {
      int64_t segsp = 0, mpad = 0;
      void *ap = nullptr;
      int *ex = nullptr;
      if ((rc = gemm_prepared_a(ctx, L.down, n, &segsp, &mpad, &ap, &ex))) return rc;
      if ((rc = launch(ctx, kKernDecOps, k_swiglu_prep, dim3((unsigned)mpad), dim3(256), 0,
                       (const float *)d->gu, n, I, segsp, segsp * kSegK, ex, (uint4 *)ap)))
        return rc;
      if ((rc = launch_matmul_nbits_prepared(ctx, L.down, n, d->tmp))) return rc;
    } else {
      if ((rc = launch(ctx, kKernDecOps, k_swiglu_rows,
                       dim3((unsigned)((I + 255) / 256), (unsigned)n), dim3(256), 0,
                       (const float *)d->gu, I, d->act)))
        return rc;
      if ((rc = launch_matmul_nbits(ctx, L.down, d->act, I, n, d->tmp))) return rc;
    }
    // x += down, and (but after the last layer) the next layer's input norm
    if (li + 1 < c.layers) {
      const mmnb_decoder::Layer &Ln = d->layers[(size_t)li + 1];
      if ((rc = norm_into(Ln.ln1, d->tmp, Ln.qkv))) return rc;
    } else if ((rc = launch(ctx, kKernDecOps, k_rmsnorm, dim3((unsigned)n), dim3(256), 0,
                            (const float *)d->x, H, (const float *)d->final_norm, eps, d->h,
                            (const float *)d->tmp, d->x))) {
      return rc;
    }
  }
  // greedy token of the last row: final norm fused into lm_head
  if ((rc = launch_dec_gemv(ctx, d->lm, d->x + (n - 1) * H, d->final_norm, eps, kDecArgmax,
                            nullptr, d->logits, d->keys)))
    return rc;
  // state: token = argmax, pos = P + n (k_dec_end advances pos by one and
  // records the token; set pos so that it lands on P + n)
  DecState hs{};
  hs.pos = (int)(P + n - 1);
  hs.step = 0;
  MMNB_HIP(hipMemcpyAsync(d->state, &hs, 8 + 4 + 4, hipMemcpyHostToDevice, s));
  if ((rc = launch(ctx, kKernDecOps, k_dec_end, dim3(1), dim3(1024), 0, d->state,
                   (const unsigned long long *)d->keys, (int)d->nkeys, d->out_tokens,
                   (int)c.max_len)))
    return rc;
  int32_t tok = 0;
  MMNB_HIP(hipMemcpyAsync(&tok, &d->state->token, 4, hipMemcpyDeviceToHost, s));
  MMNB_HIP(hipMemsetAsync(&d->state->step, 0, 4, s));
  MMNB_HIP(hipStreamSynchronize(s));
  d->pos = P + n;
  d->steps_done = 0;
  d->primed = true;
  if (next_token) *next_token = tok;
  return MMNB_OK;
}

// The (max, sum) pairs of the attention partials, after the o parts.
static float *dec_part_ml(const mmnb_decoder *d) {
  const mmnb_decoder_config &c = d->cfg;
  return d->part + c.heads * ((c.max_len + d->ks - 1) / d->ks) * c.head_dim;
}

// Decode attention of one layer: grid (splits of the cache, KV heads);
// splits past the current position exit at once.
static int launch_dec_attn(mmnb_decoder *d, const mmnb_decoder::Layer &L, float *ck, float *cv) {
  mmnb_ctx *ctx = d->ctx;
  const mmnb_decoder_config &c = d->cfg;
  const dim3 grid((unsigned)((c.max_len + d->ks - 1) / d->ks), (unsigned)c.kv_heads);
  const float scale = (float)(1.0 / std::sqrt((double)c.head_dim));
  DecAttnArgs args{(const float *)d->qkv, (int)c.heads, (int)c.kv_heads, (const float *)L.qn,
                   (const float *)L.kn, c.eps, (const float *)d->rot, ck, cv, c.max_len, scale,
                   d->part, dec_part_ml(d), (int)grid.x, d->attn};
#define MMNB_DEC_ATTN_KS(HD, KS)                                                               \
  (d->attn_defer                                                                              \
       ? launch(ctx, kKernDecAttn, k_dec_attn<HD, false, KS>, grid,                           \
                dim3(dec_attn_threads<KS>()), 0, (const DecState *)d->state, args,            \
                d->counters)                                                                  \
       : launch(ctx, kKernDecAttn, k_dec_attn<HD, true, KS>, grid,                            \
                dim3(dec_attn_threads<KS>()), 0, (const DecState *)d->state, args,            \
                d->counters))
#define MMNB_DEC_ATTN(HD)                                                                      \
  MMNB_DEC_ATTN_KS(HD, kDecKS)
  switch (c.head_dim) {
    case 32: return MMNB_DEC_ATTN(32);
    case 64: return MMNB_DEC_ATTN(64);
    case 96: return MMNB_DEC_ATTN(96);
    case 128: return MMNB_DEC_ATTN(128);
    default: return fail(MMNB_ERR_UNSUPPORTED, "decoder: head_dim");
  }
#undef MMNB_DEC_ATTN
#undef MMNB_DEC_ATTN_KS
}

static int dec_record_step(mmnb_decoder *d) {
  mmnb_ctx *ctx = d->ctx;
  const mmnb_decoder_config &c = d->cfg;
  const int64_t H = c.hidden, kvh = c.kv_heads, hd = c.head_dim, Lmax = c.max_len;
  const float eps = c.eps;
  int rc;
  if ((rc = launch(ctx, kKernDecOps, k_dec_begin, dim3(1), dim3(256), 0, d->state,
                   (const float *)d->embed, H, c.vocab, d->x, (const float *)d->cos,
                   (const float *)d->sin, (int)(c.head_dim / 2), (int)Lmax, d->rot)))
    return rc;
  for (int64_t li = 0; li < c.layers; li++) {
    const mmnb_decoder::Layer &L = d->layers[(size_t)li];
    float *ck = d->cache_k + li * kvh * Lmax * hd, *cv = d->cache_v + li * kvh * Lmax * hd;
    if ((rc = launch_dec_gemv(ctx, L.qkv, d->x, L.ln1, eps, kDecPlain, nullptr, d->qkv, nullptr)))
      return rc;
    if ((rc = launch_dec_attn(d, L, ck, cv)))
      return rc;
    if (d->attn_defer) {
      const DecAttnPartials pa{d->part, dec_part_ml(d), (int)((Lmax + d->ks - 1) / d->ks),
                               (int)hd};
      if ((rc = launch_dec_gemv_attn(ctx, L.o, pa, d->x, d->x)))
        return rc;
    } else if ((rc = launch_dec_gemv(ctx, L.o, d->attn, nullptr, eps, kDecResidual, d->x, d->x,
                                     nullptr))) {
      return rc;
    }
    if ((rc = launch_dec_gemv(ctx, L.gu, d->x, L.ln2, eps, kDecSwiglu, nullptr, d->act, nullptr)))
      return rc;
    if ((rc = launch_dec_gemv(ctx, L.down, d->act, nullptr, eps, kDecResidual, d->x, d->x,
                              nullptr)))
      return rc;
  }
  if ((rc = launch_dec_gemv(ctx, d->lm, d->x, d->final_norm, eps, kDecArgmax, nullptr, d->logits,
                            d->keys)))
    return rc;
  return launch(ctx, kKernDecOps, k_dec_end, dim3(1), dim3(1024), 0, d->state,
                (const unsigned long long *)d->keys, (int)d->nkeys, d->out_tokens,
                (int)c.max_len);
}

// `steps` greedy decode steps (graph replays); tokens[i] is the token
// generated by step i.
int mmnb_decoder_decode(mmnb_decoder *d, int64_t steps, int32_t *tokens) {
  if (!d) return fail(MMNB_ERR_ARG, "decoder: null handle");
  mmnb_ctx *ctx = d->ctx;
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "decoder: decode during graph capture");
  if (steps < 0) return fail(MMNB_ERR_ARG, "decoder: negative step count");
  if (steps == 0) return MMNB_OK;
  if (!d->primed) return fail(MMNB_ERR_ARG, "decoder: prefill first");
  if (d->pos + steps > d->cfg.max_len)
    return fail(MMNB_ERR_ARG, "decoder: steps would exceed max_len");
  if (d->steps_done + steps > d->cfg.max_len)
    return fail(MMNB_ERR_ARG, "decoder: output list full");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  hipStream_t s = ctx->stream;
  const int64_t first = d->steps_done;
  // Kernel timing takes events from each dispatch, which a graph would
  // capture and replay: with timing on, the steps launch eagerly instead.
  if (!d->use_graph || ctx->timing) {
    for (int64_t i = 0; i < steps; i++)
      if ((rc = dec_record_step(d))) return rc;
    if (tokens)
      MMNB_HIP(hipMemcpyAsync(tokens, d->out_tokens + first, (size_t)steps * 4,
                              hipMemcpyDeviceToHost, s));
    MMNB_HIP(hipStreamSynchronize(s));
    d->pos += steps;
    d->steps_done += steps;
    return MMNB_OK;
  }
  if (!d->graph) {
    MMNB_HIP(hipStreamSynchronize(s));
    MMNB_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    rc = dec_record_step(d);
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return check_hip(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&d->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      d->graph = nullptr;
      return check_hip(e, "hipGraphInstantiate");
    }
  }
  for (int64_t i = 0; i < steps; i++) MMNB_HIP(hipGraphLaunch(d->graph, s));
  if (tokens)
    MMNB_HIP(hipMemcpyAsync(tokens, d->out_tokens + first, (size_t)steps * 4,
                            hipMemcpyDeviceToHost, s));
  MMNB_HIP(hipStreamSynchronize(s));
  d->pos += steps;
  d->steps_done += steps;
  return MMNB_OK;
}

int mmnb_decoder_logits(mmnb_decoder *d, float *logits) {
  if (!d || !logits) return fail(MMNB_ERR_ARG, "decoder: null argument");
  CtxLock lk(d->ctx);
  int rc = set_device(d->ctx);
  if (rc) return rc;
  MMNB_HIP(hipMemcpyAsync(logits, d->logits, (size_t)d->cfg.vocab * 4, hipMemcpyDeviceToHost,
                          d->ctx->stream));
  MMNB_HIP(hipStreamSynchronize(d->ctx->stream));
  return MMNB_OK;
}

int mmnb_decoder_position(mmnb_decoder *d, int64_t *pos) {
  if (!d || !pos) return fail(MMNB_ERR_ARG, "decoder: null argument");
  *pos = d->pos;
  return MMNB_OK;
}

int mmnb_decoder_set_graph(mmnb_decoder *d, int use_graph) {
  if (!d) return fail(MMNB_ERR_ARG, "decoder: null handle");
  d->use_graph = use_graph != 0;
  return MMNB_OK;
}
