// MatMulNBits on gfx950: weight repack, decode-shape GEMV, activation prep
// and the MFMA prefill GEMM.
//
// Reference semantics (onnx_qlinear_ops.dart:114-156): W[k, n] =
// fl32((q[n, k] - zp[n, blk]) * scale[n, blk]), y = A * W.  The kernels
// factor the scale out of each block: y = sum_blk scale * sum_{k in blk}
// a[k] * (q - zp), which differs from the reference only in rounding.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mmnb_internal.h"

namespace mmnb {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

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
// Decode-shape GEMV on the vector ALUs (fp32 FMA), M <= 8.
//
// The K extent of a column is cut into 16-byte chunks (32 nibbles); chunk c
// = (segment s = c/2, half g = c%2) holds k = 64s + 16j + 8g + e for
// j = 0..3, e = 0..7 (dword j, nibble e).  LPC lanes share one column and
// walk its chunks with stride LPC; a wave serves G = 64/LPC columns at a time
// and U such groups, so every lane keeps U independent 16-byte weight loads
// in flight.  Per dword the lane forms sum_e a*q, then folds the block's
// zero point through sum_e a and its scale:
//     acc += scale * (sum a*q) - (scale*zp) * (sum a).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_seg_sum(float v, int lpc) {
  for (int off = 1; off < lpc; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int M, int U>
__global__ __launch_bounds__(256) void k_gemv_valu(
    const float *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W,
    int64_t col_bytes, const float *__restrict__ S, const uint8_t *__restrict__ Z,
    int nb, int bs_log2, int K, int N, float *__restrict__ Y, int chunks,
    int lpc_log2, int fast) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lpc = 1 << lpc_log2;
  const int G = 64 >> lpc_log2;
  const int gi = lane >> lpc_log2;
  const int t = lane & (lpc - 1);
  const int col0 = wave * (U * G);

  float acc[M][U];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int u = 0; u < U; u++) acc[m][u] = 0.0f;

  for (int c = t; c < chunks; c += lpc) {
    const int s = c >> 1, g = c & 1;
    const int kb = s * kSegK + g * 8;
    // weights, scales, zero points for the U columns
    uint4 wv[U];
    float sc[U][4], sz[U][4];
#pragma unroll
    for (int u = 0; u < U; u++) {
      int col = col0 + u * G + gi;
      const bool ok = col < N;
      col = ok ? col : N - 1;
      wv[u] = *(const uint4 *)(W + (int64_t)col * col_bytes + (int64_t)c * 16);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int blk = (kb + 16 * j) >> bs_log2;
        const bool inb = blk < nb;
        blk = inb ? blk : nb - 1;
        const int zi = col * nb + blk;
        float s_ = S[zi];
        int zpv = 8;
        if (Z) {
          const uint8_t zb = Z[zi >> 1];
          zpv = (zi & 1) ? (zb >> 4) : (zb & 0xF);
        }
        s_ = (inb && ok) ? s_ : 0.0f;
        sc[u][j] = s_;
        sz[u][j] = s_ * (float)zpv;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int k0 = kb + 16 * j;
      float av[M][8];
      float sa[M];
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float *ar = A + (int64_t)m * lda + k0;
        if (fast) {
          const float4 x0 = *(const float4 *)(ar);
          const float4 x1 = *(const float4 *)(ar + 4);
          av[m][0] = x0.x; av[m][1] = x0.y; av[m][2] = x0.z; av[m][3] = x0.w;
          av[m][4] = x1.x; av[m][5] = x1.y; av[m][6] = x1.z; av[m][7] = x1.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) av[m][e] = (k0 + e < K) ? ar[e] : 0.0f;
        }
        float s_ = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) s_ += av[m][e];
        sa[m] = s_;
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t w = j == 0 ? wv[u].x : j == 1 ? wv[u].y : j == 2 ? wv[u].z : wv[u].w;
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        float q[8];
        q[0] = (float)(lo & 0xFF);
        q[1] = (float)(hi & 0xFF);
        q[2] = (float)((lo >> 8) & 0xFF);
        q[3] = (float)((hi >> 8) & 0xFF);
        q[4] = (float)((lo >> 16) & 0xFF);
        q[5] = (float)((hi >> 16) & 0xFF);
        q[6] = (float)(lo >> 24);
        q[7] = (float)(hi >> 24);
#pragma unroll
        for (int m = 0; m < M; m++) {
          float d = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; e++) d = fmaf(av[m][e], q[e], d);
          acc[m][u] = fmaf(sc[u][j], d, acc[m][u]);
          acc[m][u] = fmaf(-sz[u][j], sa[m], acc[m][u]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int u = 0; u < U; u++) {
      const float v = wave_seg_sum(acc[m][u], lpc);
      const int col = col0 + u * G + gi;
      if (t == 0 && col < N) Y[(int64_t)m * N + col] = v;
    }
}

template <int M>
static int launch_gemv_m(mmnb_ctx *ctx, int u, dim3 grid, const float *A, int64_t lda,
                         const mmnb_pack *p, float *Y, int chunks, int lpc_log2, int fast,
                         int bs_log2) {
  const int nb = (int)p->n_blocks, K = (int)p->k, N = (int)p->n;
  if (u == 4)
    return launch(ctx, kKernGemv, k_gemv_valu<M, 4>, grid, dim3(256), 0, A, lda, p->d_w,
                  p->col_bytes, p->d_scales, p->d_zp, nb, bs_log2, K, N, Y, chunks, lpc_log2,
                  fast);
  if (u == 2)
    return launch(ctx, kKernGemv, k_gemv_valu<M, 2>, grid, dim3(256), 0, A, lda, p->d_w,
                  p->col_bytes, p->d_scales, p->d_zp, nb, bs_log2, K, N, Y, chunks, lpc_log2,
                  fast);
  return launch(ctx, kKernGemv, k_gemv_valu<M, 1>, grid, dim3(256), 0, A, lda, p->d_w,
                p->col_bytes, p->d_scales, p->d_zp, nb, bs_log2, K, N, Y, chunks, lpc_log2,
                fast);
}

static int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << (r + 1)) <= v) r++;
  return r;
}

static int launch_gemv(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                       int64_t m, float *d_y) {
  const int chunks = (int)(p->col_bytes / 16);
  int lpc = 1;
  while (lpc < chunks && lpc < 64) lpc <<= 1;
  const int G = 64 / lpc;
  const int64_t n = p->n;
  // columns per wave: keep >= ~4 waves per CU where N allows
  const int64_t want_waves = (int64_t)ctx->cu_count * 4;
  int u = 4;
  while (u > 1 && (n + (int64_t)u * G - 1) / ((int64_t)u * G) < want_waves) u >>= 1;
  const int64_t waves = (n + (int64_t)u * G - 1) / ((int64_t)u * G);
  const dim3 grid((unsigned)((waves + 3) / 4));
  // Aligned float4 path: every 8-float run of a chunk lies inside the row,
  // i.e. rows hold k64 values (zero padded past K by the host entry point, or
  // K itself is a multiple of 64).
  const int f = ((lda % 4 == 0) && (((uintptr_t)d_a & 15) == 0) && (lda >= p->k64)) ? 1 : 0;
  const int bs_log2 = ilog2(p->block);
  const int lpc_log2 = ilog2(lpc);
  switch (m) {
    case 1: return launch_gemv_m<1>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 2: return launch_gemv_m<2>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 3: return launch_gemv_m<3>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 4: return launch_gemv_m<4>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 5: return launch_gemv_m<5>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 6: return launch_gemv_m<6>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    case 7: return launch_gemv_m<7>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
    default: return launch_gemv_m<8>(ctx, u, grid, d_a, lda, p, d_y, chunks, lpc_log2, f, bs_log2);
  }
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
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prep_rowblock(
    const float *__restrict__ A, int64_t lda, int64_t M, int64_t K, int64_t segs,
    uint4 *__restrict__ out, int *__restrict__ row_exp) {
  __shared__ int s_exp[32];
  const int rb = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Phase 1: per-row max|a| -> exponent.  4 waves x 8 rows.
  for (int r = wave; r < 32; r += 4) {
    const int64_t row = (int64_t)rb * 32 + r;
    float mx = 0.0f;
    if (row < M) {
      const float *ar = A + row * lda;
      for (int64_t k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(ar[k]));
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) {
      int e = 0;
      if (mx > 0.0f && mx < INFINITY) e = 13 - ilogbf(mx);
      s_exp[r] = e;
      if (row < M) row_exp[row] = e;
    }
  }
  __syncthreads();
  // Phase 2: units (s, j, lane l) -> hi and lo 16-byte pieces.
  const int64_t units = segs * 4 * 64;
  for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
    const int l = (int)(u & 63);
    const int j = (int)((u >> 6) & 3);
    const int64_t s = u >> 8;
    const int r = l & 31, g = l >> 5;
    const int64_t row = (int64_t)rb * 32 + r;
    const int64_t k0 = s * kSegK + 16 * j + 8 * g;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int64_t kk = k0 + e;
      v[e] = (row < M && kk < K) ? A[row * lda + kk] : 0.0f;
    }
    const int ex = s_exp[r];
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = ldexpf(v[e], ex);
      const _Float16 h = (_Float16)x;
      hi[e] = h;
      lo[e] = (_Float16)(x - (float)h);
    }
    // permute to the dequantised-weight order {0,4,1,5,2,6,3,7}
    half8_t H = {hi[0], hi[4], hi[1], hi[5], hi[2], hi[6], hi[3], hi[7]};
    half8_t L = {lo[0], lo[4], lo[1], lo[5], lo[2], lo[6], lo[3], lo[7]};
    const int64_t base = (((int64_t)rb * segs + s) * 4 + j) * 2;
    out[(base + 0) * 64 + l] = __builtin_bit_cast(uint4, H);
    out[(base + 1) * 64 + l] = __builtin_bit_cast(uint4, L);
  }
}

// ---------------------------------------------------------------------------
// Prefill GEMM: WG tile 64 (M) x 128 (N), 4 waves in 2 x 2, wave tile
// 32 x 64 = one 32-row A block x two 32-column B blocks.  For every 16-k step
// the wave issues 2 (B blocks) x 2 (hi, lo) MFMAs into per-block partials D;
// at each quantisation-block boundary acc += scale[n, blk] * D.  The 16-byte
// weight load of a lane covers four 16-k steps (one 64-k segment).
// ---------------------------------------------------------------------------
__device__ __forceinline__ half8_t dequant8(uint32_t w, int zp) {
  const uint32_t t0 = (w & 0x000F000Fu) | 0x64006400u;
  const uint32_t t1 = (w & 0x00F000F0u) | 0x64006400u;
  const uint32_t w8 = w >> 8;
  const uint32_t t2 = (w8 & 0x000F000Fu) | 0x64006400u;
  const uint32_t t3 = (w8 & 0x00F000F0u) | 0x64006400u;
  const _Float16 z1024 = (_Float16)(1024 + zp);
  const _Float16 z64 = (_Float16)(64 + zp);
  const half2_t zz = {z1024, z1024};
  const half2_t zs = {z64, z64};
  const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2_t h0 = __builtin_bit_cast(half2_t, t0) - zz;
  const half2_t h1 = __builtin_bit_cast(half2_t, t1) * sixteenth - zs;
  const half2_t h2 = __builtin_bit_cast(half2_t, t2) - zz;
  const half2_t h3 = __builtin_bit_cast(half2_t, t3) * sixteenth - zs;
  half8_t r = {h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
  return r;
}

__device__ __forceinline__ int zp_of(const uint8_t *__restrict__ Z, int64_t zi) {
  if (!Z) return 8;
  const uint8_t zb = Z[zi >> 1];
  return (zi & 1) ? (zb >> 4) : (zb & 0xF);
}

constexpr int kGemmBM = 64;
constexpr int kGemmBN = 128;

__global__ __launch_bounds__(256) void k_gemm_mfma(
    const uint4 *__restrict__ Ap, const int *__restrict__ row_exp, int64_t segs,
    const uint8_t *__restrict__ W, int64_t col_bytes, const float *__restrict__ S,
    const uint8_t *__restrict__ Z, int64_t nb, int64_t bs, int64_t M, int64_t N,
    float *__restrict__ Y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t rb = (int64_t)blockIdx.y * (kGemmBM / 32) + wm;  // 32-row block
  const int64_t n0 = (int64_t)blockIdx.x * kGemmBN + wn * 64;
  const int cl = lane & 31, g = lane >> 5;

  int64_t col[2];
  bool colok[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    col[t] = n0 + t * 32 + cl;
    colok[t] = col[t] < N;
    if (!colok[t]) col[t] = N - 1;
  }
  float16_t acc[2], D[2];
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      acc[t][r] = 0.0f;
      D[t][r] = 0.0f;
    }
  int zpv[2] = {8, 8};
  float scl[2] = {0.0f, 0.0f};
  int64_t cur_blk = -1;

  for (int64_t s = 0; s < segs; s++) {
    uint4 wv[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
      wv[t] = *(const uint4 *)(W + col[t] * col_bytes + s * kSegBytes + g * 16);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int64_t kstep = s * kSegK + 16 * j;
      const int64_t blk = kstep / bs;
      if (blk != cur_blk) {
        cur_blk = blk;
        const bool inb = blk < nb;
        const int64_t b2 = inb ? blk : nb - 1;
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const int64_t zi = col[t] * nb + b2;
          zpv[t] = zp_of(Z, zi);
          scl[t] = inb ? S[zi] : 0.0f;
        }
      }
      const int64_t ubase = ((rb * segs + s) * 4 + j) * 2;
      const half8_t ah = __builtin_bit_cast(half8_t, Ap[(ubase + 0) * 64 + lane]);
      const half8_t al = __builtin_bit_cast(half8_t, Ap[(ubase + 1) * 64 + lane]);
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const uint32_t w = j == 0 ? wv[t].x : j == 1 ? wv[t].y : j == 2 ? wv[t].z : wv[t].w;
        const half8_t b = dequant8(w, zpv[t]);
        D[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b, D[t], 0, 0, 0);
        D[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b, D[t], 0, 0, 0);
      }
      // block boundary after this 16-k step?
      if (((kstep + 16) % bs) == 0) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            acc[t][r] = fmaf(scl[t], D[t][r], acc[t][r]);
            D[t][r] = 0.0f;
          }
      }
    }
  }
  // 32x32 f32 accumulator layout: lane l holds column l%32, rows
  // (r/4)*8 + (l/32)*4 + r%4 for r = 0..15.
#pragma unroll
  for (int t = 0; t < 2; t++) {
    if (!colok[t]) continue;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int64_t row = rb * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
      if (row < M) Y[row * N + col[t]] = ldexpf(acc[t][r], -row_exp[row]);
    }
  }
}

static int launch_gemm(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                       int64_t m, float *d_y) {
  const int64_t segs = p->k64 / kSegK;
  const int64_t mpad = (m + kGemmBM - 1) / kGemmBM * kGemmBM;
  const int64_t rblocks = mpad / 32;
  const size_t ap_bytes = (size_t)(rblocks * segs * 4 * 2 * 64) * 16;
  void *d_ap = nullptr, *d_exp = nullptr;
  int rc;
  if ((rc = scratch_get(ctx, 2, ap_bytes, &d_ap))) return rc;
  if ((rc = scratch_get(ctx, 3, (size_t)mpad * 4, &d_exp))) return rc;
  if ((rc = launch(ctx, kKernPrep, k_prep_rowblock, dim3((unsigned)rblocks), dim3(256), 0, d_a,
                    lda, m, p->k, segs, (uint4 *)d_ap, (int *)d_exp)))
    return rc;
  const dim3 grid((unsigned)((p->n + kGemmBN - 1) / kGemmBN), (unsigned)(mpad / kGemmBM));
  return launch(ctx, kKernGemm, k_gemm_mfma, grid, dim3(256), 0, (const uint4 *)d_ap,
                (const int *)d_exp, segs, p->d_w, p->col_bytes, p->d_scales, p->d_zp,
                p->n_blocks, p->block, m, p->n, d_y);
}

int launch_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                        int64_t m, float *d_y) {
  if (m <= 8) return launch_gemv(ctx, p, d_a, lda, m, d_y);
  return launch_gemm(ctx, p, d_a, lda, m, d_y);
}

}  // namespace mmnb
