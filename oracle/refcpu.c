/*
 * refcpu.c -- CPU oracle for the int4 MatMulNBits and int8
 * DynamicQuantizeLinear -> MatMulInteger path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker: it restates,
 * in plain C, the arithmetic of the reference Dart implementation so that
 * the GPU kernels can be compared against it.  Only tests/, the smoke()
 * entry and bench.py's cpu_baseline leg may load it.  The product library
 * (libmmnb.so) never links or calls it.
 *
 * Build:  gcc -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).
 * -ffp-contract=off is load-bearing: the reference forms every product and
 * every sum as separately rounded IEEE binary32 operations (Dart Float32x4
 * multiply, then Float32x4 add), so no fused multiply-add may appear.
 *
 * Each function cites the reference file:line it restates
 * (paths relative to the onnx_runtime_dart source tree).
 *
 * Parity pinning (what fixes each function, besides this restatement):
 *   ref_mmnb_dequant / ref_matmul_kernel / ref_matmul_nbits:
 *       the reference's ORT fixtures matmulnbits_{basic,zeropoints,
 *       partial_block}; an fp64 brute force (ref_matmul_nbits_f64) with the
 *       gamma_K accumulation bound; closed-form special cases (all-zero
 *       nibbles, unit scales -> integer matrix); the reference GEMM
 *       known-answer shapes (gemm_kernel_test.dart:45-78) vs fp64.
 *   ref_dql: the reference fixture dynamicquantizelinear (ints exact);
 *       closed-form IEEE properties (round-half-even ties, clamp, scale==0).
 *       The Dart-specific double-precision *scale* sequence
 *       (onnx_ops.dart:2566-2568) is not distinguished from float32 by any
 *       reference fixture: that one step is "parity unpinned" beyond this
 *       restatement and IEEE-754 semantics.
 *   ref_matmul_integer: the reference fixtures matmulinteger_{u8i8,nozp,
 *       batched,percol_bzp}, the hand case [1200, 600]
 *       (compact_tensor_test.dart:48-58), and exact int64 brute force.
 *   ref_rescale: closed form (two correctly rounded binary32 operations).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define REF_OK 0
#define REF_ERR_ARG (-1)
#define REF_ERR_UNSUPPORTED (-2)
#define REF_ERR_OOM (-4)

/* ------------------------------------------------------------------------ */
/* MatMulNBits dequantization: onnx_qlinear_ops.dart:120-149.               */
/* Writes W^T as a row-major [k x n] float buffer: bt[kk*n + col] =         */
/* fl32((q - zp) * scale).  (q - zp) is a small integer and scale a binary32 */
/* value, so the double product is exact and the store rounds once: that is */
/* exactly the binary32 product of (float)(q - zp) and scale.               */
/* Zero points are read flat: nibble index col*nBlocks+blk (:133-137), low   */
/* nibble first; absent zero points mean 8 (:132).  The partial last block  */
/* is clipped at k (:141).                                                   */
/* ------------------------------------------------------------------------ */
void ref_mmnb_dequant(const uint8_t *b, const float *scales, const uint8_t *zp,
                      int64_t k, int64_t n, int64_t block, float *bt) {
  const int64_t nblocks = (k + block - 1) / block;
  const int64_t blob = block / 2;
  for (int64_t col = 0; col < n; col++) {
    const int64_t col_base = col * nblocks * blob;
    for (int64_t blk = 0; blk < nblocks; blk++) {
      const float scale = scales[col * nblocks + blk];
      int zpv = 8;
      if (zp) {
        const int64_t zi = col * nblocks + blk;
        const uint8_t byte = zp[zi >> 1];
        zpv = (zi & 1) == 0 ? (byte & 0xF) : (byte >> 4);
      }
      const int64_t blob_base = col_base + blk * blob;
      const int64_t k_base = blk * block;
      const int64_t k_end = k_base + block < k ? k_base + block : k;
      for (int64_t kk = k_base; kk < k_end; kk++) {
        const int64_t j = kk - k_base;
        const uint8_t byte = b[blob_base + (j >> 1)];
        const int q = (j & 1) == 0 ? (byte & 0xF) : (byte >> 4);
        bt[kk * n + col] = (float)(q - zpv) * scale;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* fp32 GEMM of gemm_kernel_simd.dart:27-169 (m > 1) and _gemv :183-309     */
/* (m == 1).  For every output the reference accumulates strictly in k     */
/* order, acc = fl32(acc + fl32(a*b)), starting from +0 (Float32x4.zero, */
/* :84-87); column panels (:41-45) and 4x8 register tiles do not change that */
/* order (:13-15).  One exception: the m == 1 path with n % 4 != 0 takes   */
/* _gemvScalar (:185-190, :251-309), whose last n % 4 columns accumulate in */
/* double (:300-308) and are rounded to binary32 once at the store.          */
/* The column-panel / row-tile loop nest is kept so the CPU timing reflects */
/* the reference's memory access pattern.                                    */
/* ------------------------------------------------------------------------ */
#define PANEL_BYTES (192 * 1024)

static void gemv_f32_cols(const float *a, const float *b, float *out,
                          int64_t k, int64_t n, int64_t j0, int64_t j1) {
  /* 16-column register tiles, k-outer (gemm_kernel_simd.dart:196-246). */
  int64_t j = j0;
  for (; j + 16 <= j1; j += 16) {
    float c[16];
    for (int t = 0; t < 16; t++) c[t] = 0.0f;
    const float *br = b + j;
    for (int64_t kk = 0; kk < k; kk++) {
      const float va = a[kk];
      for (int t = 0; t < 16; t++) {
        const float p = va * br[t];
        c[t] = c[t] + p;
      }
      br += n;
    }
    for (int t = 0; t < 16; t++) out[j + t] = c[t];
  }
  for (; j + 4 <= j1; j += 4) {
    float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *br = b + j;
    for (int64_t kk = 0; kk < k; kk++) {
      const float va = a[kk];
      for (int t = 0; t < 4; t++) {
        const float p = va * br[t];
        c[t] = c[t] + p;
      }
      br += n;
    }
    for (int t = 0; t < 4; t++) out[j + t] = c[t];
  }
  /* Scalar tail in double (gemm_kernel_simd.dart:300-308). */
  for (; j < j1; j++) {
    double acc = 0.0;
    const float *br = b + j;
    for (int64_t kk = 0; kk < k; kk++) {
      acc += (double)a[kk] * (double)br[0];
      br += n;
    }
    out[j] = (float)acc;
  }
}

/* Rows [i0, i1) x all columns, panel/tile nest of :46-168. */
static void gemm_f32_rows(const float *a, const float *b, float *out,
                          int64_t m_lo, int64_t m_hi, int64_t k, int64_t n,
                          float *bp) {
  int64_t panel = PANEL_BYTES / (k * 4);
  panel = (panel >> 2) << 2;
  if (panel < 4) panel = 4;
  if (panel > n) panel = n;
  const int64_t panel_n4 = (panel + 3) >> 2;
  (void)panel_n4;
  for (int64_t p0 = 0; p0 < n; p0 += panel) {
    const int64_t pw = p0 + panel <= n ? panel : n - p0;
    const int64_t pn = ((pw + 3) >> 2) << 2; /* packed row stride */
    /* Pack this column panel of B, zero-filled tail lanes (:63-74). */
    for (int64_t kk = 0; kk < k; kk++) {
      const float *src = b + kk * n + p0;
      float *dst = bp + kk * pn;
      int64_t j = 0;
      for (; j < pw; j++) dst[j] = src[j];
      for (; j < pn; j++) dst[j] = 0.0f;
    }
    int64_t i = m_lo;
    for (; i + 4 <= m_hi; i += 4) {
      int64_t j = 0;
      for (; j + 8 <= pw; j += 8) {
        float c[4][8];
        for (int r = 0; r < 4; r++)
          for (int t = 0; t < 8; t++) c[r][t] = 0.0f;
        for (int64_t kk = 0; kk < k; kk++) {
          const float *bv = bp + kk * pn + j;
          for (int r = 0; r < 4; r++) {
            const float v = a[(i + r) * k + kk];
            for (int t = 0; t < 8; t++) {
              const float p = v * bv[t];
              c[r][t] = c[r][t] + p;
            }
          }
        }
        for (int r = 0; r < 4; r++)
          for (int t = 0; t < 8; t++) out[(i + r) * n + p0 + j + t] = c[r][t];
      }
      for (; j < pn; j += 4) {
        float c[4][4];
        for (int r = 0; r < 4; r++)
          for (int t = 0; t < 4; t++) c[r][t] = 0.0f;
        for (int64_t kk = 0; kk < k; kk++) {
          const float *bv = bp + kk * pn + j;
          for (int r = 0; r < 4; r++) {
            const float v = a[(i + r) * k + kk];
            for (int t = 0; t < 4; t++) {
              const float p = v * bv[t];
              c[r][t] = c[r][t] + p;
            }
          }
        }
        const int64_t cols = pw - j < 4 ? pw - j : 4;
        for (int r = 0; r < 4; r++)
          for (int64_t t = 0; t < cols; t++) out[(i + r) * n + p0 + j + t] = c[r][t];
      }
    }
    for (; i < m_hi; i++) {
      int64_t j = 0;
      for (; j + 8 <= pw; j += 8) {
        float c[8];
        for (int t = 0; t < 8; t++) c[t] = 0.0f;
        for (int64_t kk = 0; kk < k; kk++) {
          const float v = a[i * k + kk];
          const float *bv = bp + kk * pn + j;
          for (int t = 0; t < 8; t++) {
            const float p = v * bv[t];
            c[t] = c[t] + p;
          }
        }
        for (int t = 0; t < 8; t++) out[i * n + p0 + j + t] = c[t];
      }
      for (; j < pn; j += 4) {
        float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t kk = 0; kk < k; kk++) {
          const float v = a[i * k + kk];
          const float *bv = bp + kk * pn + j;
          for (int t = 0; t < 4; t++) {
            const float p = v * bv[t];
            c[t] = c[t] + p;
          }
        }
        const int64_t cols = pw - j < 4 ? pw - j : 4;
        for (int64_t t = 0; t < cols; t++) out[i * n + p0 + j + t] = c[t];
      }
    }
  }
}

int ref_matmul_kernel(const float *a, const float *b, float *out, int64_t m,
                      int64_t k, int64_t n) {
  if (m < 0 || k < 0 || n < 0) return REF_ERR_ARG;
  if (m == 0 || n == 0) return REF_OK;
  if (m == 1) {
    /* _gemv: aligned path when n % 4 == 0 (:185-187), else scalar path. */
    gemv_f32_cols(a, b, out, k, n, 0, n);
    return REF_OK;
  }
  int64_t panel = PANEL_BYTES / ((k > 0 ? k : 1) * 4);
  panel = (panel >> 2) << 2;
  if (panel < 4) panel = 4;
  if (panel > n) panel = n;
  const int64_t pn = ((panel + 3) >> 2) << 2;
  float *bp = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1) * (size_t)pn);
  if (!bp) return REF_ERR_OOM;
  gemm_f32_rows(a, b, out, 0, m, k, n, bp);
  free(bp);
  return REF_OK;
}

/* ------------------------------------------------------------------------ */
/* opMatMulNBits: onnx_qlinear_ops.dart:114-156.  bits != 4 is rejected     */
/* (:117-119); m = len(A) / K (:152).  Dequantize the whole weight to a     */
/* fresh K x N binary32 buffer, then run the fp32 GEMM (:151-155).          */
/* ------------------------------------------------------------------------ */
int ref_matmul_nbits(const float *a, int64_t m, const uint8_t *b,
                     const float *scales, const uint8_t *zp, int64_t k,
                     int64_t n, int64_t bits, int64_t block, float *out) {
  if (bits != 4) return REF_ERR_UNSUPPORTED;
  if (m < 0 || k <= 0 || n < 0 || block < 2 || (block & 1)) return REF_ERR_ARG;
  float *bt = (float *)calloc((size_t)k * (size_t)(n > 0 ? n : 1), sizeof(float));
  if (!bt) return REF_ERR_OOM;
  ref_mmnb_dequant(b, scales, zp, k, n, block, bt);
  memset(out, 0, sizeof(float) * (size_t)m * (size_t)n);
  int rc = ref_matmul_kernel(a, bt, out, m, k, n);
  free(bt);
  return rc;
}

/* fp64 companion for error analysis: y64[i,j] = sum_k a*W in double (long  */
/* double accumulation), with W the same binary32 dequantized weights the   */
/* reference uses, and absdot[i,j] = sum_k |a|*|W| (for the gamma_K bound). */
int ref_matmul_nbits_f64(const float *a, int64_t m, const uint8_t *b,
                         const float *scales, const uint8_t *zp, int64_t k,
                         int64_t n, int64_t block, double *y64,
                         double *absdot) {
  if (m < 0 || k <= 0 || n < 0 || block < 2 || (block & 1)) return REF_ERR_ARG;
  float *bt = (float *)calloc((size_t)k * (size_t)(n > 0 ? n : 1), sizeof(float));
  if (!bt) return REF_ERR_OOM;
  ref_mmnb_dequant(b, scales, zp, k, n, block, bt);
  for (int64_t i = 0; i < m; i++) {
    for (int64_t j = 0; j < n; j++) {
      long double s = 0.0L, sa = 0.0L;
      for (int64_t kk = 0; kk < k; kk++) {
        const long double p = (long double)a[i * k + kk] * (long double)bt[kk * n + j];
        s += p;
        sa += p < 0 ? -p : p;
      }
      y64[i * n + j] = (double)s;
      if (absdot) absdot[i * n + j] = (double)sa;
    }
  }
  free(bt);
  return REF_OK;
}

/* Column-sliced multi-threaded variant for the CPU baseline: each thread   */
/* owns a contiguous slice of output columns, the partition of the          */
/* reference's isolate pool (parallel_pool.dart:122-146, stitched :188-194). */
/* Columns are independent and each keeps its k order, so the output is     */
/* bitwise identical to ref_matmul_nbits (the pool's own invariant,         */
/* parallel_pool_test.dart:27-100).  The m==1 double tail is tied to the    */
/* global column count, so slices are cut on multiples of 16.               */
typedef struct {
  const float *a;
  const float *bt;
  float *out;
  int64_t m, k, n, j0, j1;
  const uint8_t *b;
  const float *scales;
  const uint8_t *zp;
  int64_t block;
  int phase;
} mt_job;

static void dequant_cols(const mt_job *jb) {
  const int64_t k = jb->k, n = jb->n, block = jb->block;
  const int64_t nblocks = (k + block - 1) / block, blob = block / 2;
  float *bt = (float *)jb->bt;
  for (int64_t col = jb->j0; col < jb->j1; col++) {
    for (int64_t blk = 0; blk < nblocks; blk++) {
      const float scale = jb->scales[col * nblocks + blk];
      int zpv = 8;
      if (jb->zp) {
        const int64_t zi = col * nblocks + blk;
        const uint8_t byte = jb->zp[zi >> 1];
        zpv = (zi & 1) == 0 ? (byte & 0xF) : (byte >> 4);
      }
      const int64_t bb = col * nblocks * blob + blk * blob;
      const int64_t kb = blk * block;
      const int64_t ke = kb + block < k ? kb + block : k;
      for (int64_t kk = kb; kk < ke; kk++) {
        const int64_t j = kk - kb;
        const uint8_t byte = jb->b[bb + (j >> 1)];
        const int q = (j & 1) == 0 ? (byte & 0xF) : (byte >> 4);
        bt[kk * n + col] = (float)(q - zpv) * scale;
      }
    }
  }
}

static void *mt_worker(void *p) {
  mt_job *jb = (mt_job *)p;
  dequant_cols(jb);
  if (jb->j1 <= jb->j0) return NULL;
  if (jb->m == 1) {
    /* Columns below n - n%4 are binary32; the tail is double, as in the   */
    /* single-threaded _gemvScalar.  Slices never split a 4-column group.  */
    const int64_t nf = jb->n - (jb->n % 4);
    int64_t hi = jb->j1 < nf ? jb->j1 : nf;
    if (hi > jb->j0) gemv_f32_cols(jb->a, jb->bt, jb->out, jb->k, jb->n, jb->j0, hi);
    for (int64_t j = (jb->j0 > nf ? jb->j0 : nf); j < jb->j1; j++) {
      double acc = 0.0;
      for (int64_t kk = 0; kk < jb->k; kk++)
        acc += (double)jb->a[kk] * (double)jb->bt[kk * jb->n + j];
      jb->out[j] = (float)acc;
    }
    return NULL;
  }
  /* m > 1: sequential-k binary32 per output, like the 4x8 tiles. */
  for (int64_t i = 0; i < jb->m; i++) {
    for (int64_t j0 = jb->j0; j0 < jb->j1; j0 += 8) {
      const int64_t w = jb->j1 - j0 < 8 ? jb->j1 - j0 : 8;
      float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int64_t kk = 0; kk < jb->k; kk++) {
        const float v = jb->a[i * jb->k + kk];
        const float *bv = jb->bt + kk * jb->n + j0;
        for (int64_t t = 0; t < w; t++) {
          const float p = v * bv[t];
          c[t] = c[t] + p;
        }
      }
      for (int64_t t = 0; t < w; t++) jb->out[i * jb->n + j0 + t] = c[t];
    }
  }
  return NULL;
}

int ref_matmul_nbits_mt(const float *a, int64_t m, const uint8_t *b,
                        const float *scales, const uint8_t *zp, int64_t k,
                        int64_t n, int64_t bits, int64_t block, float *out,
                        int nthreads) {
  if (bits != 4) return REF_ERR_UNSUPPORTED;
  if (m < 0 || k <= 0 || n < 0 || block < 2 || (block & 1) || nthreads < 1)
    return REF_ERR_ARG;
  if (nthreads > 256) nthreads = 256;
  float *bt = (float *)calloc((size_t)k * (size_t)(n > 0 ? n : 1), sizeof(float));
  if (!bt) return REF_ERR_OOM;
  pthread_t th[256];
  mt_job jobs[256];
  int64_t per = (n + nthreads - 1) / nthreads;
  per = ((per + 15) / 16) * 16;
  int used = 0;
  for (int t = 0; t < nthreads; t++) {
    int64_t j0 = (int64_t)t * per, j1 = j0 + per;
    if (j0 > n) j0 = n;
    if (j1 > n) j1 = n;
    jobs[t] = (mt_job){a, bt, out, m, k, n, j0, j1, b, scales, zp, block, 0};
    if (j1 > j0) {
      pthread_create(&th[t], NULL, mt_worker, &jobs[t]);
      used = t + 1;
    }
  }
  for (int t = 0; t < used; t++)
    if (jobs[t].j1 > jobs[t].j0) pthread_join(th[t], NULL);
  free(bt);
  return REF_OK;
}

/* ------------------------------------------------------------------------ */
/* _roundEven: onnx_ops.dart:2490-2497 (duplicated in                       */
/* onnx_qlinear_ops.dart:17-24).  Floor, then compare the fraction with 0.5;*/
/* ties go to the even integer.  Non-finite input makes Dart's toInt throw, */
/* so callers keep it out of contract.                                      */
/* ------------------------------------------------------------------------ */
static int64_t round_even(double v) {
  const double f = floor(v);
  const double frac = v - f;
  if (frac > 0.5) return (int64_t)f + 1;
  if (frac < 0.5) return (int64_t)f;
  const int64_t i = (int64_t)f;
  return (i % 2 == 0) ? i : i + 1;
}

/* ------------------------------------------------------------------------ */
/* opDynamicQuantizeLinear: onnx_ops.dart:2556-2583.                         */
/*   mn = min(0, x), mx = max(0, x) in double; NaN never passes < or >.    */
/*   scale = fl32((mx - mn) / 255.0)  -- the subtraction and the division  */
/*           are double operations, then one rounding to binary32.         */
/*   zpF   = fl32(-mn / scale) (0 when scale == 0); zp = roundEven(clamp). */
/*   y[k]  = clamp(roundEven(fl32(x[k] / scale)) + zp, 0, 255); when       */
/*           scale == 0 every y is zp.                                     */
/* Returns the rounding-exact values; zp as int64 like Tensor.scalarInt.    */
/* Non-finite input: when scale != 0, a NaN or infinite x[k] makes the      */
/* quotient non-finite (an infinity also makes scale infinite, and          */
/* inf / inf is NaN), and _roundEven's toInt() throws UnsupportedError:     */
/* REF_ERR_UNSUPPORTED, outputs unspecified.  When scale == 0 (NaN among    */
/* zeros) no element is rounded and the reference returns zp everywhere.    */
/* ------------------------------------------------------------------------ */
int ref_dql(const float *x, int64_t n, uint8_t *y, float *scale_out,
            int64_t *zp_out) {
  double mn = 0.0, mx = 0.0;
  for (int64_t k = 0; k < n; k++) {
    const double v = (double)x[k];
    if (v < mn) mn = v;
    if (v > mx) mx = v;
  }
  const float scale_f = (float)((mx - mn) / 255.0);
  const double scale = (double)scale_f;
  const float zpf = scale == 0.0 ? 0.0f : (float)(-mn / scale);
  double zc = (double)zpf;
  if (zc < 0.0) zc = 0.0;
  if (zc > 255.0) zc = 255.0;
  const int64_t zp = round_even(zc);
  for (int64_t k = 0; k < n; k++) {
    int64_t q;
    if (scale == 0.0) {
      q = zp;
    } else {
      const float r = (float)((double)x[k] / scale);
      if (!isfinite(r)) return REF_ERR_UNSUPPORTED; /* toInt() of NaN / inf */
      q = round_even((double)r) + zp;
    }
    y[k] = (uint8_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
  }
  *scale_out = scale_f;
  *zp_out = zp;
  return REF_OK;
}

/* ------------------------------------------------------------------------ */
/* opMatMulInteger: onnx_qlinear_ops.dart:30-79.                            */
/*   Y[bb,i,j] = sum_k (A[i,k] - azp) * (B[k,j] - bzp), exact (int64 here, */
/*   int32 semantics in the op contract).  Zero points: absent, scalar     */
/*   (len 1), per-row [M] for A (only when M != 1) or per-column [N] for B */
/*   (only when N != 1); any other length is UnsupportedError (:35-43).    */
/*   Batch: A and B batch counts equal or 1 (:44-47).                      */
/* a_signed / b_signed select int8 vs uint8 element reading.                */
/* ------------------------------------------------------------------------ */
static inline int64_t rd8(const uint8_t *p, int64_t i, int is_signed) {
  return is_signed ? (int64_t)(int8_t)p[i] : (int64_t)p[i];
}

int ref_matmul_integer(const uint8_t *a, int a_signed, int64_t a_batch,
                       int64_t m, int64_t k, const uint8_t *b, int b_signed,
                       int64_t b_batch, int64_t n, const int64_t *azp,
                       int64_t azp_len, const int64_t *bzp, int64_t bzp_len,
                       int64_t *out) {
  if (m < 0 || k < 0 || n < 0 || a_batch < 1 || b_batch < 1) return REF_ERR_ARG;
  if ((azp_len != 0 && azp_len != 1 && azp_len != m) ||
      (bzp_len != 0 && bzp_len != 1 && bzp_len != n))
    return REF_ERR_UNSUPPORTED;
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  if ((a_batch != batch && a_batch != 1) || (b_batch != batch && b_batch != 1))
    return REF_ERR_ARG;
  const int64_t az = (azp_len == 1) ? azp[0] : 0;
  const int64_t *az_row = (azp_len == m && m != 1) ? azp : NULL;
  const int64_t bz = (bzp_len == 1) ? bzp[0] : 0;
  const int64_t *bz_col = (bzp_len == n && n != 1) ? bzp : NULL;
  memset(out, 0, sizeof(int64_t) * (size_t)(batch * m * n));
  for (int64_t bb = 0; bb < batch; bb++) {
    const int64_t a_off = (a_batch == 1 ? 0 : bb) * m * k;
    const int64_t b_off = (b_batch == 1 ? 0 : bb) * k * n;
    const int64_t o_off = bb * m * n;
    for (int64_t i = 0; i < m; i++) {
      const int64_t azi = az_row ? az_row[i] : az;
      for (int64_t kk = 0; kk < k; kk++) {
        const int64_t av = rd8(a, a_off + i * k + kk, a_signed) - azi;
        if (av == 0) continue;
        const int64_t b_row = b_off + kk * n;
        int64_t *o_row = out + o_off + i * n;
        for (int64_t j = 0; j < n; j++) {
          const int64_t z = bz_col ? bz_col[j] : bz;
          o_row[j] += av * (rd8(b, b_row + j, b_signed) - z);
        }
      }
    }
  }
  return REF_OK;
}

/* ------------------------------------------------------------------------ */
/* fp32 rescale of the dynamic-quant export pattern: Cast(to=FLOAT) of the  */
/* MatMulInteger result (opCast onnx_ops.dart:579-606 -> asFloatList        */
/* tensor.dart:118-126: int -> double -> binary32, one rounding), the scale */
/* product Mul(a_scale, b_scale) and Mul(cast, product) (opMul ->           */
/* _arithFloatFast onnx_ops.dart:99-135, :399-401: binary32 products).      */
/*   s_j  = fl32(a_scale * b_scale[j or 0])                                 */
/*   y    = fl32(fl32(acc) * s_j)                                           */
/* b_scale_len is 1 (per tensor) or n (per output column).                  */
/* ------------------------------------------------------------------------ */
void ref_rescale(const int64_t *acc, int64_t rows, int64_t n, float a_scale,
                 const float *b_scale, int64_t b_scale_len, float *y) {
  for (int64_t i = 0; i < rows; i++) {
    for (int64_t j = 0; j < n; j++) {
      const float s = a_scale * b_scale[b_scale_len == 1 ? 0 : j];
      const float c = (float)acc[i * n + j];
      y[i * n + j] = c * s;
    }
  }
}
