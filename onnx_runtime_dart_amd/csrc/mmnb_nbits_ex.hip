// MatMulNBits beyond the reference's 4-bit form: bits = 8, g_idx
// (act-order groups), bias, floating-point zero points, fp16 scales and
// bias, and ORT's per-column zero-point layout.
//
// Everything is mapped onto the 4-bit kernels at pack time ("virtual"
// 4-bit weight of Kv rows), plus an optional A gather before and one
// correction pass after the product:
//
//   bits = 8:  q8 = 16 hi + lo, so (q8 - z) s = (hi - 8)(16 s) + (lo - 8) s
//              + (136 - z) s.  The virtual weight stacks the hi plane (scale
//              16 s, exact) over the lo plane (scale s), both with zero
//              point 8, over Kv = 2 * ceil(K/bs) * bs rows; A is gathered as
//              [A | A]; the last term is the correction below.
//   float zp:  (q - z) s = q s - z s: the kernels run with zero point 0 and
//              the correction adds -z s per block.
//   g_idx:     the rows are sorted by group (stable), so every group is one
//              block of the virtual weight; A is gathered in the same order.
//              Each group must hold exactly block_size rows.
//   bias:      added in the correction pass.
//
// Correction: y[m, n] += bias[n] + sum_b c[b][n] * asum[m][b], with asum the
// block sums of the (gathered) A over the first corr_nb blocks.  c is built
// in double and rounded once to fp32.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "mmnb_host.h"
#include "mmnb_internal.h"

using namespace mmnb;

namespace mmnb {

// out[m, j] = A[m, src[j]] for j < kv (src[j] < 0: 0), zero for kv <= j < ldo.
__global__ __launch_bounds__(256) void k_gather_a(const float *__restrict__ A, int64_t lda,
                                                  int64_t M, const int32_t *__restrict__ src,
                                                  int64_t kv, int64_t ldo,
                                                  float *__restrict__ out) {
  const int64_t total = M * ldo;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / ldo, j = i % ldo;
    const int s = src[j < kv ? j : 0];
    const bool ok = j < kv && s >= 0;
    const float v = A[m * lda + (ok ? s : 0)];
    out[i] = ok ? v : 0.0f;
  }
}

// asum[m][b] = sum of A[m, b*bs .. min((b+1)*bs, ka) - 1]; one wave per (b, m).
__global__ __launch_bounds__(64) void k_block_sums(const float *__restrict__ A, int64_t lda,
                                                   int64_t ka, int64_t bs, int64_t nb,
                                                   float *__restrict__ asum) {
  const int64_t b = blockIdx.x, m = blockIdx.y;
  const int64_t k0 = b * bs, k1 = std::min(ka, k0 + bs);
  float s = 0.0f;
  for (int64_t kk = k0 + threadIdx.x; kk < k1; kk += 64) s += A[m * lda + kk];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (threadIdx.x == 0) asum[m * nb + b] = s;
}

// y[m, n] += bias[n] + sum_b corr[b][n] * asum[m][b]
__global__ __launch_bounds__(256) void k_nbits_correct(float *__restrict__ Y, int64_t N,
                                                       const float *__restrict__ bias,
                                                       const float *__restrict__ corr,
                                                       int64_t nb,
                                                       const float *__restrict__ asum) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
  if (n >= N) return;
  float v = bias ? bias[n] : 0.0f;
  if (corr) {
    const float *as = asum + m * nb;
    for (int64_t b = 0; b < nb; b++) v = fmaf(corr[b * N + n], as[b], v);
  }
  Y[m * N + n] += v;
}

// The same correction for few rows, with the block sums of row m formed in
// LDS by the workgroup itself (one launch instead of two; every column
// workgroup re-reads its row, which is cheap for M <= 8).  A workgroup takes
// 64 columns; its 4 waves split the blocks (wave w: b = w, w + 4, ...) with
// eight loads of corr in flight per lane, then add their partial sums in a
// fixed order through LDS (a single chain over all blocks waited on every
// load in turn).
constexpr int kFusedMaxBlocks = 8192;
constexpr int kCorrCols = 64;

__global__ __launch_bounds__(256) void k_nbits_correct_rows(
    float *__restrict__ Y, int64_t N, const float *__restrict__ bias,
    const float *__restrict__ corr, int64_t nb, const float *__restrict__ A, int64_t lda,
    int64_t ka, int64_t bs) {
  __shared__ float sas[kFusedMaxBlocks];
  __shared__ float spart[4][kCorrCols];
  const int64_t m = blockIdx.y;
  const int w = threadIdx.x >> 6, ln = threadIdx.x & 63;
  if (corr) {
    for (int64_t b = w; b < nb; b += 4) {
      const int64_t k0 = b * bs, k1 = std::min(ka, k0 + bs);
      float s = 0.0f;
      for (int64_t kk = k0 + ln; kk < k1; kk += 64) s += A[m * lda + kk];
      for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
      if (ln == 0) sas[b] = s;
    }
    __syncthreads();
  }
  const int64_t n = (int64_t)blockIdx.x * kCorrCols + ln;
  const int64_t nc = n < N ? n : N - 1;
  float v = 0.0f;
  if (corr) {
    int64_t b = w;
    for (; b + 28 < nb; b += 32) {
      float c[8];
#pragma unroll
      for (int u = 0; u < 8; u++) c[u] = corr[(b + 4 * u) * N + nc];
#pragma unroll
      for (int u = 0; u < 8; u++) v = fmaf(c[u], sas[b + 4 * u], v);
    }
    for (; b < nb; b += 4) v = fmaf(corr[b * N + nc], sas[b], v);
  }
  spart[w][ln] = v;
  __syncthreads();
  if (w == 0 && n < N) {
    float t = bias ? bias[n] : 0.0f;
    t += ((spart[0][ln] + spart[1][ln]) + spart[2][ln]) + spart[3][ln];
    Y[m * N + n] += t;
  }
}

int run_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                     int64_t m, float *d_y) {
  if (!p->ext) return launch_matmul_nbits(ctx, p, d_a, lda, m, d_y);
  int rc;
  const float *a2 = d_a;
  int64_t lda2 = lda, ka = p->k_in;
  if (p->d_asrc) {
    void *buf = nullptr;
    if ((rc = scratch_get(ctx, 9, (size_t)(m * p->k64) * 4, &buf))) return rc;
    int64_t blocks = (m * p->k64 + 255) / 256;
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, 16384));
    if ((rc = launch(ctx, kKernNbitsEx, k_gather_a, dim3((unsigned)blocks), dim3(256), 0, d_a, lda,
                     m, (const int32_t *)p->d_asrc, p->k, p->k64, (float *)buf)))
      return rc;
    a2 = (const float *)buf;
    lda2 = p->k64;
    ka = p->k;
  }
  if ((rc = launch_matmul_nbits(ctx, p, a2, lda2, m, d_y))) return rc;
  if (m <= 8 && p->corr_nb <= kFusedMaxBlocks)
    return launch(ctx, kKernNbitsEx, k_nbits_correct_rows,
                  dim3((unsigned)((p->n + kCorrCols - 1) / kCorrCols), (unsigned)m), dim3(256), 0,
                  d_y, p->n,
                  (const float *)p->d_bias, (const float *)p->d_corr, p->corr_nb, a2, lda2, ka,
                  p->block);
  const float *d_asum = nullptr;
  if (p->d_corr) {
    void *buf = nullptr;
    if ((rc = scratch_get(ctx, 7, (size_t)(m * p->corr_nb) * 4, &buf))) return rc;
    if ((rc = launch(ctx, kKernNbitsEx, k_block_sums, dim3((unsigned)p->corr_nb, (unsigned)m),
                     dim3(64), 0, a2, lda2, ka, p->block, p->corr_nb, (float *)buf)))
      return rc;
    d_asum = (const float *)buf;
  }
  return launch(ctx, kKernNbitsEx, k_nbits_correct,
                dim3((unsigned)((p->n + 255) / 256), (unsigned)m), dim3(256), 0, d_y, p->n,
                (const float *)p->d_bias, (const float *)p->d_corr, p->corr_nb, d_asum);
}

}  // namespace mmnb

namespace {

template <typename T>
int upload(mmnb_pack *p, const std::vector<T> &v, T **dst) {
  int rc = device_alloc(v.size() * sizeof(T), (void **)dst);
  if (rc) return rc;
  MMNB_HIP(hipMemcpy(*dst, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  p->bytes += (int64_t)(v.size() * sizeof(T));
  return MMNB_OK;
}

}  // namespace

int mmnb_pack_nbits_ex(mmnb_ctx *ctx, const mmnb_nbits_desc *d, mmnb_pack **out) {
  MMNB_GUARD_CTX(ctx);
  if (!out || !d) return fail(MMNB_ERR_ARG, "mmnb_pack_nbits_ex: null argument");
  *out = nullptr;
  // validation and the virtual 4-bit weight: host code (mmnb_host.cpp)
  NbitsHost h;
  int rc = nbits_prepare(d, &h);
  if (rc) return rc;
  mmnb_pack *p = nullptr;
  int urc = MMNB_OK;
  {
    CtxLock lk(ctx);
    if ((rc = set_device(ctx))) return rc;
    // the reference's own form takes any even block size (pack_nbits_any);
    // the extensions run on power-of-two blocks (nbits_prepare checks)
    const bool plain = h.asrc.empty() && h.corr.empty() && h.bias.empty();
    const uint8_t *vz = h.vz.empty() ? nullptr : h.vz.data();
    rc = plain ? pack_nbits_any(ctx, h.vb.data(), h.vs.data(), vz, h.zfill, h.kv, h.n, h.block, &p)
               : pack_nbits_core(ctx, h.vb.data(), h.vs.data(), vz, h.zfill, h.kv, h.n, h.block,
                                 &p);
    if (rc) return rc;
    p->k_in = h.k;
    p->ext = !h.asrc.empty() || !h.corr.empty() || !h.bias.empty();
    if (!h.asrc.empty()) urc = upload(p, h.asrc, &p->d_asrc);
    if (!urc && !h.corr.empty()) {
      std::vector<float> c32(h.corr.begin(), h.corr.end());
      urc = upload(p, c32, &p->d_corr);
      p->corr_nb = h.n_blocks;
    }
    if (!urc && !h.bias.empty()) urc = upload(p, h.bias, &p->d_bias);
  }
  if (urc) {
    (void)mmnb_pack_free(p);  // takes the context lock itself
    return urc;
  }
  *out = p;
  return MMNB_OK;
}
