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
// workgroup re-reads its row, which is cheap for M <= 8).
constexpr int kFusedMaxBlocks = 8192;

__global__ __launch_bounds__(256) void k_nbits_correct_rows(
    float *__restrict__ Y, int64_t N, const float *__restrict__ bias,
    const float *__restrict__ corr, int64_t nb, const float *__restrict__ A, int64_t lda,
    int64_t ka, int64_t bs) {
  __shared__ float sas[kFusedMaxBlocks];
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
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float v = bias ? bias[n] : 0.0f;
  if (corr)
    for (int64_t b = 0; b < nb; b++) v = fmaf(corr[b * N + n], sas[b], v);
  Y[m * N + n] += v;
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
                  dim3((unsigned)((p->n + 255) / 256), (unsigned)m), dim3(256), 0, d_y, p->n,
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

// IEEE-754 binary16 -> binary32 (exact): subnormals m * 2^-24, normals
// (1024 + m) * 2^(e - 25), e = 31 infinities / NaN.
float half_to_float(uint16_t h) {
  const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? std::nanf("") : INFINITY;
  else v = std::ldexp((float)(1024 + m), e - 25);
  return sign ? -v : v;
}

int read_floats(const void *p, int64_t len, int type, int64_t need, const char *what,
                std::vector<float> *out) {
  if (!p || len < need)
    return fail(MMNB_ERR_ARG, std::string("MatMulNBits: ") + what + " has " +
                                  std::to_string(p ? len : 0) + " values, need " +
                                  std::to_string(need));
  out->resize((size_t)need);
  if (type == MMNB_DT_F32) {
    std::memcpy(out->data(), p, (size_t)need * 4);
  } else if (type == MMNB_DT_F16) {
    const uint16_t *h = (const uint16_t *)p;
    for (int64_t i = 0; i < need; i++) (*out)[(size_t)i] = half_to_float(h[i]);
  } else {
    return fail(MMNB_ERR_UNSUPPORTED, std::string("MatMulNBits: ") + what +
                                          " must be float32 or float16");
  }
  return MMNB_OK;
}

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
  const int64_t k = d->k, n = d->n, bits = d->bits, bs = d->block_size;
  if (bits != 4 && bits != 8)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: bits must be 4 or 8, got " + std::to_string(bits));
  if (k <= 0 || n <= 0) return fail(MMNB_ERR_ARG, "MatMulNBits: K and N must be positive");
  if (bs < 16 || (bs & (bs - 1)) != 0)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: block_size must be a power of two >= 16, got " +
                    std::to_string(bs));
  const int64_t nb = (k + bs - 1) / bs;
  const int64_t blob = bs * bits / 8;
  if (!d->b_q || d->b_q_len < n * nb * blob)
    return fail(MMNB_ERR_ARG, "MatMulNBits: B has " + std::to_string(d->b_q_len) +
                                  " bytes, need " + std::to_string(n * nb * blob));
  int rc;
  std::vector<float> s;
  if ((rc = read_floats(d->scales, d->scales_len, d->scales_type, n * nb, "scales", &s)))
    return rc;
  // ---- zero points: integers (zi) or floats (zf), one per (column, block)
  std::vector<int32_t> zi;
  std::vector<float> zf;
  if (d->zero_points) {
    if (d->zero_points_type == MMNB_DT_U8) {
      const uint8_t *z = (const uint8_t *)d->zero_points;
      zi.resize((size_t)(n * nb));
      if (bits == 8) {
        if (d->zero_points_len < n * nb)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs N*n_blocks bytes");
        for (int64_t i = 0; i < n * nb; i++) zi[(size_t)i] = z[i];
      } else if (d->zero_points_layout == MMNB_ZP_PER_COLUMN) {
        const int64_t row = (nb + 1) / 2;
        if (d->zero_points_len < n * row)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs N*ceil(n_blocks/2) bytes");
        for (int64_t c = 0; c < n; c++)
          for (int64_t b = 0; b < nb; b++) {
            const uint8_t byte = z[c * row + b / 2];
            zi[(size_t)(c * nb + b)] = (b & 1) ? byte >> 4 : byte & 15;
          }
      } else if (d->zero_points_layout == MMNB_ZP_FLAT) {
        if (d->zero_points_len < (n * nb + 1) / 2)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs ceil(N*n_blocks/2) bytes");
        for (int64_t i = 0; i < n * nb; i++) {
          const uint8_t byte = z[i >> 1];
          zi[(size_t)i] = (i & 1) ? byte >> 4 : byte & 15;
        }
      } else {
        return fail(MMNB_ERR_ARG, "MatMulNBits: unknown zero-point layout");
      }
    } else if ((rc = read_floats(d->zero_points, d->zero_points_len, d->zero_points_type,
                                 n * nb, "zero_points", &zf))) {
      return rc;
    }
  }
  std::vector<float> bias;
  if (d->bias && (rc = read_floats(d->bias, d->bias_len, d->bias_type, n, "bias", &bias)))
    return rc;
  // ---- g_idx: a stable sort of the rows by group, unless it is k / bs
  std::vector<int32_t> perm;
  if (d->g_idx) {
    if (d->g_idx_len != k) return fail(MMNB_ERR_ARG, "MatMulNBits: g_idx needs K entries");
    bool trivial = true;
    std::vector<int64_t> count((size_t)nb, 0);
    for (int64_t i = 0; i < k; i++) {
      const int32_t g = d->g_idx[i];
      if (g < 0 || g >= nb) return fail(MMNB_ERR_ARG, "MatMulNBits: g_idx out of range");
      count[(size_t)g]++;
      trivial = trivial && g == i / bs;
    }
    if (!trivial) {
      if (bits != 4)
        return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx with bits=8 is not supported");
      if (k % bs)
        return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx needs K a multiple of block_size");
      for (int64_t g = 0; g < nb; g++)
        if (count[(size_t)g] != bs)
          return fail(MMNB_ERR_UNSUPPORTED,
                      "MatMulNBits: g_idx groups must hold block_size rows each");
      perm.resize((size_t)k);
      for (int64_t i = 0; i < k; i++) perm[(size_t)i] = (int32_t)i;
      std::stable_sort(perm.begin(), perm.end(), [&](int32_t a, int32_t b) {
        return d->g_idx[a] < d->g_idx[b];
      });
    }
  }
  // ---- the virtual 4-bit weight
  const uint8_t *B = d->b_q;
  const int64_t kp = nb * bs;
  const int64_t kv = bits == 8 ? 2 * kp : k;
  const int64_t nbv = (kv + bs - 1) / bs;
  const int64_t vblob = bs / 2;
  std::vector<uint8_t> vb;
  std::vector<float> vs = s;
  std::vector<uint8_t> vz;        // flat packed nibbles, or empty
  int zfill = 0x88;
  std::vector<double> corr;       // [nb][n], empty when none
  std::vector<int32_t> asrc;      // [kv], empty when A is used as is
  auto nib4 = [&](int64_t c, int64_t kk) -> int {  // 4-bit q of column c, row kk
    const uint8_t byte = B[c * nb * blob + (kk / bs) * blob + (kk % bs) / 2];
    return (kk & 1) ? byte >> 4 : byte & 15;
  };
  auto put = [&](int64_t c, int64_t j, int q) {
    uint8_t &byte = vb[(size_t)(c * nbv * vblob + (j / bs) * vblob + (j % bs) / 2)];
    byte = (j & 1) ? (uint8_t)((byte & 0x0F) | (q << 4)) : (uint8_t)((byte & 0xF0) | q);
  };
  if (bits == 8) {
    vb.assign((size_t)(n * nbv * vblob), 0x88);
    for (int64_t c = 0; c < n; c++)
      for (int64_t kk = 0; kk < k; kk++) {
        const int q8 = B[c * nb * bs + kk];
        put(c, kk, q8 >> 4);
        put(c, kp + kk, q8 & 15);
      }
    vs.resize((size_t)(n * nbv));
    for (int64_t c = 0; c < n; c++)
      for (int64_t b = 0; b < nb; b++) {
        vs[(size_t)(c * nbv + b)] = 16.0f * s[(size_t)(c * nb + b)];
        vs[(size_t)(c * nbv + nb + b)] = s[(size_t)(c * nb + b)];
      }
    corr.assign((size_t)(nb * n), 0.0);
    for (int64_t c = 0; c < n; c++)
      for (int64_t b = 0; b < nb; b++) {
        const double z = !zf.empty() ? (double)zf[(size_t)(c * nb + b)]
                                     : !zi.empty() ? (double)zi[(size_t)(c * nb + b)] : 128.0;
        corr[(size_t)(b * n + c)] = (136.0 - z) * (double)s[(size_t)(c * nb + b)];
      }
    asrc.resize((size_t)kv);
    for (int64_t j = 0; j < kv; j++) {
      const int64_t kk = j < kp ? j : j - kp;
      asrc[(size_t)j] = kk < k ? (int32_t)kk : -1;
    }
  } else {
    if (perm.empty()) {
      vb.assign(B, B + n * nb * blob);
    } else {
      vb.assign((size_t)(n * nbv * vblob), 0);
      for (int64_t c = 0; c < n; c++)
        for (int64_t j = 0; j < k; j++) put(c, j, nib4(c, perm[(size_t)j]));
      asrc = perm;
    }
    if (!zf.empty()) {
      zfill = 0x00;  // the kernels see zero point 0; -z s goes to the correction
      corr.assign((size_t)(nb * n), 0.0);
      for (int64_t c = 0; c < n; c++)
        for (int64_t b = 0; b < nb; b++)
          corr[(size_t)(b * n + c)] =
              -(double)zf[(size_t)(c * nb + b)] * (double)s[(size_t)(c * nb + b)];
    } else if (!zi.empty()) {
      vz.assign((size_t)((n * nb + 1) / 2), 0);
      for (int64_t i = 0; i < n * nb; i++)
        vz[(size_t)(i >> 1)] |= (uint8_t)(zi[(size_t)i] << ((i & 1) * 4));
    }
  }
  mmnb_pack *p = nullptr;
  int urc = MMNB_OK;
  {
    CtxLock lk(ctx);
    if ((rc = set_device(ctx))) return rc;
    if ((rc = pack_nbits_core(ctx, vb.data(), vs.data(), vz.empty() ? nullptr : vz.data(),
                              zfill, kv, n, bs, &p)))
      return rc;
    p->k_in = k;
    p->ext = !asrc.empty() || !corr.empty() || !bias.empty();
    if (!asrc.empty()) urc = upload(p, asrc, &p->d_asrc);
    if (!urc && !corr.empty()) {
      std::vector<float> c32(corr.begin(), corr.end());
      urc = upload(p, c32, &p->d_corr);
      p->corr_nb = nb;
    }
    if (!urc && !bias.empty()) urc = upload(p, bias, &p->d_bias);
  }
  if (urc) {
    (void)mmnb_pack_free(p);  // takes the context lock itself
    return urc;
  }
  *out = p;
  return MMNB_OK;
}
