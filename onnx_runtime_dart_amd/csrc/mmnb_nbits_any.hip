// MatMulNBits for every even block size the reference accepts.
//
// The reference takes any block_size: n_blocks = ceil(K / bs), each block a
// run of bs / 2 bytes, low nibble first, the last block clipped at K
// (onnx_qlinear_ops.dart:120-121, :139-146).  For an even bs a column's bytes
// are therefore just its k run two to a byte: byte k / 2 holds k, in the low
// nibble when k is even.  The fast kernels take power-of-two blocks >= 16;
// every other even size is packed here:
//
//  - bs a multiple of 16 (48, 80, 96, 192, ...): the pack re-blocks to v, the
//    largest power of two dividing bs.  Virtual block j (k in [j v, (j+1) v))
//    lies inside reference block j v / bs, so it takes that block's scale and
//    zero point; the weight bytes are not touched (the repack reads columns
//    of the reference's n_blocks * bs / 2 bytes).  Same kernels and the same
//    accumulation bound as a power-of-two block.
//  - any other even bs (2 .. 14, 18, 20, 22, 24, ...): the pack keeps the
//    reference's bytes, scales and zero points as they are, and k_nbits_generic
//    computes every output in the reference's own order: w = fl32((q - zp) *
//    scale) per weight (the exact product of a small integer and a binary32
//    value, rounded once, as the Float32List store of :146 rounds it), then
//    acc = fl32(acc + fl32(a * w)) over k ascending from +0 (matmulKernel,
//    gemm_kernel_simd.dart:89-104), and for M = 1 the last N % 4 columns in
//    double (_gemvScalar's tail, :300-308).  Its results are the reference's
//    bits.  It reads the weights once per 16 rows and is far slower than the
//    fast kernels; exporters use power-of-two blocks (ONNX Runtime's
//    MatMulNBits requires them), so this path exists for parity, not speed.
//
// Odd block sizes are rejected (MMNB_ERR_UNSUPPORTED): the reference's
// blob = bs ~/ 2 bytes cannot hold bs nibbles, so its byte index j >> 1 runs
// into the next block's bytes (and past the end of B for the last one).
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
#include <vector>

#include "mmnb_internal.h"

namespace mmnb {

constexpr int kGenCols = 64;                 // columns per workgroup (lane = column)
constexpr int kGenWaves = 4;                 // waves per workgroup, RW rows each
constexpr int kGenK = 64;                    // k per staged chunk
constexpr int kGenMaxBlk = kGenK / 2 + 1;    // blocks one chunk can touch (bs >= 2)

// y[m, n] for a tile of 64 columns x (4 * RW) rows.  Each chunk of 64 k stages
// the tile's weight bytes (8 dwords per column), the scales and zero points of
// the blocks the chunk touches, and the rows' activations in LDS; then lane c
// walks the chunk block by block (wave-uniform bounds) for its column.
// Output (m, n) with m == 0, M == 1 and n >= dtail_from accumulates in double.
template <int RW>
__global__ __launch_bounds__(kGenCols * kGenWaves) void k_nbits_generic(
    const float *__restrict__ A, int64_t lda, const uint8_t *__restrict__ B, int64_t col_bytes,
    const float *__restrict__ S, const uint8_t *__restrict__ Z, int nb, int bs, int K, int M,
    int N, float *__restrict__ Y, int dtail_from) {
  __shared__ uint32_t sw[kGenCols][9];
  __shared__ float ss[kGenCols][kGenMaxBlk];
  __shared__ int sz[kGenCols][kGenMaxBlk];
  __shared__ float sa[kGenWaves * RW][kGenK];
  const int t = threadIdx.x;
  const int c = t & 63, w = t >> 6;
  const int col0 = blockIdx.x * kGenCols;
  const int row0 = blockIdx.y * (kGenWaves * RW);
  const int col = col0 + c;
  const bool dbl = col >= dtail_from;
  float acc[RW];
  double accd[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) {
    acc[r] = 0.0f;
    accd[r] = 0.0;
  }
  for (int k0 = 0; k0 < K; k0 += kGenK) {
    const int kend = min(k0 + kGenK, K);
    const int b0 = k0 / bs;
    const int b1 = min(nb - 1, (kend - 1) / bs);
    const int nbc = b1 - b0 + 1;
    {  // weight bytes: 4 threads per column, 8 bytes each (zero past the column)
      const int cc = t >> 2, part = t & 3;
      const int colg = min(col0 + cc, N - 1);
      const uint8_t *src = B + (int64_t)colg * col_bytes;
      uint32_t d[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int64_t byte = (int64_t)(k0 >> 1) + part * 8 + i;
        const uint32_t v = byte < col_bytes ? (uint32_t)src[byte] : 0u;
        d[i >> 2] |= v << (8 * (i & 3));
      }
      sw[cc][2 * part] = d[0];
      sw[cc][2 * part + 1] = d[1];
    }
    for (int i = t; i < kGenCols * nbc; i += kGenCols * kGenWaves) {
      const int cc = i / nbc, b = i % nbc;
      const int64_t zi = (int64_t)min(col0 + cc, N - 1) * nb + b0 + b;
      ss[cc][b] = S[zi];
      sz[cc][b] = (int)((Z[zi >> 1] >> (4 * (int)(zi & 1))) & 0xF);
    }
    for (int i = t; i < kGenWaves * RW * kGenK; i += kGenCols * kGenWaves) {
      const int r = i / kGenK, kk = i % kGenK;
      const int row = min(row0 + r, M - 1);
      const int k = k0 + kk;
      sa[r][kk] = k < K ? A[(int64_t)row * lda + k] : 0.0f;
    }
    __syncthreads();
    for (int b = 0; b < nbc; b++) {
      // the reference's separately rounded multiply and add: no contraction
      // into an FMA (HIP compiles with -ffp-contract=fast)
#pragma clang fp contract(off)
      const int lo = max(k0, (b0 + b) * bs);
      const int hi = min(kend, (b0 + b + 1) * bs);
      const float s = ss[c][b];
      const int z = sz[c][b];
      for (int k = lo; k < hi; k++) {
        const int i = k - k0;
        const int q = (int)((sw[c][i >> 3] >> (4 * (i & 7))) & 0xFu);
        const float wv = (float)(q - z) * s;
#pragma unroll
        for (int r = 0; r < RW; r++) {
          const float a = sa[w * RW + r][i];
          if (dbl)
            accd[r] = accd[r] + (double)a * (double)wv;
          else
            acc[r] = acc[r] + a * wv;
        }
      }
    }
    __syncthreads();
  }
  if (col < N) {
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const int row = row0 + w * RW + r;
      if (row < M) Y[(int64_t)row * N + col] = dbl ? (float)accd[r] : acc[r];
    }
  }
}

bool nbits_block_native(int64_t bs) { return bs >= 16 && (bs & (bs - 1)) == 0; }

int launch_nbits_generic(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                         int64_t m, float *d_y) {
  const int n = (int)p->n;
  // the reference's m == 1 path sends the last n % 4 columns through
  // _gemvScalar's double accumulator (gemm_kernel_simd.dart:185-190, :300-308)
  const int dtail_from = m == 1 ? n - n % 4 : n;
  const unsigned gx = (unsigned)((n + kGenCols - 1) / kGenCols);
  if (m < 16) {
    const unsigned gy = (unsigned)((m + kGenWaves - 1) / kGenWaves);
    return launch(ctx, kKernNbitsAny, k_nbits_generic<1>, dim3(gx, gy), dim3(kGenCols * kGenWaves),
                  0, d_a, lda, (const uint8_t *)p->d_w, p->col_bytes, (const float *)p->d_scales,
                  (const uint8_t *)p->d_zp, (int)p->n_blocks, (int)p->block, (int)p->k, (int)m, n,
                  d_y, dtail_from);
  }
  const unsigned gy = (unsigned)((m + 4 * kGenWaves - 1) / (4 * kGenWaves));
  return launch(ctx, kKernNbitsAny, k_nbits_generic<4>, dim3(gx, gy), dim3(kGenCols * kGenWaves),
                0, d_a, lda, (const uint8_t *)p->d_w, p->col_bytes, (const float *)p->d_scales,
                (const uint8_t *)p->d_zp, (int)p->n_blocks, (int)p->block, (int)p->k, (int)m, n,
                d_y, dtail_from);
}

// A pack of the reference's own bytes, scales and zero points for the generic
// kernel (lock held).
static int pack_nbits_generic(mmnb_ctx *ctx, const uint8_t *b_q, const float *scales,
                              const uint8_t *zero_points, int zp_fill, int64_t k, int64_t n,
                              int64_t bs, mmnb_pack **out) {
  const int64_t nb = (k + bs - 1) / bs;
  const int64_t src_col = nb * (bs / 2);
  const int64_t zp_need = (n * nb + 1) / 2;
  mmnb_pack *p = new (std::nothrow) mmnb_pack();
  if (!p) return fail(MMNB_ERR_OOM, "out of host memory");
  p->ctx = ctx;
  p->kind = kPackNBits;
  p->generic = true;
  p->k = k;
  p->k_in = k;
  p->n = n;
  p->block = bs;
  p->n_blocks = nb;
  p->k64 = k;  // rows of A are read as they are (no padding)
  p->col_bytes = src_col;
  p->has_zp = zero_points != nullptr || zp_fill != 0x88;
  int rc;
  auto cleanup = [&](int code) {
    if (p->d_w) (void)hipFree(p->d_w);
    if (p->d_scales) (void)hipFree(p->d_scales);
    if (p->d_zp) (void)hipFree(p->d_zp);
    delete p;
    return code;
  };
  if ((rc = device_alloc((size_t)(n * src_col), (void **)&p->d_w))) return cleanup(rc);
  if ((rc = device_alloc((size_t)(n * nb) * 4, (void **)&p->d_scales))) return cleanup(rc);
  if ((rc = device_alloc((size_t)zp_need, (void **)&p->d_zp))) return cleanup(rc);
  hipError_t e;
  if ((e = hipMemcpyAsync(p->d_w, b_q, (size_t)(n * src_col), hipMemcpyHostToDevice,
                          ctx->stream)) != hipSuccess ||
      (e = hipMemcpyAsync(p->d_scales, scales, (size_t)(n * nb) * 4, hipMemcpyHostToDevice,
                          ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(generic pack)"));
  if (zero_points)
    e = hipMemcpyAsync(p->d_zp, zero_points, (size_t)zp_need, hipMemcpyHostToDevice,
                       ctx->stream);
  else
    e = hipMemsetAsync(p->d_zp, zp_fill, (size_t)zp_need, ctx->stream);
  if (e != hipSuccess) return cleanup(check_hip(e, "zero points (generic pack)"));
  if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipStreamSynchronize(generic pack)"));
  p->bytes = n * src_col + n * nb * 4 + zp_need;
  ctx->live_packs++;
  *out = p;
  return MMNB_OK;
}

int pack_nbits_any(mmnb_ctx *ctx, const uint8_t *b_q, const float *scales,
                   const uint8_t *zero_points, int zp_fill, int64_t k, int64_t n, int64_t bs,
                   mmnb_pack **out) {
  if (bs < 2 || (bs & 1))
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: block_size must be even, got " + std::to_string(bs));
  if (nbits_block_native(bs))
    return pack_nbits_core(ctx, b_q, scales, zero_points, zp_fill, k, n, bs, out);
  if (bs % 16 != 0)
    return pack_nbits_generic(ctx, b_q, scales, zero_points, zp_fill, k, n, bs, out);
  // re-block to v = the largest power of two dividing bs (>= 16)
  const int64_t v = bs & -bs;
  const int64_t nb = (k + bs - 1) / bs, nbv = (k + v - 1) / v;
  const int64_t ratio = bs / v;
  std::vector<float> sv;
  std::vector<uint8_t> zv;
  try {
    sv.resize((size_t)(n * nbv));
    if (zero_points) zv.assign((size_t)((n * nbv + 1) / 2), 0);
  } catch (const std::bad_alloc &) {
    return fail(MMNB_ERR_OOM, "MatMulNBits: out of host memory re-blocking the scales");
  }
  for (int64_t c = 0; c < n; c++)
    for (int64_t j = 0; j < nbv; j++) {
      const int64_t src = c * nb + j / ratio, dst = c * nbv + j;
      sv[(size_t)dst] = scales[src];
      if (zero_points) {
        const int zq = (zero_points[src >> 1] >> (4 * (int)(src & 1))) & 0xF;
        zv[(size_t)(dst >> 1)] |= (uint8_t)(zq << (4 * (int)(dst & 1)));
      }
    }
  return pack_nbits_core(ctx, b_q, sv.data(), zero_points ? zv.data() : nullptr, zp_fill, k, n,
                         v, out, nb * (bs / 2));
}

}  // namespace mmnb
