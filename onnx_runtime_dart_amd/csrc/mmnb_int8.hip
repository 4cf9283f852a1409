// Int8 dynamic-quantisation path on gfx950: DynamicQuantizeLinear and
// MatMulInteger (i8 MFMA, exact int32) with the optional fp32 rescale.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mmnb_device.h"
#include "mmnb_internal.h"

namespace mmnb {

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear (onnx_ops.dart:2556-2583), bit-exact:
//   pass 1  per-block min/max partials, starting from 0 (:2558-2562); NaN is
//           skipped because it never compares below/above (Dart `<`/`>`).
//   pass 2  every block reduces the partials itself (deterministic, no
//           atomics), derives scale/zero point in double exactly as the
//           reference, then quantises its slice:
//             scale = fl32((mx - mn) / 255.0)           (double ops)
//             zp    = roundEven(clamp(fl32(-mn / scale), 0, 255))
//             y     = clamp(rint(fl32(x / scale)) + zp, 0, 255)
//           fl32(x / scale) of two binary32 operands equals the reference's
//           double quotient rounded to binary32 (double rounding is
//           innocuous for division at these precisions), so __fdiv_rn gives
//           the same bits.  rint is round-half-even, as _roundEven
//           (onnx_ops.dart:2490-2497) for finite input.
// Non-finite input: the reference throws (toInt() of a NaN / infinite
// quotient in _roundEven) whenever scale != 0 and some x is NaN or infinite;
// an infinity makes mn or mx infinite, a NaN is flagged by pass 1.  Then the
// scale is written as NaN, the marker the host entry point turns into
// MMNB_ERR_UNSUPPORTED, and every quantised byte is defined (NaN -> 0).  With
// scale == 0 (NaN among zeros) the reference rounds nothing and returns zp
// everywhere, and so do the kernels.
// ---------------------------------------------------------------------------
constexpr int kDqlThreads = 256;
constexpr int kDqlMaxBlocks = 1024;
// 16-byte loads a thread issues before using any: 2 gives twice the
// workgroups of 4 at the same bytes (at [512,1024] 512 against 256; the two
// launches took 5.65 against 6.2 us, and 5.9 at 1, 7.6 at 8)
constexpr int kDqlUnroll = 2;

// Per-block min/max partials.  Each thread issues kDqlUnroll float4 loads
// (indices clamped into range: a repeated element changes neither extreme)
// before comparing any, so a grid-stride pass is one round trip per
// kDqlUnroll loads instead of one per load.
__global__ __launch_bounds__(kDqlThreads) void k_dql_minmax(const float *__restrict__ x,
                                                            int64_t n,
                                                            float2 *__restrict__ part,
                                                            int *__restrict__ part_nan,
                                                            int nblocks) {
  // every argument in SGPRs up front (one round of scalar loads; the grid
  // size as an argument, gridDim.x being a vector load of the hidden ones)
  kernarg_fence(x, n, part, part_nan, nblocks);
  float mn = 0.0f, mx = 0.0f;
  bool nan = false;
  const int64_t stride = (int64_t)nblocks * kDqlThreads;
  const int64_t tid = (int64_t)blockIdx.x * kDqlThreads + threadIdx.x;
  const bool vec = (((uintptr_t)x) & 15) == 0;
  int64_t done = 0;
  if (vec && n >= 4) {
    const int64_t n4 = n >> 2;
    const float4 *x4 = (const float4 *)x;
    for (int64_t base = tid; base < n4; base += stride * kDqlUnroll) {
      float4 v[kDqlUnroll];
#pragma unroll
      for (int u = 0; u < kDqlUnroll; u++) {
        const int64_t i = base + u * stride;
        v[u] = x4[i < n4 ? i : n4 - 1];
      }
#pragma unroll
      for (int u = 0; u < kDqlUnroll; u++) {
        mn = v[u].x < mn ? v[u].x : mn; mx = v[u].x > mx ? v[u].x : mx;
        mn = v[u].y < mn ? v[u].y : mn; mx = v[u].y > mx ? v[u].y : mx;
        mn = v[u].z < mn ? v[u].z : mn; mx = v[u].z > mx ? v[u].z : mx;
        mn = v[u].w < mn ? v[u].w : mn; mx = v[u].w > mx ? v[u].w : mx;
        nan |= (v[u].x != v[u].x) | (v[u].y != v[u].y) | (v[u].z != v[u].z) |
               (v[u].w != v[u].w);
      }
    }
    done = n4 << 2;
  }
  for (int64_t i = done + tid; i < n; i += stride) {
    const float v = x[i];
    mn = v < mn ? v : mn;
    mx = v > mx ? v : mx;
    nan |= v != v;
  }
  const bool wave_nan = __any(nan);
  for (int off = 32; off > 0; off >>= 1) {
    const float a = __shfl_xor(mn, off, 64), b = __shfl_xor(mx, off, 64);
    mn = a < mn ? a : mn;
    mx = b > mx ? b : mx;
  }
  __shared__ float2 s[kDqlThreads / 64];
  __shared__ int s_nan[kDqlThreads / 64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    s[wave] = make_float2(mn, mx);
    s_nan[wave] = wave_nan ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int any_nan = s_nan[0];
    for (int w = 1; w < kDqlThreads / 64; w++) {
      mn = s[w].x < mn ? s[w].x : mn;
      mx = s[w].y > mx ? s[w].y : mx;
      any_nan |= s_nan[w];
    }
    part[blockIdx.x] = make_float2(mn, mx);
    part_nan[blockIdx.x] = any_nan;
  }
}

__device__ __forceinline__ uint8_t dql_q(float v, float scale, int zp) {
  if (scale == 0.0f) return (uint8_t)zp;
  const float r = rintf(__fdiv_rn(v, scale));
  // r is an integral float; clamp before converting (|r| <= ~2^8 for finite
  // in-contract input; NaN, reached only out of contract, goes to 0).
  float q = r + (float)zp;
  q = q >= 0.0f ? (q > 255.0f ? 255.0f : q) : 0.0f;
  return (uint8_t)(int)q;
}

__global__ __launch_bounds__(kDqlThreads) void k_dql_quant(
    const float *__restrict__ x, int64_t n, const float2 *__restrict__ part,
    const int *__restrict__ part_nan, int nparts, uint8_t *__restrict__ y,
    float *__restrict__ out_scale, int32_t *__restrict__ out_zp, int nblocks) {
  __shared__ float2 s[kDqlThreads / 64];
  __shared__ int s_nan[kDqlThreads / 64];
  __shared__ float s_scale;
  __shared__ int s_zp;
  kernarg_fence(x, n, part, part_nan, nparts, y, out_scale, out_zp, nblocks);
  const int64_t stride = (int64_t)nblocks * kDqlThreads;
  const int64_t tid = (int64_t)blockIdx.x * kDqlThreads + threadIdx.x;
  const bool vec = ((((uintptr_t)x) & 15) == 0) && ((((uintptr_t)y) & 3) == 0);
  const int64_t n4 = (vec && n >= 4) ? n >> 2 : 0;
  const float4 *x4 = (const float4 *)x;
  // the thread's first batch of x is loaded before the scale is known (it
  // does not depend on it), so its round trip overlaps the partials' one
  float4 v[kDqlUnroll];
  if (n4 > 0) {  // workgroup-uniform
#pragma unroll
    for (int u = 0; u < kDqlUnroll; u++) {
      const int64_t i = tid + u * stride;
      v[u] = x4[i < n4 ? i : n4 - 1];
    }
  }
  float mn = 0.0f, mx = 0.0f;
  bool nan = false;
  for (int i = threadIdx.x; i < nparts; i += kDqlThreads) {
    const float2 p = part[i];
    mn = p.x < mn ? p.x : mn;
    mx = p.y > mx ? p.y : mx;
    nan |= part_nan[i] != 0;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float a = __shfl_xor(mn, off, 64), b = __shfl_xor(mx, off, 64);
    mn = a < mn ? a : mn;
    mx = b > mx ? b : mx;
  }
  const bool wave_nan = __any(nan);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    s[wave] = make_float2(mn, mx);
    s_nan[wave] = wave_nan ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int any_nan = s_nan[0];
    for (int w = 1; w < kDqlThreads / 64; w++) {
      mn = s[w].x < mn ? s[w].x : mn;
      mx = s[w].y > mx ? s[w].y : mx;
      any_nan |= s_nan[w];
    }
    const double dmn = (double)mn, dmx = (double)mx;
    float scale = (float)((dmx - dmn) / 255.0);
    // out of contract (the reference throws): NaN scale marks it
    if (scale != 0.0f && (any_nan || __builtin_isinf(mn) || __builtin_isinf(mx)))
      scale = __builtin_nanf("");
    const double ds = (double)scale;
    const float zpf = ds == 0.0 ? 0.0f : (float)(-dmn / ds);
    double zc = (double)zpf;
    zc = zc >= 0.0 ? (zc > 255.0 ? 255.0 : zc) : 0.0;  // NaN (out of contract) -> 0
    const int zp = (int)rint(zc);
    s_scale = scale;
    s_zp = zp;
    if (blockIdx.x == 0) {
      *out_scale = scale;
      *out_zp = zp;
    }
  }
  __syncthreads();
  const float scale = s_scale;
  const int zp = s_zp;
  if (n4 > 0) {
    uint32_t *y4 = (uint32_t *)y;
    // kDqlUnroll loads in flight per thread (clamped indices; only the
    // in-range results are stored)
    for (int64_t base = tid; base < n4; base += stride * kDqlUnroll) {
      if (base != tid) {
#pragma unroll
        for (int u = 0; u < kDqlUnroll; u++) {
          const int64_t i = base + u * stride;
          v[u] = x4[i < n4 ? i : n4 - 1];
        }
      }
#pragma unroll
      for (int u = 0; u < kDqlUnroll; u++) {
        const int64_t i = base + u * stride;
        const uint32_t b = (uint32_t)dql_q(v[u].x, scale, zp) |
                           ((uint32_t)dql_q(v[u].y, scale, zp) << 8) |
                           ((uint32_t)dql_q(v[u].z, scale, zp) << 16) |
                           ((uint32_t)dql_q(v[u].w, scale, zp) << 24);
        if (i < n4) y4[i] = b;
      }
    }
  }
  for (int64_t i = (n4 << 2) + tid; i < n; i += stride) y[i] = dql_q(x[i], scale, zp);
}

int launch_dql(mmnb_ctx *ctx, const float *d_x, int64_t n, uint8_t *d_y, float *d_scale,
               int32_t *d_zp) {
  void *d_part = nullptr;
  int rc;
  // partials: kDqlMaxBlocks (min, max) pairs, then kDqlMaxBlocks NaN flags
  if ((rc = scratch_get(ctx, 3, (sizeof(float2) + sizeof(int)) * kDqlMaxBlocks, &d_part)))
    return rc;
  int *d_part_nan = (int *)((float2 *)d_part + kDqlMaxBlocks);
  // one batch of kDqlUnroll float4 per thread when the grid allows
  const int64_t per_block = (int64_t)kDqlThreads * kDqlUnroll * 4;
  int64_t blocks = (n + per_block - 1) / per_block;
  if (blocks < 1) blocks = 1;
  if (blocks > kDqlMaxBlocks) blocks = kDqlMaxBlocks;
  if ((rc = launch(ctx, kKernDqlMinmax, k_dql_minmax, dim3((unsigned)blocks), dim3(kDqlThreads),
                    0, d_x, n, (float2 *)d_part, d_part_nan, (int)blocks)))
    return rc;
  int64_t qblocks = (n + per_block - 1) / per_block;
  if (qblocks < 1) qblocks = 1;
  if (qblocks > 4096) qblocks = 4096;
  return launch(ctx, kKernDqlQuant, k_dql_quant, dim3((unsigned)qblocks), dim3(kDqlThreads), 0,
                d_x, n, (const float2 *)d_part, (const int *)d_part_nan, (int)blocks, d_y,
                d_scale, d_zp, (int)qblocks);
}

// ---------------------------------------------------------------------------
// MatMulInteger (onnx_qlinear_ops.dart:30-79) on v_mfma_i32_16x16x64_i8.
//
// The i8 MFMA multiplies signed bytes.  Operands are offset into int8:
//   A' = A xor 0x80 = A - 128 (uint8 A) or A (int8 A);  A - azp = A' + c_m,
//        c_m = (uint8 ? 128 : 0) - azp_m
//   B' = B xor 0x80 (uint8 B) or B;                      B - bzp = B' + e_n,
//        e_n = (uint8 ? 128 : 0) - bzp_n
// so  Y = sum A'B' + e_n sum_k A'_m + c_m sum_k B'_n + K c_m e_n,
// every term an exact integer; the sum is evaluated modulo 2^32, which is
// exact whenever the true result fits int32 (|Y| <= 255*255*K, K <= 33025).
// B' is prepared once per pack as [batch][n][kpad] (k contiguous, zero
// padded) with its column sums; row sums of A' come from v_dot4 on the
// operand registers.
// ---------------------------------------------------------------------------
// One 64 (k) x 64 (column) tile per workgroup: the source bytes are read
// along whichever axis is contiguous (columns of a [batch, k, n] B, k of a
// transposed [batch, n, k] convolution weight), turned through LDS, and
// written k-contiguous per column as 16-byte stores; each column's partial
// sum over the tile is added to colsum (zeroed beforehand; integer adds, so
// the order does not matter).
__global__ __launch_bounds__(256) void k_prep_int_b(const uint8_t *__restrict__ src,
                                                    int b_signed, int b_trans, int64_t k,
                                                    int64_t n, int64_t kpad,
                                                    int8_t *__restrict__ bt,
                                                    int32_t *__restrict__ colsum) {
  __shared__ int8_t tile[64][64 + 4];  // [column][k]
  const int64_t c0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  const int64_t b = blockIdx.z;
  const int t = threadIdx.x;
  // load: thread t takes 16 consecutive elements along the contiguous axis
  const int lo = (t & 3) * 16, hi = t >> 2;  // 16 along the fast axis, 1 along the slow
#pragma unroll
  for (int e = 0; e < 16; e++) {
    // (kk, col) of this element
    const int64_t kk = b_trans ? k0 + lo + e : k0 + hi;
    const int64_t col = b_trans ? c0 + hi : c0 + lo + e;
    int v = 0;
    if (kk < k && col < n) {
      const uint8_t raw = b_trans ? src[(b * n + col) * k + kk] : src[(b * k + kk) * n + col];
      v = b_signed ? (int)(int8_t)raw : (int)raw - 128;
    }
    if (b_trans)
      tile[hi][lo + e] = (int8_t)v;
    else
      tile[lo + e][hi] = (int8_t)v;
  }
  __syncthreads();
  // store: thread t writes k = k0 + lo .. +15 of column c0 + hi
  const int64_t col = c0 + hi;
  int sum = 0;
  uint32_t w[4];
#pragma unroll
  for (int d = 0; d < 4; d++) {
    uint32_t x = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int8_t v = tile[hi][lo + 4 * d + e];
      sum += v;
      x |= (uint32_t)(uint8_t)v << (8 * e);
    }
    w[d] = x;
  }
  if (col < n) {
    *(uint4 *)(bt + (b * n + col) * kpad + k0 + lo) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  // the four threads of a column: lanes 4j .. 4j+3
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  if ((t & 3) == 0 && col < n) atomicAdd(&colsum[b * n + col], sum);
}

// e = (uint8 ? 128 : 0) - b_zp for each of `cnt` columns (n, or batch*n
// when the zero points differ per batch).
__global__ void k_prep_int_e(int b_signed, int64_t cnt, const int32_t *__restrict__ bzp,
                             int64_t bzp_len, int32_t *__restrict__ ecol) {
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= cnt) return;
  int32_t z = 0;
  if (bzp_len == 1) z = bzp[0];
  else if (bzp_len == cnt && cnt != 1) z = bzp[col];
  ecol[col] = (b_signed ? 0 : 128) - z;
}

int prepare_integer_b(mmnb_ctx *ctx, const uint8_t *d_src, int b_signed, int b_trans,
                      int64_t batch, int64_t k, int64_t n, int64_t kpad, const int32_t *d_bzp,
                      int64_t bzp_len, int8_t *d_bt, int32_t *d_colsum, int32_t *d_ecol) {
  const int threads = 256;
  MMNB_HIP(hipMemsetAsync(d_colsum, 0, (size_t)(batch * n) * 4, ctx->stream));
  int rc = launch(ctx, kKernPrepIntB, k_prep_int_b,
                  dim3((unsigned)((n + 63) / 64), (unsigned)(kpad / 64), (unsigned)batch),
                  dim3(threads), 0, d_src, b_signed, b_trans, k, n, kpad, d_bt, d_colsum);
  if (rc) return rc;
  const int64_t cnt = (bzp_len == batch * n && batch > 1) ? batch * n : n;
  return launch(ctx, kKernPrepIntB, k_prep_int_e, dim3((unsigned)((cnt + threads - 1) / threads)),
                dim3(threads), 0, b_signed, cnt, d_bzp, bzp_len, d_ecol);
}

typedef int int4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Epilogue operands of one lane: A's zero point for each of its 8 rows, and
// per column (2 of them) the pack's zero-point terms, the fp32 rescale's B
// scale and the requantisation's multiplier and bias.  Loaded at the start of
// the kernel, unconditionally (clamped indices; arrays a call does not use are
// read from the zero page `pad`), so they arrive during the K loop instead of
// as a chain of dependent round trips after it (a load under a branch ends in
// a full wait).
struct MmiEpiIn {
  int32_t z[2][4];
  int32_t e[2], cs[2];
  float bs[2];
  double mch[2];
  int32_t bias[2];
  float as;
};

template <int TI = 2>
__device__ __forceinline__ void mmi_epi_load(MmiEpiIn &in, int64_t bz, int64_t M, int64_t N,
                                             int64_t m0, int64_t n0, int lane,
                                             const int32_t *__restrict__ colsum,
                                             int64_t cs_bstride, const int32_t *__restrict__ ecol,
                                             const int32_t *__restrict__ azp, int64_t azp_len,
                                             const MmiEpi &o, const void *pad) {
  const int r16 = lane & 15, q = lane >> 4;
  const bool zload = azp_len > 0 && !o.azp_is_const;
  const int32_t *zp = zload ? azp : (const int32_t *)pad;
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      int64_t row = m0 + i * 16 + q * 4 + r;
      row = row < M ? row : M - 1;
      in.z[i][r] = zp[(zload && azp_len > 1) ? row : 0];
    }
  const bool fy = o.yf != nullptr;
  in.as = (fy ? o.a_scale : (const float *)pad)[0];
  const float *bsp = fy ? o.b_scale : (const float *)pad;
  const bool rq2 = o.rq_mode == 2, hb = rq2 && o.rq_bias != nullptr;
  const double *mp = rq2 ? o.rq_mult_ch : (const double *)pad;
  const int32_t *bp = hb ? o.rq_bias : (const int32_t *)pad;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    int64_t col = n0 + j * 16 + r16;
    col = col < N ? col : N - 1;
    in.e[j] = ecol[bz * o.ecol_bstride + col];
    in.cs[j] = colsum[bz * cs_bstride + col];
    in.bs[j] = bsp[(fy && o.b_scale_len != 1) ? col : 0];
    const int64_t ch = o.trans ? bz * N + col : col;  // output channel (requant mode 2)
    in.mch[j] = mp[rq2 ? ch : 0];
    in.bias[j] = bp[hb ? ch : 0];
  }
}

// 8-bit requantisation of one exact accumulator v (QLinearMatMul /
// QLinearConv): mode 1 rounds v * mult through binary32 as the reference's
// float path does, otherwise (v + bias) * mult_ch in double; then round half
// to even, add the output zero point and saturate.
__device__ __forceinline__ uint32_t mmi_requant(uint32_t v, double mch, double bias,
                                                const MmiEpi &o) {
  double x;
  if (o.rq_mode == 1) {
    x = (double)(float)((double)(int32_t)v * (double)o.rq_mult);
  } else {
    x = ((double)(int32_t)v + bias) * mch;
  }
  double t = rint(x) + (double)o.yzp;
  t = t < (double)o.lo ? (double)o.lo : (t > (double)o.hi ? (double)o.hi : t);
  return (uint32_t)(uint8_t)(int32_t)t;
}

// Epilogue shared by both MatMulInteger kernels: completes the row sums,
// applies the exact integer zero-point corrections and stores what `o` asks
// for (int32, the fused fp32 rescale, 8-bit requantisation).  16x16 i32
// accumulator layout: lane l holds column l%16 and rows 4*(l/16) + r.
template <int TI = 2>
__device__ __forceinline__ void mmi_epilogue(const int4v (&acc)[TI][2], int (&rsum)[TI],
                                             const MmiEpiIn &in, int a_signed, int64_t bz,
                                             int64_t M, int64_t K, int64_t N, int64_t m0,
                                             int64_t n0, int lane, int64_t azp_len,
                                             const MmiEpi &o) {
  const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < TI; t++) {
    rsum[t] += __shfl_xor(rsum[t], 16, 64);
    rsum[t] += __shfl_xor(rsum[t], 32, 64);
  }
#pragma unroll
  for (int i = 0; i < TI; i++) {
    int32_t rs[4], cm[4];
    int64_t row[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      rs[r] = __shfl(rsum[i], q * 4 + r, 64);  // lane holding that row's sum
      row[r] = m0 + i * 16 + q * 4 + r;
      const int32_t z = o.azp_is_const ? o.azp_const : (azp_len > 0 ? in.z[i][r] : 0);
      cm[r] = (a_signed ? 0 : 128) - z;
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int64_t col = n0 + j * 16 + r16;
      if (col >= N) continue;
      const uint32_t e = (uint32_t)in.e[j];
      const uint32_t cs = (uint32_t)in.cs[j];
      const float sj = in.as * in.bs[j];
      const double mch = in.mch[j], bias = (double)in.bias[j];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        if (row[r] >= M) continue;
        const uint32_t c = (uint32_t)cm[r];
        const uint32_t v = (uint32_t)acc[i][j][r] + e * (uint32_t)rs[r] + c * cs +
                           (uint32_t)K * c * e;
        const int64_t oi = o.trans ? (bz * N + col) * M + row[r] : (bz * M + row[r]) * N + col;
        if (o.y) o.y[oi] = (int32_t)v;
        if (o.yf) o.yf[oi] = (float)(int32_t)v * sj;
        if (o.yq) o.yq[oi] = (uint8_t)mmi_requant(v, mch, bias, o);
      }
    }
  }
}

// Epilogue of the row-major int32 / fp32 outputs through LDS: the exact
// zero-point corrections of mmi_epilogue, then the wave's (16 TI) x 32 tile
// parked in `tiles` (two (16 TI) x 33 arrays: int32 and fp32; 4224 TI bytes
// per wave) and stored back as 16 bytes per lane, 8 full 128-byte rows per
// instruction (the MFMA layout would write 64-byte row pieces 16 columns
// wide).  With the 8-bit output (only: the launcher sends y / yf with yq
// to mmi_epilogue) the requantised bytes go through the int32 tile and each
// lane stores 8 of them.  The caller's LDS must be free of other readers (a
// barrier after the K loop).
template <int TI = 2>
__device__ __forceinline__ void mmi_epilogue_lds(const int4v (&acc)[TI][2], int (&rsum)[TI],
                                                 const MmiEpiIn &ein, int a_signed, int64_t bz,
                                                 int64_t M, int64_t K, int64_t N, int64_t m0,
                                                 int64_t n0, int lane, int64_t azp_len,
                                                 const MmiEpi &o, uint32_t *tiles) {
  const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < TI; t++) {
    rsum[t] += __shfl_xor(rsum[t], 16, 64);
    rsum[t] += __shfl_xor(rsum[t], 32, 64);
  }
  uint32_t *ti = tiles;                          // int32 tile [16 TI][33]
  float *tf = (float *)(tiles + 16 * TI * 33);  // fp32 tile [16 TI][33]
#pragma unroll
  for (int i = 0; i < TI; i++) {
    int32_t rs[4], cm[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      rs[r] = __shfl(rsum[i], q * 4 + r, 64);
      const int32_t z = o.azp_is_const ? o.azp_const : (azp_len > 0 ? ein.z[i][r] : 0);
      cm[r] = (a_signed ? 0 : 128) - z;
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t e = (uint32_t)ein.e[j], csum = (uint32_t)ein.cs[j];
      const float sj = ein.as * ein.bs[j];
      const double mch = ein.mch[j], bias = (double)ein.bias[j];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t c = (uint32_t)cm[r];
        const uint32_t v = (uint32_t)acc[i][j][r] + e * (uint32_t)rs[r] + c * csum +
                           (uint32_t)K * c * e;
        const int at = (i * 16 + q * 4 + r) * 33 + j * 16 + r16;
        if (o.yq) {
          ti[at] = mmi_requant(v, mch, bias, o);
        } else {
          ti[at] = v;
          tf[at] = (float)(int32_t)v * sj;
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS writes, read back by its own lanes
  if (o.yq) {
    // lane l -> row 16 pass + l/4, columns 8 (l % 4) .. +7
    const int c8 = (lane & 3) * 8;
    const bool vq = n0 + 32 <= N && (N & 7) == 0 && (((uintptr_t)o.yq) & 7) == 0;
#pragma unroll
    for (int pass = 0; pass < TI; pass++) {
      const int rr = pass * 16 + (lane >> 2);
      const int64_t row = m0 + rr;
      uint32_t b[8];
#pragma unroll
      for (int u = 0; u < 8; u++) b[u] = ti[rr * 33 + c8 + u];
      if (row >= M) continue;
      const int64_t base = (bz * M + row) * N + n0 + c8;
      if (vq) {
        *(uint2 *)(o.yq + base) = make_uint2(b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24,
                                             b[4] | b[5] << 8 | b[6] << 16 | b[7] << 24);
      } else {
#pragma unroll
        for (int u = 0; u < 8; u++)
          if (n0 + c8 + u < N) o.yq[base + u] = (uint8_t)b[u];
      }
    }
    return;
  }
  // ---- stores: lane l -> row 8 pass + l/8, columns 4 (l % 8) .. +3
  const int sc0 = (lane & 7) * 4;
  const bool vec = n0 + 32 <= N && (N & 3) == 0 &&
                   ((((uintptr_t)o.y) | ((uintptr_t)o.yf)) & 15) == 0;
#pragma unroll
  for (int pass = 0; pass < 2 * TI; pass++) {
    const int rr = pass * 8 + (lane >> 3);
    const int64_t row = m0 + rr;
    uint32_t v[4];
    float f[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      v[u] = ti[rr * 33 + sc0 + u];
      f[u] = tf[rr * 33 + sc0 + u];
    }
    if (row >= M) continue;
    const int64_t base = (bz * M + row) * N + n0 + sc0;
    if (vec) {
      // non-temporal: the outputs are not read again by this kernel (at
      // [512,1024] x [1024,3072] the kernel went from 8.98 to 8.51 us)
      if (o.y)
        __builtin_nontemporal_store((u32x4){v[0], v[1], v[2], v[3]}, (u32x4 *)(o.y + base));
      if (o.yf)
        __builtin_nontemporal_store((f32x4){f[0], f[1], f[2], f[3]}, (f32x4 *)(o.yf + base));
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        if (n0 + sc0 + u >= N) continue;
        if (o.y) o.y[base + u] = (int32_t)v[u];
        if (o.yf) o.yf[base + u] = f[u];
      }
    }
  }
}

// WG tile 64 x 64 (4 waves, 2 x 2), wave tile 32 x 32 = 2 x 2 MFMA tiles of
// 16 x 16; K steps of 64.  Operand lanes: l%16 = row (A) / column (B),
// l/16 = which 16-byte quarter of the 64-k step.
__global__ __launch_bounds__(256) void k_mmi_mfma(
    const uint8_t *__restrict__ A, int a_signed, int64_t a_bstride, int64_t M, int64_t K,
    const int8_t *__restrict__ Bt, int64_t b_bstride, int64_t kpad,
    const int32_t *__restrict__ colsum, int64_t cs_bstride, const int32_t *__restrict__ ecol,
    int64_t N, const int32_t *__restrict__ azp, int64_t azp_len, MmiEpi o, int fast,
    const void *__restrict__ pad) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t bz = blockIdx.z;
  const uint8_t *Ab = A + bz * a_bstride;
  const int8_t *Bb = Bt + bz * b_bstride;
  const int64_t m0 = (int64_t)blockIdx.y * 64 + wm * 32;
  const int64_t n0 = (int64_t)blockIdx.x * 64 + wn * 32;
  const int r16 = lane & 15, q = lane >> 4;
  const uint32_t flip = a_signed ? 0u : 0x80808080u;

  int64_t arow[2], bcol[2];
  bool arok[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    arow[t] = m0 + t * 16 + r16;
    arok[t] = arow[t] < M;
    if (!arok[t]) arow[t] = M - 1;
    bcol[t] = n0 + t * 16 + r16;
    if (bcol[t] >= N) bcol[t] = N - 1;
  }
  int4v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (int4v){0, 0, 0, 0};
  int rsum[2] = {0, 0};
  MmiEpiIn ein;
  mmi_epi_load(ein, bz, M, N, m0, n0, lane, colsum, cs_bstride, ecol, azp, azp_len, o, pad);

  for (int64_t k0 = 0; k0 < kpad; k0 += 64) {
    const int64_t kq = k0 + q * 16;
    int4v av[2], bv[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      uint32_t w[4];
      if (fast) {
        // K % 16 == 0 and 16-byte aligned rows: whole quarters are in range
        // or entirely past K.
        if (kq < K) {
          const uint4 v = *(const uint4 *)(Ab + arow[t] * K + kq);
          w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else {
          w[0] = w[1] = w[2] = w[3] = flip;  // becomes 0 after the flip
        }
      } else {
#pragma unroll
        for (int d = 0; d < 4; d++) {
          uint32_t x = 0;
#pragma unroll
          for (int b = 0; b < 4; b++) {
            const int64_t kk = kq + d * 4 + b;
            const uint32_t byte = kk < K ? (uint32_t)Ab[arow[t] * K + kk] : (flip & 0xFFu);
            x |= byte << (8 * b);
          }
          w[d] = x;
        }
      }
#pragma unroll
      for (int d = 0; d < 4; d++) {
        w[d] ^= flip;
        rsum[t] = __builtin_amdgcn_sdot4((int)w[d], 0x01010101, rsum[t], false);
      }
      av[t] = (int4v){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      const uint4 bb = *(const uint4 *)(Bb + bcol[t] * kpad + kq);
      bv[t] = (int4v){(int)bb.x, (int)bb.y, (int)bb.z, (int)bb.w};
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
  }
  mmi_epilogue(acc, rsum, ein, a_signed, bz, M, K, N, m0, n0, lane, azp_len, o);
}


// MatMulInteger with LDS staging by direct global->LDS DMA
// (buffer_load_dwordx4 ... lds, 16 B per lane, no VGPR round trip).  Workgroup
// tile TM x TN, WM x (TN/32) waves, wave tile (TM/WM) x 32 of 16 x 16 MFMA
// tiles, K steps of 64 as k_mmi_mfma.  The launcher uses 32 x 64 and 64 x 64
// on 2 x 2 waves; 64 x 128 on 4 x 4 or 2 x 4 waves, 32 x 128, 64 x 64 on 4 x 2
// and 128 x 64 were all parity-green and 1-10% slower at [512,1024] x
// [1024,3072].  K moves in chunks of
// kMmiKc bytes through a two-slot ring: the next chunk is in flight while the
// current one is multiplied (every thread issues the same number of DMA
// loads per chunk, so "chunk c has landed" is vmcnt <= that number while
// chunk c+1 is pending; a barrier then publishes it, another frees its
// slot).  LDS rows hold kMmiPieces 16-byte pieces; piece c of row r is
// stored at slot c ^ (r & 15) so the 16 rows an MFMA operand read touches
// land in 16 different bank groups.  Pieces past K (or rows past M) are read
// from clamped in-range addresses and A's pieces past K zeroed when read.
// Requires K % 16 == 0 (K > 0), a 16-byte aligned A and per-batch operands
// below 2 GB (31-bit buffer offsets).
//
// TM = 32 doubles the workgroups for the same output: L2 -> LDS streaming
// rises with the waves per CU (three 48 KB workgroups fit a CU where two
// 64 KB ones did), which outweighs re-reading B twice as often.
constexpr int kMmiKc = 256;
constexpr int kMmiPieces = kMmiKc / 16;  // per row

template <bool LDS_EPI, int TM, int TN, int WM>
__global__ __launch_bounds__(64 * WM * (TN / 32)) void k_mmi_lds(
    const uint8_t *__restrict__ A, int a_signed, int64_t a_bstride, int64_t M, int64_t K,
    const int8_t *__restrict__ Bt, int64_t b_bstride, int64_t kpad,
    const int32_t *__restrict__ colsum, int64_t cs_bstride, const int32_t *__restrict__ ecol,
    int64_t N, const int32_t *__restrict__ azp, int64_t azp_len, MmiEpi o,
    const uint8_t *__restrict__ pad) {
  constexpr int WN = TN / 32;                      // waves across the tile's columns
  constexpr int NW = WM * WN;                      // waves per workgroup
  constexpr int TI = TM / (16 * WM);               // 16-row blocks per wave
  constexpr int kSA = TM * kMmiPieces;             // uint4 per A slot
  constexpr int kSB = TN * kMmiPieces;             // uint4 per B slot
  constexpr int kLoads = (kSA + kSB) / 64 / NW;    // DMA loads per thread per chunk
  static_assert(TI >= 1 && TM == 16 * TI * WM, "wave rows");
  static_assert((kSA / 64) % NW == 0 && (kSB / 64) % NW == 0, "whole DMA rounds per wave");
  // one array: the A ring (two slots of kSA) then the B ring (two of kSB),
  // which the LDS epilogue reuses whole
  __shared__ uint4 smem[2 * (kSA + kSB)];
  uint4 *sA0 = smem, *sB0 = smem + 2 * kSA;
  // the operand arguments in SGPRs up front (one round of scalar loads)
  kernarg_fence(A, a_signed, a_bstride, M, K, Bt, b_bstride, kpad, colsum, cs_bstride, ecol, N,
                azp, azp_len);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t bz = blockIdx.z;
  const uint8_t *Ab = A + bz * a_bstride;
  const int8_t *Bb = Bt + bz * b_bstride;
  const int64_t m0 = (int64_t)blockIdx.y * TM + wm * (16 * TI);
  const int64_t n0 = (int64_t)blockIdx.x * TN + wn * 32;
  const int64_t mt0 = (int64_t)blockIdx.y * TM, nt0 = (int64_t)blockIdx.x * TN;
  const int r16 = lane & 15, q = lane >> 4;
  const uint32_t flip = a_signed ? 0u : 0x80808080u;
  const int nchunks = (int)((kpad + kMmiKc - 1) / kMmiKc);
  // the operands as buffer resources (the launcher keeps every offset below
  // 2^31): DMA through buffer_load_dwordx4 ... lds, which the compiler
  // counts on vmcnt only.  Through global_load_lds it waited vmcnt(0) before
  // every step's LDS reads, i.e. for the next chunk's DMA too, so a
  // workgroup never overlapped a chunk's MFMAs with the next chunk's DMA.
  const __amdgpu_buffer_rsrc_t a_rs = buf_rsrc(Ab);
  const __amdgpu_buffer_rsrc_t b_rs = buf_rsrc(Bb);

  // DMA of chunk c into slot s: instruction i of a wave fills LDS slots
  // [64 i, 64 i + 64) of an operand.  Pieces past K (A) or past kpad (B),
  // and rows past M, read clamped in-range bytes: A pieces past K are zeroed
  // when read (so neither the products nor the row sums see them), which
  // also cancels whatever B holds there; rows past M feed only rows that are
  // not stored.
  auto issue = [&](int c, int s) {
    const int64_t k0 = (int64_t)c * kMmiKc;
#pragma unroll
    for (int u = 0; u < kSA / 64 / NW; u++) {
      const int i = wave + NW * u;
      const int slot = i * 64 + lane;
      const int r = slot / kMmiPieces, cs_ = slot % kMmiPieces;
      const int64_t kk = min(k0 + (int64_t)(cs_ ^ (r & 15)) * 16, K - 16);
      const int64_t arow = min(mt0 + r, M - 1);
      dma16_buf(a_rs, (uint32_t)(arow * K + kk), 0u, sA0 + s * kSA + i * 64);
    }
#pragma unroll
    for (int u = 0; u < kSB / 64 / NW; u++) {
      const int i = wave + NW * u;
      const int slot = i * 64 + lane;
      const int r = slot / kMmiPieces, cs_ = slot % kMmiPieces;
      const int64_t kk = min(k0 + (int64_t)(cs_ ^ (r & 15)) * 16, kpad - 16);
      const int64_t bcol = min(nt0 + r, N - 1);
      dma16_buf(b_rs, (uint32_t)(bcol * kpad + kk), 0u, sB0 + s * kSB + i * 64);
    }
  };

  int4v acc[TI][2];
#pragma unroll
  for (int i = 0; i < TI; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (int4v){0, 0, 0, 0};
  int rsum[TI];
#pragma unroll
  for (int i = 0; i < TI; i++) rsum[i] = 0;
  // issued before the first chunk, so the chunk waits below cover them too
  MmiEpiIn ein;
  mmi_epi_load<TI>(ein, bz, M, N, m0, n0, lane, colsum, cs_bstride, ecol, azp, azp_len, o, pad);

  issue(0, 0);
  if (nchunks > 1) issue(1, 1);
  for (int c = 0; c < nchunks; c++) {
    const int s = c & 1;
    if (c + 1 < nchunks)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kLoads));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    const uint4 *sA = sA0 + s * kSA, *sB = sB0 + s * kSB;
    const int64_t kc = kpad - (int64_t)c * kMmiKc < kMmiKc ? kpad - (int64_t)c * kMmiKc
                                                            : kMmiKc;  // multiple of 64
    // chunks reaching past K zero the A pieces there (clamped DMA sources)
    const bool tail = (int64_t)(c + 1) * kMmiKc > K;
    for (int st = 0; st < kc / 64; st++) {
      int4v av[TI], bv[2];
      uint32_t keep = ~0u;
      if (tail) keep = (int64_t)c * kMmiKc + (st * 4 + q) * 16 < K ? ~0u : 0u;
      // LDS reads as vector-type loads: read through the uint4 struct the
      // compiler put vmcnt(0) (a wait for every outstanding DMA, the next
      // chunk's too) before each step's reads; the ring's own vmcnt waits
      // and barriers already order these reads after their chunk's DMA
      const u32x4 *sAv = (const u32x4 *)sA, *sBv = (const u32x4 *)sB;
#pragma unroll
      for (int t = 0; t < TI; t++) {
        const int ra = wm * (16 * TI) + t * 16 + r16;
        const u32x4 x = sAv[ra * kMmiPieces + ((st * 4 + q) ^ (ra & 15))];
        uint32_t w[4] = {(x.x ^ flip) & keep, (x.y ^ flip) & keep, (x.z ^ flip) & keep,
                         (x.w ^ flip) & keep};
#pragma unroll
        for (int d = 0; d < 4; d++)
          rsum[t] = __builtin_amdgcn_sdot4((int)w[d], 0x01010101, rsum[t], false);
        av[t] = (int4v){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      }
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int rb = wn * 32 + t * 16 + r16;
        const u32x4 y = sBv[rb * kMmiPieces + ((st * 4 + q) ^ (rb & 15))];
        bv[t] = (int4v){(int)y.x, (int)y.y, (int)y.z, (int)y.w};
      }
#pragma unroll
      for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (c + 2 < nchunks) {
      __builtin_amdgcn_s_barrier();  // every wave is done with slot s
      issue(c + 2, s);
    }
  }
  if constexpr (LDS_EPI) {
    static_assert(NW * 2 * 16 * TI * 33 * 4 <= (int)sizeof(smem), "epilogue tiles fit the ring");
    __syncthreads();  // the ring is free: it holds the output tiles now
    mmi_epilogue_lds<TI>(acc, rsum, ein, a_signed, bz, M, K, N, m0, n0, lane, azp_len, o,
                         (uint32_t *)smem + wave * 2 * 16 * TI * 33);
  } else {
    mmi_epilogue<TI>(acc, rsum, ein, a_signed, bz, M, K, N, m0, n0, lane, azp_len, o);
  }
}

int launch_matmul_integer(mmnb_ctx *ctx, const mmnb_pack *p, const void *d_a, int a_signed,
                          int64_t a_batch, int64_t m, const int32_t *d_azp, int64_t azp_len,
                          const MmiEpi &out) {
  const int64_t batch = a_batch > p->batch ? a_batch : p->batch;
  const int64_t k = p->k, n = p->n;
  if (!out.y && !out.yf && !out.yq) return fail(MMNB_ERR_ARG, "MatMulInteger: no output");
  MmiEpi o = out;
  o.ecol_bstride = p->ecol_bstride;
  if (m <= 0 || n <= 0 || batch <= 0) return MMNB_OK;
  // the LDS-staged kernel: K a multiple of 16, a 16-byte aligned A, and
  // per-batch operands small enough for 31-bit buffer offsets
  const int fast = k > 0 && (k % 16 == 0) && ((((uintptr_t)d_a) & 15) == 0) &&
                   m * k < ((int64_t)1 << 31) && n * p->kpad < ((int64_t)1 << 31);
  const dim3 grid((unsigned)((n + 63) / 64), (unsigned)((m + 63) / 64), (unsigned)batch);
  if (fast && ctx->d_pad) {
    // 32-row tiles when 64-row ones would leave fewer than three workgroups
    // per CU (tuning override: MMNB_MMI_TM)
    const int64_t tiles64 = (int64_t)grid.x * grid.y * grid.z;
    const int tm = ctx->mmi_tm ? ctx->mmi_tm : (tiles64 < 3 * (int64_t)ctx->cu_count ? 32 : 64);
    // the LDS epilogue: row-major outputs, the 8-bit one only on its own
    const bool le = !o.trans && (!o.yq || (!o.y && !o.yf));
    auto kern = le ? k_mmi_lds<true, 64, 64, 2> : k_mmi_lds<false, 64, 64, 2>;
    dim3 g = grid;
    if (tm == 32) {
      kern = le ? k_mmi_lds<true, 32, 64, 2> : k_mmi_lds<false, 32, 64, 2>;
      g.y = (unsigned)((m + 31) / 32);
    }
    return launch(ctx, kKernMmi, kern, g, dim3(256), 0, (const uint8_t *)d_a, a_signed,
                  a_batch == 1 ? (int64_t)0 : m * k, m, k, (const int8_t *)p->d_bt,
                  p->batch == 1 ? (int64_t)0 : n * p->kpad, p->kpad,
                  (const int32_t *)p->d_colsum, p->batch == 1 ? (int64_t)0 : n,
                  (const int32_t *)p->d_ecol, n, d_azp, azp_len, o,
                  (const uint8_t *)ctx->d_pad);
  }
  return launch(ctx, kKernMmi, k_mmi_mfma, grid, dim3(256), 0, (const uint8_t *)d_a, a_signed,
                a_batch == 1 ? (int64_t)0 : m * k, m, k, (const int8_t *)p->d_bt,
                p->batch == 1 ? (int64_t)0 : n * p->kpad, p->kpad, (const int32_t *)p->d_colsum,
                p->batch == 1 ? (int64_t)0 : n, (const int32_t *)p->d_ecol, n, d_azp, azp_len, o,
                fast, (const void *)ctx->d_pad);
}

// ---------------------------------------------------------------------------
// Platform calibration: an empty kernel, and a streaming read with four
// independent 16-byte non-temporal loads per thread (bounds-checked) whose
// xor is kept live by a never-taken store.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_probe_empty(int *sink, unsigned key) {
  if (threadIdx.x == key) sink[0] = 1;  // key is out of range: never stores
}

__global__ __launch_bounds__(256) void k_probe_read(const uint4 *__restrict__ p, size_t n16,
                                                    int *sink, unsigned key) {
  const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
  uint4 v[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const size_t i = base + (size_t)u * 256;
    // non-temporal, as the GEMVs read their weights (the faster way to
    // stream bytes read once: 8.95 MB back to back 3.33 -> 3.04 us, 134 MB
    // 23.4 -> 21.4 us)
    const u32x4 x = __builtin_nontemporal_load((const u32x4 *)(p + (i < n16 ? i : 0)));
    v[u] = i < n16 ? make_uint4(x.x, x.y, x.z, x.w) : make_uint4(0, 0, 0, 0);
  }
  unsigned x = 0;
#pragma unroll
  for (int u = 0; u < 4; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (x == key) sink[0] = (int)x;  // practically never; keeps the loads live
}

int launch_probe_empty(mmnb_ctx *ctx, int blocks) {
  return launch(ctx, kKernProbeEmpty, k_probe_empty, dim3((unsigned)blocks), dim3(256), 0,
                (int *)((char *)ctx->d_pad + 2048), 4096u);
}

int launch_probe_read(mmnb_ctx *ctx, const void *d_buf, size_t bytes) {
  const size_t n16 = bytes / 16;
  const size_t grid = (n16 + 1023) / 1024;
  return launch(ctx, kKernProbeRead, k_probe_read, dim3((unsigned)grid), dim3(256), 0,
                (const uint4 *)d_buf, n16, (int *)((char *)ctx->d_pad + 2048), 0x9E3779B9u);
}

}  // namespace mmnb
