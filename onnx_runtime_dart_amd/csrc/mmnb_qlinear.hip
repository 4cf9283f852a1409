// QLinearMatMul, ConvInteger and QLinearConv on the MatMulInteger kernels.
//
// QLinearMatMul (onnx_qlinear_ops.dart:83-106) is MatMulInteger with an
// 8-bit requantising epilogue.  A convolution (:157-308) runs as one
// MatMulInteger per image: an im2col pass writes A[g][p][kc] (p an output
// position, kc = (c*kh + ky)*kw + kx, out-of-image taps set to the input zero
// point so that (x - x_zp) = 0 there, which is the reference's skipping of
// them), the weight w[m][c/g][kh][kw] is a MatMulInteger pack of B^T per
// group (batch = group), and the epilogue stores channel-major
// y[m][oy][ox] directly (MmiEpi::trans), requantising per output channel for
// QLinearConv.
#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

#include "mmnb_internal.h"

using namespace mmnb;

namespace mmnb {

// One image: x [C][H][W] bytes -> out [groups][oh*ow][cg*kh*kw].  Grid
// (items / 256, groups); 32-bit index arithmetic (the host checks that
// groups * oh*ow * cg*kh*kw fits); the source index is clamped so every load
// is in bounds.
__global__ __launch_bounds__(256) void k_im2col(const uint8_t *__restrict__ x, int H, int W,
                                                int cg, int kh, int kw, int ow, int sh, int sw,
                                                int ph, int pw, int dh, int dw, uint32_t zp,
                                                int items, int per, uint8_t *__restrict__ out) {
  // the group's output [P][kcn] is contiguous: thread item i owns bytes
  // per*i .. per*i + per - 1 of it (per = 4 when kcn % 4 == 0, one 32-bit
  // store; else 1), all of whose source bytes are loaded before any store
  const unsigned item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (unsigned)items) return;
  const int g = blockIdx.y;
  const int kcn = cg * kh * kw, khw = kh * kw;
  const int e0 = (int)item * per;
  const int p = e0 / kcn, kc0 = e0 - p * kcn;
  const int oy = p / ow, ox = p - oy * ow;
  uint32_t v[4];
  bool in[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int kc = kc0 + (u < per ? u : 0);
    const int c = kc / khw, r = kc - c * khw;
    const int ky = r / kw, kx = r - ky * kw;
    const int iy = oy * sh - ph + ky * dh, ix = ox * sw - pw + kx * dw;
    in[u] = iy >= 0 && iy < H && ix >= 0 && ix < W;
    v[u] = x[((size_t)(g * cg + c) * H + (in[u] ? iy : 0)) * W + (in[u] ? ix : 0)];
  }
  uint8_t *o = out + (size_t)g * items * per + e0;
  if (per == 4) {
    uint32_t word = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) word |= (in[u] ? v[u] : zp) << (8 * u);
    *(uint32_t *)o = word;
  } else {
    o[0] = (uint8_t)(in[0] ? v[0] : zp);
  }
}

}  // namespace mmnb

namespace {

struct ConvShape {
  int64_t n, c, h, w, oh, ow;
  int sh, sw, ph, pw, dh, dw;
};

// Output size per axis, `(in + pad_begin + pad_end - window) ~/ stride + 1`
// (onnx_qlinear_ops.dart:222-231); strides, dilations >= 1, pads >= 0.
int conv_shape(const mmnb_pack *p, int64_t n, int64_t c, int64_t h, int64_t w,
               const mmnb_conv_params *prm, ConvShape *s) {
  if (!p || p->kind != kPackConv) return fail(MMNB_ERR_ARG, "conv: not a convolution pack");
  if (!prm) return fail(MMNB_ERR_ARG, "conv: null parameters");
  if (n < 0 || h < 1 || w < 1) return fail(MMNB_ERR_ARG, "conv: bad input shape");
  if (c != p->conv_cg * p->conv_group)
    return fail(MMNB_ERR_ARG, "conv: input channels != weight channels * group");
  for (int a = 0; a < 2; a++)
    if (prm->strides[a] < 1 || prm->dilations[a] < 1)
      return fail(MMNB_ERR_ARG, "conv: strides and dilations must be >= 1");
  for (int a = 0; a < 4; a++)
    if (prm->pads[a] < 0) return fail(MMNB_ERR_ARG, "conv: negative pad");
  const int64_t kdim[2] = {p->conv_kh, p->conv_kw}, in[2] = {h, w};
  int64_t out[2];
  for (int a = 0; a < 2; a++) {
    const int64_t window = prm->dilations[a] * (kdim[a] - 1) + 1;
    const int64_t span = in[a] + prm->pads[a] + prm->pads[2 + a] - window;
    if (span < 0) return fail(MMNB_ERR_ARG, "conv: kernel window larger than the padded input");
    out[a] = span / prm->strides[a] + 1;
  }
  if (prm->strides[0] > INT32_MAX || prm->strides[1] > INT32_MAX ||
      prm->pads[0] > INT32_MAX || prm->pads[1] > INT32_MAX ||
      prm->dilations[0] > INT32_MAX || prm->dilations[1] > INT32_MAX)
    return fail(MMNB_ERR_UNSUPPORTED, "conv: parameter beyond int32");
  *s = ConvShape{n, c, h, w, out[0], out[1], (int)prm->strides[0], (int)prm->strides[1],
                 (int)prm->pads[0], (int)prm->pads[1], (int)prm->dilations[0],
                 (int)prm->dilations[1]};
  return MMNB_OK;
}

int check_zp(int64_t v, int is_signed, const char *what) {
  const int64_t lo = is_signed ? -128 : 0, hi = is_signed ? 127 : 255;
  if (v < lo || v > hi) return fail(MMNB_ERR_ARG, std::string(what) + " out of range");
  return MMNB_OK;
}

// Device side of a convolution: per image, im2col then the MatMulInteger
// kernel with a channel-major epilogue.  `o` carries the output pointers of
// image 0; each image's output follows the previous one's m*oh*ow values.
// Scratch: slot 6 = im2col.
int conv_run(mmnb_ctx *ctx, const mmnb_pack *p, const uint8_t *d_x, int x_signed,
             const ConvShape &s, int64_t x_zp, MmiEpi o) {
  const int64_t P = s.oh * s.ow, kcn = p->k, g = p->conv_group, m = p->conv_m;
  if (s.n == 0 || P == 0) return MMNB_OK;
  if (kcn > 65535 * 256 || g > 65535 || g * P * kcn > INT32_MAX ||
      s.c * s.h * s.w > INT32_MAX)
    return fail(MMNB_ERR_UNSUPPORTED, "conv: image too large for one launch");
  void *d_col = nullptr;
  int rc;
  if ((rc = scratch_get(ctx, 6, (size_t)(g * P * kcn) + 256, &d_col))) return rc;
  o.azp_is_const = 1;
  o.azp_const = (int32_t)x_zp;
  const uint32_t zbyte = (uint32_t)(x_zp & 0xFF);
  // 4 bytes per thread when the rows are whole dwords (the scratch buffer
  // is 256-byte aligned, so then every dword is aligned)
  const int per = kcn % 4 == 0 ? 4 : 1;
  const int items = (int)(P * kcn / per);
  const dim3 grid((unsigned)((items + 255) / 256), (unsigned)g);
  for (int64_t b = 0; b < s.n; b++) {
    const uint8_t *xb = d_x + b * s.c * s.h * s.w;
    if ((rc = launch(ctx, kKernIm2col, k_im2col, grid, dim3(256), 0, xb, (int)s.h, (int)s.w,
                     (int)p->conv_cg, (int)p->conv_kh, (int)p->conv_kw, (int)s.ow, s.sh, s.sw,
                     s.ph, s.pw, s.dh, s.dw, zbyte, items, per, (uint8_t *)d_col)))
      return rc;
    MmiEpi ob = o;
    ob.trans = 1;
    const int64_t off = b * m * P;
    if (o.y) ob.y = o.y + off;
    if (o.yq) ob.yq = o.yq + off;
    if ((rc = launch_matmul_integer(ctx, p, d_col, x_signed, g, P, (const int32_t *)ctx->d_pad,
                                    1, ob)))
      return rc;
  }
  return MMNB_OK;
}

}  // namespace

// -------------------------------------------------------------- QLinearMatMul

// mult = fl32(fl32(a_scale * b_scale) / y_scale), the reference's two
// binary32 roundings (onnx_qlinear_ops.dart:93-96).
static int qmm_mult(float a_scale, float b_scale, float y_scale, float *mult) {
  if (!std::isfinite(a_scale) || !std::isfinite(b_scale) || !std::isfinite(y_scale) ||
      y_scale == 0.0f)
    return fail(MMNB_ERR_ARG, "QLinearMatMul: scales must be finite and y_scale non-zero");
  const float ab = (float)((double)a_scale * (double)b_scale);
  *mult = (float)((double)ab / (double)y_scale);
  if (!std::isfinite(*mult)) return fail(MMNB_ERR_ARG, "QLinearMatMul: multiplier overflows");
  return MMNB_OK;
}

static int qmm_check(mmnb_ctx *ctx, const mmnb_pack *p, int64_t a_batch, int64_t m,
                     int64_t azl) {
  if (!p || p->kind != kPackInteger)
    return fail(MMNB_ERR_ARG, "QLinearMatMul: not a MatMulInteger pack");
  if (p->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if (a_batch < 1 || m < 0) return fail(MMNB_ERR_ARG, "QLinearMatMul: bad A shape");
  if (azl != 0 && azl != 1 && azl != m)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                "per-column [N] for B");
  const int64_t batch = a_batch > p->batch ? a_batch : p->batch;
  if ((a_batch != batch && a_batch != 1) || (p->batch != batch && p->batch != 1))
    return fail(MMNB_ERR_ARG, "MatMulInteger batch mismatch");
  return MMNB_OK;
}

int mmnb_qlinear_matmul_dev(mmnb_ctx *ctx, const mmnb_pack *pack, const void *d_a,
                            int a_is_signed, int64_t a_batch, int64_t m,
                            const int32_t *d_a_zero_point, int64_t a_zero_point_len,
                            float a_scale, float b_scale, float y_scale, int64_t y_zero_point,
                            int y_is_signed, void *d_y) {
  MMNB_GUARD_CTX(ctx);
  const int64_t azl = d_a_zero_point ? a_zero_point_len : 0;
  int rc = qmm_check(ctx, pack, a_batch, m, azl);
  if (rc) return rc;
  float mult;
  if ((rc = qmm_mult(a_scale, b_scale, y_scale, &mult))) return rc;
  if ((rc = check_zp(y_zero_point, y_is_signed, "QLinearMatMul: y zero point"))) return rc;
  if (m == 0) return MMNB_OK;
  if (!d_y || (!d_a && pack->k > 0)) return fail(MMNB_ERR_ARG, "QLinearMatMul: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  MmiEpi o;
  o.yq = (uint8_t *)d_y;
  o.rq_mode = 1;
  o.rq_mult = mult;
  o.yzp = (int32_t)y_zero_point;
  o.lo = y_is_signed ? -128 : 0;
  o.hi = y_is_signed ? 127 : 255;
  return launch_matmul_integer(ctx, pack, d_a, a_is_signed ? 1 : 0, a_batch, m, d_a_zero_point,
                               azl, o);
}

int mmnb_qlinear_matmul(mmnb_ctx *ctx, const mmnb_pack *pack, const void *a, int a_is_signed,
                        int64_t a_batch, int64_t m, const int64_t *a_zero_point,
                        int64_t a_zero_point_len, float a_scale, float b_scale, float y_scale,
                        int64_t y_zero_point, int y_is_signed, void *y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  const int64_t azl = a_zero_point ? a_zero_point_len : 0;
  int rc = qmm_check(ctx, pack, a_batch, m, azl);
  if (rc) return rc;
  float mult;
  if ((rc = qmm_mult(a_scale, b_scale, y_scale, &mult))) return rc;
  if ((rc = check_zp(y_zero_point, y_is_signed, "QLinearMatMul: y zero point"))) return rc;
  if (m == 0) return MMNB_OK;
  if (!y || (!a && pack->k > 0)) return fail(MMNB_ERR_ARG, "QLinearMatMul: null buffer");
  std::vector<int32_t> az((size_t)(azl ? azl : 1));
  for (int64_t i = 0; i < azl; i++) {
    if ((rc = check_zp(a_zero_point[i], a_is_signed, "QLinearMatMul: A zero point"))) return rc;
    az[(size_t)i] = (int32_t)a_zero_point[i];
  }
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  const int64_t k = pack->k, n = pack->n;
  const int64_t batch = a_batch > pack->batch ? a_batch : pack->batch;
  void *d_a = nullptr, *d_y = nullptr, *d_az = nullptr;
  if ((rc = scratch_get(ctx, 0, (size_t)(a_batch * m * k) + 256, &d_a))) return rc;
  if ((rc = scratch_get(ctx, 1, (size_t)(batch * m * n), &d_y))) return rc;
  if ((rc = scratch_get(ctx, 5, az.size() * 4, &d_az))) return rc;
  if (a_batch * m * k)
    MMNB_HIP(hipMemcpyAsync(d_a, a, (size_t)(a_batch * m * k), hipMemcpyHostToDevice,
                            ctx->stream));
  if (azl)
    MMNB_HIP(hipMemcpyAsync(d_az, az.data(), (size_t)azl * 4, hipMemcpyHostToDevice,
                            ctx->stream));
  MmiEpi o;
  o.yq = (uint8_t *)d_y;
  o.rq_mode = 1;
  o.rq_mult = mult;
  o.yzp = (int32_t)y_zero_point;
  o.lo = y_is_signed ? -128 : 0;
  o.hi = y_is_signed ? 127 : 255;
  if ((rc = launch_matmul_integer(ctx, pack, d_a, a_is_signed ? 1 : 0, a_batch, m,
                                  azl ? (const int32_t *)d_az : nullptr, azl, o)))
    return rc;
  MMNB_HIP(hipMemcpyAsync(y, d_y, (size_t)(batch * m * n), hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}

// ------------------------------------------------------------- convolutions

int mmnb_pack_conv(mmnb_ctx *ctx, const void *w, int w_is_signed, int64_t m,
                   int64_t c_per_group, int64_t kh, int64_t kw, int64_t group,
                   const int64_t *w_zero_point, int64_t w_zero_point_len, mmnb_pack **out) {
  MMNB_GUARD_CTX(ctx);
  if (!out) return fail(MMNB_ERR_ARG, "mmnb_pack_conv: out is null");
  *out = nullptr;
  if (m < 1 || c_per_group < 1 || kh < 1 || kw < 1 || group < 1)
    return fail(MMNB_ERR_ARG, "conv: bad weight shape");
  if (m % group) return fail(MMNB_ERR_ARG, "conv: output channels not divisible by group");
  if (!w) return fail(MMNB_ERR_ARG, "conv: weight is null");
  const int64_t wzl = w_zero_point ? w_zero_point_len : 0;
  if (wzl != 0 && wzl != 1 && wzl != m)
    return fail(MMNB_ERR_UNSUPPORTED,
                "ConvInteger: weight zero point must be scalar or per-output-channel");
  const int64_t k = c_per_group * kh * kw, n = m / group;
  if (k > 33025) return fail(MMNB_ERR_UNSUPPORTED, "conv: c/group*kh*kw > 33025 may overflow int32");
  std::vector<int32_t> zp((size_t)(wzl ? wzl : 1));
  int rc;
  for (int64_t i = 0; i < wzl; i++) {
    if ((rc = check_zp(w_zero_point[i], w_is_signed, "conv: weight zero point"))) return rc;
    zp[(size_t)i] = (int32_t)w_zero_point[i];
  }
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  mmnb_pack *p = new (std::nothrow) mmnb_pack();
  if (!p) return fail(MMNB_ERR_OOM, "out of host memory");
  p->ctx = ctx;
  p->kind = kPackConv;
  p->batch = group;
  p->k = k;
  p->n = n;
  p->kpad = (k + 63) / 64 * 64;
  p->b_signed = w_is_signed ? 1 : 0;
  p->conv_m = m;
  p->conv_cg = c_per_group;
  p->conv_kh = kh;
  p->conv_kw = kw;
  p->conv_group = group;
  // per-channel zero points differ between groups: one offset per (group, column)
  const bool per_batch = wzl == m && m != 1 && group > 1;
  p->ecol_bstride = per_batch ? n : 0;
  auto cleanup = [&](int code) {
    if (p->d_bt) (void)hipFree(p->d_bt);
    if (p->d_colsum) (void)hipFree(p->d_colsum);
    if (p->d_ecol) (void)hipFree(p->d_ecol);
    delete p;
    return code;
  };
  const size_t bt_bytes = (size_t)(group * n * p->kpad);
  if ((rc = device_alloc(bt_bytes, (void **)&p->d_bt))) return cleanup(rc);
  if ((rc = device_alloc((size_t)(group * n) * 4, (void **)&p->d_colsum))) return cleanup(rc);
  if ((rc = device_alloc((size_t)(per_batch ? m : n) * 4, (void **)&p->d_ecol)))
    return cleanup(rc);
  const size_t raw_bytes = (size_t)(m * k);
  void *d_raw = nullptr, *d_zp = nullptr;
  if ((rc = scratch_get(ctx, 4, raw_bytes + 256, &d_raw))) return cleanup(rc);
  if ((rc = scratch_get(ctx, 5, zp.size() * 4, &d_zp))) return cleanup(rc);
  hipError_t e;
  if ((e = hipMemcpyAsync(d_raw, w, raw_bytes, hipMemcpyHostToDevice, ctx->stream)) !=
      hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(w)"));
  if (wzl && (e = hipMemcpyAsync(d_zp, zp.data(), (size_t)wzl * 4, hipMemcpyHostToDevice,
                                 ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(w_zp)"));
  // zero points per (group, column) are the flat per-channel list
  if ((rc = prepare_integer_b(ctx, (const uint8_t *)d_raw, p->b_signed, 1, group, k, n, p->kpad,
                              (const int32_t *)d_zp, wzl,
                              p->d_bt, p->d_colsum, p->d_ecol)))
    return cleanup(rc);
  if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipStreamSynchronize(pack)"));
  p->bytes = (int64_t)bt_bytes + group * n * 4 + (per_batch ? m : n) * 4;
  ctx->live_packs++;
  *out = p;
  return MMNB_OK;
}

int mmnb_conv_output_shape(const mmnb_pack *w, int64_t n, int64_t c, int64_t h, int64_t wd,
                           const mmnb_conv_params *prm, int64_t *oh, int64_t *ow) {
  ConvShape s;
  int rc = conv_shape(w, n, c, h, wd, prm, &s);
  if (rc) return rc;
  if (oh) *oh = s.oh;
  if (ow) *ow = s.ow;
  return MMNB_OK;
}

int mmnb_conv_integer_dev(mmnb_ctx *ctx, const mmnb_pack *w, const void *d_x, int x_is_signed,
                          int64_t n, int64_t c, int64_t h, int64_t wd, int64_t x_zero_point,
                          const mmnb_conv_params *prm, int32_t *d_y) {
  MMNB_GUARD_CTX(ctx);
  ConvShape s;
  int rc = conv_shape(w, n, c, h, wd, prm, &s);
  if (rc) return rc;
  if (w->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if ((rc = check_zp(x_zero_point, x_is_signed, "ConvInteger: x zero point"))) return rc;
  if (!d_x || !d_y) return fail(MMNB_ERR_ARG, "ConvInteger: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  MmiEpi o;
  o.y = d_y;
  return conv_run(ctx, w, (const uint8_t *)d_x, x_is_signed ? 1 : 0, s, x_zero_point, o);
}

int mmnb_conv_integer(mmnb_ctx *ctx, const mmnb_pack *w, const void *x, int x_is_signed,
                      int64_t n, int64_t c, int64_t h, int64_t wd, int64_t x_zero_point,
                      const mmnb_conv_params *prm, int32_t *y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  ConvShape s;
  int rc = conv_shape(w, n, c, h, wd, prm, &s);
  if (rc) return rc;
  if (w->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if ((rc = check_zp(x_zero_point, x_is_signed, "ConvInteger: x zero point"))) return rc;
  if (!x || !y) return fail(MMNB_ERR_ARG, "ConvInteger: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  const size_t xb = (size_t)(n * c * h * wd), yn = (size_t)(n * w->conv_m * s.oh * s.ow);
  void *d_x = nullptr, *d_y = nullptr;
  if ((rc = scratch_get(ctx, 0, xb + 256, &d_x))) return rc;
  if ((rc = scratch_get(ctx, 1, yn * 4, &d_y))) return rc;
  if (xb) MMNB_HIP(hipMemcpyAsync(d_x, x, xb, hipMemcpyHostToDevice, ctx->stream));
  MmiEpi o;
  o.y = (int32_t *)d_y;
  if ((rc = conv_run(ctx, w, (const uint8_t *)d_x, x_is_signed ? 1 : 0, s, x_zero_point, o)))
    return rc;
  if (yn) MMNB_HIP(hipMemcpyAsync(y, d_y, yn * 4, hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}

// Per-channel requantisation parameters of QLinearConv, in double as the
// reference computes them (onnx_qlinear_ops.dart:295-305): mult[c] =
// x_scale * w_scale[c] / y_scale, bias[c] (int32, optional).  Written to
// scratch slot 8 as [m doubles][m int32].
static int qconv_params(mmnb_ctx *ctx, int64_t m, float x_scale, const float *w_scale,
                        int64_t w_scale_len, float y_scale, const int32_t *bias,
                        const double **d_mult, const int32_t **d_bias) {
  if (!w_scale || (w_scale_len != 1 && w_scale_len != m))
    return fail(MMNB_ERR_ARG, "QLinearConv: w_scale must have 1 or M values");
  if (!std::isfinite(x_scale) || !std::isfinite(y_scale) || y_scale == 0.0f)
    return fail(MMNB_ERR_ARG, "QLinearConv: scales must be finite and y_scale non-zero");
  std::vector<char> buf((size_t)m * 12);
  double *mult = (double *)buf.data();
  int32_t *bb = (int32_t *)(buf.data() + m * 8);
  for (int64_t c = 0; c < m; c++) {
    const double ws = (double)w_scale[w_scale_len == 1 ? 0 : c];
    mult[c] = (double)x_scale * ws / (double)y_scale;
    if (!std::isfinite(mult[c])) return fail(MMNB_ERR_ARG, "QLinearConv: non-finite scale");
    bb[c] = bias ? bias[c] : 0;
  }
  void *d = nullptr;
  int rc = scratch_get(ctx, 8, buf.size(), &d);
  if (rc) return rc;
  MMNB_HIP(hipMemcpyAsync(d, buf.data(), buf.size(), hipMemcpyHostToDevice, ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));  // `buf` is about to go away
  *d_mult = (const double *)d;
  *d_bias = bias ? (const int32_t *)((char *)d + m * 8) : nullptr;
  return MMNB_OK;
}

int mmnb_qlinear_conv_dev(mmnb_ctx *ctx, const mmnb_pack *w, const void *d_x, int x_is_signed,
                          int64_t n, int64_t c, int64_t h, int64_t wd, int64_t x_zero_point,
                          float x_scale, const float *w_scale, int64_t w_scale_len,
                          float y_scale, int64_t y_zero_point, int y_is_signed,
                          const int32_t *bias, const mmnb_conv_params *prm, void *d_y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "QLinearConv uploads its parameters: not capturable");
  ConvShape s;
  int rc = conv_shape(w, n, c, h, wd, prm, &s);
  if (rc) return rc;
  if (w->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if ((rc = check_zp(x_zero_point, x_is_signed, "QLinearConv: x zero point"))) return rc;
  if ((rc = check_zp(y_zero_point, y_is_signed, "QLinearConv: y zero point"))) return rc;
  if (!d_x || !d_y) return fail(MMNB_ERR_ARG, "QLinearConv: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  MmiEpi o;
  if ((rc = qconv_params(ctx, w->conv_m, x_scale, w_scale, w_scale_len, y_scale, bias,
                         &o.rq_mult_ch, &o.rq_bias)))
    return rc;
  o.yq = (uint8_t *)d_y;
  o.rq_mode = 2;
  o.yzp = (int32_t)y_zero_point;
  o.lo = y_is_signed ? -128 : 0;
  o.hi = y_is_signed ? 127 : 255;
  return conv_run(ctx, w, (const uint8_t *)d_x, x_is_signed ? 1 : 0, s, x_zero_point, o);
}

int mmnb_qlinear_conv(mmnb_ctx *ctx, const mmnb_pack *w, const void *x, int x_is_signed,
                      int64_t n, int64_t c, int64_t h, int64_t wd, int64_t x_zero_point,
                      float x_scale, const float *w_scale, int64_t w_scale_len, float y_scale,
                      int64_t y_zero_point, int y_is_signed, const int32_t *bias,
                      const mmnb_conv_params *prm, void *y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  ConvShape s;
  int rc = conv_shape(w, n, c, h, wd, prm, &s);
  if (rc) return rc;
  if (w->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if ((rc = check_zp(x_zero_point, x_is_signed, "QLinearConv: x zero point"))) return rc;
  if ((rc = check_zp(y_zero_point, y_is_signed, "QLinearConv: y zero point"))) return rc;
  if (!x || !y) return fail(MMNB_ERR_ARG, "QLinearConv: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  const size_t xb = (size_t)(n * c * h * wd), yn = (size_t)(n * w->conv_m * s.oh * s.ow);
  void *d_x = nullptr, *d_y = nullptr;
  if ((rc = scratch_get(ctx, 0, xb + 256, &d_x))) return rc;
  if ((rc = scratch_get(ctx, 1, yn + 256, &d_y))) return rc;
  MmiEpi o;
  if ((rc = qconv_params(ctx, w->conv_m, x_scale, w_scale, w_scale_len, y_scale, bias,
                         &o.rq_mult_ch, &o.rq_bias)))
    return rc;
  if (xb) MMNB_HIP(hipMemcpyAsync(d_x, x, xb, hipMemcpyHostToDevice, ctx->stream));
  o.yq = (uint8_t *)d_y;
  o.rq_mode = 2;
  o.yzp = (int32_t)y_zero_point;
  o.lo = y_is_signed ? -128 : 0;
  o.hi = y_is_signed ? 127 : 255;
  if ((rc = conv_run(ctx, w, (const uint8_t *)d_x, x_is_signed ? 1 : 0, s, x_zero_point, o)))
    return rc;
  if (yn) MMNB_HIP(hipMemcpyAsync(y, d_y, yn, hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}
