// C ABI of libmmnb: contexts, weight packs, host/device entry points.
//
// The operator entry points mirror the reference's Dart op functions
// (argument meaning and error behaviour); see include/mmnb.h for the
// file:line each one replaces.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "mmnb_internal.h"

namespace mmnb {

static thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_hip(hipError_t e, const char *what) {
  std::string m = std::string("HIP error in ") + what + ": " + hipGetErrorString(e);
  return fail(e == hipErrorOutOfMemory ? MMNB_ERR_OOM : MMNB_ERR_DEVICE, m);
}

int scratch_get(mmnb_ctx *ctx, int slot, size_t bytes, void **out) {
  Scratch &s = ctx->scratch[slot];
  if (bytes == 0) bytes = 1;
  if (s.cap < bytes) {
    if (ctx->capturing)
      return fail(MMNB_ERR_ARG,
                  "device scratch must grow during graph capture: run the call once "
                  "before capturing it");
    if (s.ptr) {
      // The stream may still read the old buffer: drain it first.
      MMNB_HIP(hipStreamSynchronize(ctx->stream));
      MMNB_HIP(hipFree(s.ptr));
      s.ptr = nullptr;
      s.cap = 0;
    }
    size_t cap = bytes + kTailPad;
    cap = (cap + 4095) & ~size_t(4095);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, cap);
    if (e != hipSuccess) return check_hip(e, "hipMalloc(scratch)");
    s.ptr = p;
    s.cap = cap - kTailPad;
  }
  *out = s.ptr;
  return MMNB_OK;
}

int device_alloc(size_t bytes, void **p) {
  size_t cap = bytes + kTailPad;
  hipError_t e = hipMalloc(p, cap);
  if (e != hipSuccess) return check_hip(e, "hipMalloc");
  return MMNB_OK;
}

}  // namespace mmnb

using namespace mmnb;


extern "C" {

int mmnb_abi_version(void) { return MMNB_ABI_VERSION; }

const char *mmnb_last_error(void) { return g_last_error.c_str(); }

int mmnb_init(int device, mmnb_ctx **out) {
  if (!out) return fail(MMNB_ERR_ARG, "mmnb_init: out is null");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(MMNB_ERR_DEVICE, "mmnb_init: no HIP device available");
  if (device < 0 || device >= count)
    return fail(MMNB_ERR_ARG, "mmnb_init: device index out of range");
  MMNB_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  MMNB_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return fail(MMNB_ERR_UNSUPPORTED,
                std::string("mmnb_init: kernels are built for gfx950, device is ") +
                    prop.gcnArchName);
  }
  mmnb_ctx *ctx = new (std::nothrow) mmnb_ctx();
  if (!ctx) return fail(MMNB_ERR_OOM, "mmnb_init: out of host memory");
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) ==
            hipSuccess &&
        v > 0)
      ctx->lds_max = v;
  }
  if (const char *r = std::getenv("MMNB_GEMV_R")) {
    const int v = std::atoi(r);
    if (v == 1 || v == 2 || v == 4 || v == 8) ctx->gemv_r = v;
  }
  if (const char *r = std::getenv("MMNB_GEMM_STAGES")) {
    const int v = std::atoi(r);
    if (v == 2 || v == 3) ctx->gemm_stages = v;
  }
  if (const char *r = std::getenv("MMNB_GEMM_CB")) {
    const int v = std::atoi(r);
    if (v == 1 || v == 2) ctx->gemm_cb = v;
  }
  if (const char *r = std::getenv("MMNB_GEMM_KSPLIT")) {
    const int v = std::atoi(r);
    if (v == 1 || v == 2 || v == 4 || v == 8) ctx->gemm_ksplit = v;
  }
  if (const char *r = std::getenv("MMNB_MMI_TM")) {
    const int v = std::atoi(r);
    if (v == 32 || v == 64) ctx->mmi_tm = v;
  }
  if (const char *r = std::getenv("MMNB_GEMV_CG")) {
    const int v = std::atoi(r);
    if (v >= 1 && v <= 8) ctx->gemv_cg = v;
  }
  if (const char *r = std::getenv("MMNB_ATTN_MFMA")) {
    const int v = std::atoi(r);
    if (v == 0 || v == 1) ctx->attn_mfma = v;
  }
  if (const char *r = std::getenv("MMNB_PREP_FUSE")) {
    const int v = std::atoi(r);
    if (v == 0 || v == 1) ctx->prep_fuse = v;
  }
  if (const char *r = std::getenv("MMNB_DEC_ATTN_DEFER")) {
    const int v = std::atoi(r);
    if (v == 0 || v == 1) ctx->dec_attn_defer = v;
  }
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return check_hip(e, "hipStreamCreateWithFlags");
  }
  for (auto &ev : ctx->events) {
    e = hipEventCreate(&ev);
    if (e != hipSuccess) {
      delete ctx;
      return check_hip(e, "hipEventCreate");
    }
  }
  e = hipMalloc(&ctx->d_pad, 4096);
  if (e == hipSuccess) e = hipMemset(ctx->d_pad, 0, 1024);
  if (e == hipSuccess) e = hipMemset((char *)ctx->d_pad + 1024, 0x80, 1024);
  if (e == hipSuccess) e = hipMemset((char *)ctx->d_pad + 2048, 0, 2048);
  if (e == hipSuccess) e = hipMalloc((void **)&ctx->d_gemm_cnt, kGemmMaxSplitTiles * sizeof(int));
  if (e == hipSuccess) e = hipMemset(ctx->d_gemm_cnt, 0, kGemmMaxSplitTiles * sizeof(int));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    if (ctx->d_pad) (void)hipFree(ctx->d_pad);
    if (ctx->d_gemm_cnt) (void)hipFree(ctx->d_gemm_cnt);
    delete ctx;
    return check_hip(e, "hipMalloc(pad page, GEMM counters)");
  }
  // The fixed workspace serves only mmnb_matmul_nbits_dev_noalloc: when it
  // cannot be resolved the context still opens, and that entry point reports
  // the reason (kept here) on every call.
  if (noalloc_setup(ctx) != MMNB_OK) {
    ctx->noalloc_ws = nullptr;
    ctx->noalloc_err = mmnb_last_error();
    (void)hipGetLastError();  // clear the sticky HIP error of the failed lookup
  }
  *out = ctx;
  return MMNB_OK;
}

int mmnb_shutdown(mmnb_ctx *ctx) {
  MMNB_GUARD_CTX(ctx);
  {
    CtxLock lk(ctx);
    if (ctx->live_packs != 0)
      return fail(MMNB_ERR_ARG, "mmnb_shutdown: packs still alive");
    int rc = set_device(ctx);
    if (rc) return rc;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &s : ctx->scratch)
      if (s.ptr) (void)hipFree(s.ptr);
    if (ctx->d_pad) (void)hipFree(ctx->d_pad);
    if (ctx->d_gemm_cnt) (void)hipFree(ctx->d_gemm_cnt);
    for (auto &ev : ctx->events)
      if (ev) (void)hipEventDestroy(ev);
    for (auto &ev : ctx->tev) (void)hipEventDestroy(ev);
    (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return MMNB_OK;
}

int mmnb_device_info(mmnb_ctx *ctx, char *name, size_t name_len,
                     int *compute_units, int64_t *hbm_bytes) {
  MMNB_GUARD_CTX(ctx);
  hipDeviceProp_t prop;
  MMNB_HIP(hipGetDeviceProperties(&prop, ctx->device));
  if (name && name_len) {
    std::snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (compute_units) *compute_units = prop.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = (int64_t)prop.totalGlobalMem;
  return MMNB_OK;
}

// ---------------------------------------------------------------- MatMulNBits

}  // extern "C"

int mmnb::pack_nbits_core(mmnb_ctx *ctx, const uint8_t *b_q, const float *scales,
                    const uint8_t *zero_points, int zp_fill, int64_t k, int64_t n,
                    int64_t block_size, mmnb_pack **out, int64_t src_col) {
  const int64_t nb = (k + block_size - 1) / block_size;
  if (src_col <= 0) src_col = nb * (block_size / 2);
  const int64_t zp_need = (n * nb + 1) / 2;
  int rc;
  mmnb_pack *p = new (std::nothrow) mmnb_pack();
  if (!p) return fail(MMNB_ERR_OOM, "out of host memory");
  p->ctx = ctx;
  p->kind = kPackNBits;
  p->k = k;
  p->n = n;
  p->block = block_size;
  p->n_blocks = nb;
  int64_t kp = nb * block_size;
  p->k64 = (kp + kSegK - 1) / kSegK * kSegK;
  p->col_bytes = p->k64 / 2;
  auto cleanup = [&](int code) {
    if (p->d_w) (void)hipFree(p->d_w);
    if (p->d_scales) (void)hipFree(p->d_scales);
    if (p->d_zp) (void)hipFree(p->d_zp);
    if (p->d_st) (void)hipFree(p->d_st);  // d_zt lies inside it
    delete p;
    return code;
  };
  const size_t wbytes = (size_t)(n * p->col_bytes);
  if ((rc = device_alloc(wbytes, (void **)&p->d_w))) return cleanup(rc);
  if ((rc = device_alloc((size_t)(n * nb) * 4, (void **)&p->d_scales))) return cleanup(rc);
  p->has_zp = zero_points != nullptr || zp_fill != 0x88;
  if ((rc = device_alloc((size_t)zp_need, (void **)&p->d_zp))) return cleanup(rc);
  // Upload the raw B into scratch, repack on the device.
  void *d_raw = nullptr;
  if ((rc = scratch_get(ctx, 4, (size_t)(n * src_col), &d_raw))) return cleanup(rc);
  hipError_t e;
  if ((e = hipMemcpyAsync(d_raw, b_q, (size_t)(n * src_col), hipMemcpyHostToDevice,
                          ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(B)"));
  if ((rc = repack_nbits_weights(ctx, (const uint8_t *)d_raw, n, k, src_col, p->col_bytes,
                                 p->d_w)))
    return cleanup(rc);
  if ((e = hipMemcpyAsync(p->d_scales, scales, (size_t)(n * nb) * 4,
                          hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(scales)"));
  if (zero_points) {
    if ((e = hipMemcpyAsync(p->d_zp, zero_points, (size_t)zp_need, hipMemcpyHostToDevice,
                            ctx->stream)) != hipSuccess)
      return cleanup(check_hip(e, "hipMemcpyAsync(zero_points)"));
  } else if ((e = hipMemsetAsync(p->d_zp, zp_fill, (size_t)zp_need, ctx->stream)) !=
             hipSuccess) {
    return cleanup(check_hip(e, "hipMemsetAsync(zero_points)"));
  }
  if ((rc = build_gemm_sz(ctx, p))) return cleanup(rc);
  if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipStreamSynchronize(pack)"));
  p->bytes = (int64_t)wbytes + n * nb * 4 + zp_need + p->ldsz * nb * 8;
  p->k_in = k;
  ctx->live_packs++;
  *out = p;
  return MMNB_OK;
}

extern "C" {

int mmnb_pack_nbits(mmnb_ctx *ctx, const uint8_t *b_q, int64_t b_q_len,
                    const float *scales, int64_t scales_len,
                    const uint8_t *zero_points, int64_t zero_points_len,
                    int64_t k, int64_t n, int64_t bits, int64_t block_size,
                    mmnb_pack **out) {
  MMNB_GUARD_CTX(ctx);
  if (!out) return fail(MMNB_ERR_ARG, "mmnb_pack_nbits: out is null");
  *out = nullptr;
  if (bits != 4)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: only bits=4 supported, got " + std::to_string(bits));
  if (k <= 0 || n <= 0)
    return fail(MMNB_ERR_ARG, "MatMulNBits: K and N must be positive");
  if (k > INT32_MAX / 2 || n > INT32_MAX)
    return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: K or N too large for the kernels");
  // any even block size, as the reference (onnx_qlinear_ops.dart:120-121);
  // an odd one cannot hold its nibbles in block_size ~/ 2 bytes
  if (block_size < 2 || (block_size & 1))
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: block_size must be even, got " + std::to_string(block_size));
  if (block_size > (int64_t(1) << 30))
    return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: block_size above 2^30");
  const int64_t nb = (k + block_size - 1) / block_size;
  const int64_t src_col = nb * (block_size / 2);
  if (!b_q || b_q_len < n * src_col)
    return fail(MMNB_ERR_ARG, "MatMulNBits: B has " + std::to_string(b_q_len) +
                                  " bytes, need N*ceil(K/block)*block/2 = " +
                                  std::to_string(n * src_col));
  if (!scales || scales_len < n * nb)
    return fail(MMNB_ERR_ARG, "MatMulNBits: scales has " + std::to_string(scales_len) +
                                  " values, need " + std::to_string(n * nb));
  const int64_t zp_need = (n * nb + 1) / 2;
  if (zero_points && zero_points_len < zp_need)
    return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points has " +
                                  std::to_string(zero_points_len) + " bytes, need " +
                                  std::to_string(zp_need));
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return pack_nbits_any(ctx, b_q, scales, zero_points, 0x88, k, n, block_size, out);
}

static int check_nbits_pack(const mmnb_ctx *ctx, const mmnb_pack *p) {
  if (!p || p->kind != kPackNBits)
    return fail(MMNB_ERR_ARG, "MatMulNBits: not a MatMulNBits pack");
  if (p->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  return MMNB_OK;
}

int mmnb_matmul_nbits_dev(mmnb_ctx *ctx, const mmnb_pack *pack, const float *d_a,
                          int64_t m, float *d_y) {
  MMNB_GUARD_CTX(ctx);
  int rc = check_nbits_pack(ctx, pack);
  if (rc) return rc;
  if (m < 0) return fail(MMNB_ERR_ARG, "MatMulNBits: negative M");
  if (m == 0) return MMNB_OK;
  if (!d_a || !d_y) return fail(MMNB_ERR_ARG, "MatMulNBits: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  return run_matmul_nbits(ctx, pack, d_a, pack->k_in, m, d_y);
}

int mmnb_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *pack, const float *a,
                      int64_t m, float *y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  int rc = check_nbits_pack(ctx, pack);
  if (rc) return rc;
  if (m < 0) return fail(MMNB_ERR_ARG, "MatMulNBits: negative M");
  if (m == 0) return MMNB_OK;
  if (!a || !y) return fail(MMNB_ERR_ARG, "MatMulNBits: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  const int64_t k = pack->k_in, n = pack->n;
  // Stage A with rows padded to k64 (zero tail) so the kernels take their
  // aligned full-segment path (an extended pack gathers A itself).
  const int64_t lda = pack->ext ? k : pack->k64;
  void *d_a = nullptr, *d_y = nullptr;
  if ((rc = scratch_get(ctx, 0, (size_t)(m * lda) * 4, &d_a))) return rc;
  if ((rc = scratch_get(ctx, 1, (size_t)(m * n) * 4, &d_y))) return rc;
  if (lda != k) {
    MMNB_HIP(hipMemsetAsync(d_a, 0, (size_t)(m * lda) * 4, ctx->stream));
    MMNB_HIP(hipMemcpy2DAsync(d_a, (size_t)lda * 4, a, (size_t)k * 4, (size_t)k * 4,
                              (size_t)m, hipMemcpyHostToDevice, ctx->stream));
  } else {
    MMNB_HIP(hipMemcpyAsync(d_a, a, (size_t)(m * k) * 4, hipMemcpyHostToDevice,
                            ctx->stream));
  }
  if ((rc = run_matmul_nbits(ctx, pack, (const float *)d_a, lda, m, (float *)d_y)))
    return rc;
  MMNB_HIP(hipMemcpyAsync(y, d_y, (size_t)(m * n) * 4, hipMemcpyDeviceToHost,
                          ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}

// ------------------------------------------------------ DynamicQuantizeLinear

int mmnb_dynamic_quantize_linear_dev(mmnb_ctx *ctx, const float *d_x, int64_t n,
                                     uint8_t *d_y, float *d_scale,
                                     int32_t *d_zero_point) {
  MMNB_GUARD_CTX(ctx);
  if (n < 0) return fail(MMNB_ERR_ARG, "DynamicQuantizeLinear: negative length");
  if ((n > 0 && (!d_x || !d_y)) || !d_scale || !d_zero_point)
    return fail(MMNB_ERR_ARG, "DynamicQuantizeLinear: null buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch_dql(ctx, d_x, n, d_y, d_scale, d_zero_point);
}

int mmnb_dynamic_quantize_linear(mmnb_ctx *ctx, const float *x, int64_t n,
                                 uint8_t *y, float *scale, int64_t *zero_point) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  if (n < 0) return fail(MMNB_ERR_ARG, "DynamicQuantizeLinear: negative length");
  if ((n > 0 && (!x || !y)) || !scale || !zero_point)
    return fail(MMNB_ERR_ARG, "DynamicQuantizeLinear: null buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  void *d_x = nullptr, *d_y = nullptr, *d_sz = nullptr;
  if ((rc = scratch_get(ctx, 0, (size_t)n * 4, &d_x))) return rc;
  if ((rc = scratch_get(ctx, 1, (size_t)n, &d_y))) return rc;
  if ((rc = scratch_get(ctx, 5, 64, &d_sz))) return rc;
  if (n) MMNB_HIP(hipMemcpyAsync(d_x, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
  float *d_scale = (float *)d_sz;
  int32_t *d_zp = (int32_t *)((char *)d_sz + 16);
  if ((rc = launch_dql(ctx, (const float *)d_x, n, (uint8_t *)d_y, d_scale, d_zp))) return rc;
  float hs = 0.0f;
  int32_t hz = 0;
  if (n) MMNB_HIP(hipMemcpyAsync(y, d_y, (size_t)n, hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipMemcpyAsync(&hs, d_scale, 4, hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipMemcpyAsync(&hz, d_zp, 4, hipMemcpyDeviceToHost, ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  // a NaN scale is the kernels' marker for input the reference rejects
  if (hs != hs)
    return fail(MMNB_ERR_UNSUPPORTED,
                "DynamicQuantizeLinear: NaN or infinite input (roundEven of a non-finite "
                "quotient)");
  *scale = hs;
  *zero_point = hz;
  return MMNB_OK;
}

// -------------------------------------------------------------- MatMulInteger

int mmnb_pack_integer(mmnb_ctx *ctx, const void *b, int b_is_signed, int64_t b_batch,
                      int64_t k, int64_t n, const int64_t *b_zero_point,
                      int64_t b_zero_point_len, mmnb_pack **out) {
  MMNB_GUARD_CTX(ctx);
  if (!out) return fail(MMNB_ERR_ARG, "mmnb_pack_integer: out is null");
  *out = nullptr;
  if (b_batch < 1 || k < 0 || n < 1)
    return fail(MMNB_ERR_ARG, "MatMulInteger: bad B shape");
  if (!b && k > 0) return fail(MMNB_ERR_ARG, "MatMulInteger: B is null");
  const int64_t bzl = b_zero_point ? b_zero_point_len : 0;
  if (bzl != 0 && bzl != 1 && bzl != n)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                "per-column [N] for B");
  // Exact int32 accumulation holds while 255*255*K < 2^31.
  if (k > 33025)
    return fail(MMNB_ERR_UNSUPPORTED, "MatMulInteger: K > 33025 may overflow int32");
  std::vector<int32_t> zp;
  if (bzl) {
    zp.resize((size_t)bzl);
    const int64_t lo = b_is_signed ? -128 : 0, hi = b_is_signed ? 127 : 255;
    for (int64_t i = 0; i < bzl; i++) {
      if (b_zero_point[i] < lo || b_zero_point[i] > hi)
        return fail(MMNB_ERR_ARG, "MatMulInteger: B zero point out of range");
      zp[(size_t)i] = (int32_t)b_zero_point[i];
    }
  }
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  mmnb_pack *p = new (std::nothrow) mmnb_pack();
  if (!p) return fail(MMNB_ERR_OOM, "out of host memory");
  p->ctx = ctx;
  p->kind = kPackInteger;
  p->batch = b_batch;
  p->k = k;
  p->n = n;
  p->kpad = (k + 63) / 64 * 64;
  if (p->kpad == 0) p->kpad = 64;
  p->b_signed = b_is_signed ? 1 : 0;
  auto cleanup = [&](int code) {
    if (p->d_bt) (void)hipFree(p->d_bt);
    if (p->d_colsum) (void)hipFree(p->d_colsum);
    if (p->d_ecol) (void)hipFree(p->d_ecol);
    delete p;
    return code;
  };
  const size_t bt_bytes = (size_t)(b_batch * n * p->kpad);
  if ((rc = device_alloc(bt_bytes, (void **)&p->d_bt))) return cleanup(rc);
  if ((rc = device_alloc((size_t)(b_batch * n) * 4, (void **)&p->d_colsum))) return cleanup(rc);
  if ((rc = device_alloc((size_t)n * 4, (void **)&p->d_ecol))) return cleanup(rc);
  const size_t raw_bytes = (size_t)(b_batch * k * n);
  void *d_raw = nullptr, *d_zp = nullptr;
  if ((rc = scratch_get(ctx, 4, raw_bytes + 256, &d_raw))) return cleanup(rc);
  if ((rc = scratch_get(ctx, 5, (size_t)(bzl ? bzl : 1) * 4, &d_zp))) return cleanup(rc);
  hipError_t e;
  if (raw_bytes &&
      (e = hipMemcpyAsync(d_raw, b, raw_bytes, hipMemcpyHostToDevice, ctx->stream)) !=
          hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(B)"));
  if (bzl && (e = hipMemcpyAsync(d_zp, zp.data(), (size_t)bzl * 4, hipMemcpyHostToDevice,
                                 ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipMemcpyAsync(b_zp)"));
  if ((rc = prepare_integer_b(ctx, (const uint8_t *)d_raw, p->b_signed, 0, b_batch, k, n,
                              p->kpad, (const int32_t *)d_zp, bzl, p->d_bt, p->d_colsum,
                              p->d_ecol)))
    return cleanup(rc);
  if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
    return cleanup(check_hip(e, "hipStreamSynchronize(pack)"));
  p->bytes = (int64_t)bt_bytes + b_batch * n * 4 + n * 4;
  ctx->live_packs++;
  *out = p;
  return MMNB_OK;
}

static int check_int_args(const mmnb_ctx *ctx, const mmnb_pack *p, int64_t a_batch,
                          int64_t m, int64_t azp_len) {
  if (!p || p->kind != kPackInteger)
    return fail(MMNB_ERR_ARG, "MatMulInteger: not a MatMulInteger pack");
  if (p->ctx != ctx) return fail(MMNB_ERR_ARG, "pack belongs to another context");
  if (a_batch < 1 || m < 0) return fail(MMNB_ERR_ARG, "MatMulInteger: bad A shape");
  if (azp_len != 0 && azp_len != 1 && azp_len != m)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                "per-column [N] for B");
  const int64_t batch = a_batch > p->batch ? a_batch : p->batch;
  if ((a_batch != batch && a_batch != 1) || (p->batch != batch && p->batch != 1))
    return fail(MMNB_ERR_ARG, "MatMulInteger batch mismatch");
  return MMNB_OK;
}

int mmnb_matmul_integer_dev(mmnb_ctx *ctx, const mmnb_pack *pack, const void *d_a,
                            int a_is_signed, int64_t a_batch, int64_t m,
                            const int32_t *d_a_zero_point, int64_t a_zero_point_len,
                            int32_t *d_y) {
  MMNB_GUARD_CTX(ctx);
  const int64_t azl = d_a_zero_point ? a_zero_point_len : 0;
  int rc = check_int_args(ctx, pack, a_batch, m, azl);
  if (rc) return rc;
  if (m == 0) return MMNB_OK;
  if (!d_y || (!d_a && pack->k > 0)) return fail(MMNB_ERR_ARG, "MatMulInteger: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  MmiEpi o;
  o.y = d_y;
  return launch_matmul_integer(ctx, pack, d_a, a_is_signed ? 1 : 0, a_batch, m,
                               d_a_zero_point, azl, o);
}

int mmnb_matmul_integer(mmnb_ctx *ctx, const mmnb_pack *pack, const void *a,
                        int a_is_signed, int64_t a_batch, int64_t m,
                        const int64_t *a_zero_point, int64_t a_zero_point_len,
                        int32_t *y) {
  MMNB_GUARD_CTX(ctx);
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "host entry point during graph capture");
  const int64_t azl = a_zero_point ? a_zero_point_len : 0;
  int rc = check_int_args(ctx, pack, a_batch, m, azl);
  if (rc) return rc;
  if (m == 0) return MMNB_OK;
  if (!y || (!a && pack->k > 0)) return fail(MMNB_ERR_ARG, "MatMulInteger: null buffer");
  std::vector<int32_t> az((size_t)(azl ? azl : 1));
  {
    const int64_t lo = a_is_signed ? -128 : 0, hi = a_is_signed ? 127 : 255;
    for (int64_t i = 0; i < azl; i++) {
      if (a_zero_point[i] < lo || a_zero_point[i] > hi)
        return fail(MMNB_ERR_ARG, "MatMulInteger: A zero point out of range");
      az[(size_t)i] = (int32_t)a_zero_point[i];
    }
  }
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  const int64_t k = pack->k, n = pack->n;
  const int64_t batch = a_batch > pack->batch ? a_batch : pack->batch;
  void *d_a = nullptr, *d_y = nullptr, *d_az = nullptr;
  if ((rc = scratch_get(ctx, 0, (size_t)(a_batch * m * k) + 256, &d_a))) return rc;
  if ((rc = scratch_get(ctx, 1, (size_t)(batch * m * n) * 4, &d_y))) return rc;
  if ((rc = scratch_get(ctx, 5, az.size() * 4, &d_az))) return rc;
  if (a_batch * m * k)
    MMNB_HIP(hipMemcpyAsync(d_a, a, (size_t)(a_batch * m * k), hipMemcpyHostToDevice,
                            ctx->stream));
  if (azl)
    MMNB_HIP(hipMemcpyAsync(d_az, az.data(), (size_t)azl * 4, hipMemcpyHostToDevice,
                            ctx->stream));
  MmiEpi o;
  o.y = (int32_t *)d_y;
  if ((rc = launch_matmul_integer(ctx, pack, d_a, a_is_signed ? 1 : 0, a_batch, m,
                                  (const int32_t *)d_az, azl, o)))
    return rc;
  MMNB_HIP(hipMemcpyAsync(y, d_y, (size_t)(batch * m * n) * 4, hipMemcpyDeviceToHost,
                          ctx->stream));
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}

int mmnb_dynamic_matmul_dev(mmnb_ctx *ctx, const mmnb_pack *pack, const float *d_x,
                            int64_t m, const float *d_b_scale, int64_t b_scale_len,
                            uint8_t *d_a_q, float *d_a_scale, int32_t *d_a_zero_point,
                            int32_t *d_acc, float *d_y) {
  MMNB_GUARD_CTX(ctx);
  int rc = check_int_args(ctx, pack, 1, m, 1);
  if (rc) return rc;
  if (pack->batch != 1)
    return fail(MMNB_ERR_UNSUPPORTED, "dynamic matmul: batched B not supported");
  if (b_scale_len != 1 && b_scale_len != pack->n)
    return fail(MMNB_ERR_ARG, "dynamic matmul: b_scale must have 1 or N values");
  if (!d_b_scale || !d_a_q || !d_a_scale || !d_a_zero_point || !d_y)
    return fail(MMNB_ERR_ARG, "dynamic matmul: null buffer");
  if (m == 0) return MMNB_OK;
  if (!d_x) return fail(MMNB_ERR_ARG, "dynamic matmul: null buffer");
  CtxLock lk(ctx);
  if ((rc = set_device(ctx))) return rc;
  if ((rc = launch_dql(ctx, d_x, m * pack->k, d_a_q, d_a_scale, d_a_zero_point))) return rc;
  MmiEpi o;
  o.y = d_acc;
  o.yf = d_y;
  o.a_scale = d_a_scale;
  o.b_scale = d_b_scale;
  o.b_scale_len = b_scale_len;
  return launch_matmul_integer(ctx, pack, d_a_q, 0, 1, m, d_a_zero_point, 1, o);
}

// ---------------------------------------------------------------------- packs

int mmnb_pack_dims(const mmnb_pack *p, int64_t *k, int64_t *n, int64_t *batch) {
  if (!p) return fail(MMNB_ERR_ARG, "null pack");
  if (k) *k = p->kind == kPackNBits ? p->k_in : p->k;
  if (n) *n = p->kind == kPackConv ? p->conv_m : p->n;
  if (batch) *batch = p->kind == kPackNBits ? 1 : p->batch;
  return MMNB_OK;
}

int mmnb_pack_free(mmnb_pack *p) {
  if (!p) return MMNB_OK;
  mmnb_ctx *ctx = p->ctx;
  {
    CtxLock lk(ctx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (p->d_w) (void)hipFree(p->d_w);
    if (p->d_scales) (void)hipFree(p->d_scales);
    if (p->d_zp) (void)hipFree(p->d_zp);
    if (p->d_st) (void)hipFree(p->d_st);  // d_zt lies inside it
    if (p->d_bt) (void)hipFree(p->d_bt);
    if (p->d_colsum) (void)hipFree(p->d_colsum);
    if (p->d_ecol) (void)hipFree(p->d_ecol);
    if (p->d_asrc) (void)hipFree(p->d_asrc);
    if (p->d_corr) (void)hipFree(p->d_corr);
    if (p->d_bias) (void)hipFree(p->d_bias);
    ctx->live_packs--;
  }
  delete p;
  return MMNB_OK;
}

int64_t mmnb_pack_device_bytes(const mmnb_pack *p) { return p ? p->bytes : 0; }

// ------------------------------------------------------ device memory/timing

int mmnb_device_alloc(mmnb_ctx *ctx, size_t bytes, void **d_ptr) {
  MMNB_GUARD_CTX(ctx);
  if (!d_ptr) return fail(MMNB_ERR_ARG, "null out pointer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return device_alloc(bytes ? bytes : 1, d_ptr);
}

int mmnb_device_free(mmnb_ctx *ctx, void *d_ptr) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  if (d_ptr) MMNB_HIP(hipFree(d_ptr));
  return MMNB_OK;
}

int mmnb_memcpy_h2d(mmnb_ctx *ctx, void *d_dst, const void *src, size_t bytes) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (bytes) {
    MMNB_HIP(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    MMNB_HIP(hipStreamSynchronize(ctx->stream));
  }
  return MMNB_OK;
}

int mmnb_memcpy_d2h(mmnb_ctx *ctx, void *dst, const void *d_src, size_t bytes) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (bytes) {
    MMNB_HIP(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    MMNB_HIP(hipStreamSynchronize(ctx->stream));
  }
  return MMNB_OK;
}

int mmnb_memcpy_d2d(mmnb_ctx *ctx, void *d_dst, const void *d_src, size_t bytes) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (bytes) MMNB_HIP(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return MMNB_OK;
}

int mmnb_memset_dev(mmnb_ctx *ctx, void *d_dst, int value, size_t bytes) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (bytes) MMNB_HIP(hipMemsetAsync(d_dst, value, bytes, ctx->stream));
  return MMNB_OK;
}

int mmnb_synchronize(mmnb_ctx *ctx) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  return MMNB_OK;
}

int mmnb_event_record(mmnb_ctx *ctx, int slot) {
  MMNB_GUARD_CTX(ctx);
  if (slot < 0 || slot >= 16) return fail(MMNB_ERR_ARG, "event slot out of range");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipEventRecord(ctx->events[slot], ctx->stream));
  return MMNB_OK;
}

int mmnb_event_elapsed_ms(mmnb_ctx *ctx, int slot_start, int slot_end, float *ms) {
  MMNB_GUARD_CTX(ctx);
  if (slot_start < 0 || slot_start >= 16 || slot_end < 0 || slot_end >= 16 || !ms)
    return fail(MMNB_ERR_ARG, "event slot out of range");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipEventSynchronize(ctx->events[slot_end]));
  MMNB_HIP(hipEventElapsedTime(ms, ctx->events[slot_start], ctx->events[slot_end]));
  return MMNB_OK;
}

static const char *kKernelNames[kKernCount] = {
    "k_gemv_valu", "k_prep_a", "k_gemm_mfma", "k_dql_minmax",
    "k_dql_quant", "k_mmi_mfma", "k_repack_nbits", "k_prep_int_b", "k_probe_empty",
    "k_probe_read", "k_dec_gemv", "k_dec_attn", "k_dec_ops", "k_dec_gemv_res",
    "k_dec_gemv_glu", "k_dec_gemv_lm", "k_im2col", "k_nbits_ex", "k_nbits_generic"};

const char *mmnb_kernel_name(int kernel_id) {
  if (kernel_id < 0 || kernel_id >= kKernCount) return nullptr;
  return kKernelNames[kernel_id];
}

int mmnb_kernel_timing(mmnb_ctx *ctx, int enable, int max_launches) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (!enable) {
    ctx->timing = false;
    return MMNB_OK;
  }
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "kernel timing during graph capture");
  if (max_launches < 1 || max_launches > (1 << 20))
    return fail(MMNB_ERR_ARG, "max_launches out of range");
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  while (ctx->tev.size() < (size_t)max_launches * 2) {
    hipEvent_t ev;
    MMNB_HIP(hipEventCreate(&ev));
    ctx->tev.push_back(ev);
  }
  ctx->tkid.assign((size_t)max_launches, -1);
  ctx->tused = 0;
  ctx->timing = true;
  return MMNB_OK;
}

int mmnb_kernel_timing_read(mmnb_ctx *ctx, int kernel_id, int64_t *count, double *total_ms,
                            double *min_ms, double *max_ms) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  int64_t c = 0;
  double tot = 0.0, mn = 0.0, mx = 0.0;
  for (size_t i = 0; i < ctx->tused; i++) {
    if (ctx->tkid[i] != kernel_id) continue;
    float ms = 0.0f;
    MMNB_HIP(hipEventElapsedTime(&ms, ctx->tev[2 * i], ctx->tev[2 * i + 1]));
    if (c == 0 || ms < mn) mn = ms;
    if (c == 0 || ms > mx) mx = ms;
    tot += ms;
    c++;
  }
  if (count) *count = c;
  if (total_ms) *total_ms = tot;
  if (min_ms) *min_ms = mn;
  if (max_ms) *max_ms = mx;
  return MMNB_OK;
}

int mmnb_kernel_timing_samples(mmnb_ctx *ctx, int kernel_id, float *ms_out, int64_t cap,
                               int64_t *count) {
  MMNB_GUARD_CTX(ctx);
  if (cap < 0 || (cap > 0 && !ms_out) || !count)
    return fail(MMNB_ERR_ARG, "mmnb_kernel_timing_samples: bad output buffer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipStreamSynchronize(ctx->stream));
  int64_t c = 0;
  for (size_t i = 0; i < ctx->tused; i++) {
    if (ctx->tkid[i] != kernel_id) continue;
    if (c < cap) {
      float ms = 0.0f;
      MMNB_HIP(hipEventElapsedTime(&ms, ctx->tev[2 * i], ctx->tev[2 * i + 1]));
      ms_out[c] = ms;
    }
    c++;
  }
  *count = c;
  return MMNB_OK;
}

int mmnb_probe_empty(mmnb_ctx *ctx, int blocks) {
  MMNB_GUARD_CTX(ctx);
  if (blocks < 1 || blocks > (1 << 20)) return fail(MMNB_ERR_ARG, "blocks out of range");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch_probe_empty(ctx, blocks);
}

int mmnb_probe_stream_read(mmnb_ctx *ctx, const void *d_buf, size_t bytes) {
  MMNB_GUARD_CTX(ctx);
  if (!d_buf || bytes == 0 || (bytes & 15) || (((uintptr_t)d_buf) & 15))
    return fail(MMNB_ERR_ARG, "probe buffer must be 16-byte aligned, size a multiple of 16");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch_probe_read(ctx, d_buf, bytes);
}

int mmnb_graph_begin(mmnb_ctx *ctx) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (ctx->capturing) return fail(MMNB_ERR_ARG, "graph capture already active");
  if (ctx->timing) return fail(MMNB_ERR_ARG, "graph capture while kernel timing is on");
  MMNB_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  return MMNB_OK;
}

int mmnb_graph_end(mmnb_ctx *ctx, void **graph_exec) {
  MMNB_GUARD_CTX(ctx);
  if (!graph_exec) return fail(MMNB_ERR_ARG, "null out pointer");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (!ctx->capturing) return fail(MMNB_ERR_ARG, "no graph capture active");
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  MMNB_HIP(hipStreamEndCapture(ctx->stream, &g));
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return check_hip(e, "hipGraphInstantiate");
  *graph_exec = (void *)ex;
  return MMNB_OK;
}

int mmnb_graph_launch(mmnb_ctx *ctx, void *graph_exec) {
  MMNB_GUARD_CTX(ctx);
  if (!graph_exec) return fail(MMNB_ERR_ARG, "null graph");
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  MMNB_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream));
  return MMNB_OK;
}

int mmnb_graph_destroy(mmnb_ctx *ctx, void *graph_exec) {
  MMNB_GUARD_CTX(ctx);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  if (graph_exec) {
    MMNB_HIP(hipStreamSynchronize(ctx->stream));
    MMNB_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  }
  return MMNB_OK;
}

}  // extern "C"
