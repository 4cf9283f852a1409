/*
 * mmnb.h -- C ABI of libmmnb: MI355X (gfx950) kernels for the quantized
 * matrix-multiply path of onnx_runtime_dart.
 *
 *   MatMulNBits            int4 block-quantized weights, fp32 activations
 *   DynamicQuantizeLinear  fp32 -> uint8 with data-derived scale/zero point
 *   MatMulInteger          uint8/int8 x uint8/int8 -> int32, exact
 *
 * Plain C types only (pointers, sizes, status codes): this is the surface a
 * dart:ffi binding (or ctypes, or C++) calls.  Each operator entry point
 * names the reference function it replaces; paths are relative to the
 * onnx_runtime_dart source tree.
 *
 * Conventions
 *  - Every function returns an int status: MMNB_OK (0) or a negative code.
 *    mmnb_last_error() returns a message for the calling thread's last
 *    failure.  The codes map onto the reference's exception types:
 *    MMNB_ERR_ARG -> ArgumentError / AssertionError, MMNB_ERR_UNSUPPORTED ->
 *    UnsupportedError; device and allocation failures have no reference
 *    counterpart (the reference never leaves the CPU).
 *  - "host" entry points take host buffers and are synchronous: they return
 *    after the result is back in the caller's memory (the reference ops are
 *    pure synchronous functions).
 *  - "_dev" entry points take device pointers and enqueue work on the
 *    context's stream without waiting; call mmnb_synchronize() before
 *    reading results.  Device buffers come from mmnb_device_alloc().
 *  - Weight packs live in device memory (HBM) from mmnb_pack_* until
 *    mmnb_pack_free(): weights are uploaded once and stay resident across
 *    calls, like the initializer Tensors the reference keeps for the
 *    lifetime of a model (onnx_graph.dart:90-93, :553).
 *  - A context may be used from several threads; calls on one context are
 *    serialised by an internal mutex.
 */
#ifndef MMNB_H
#define MMNB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MMNB_OK 0
#define MMNB_ERR_ARG (-1)
#define MMNB_ERR_UNSUPPORTED (-2)
#define MMNB_ERR_DEVICE (-3)
#define MMNB_ERR_OOM (-4)

#define MMNB_ABI_VERSION 1

typedef struct mmnb_ctx mmnb_ctx;
typedef struct mmnb_pack mmnb_pack;

/* ---- library / context ------------------------------------------------ */

/* ABI version of the loaded library (MMNB_ABI_VERSION). */
int mmnb_abi_version(void);

/* Message describing the calling thread's most recent failure ("" if none). */
const char *mmnb_last_error(void);

/* Open a context on HIP device `device` (one stream, default priority).
 * Replaces: nothing in the reference (its ops run on the calling isolate);
 * the Dart binding opens one context per process and keeps it alive while
 * any OnnxModel holds a pack (OnnxModel.fromBytes,
 * lib/onnx_runtime_dart.dart:65-88). */
int mmnb_init(int device, mmnb_ctx **out);

/* Release the context, its stream and scratch memory.  Packs must be freed
 * first.  Mirrors OnnxModel.dispose (lib/onnx_runtime_dart.dart:140). */
int mmnb_shutdown(mmnb_ctx *ctx);

/* Device name, compute-unit count and HBM bytes of the context's GPU. */
int mmnb_device_info(mmnb_ctx *ctx, char *name, size_t name_len,
                     int *compute_units, int64_t *hbm_bytes);

/* ---- MatMulNBits ------------------------------------------------------- */

/* Upload a MatMulNBits weight to HBM.
 *   b_q          uint8 [n, ceil(k/block_size), block_size/2], low nibble =
 *                even k (onnx_qlinear_ops.dart:121, :144-145)
 *   scales       fp32, n*ceil(k/block_size) values read flat (:123, :131)
 *   zero_points  NULL (zero point 8, :132) or packed uint4, nibble index
 *                col*n_blocks+blk, low nibble first (:133-137)
 *   bits         must be 4 (:117-119 -> MMNB_ERR_UNSUPPORTED)
 * The lengths are element counts of the caller's buffers and are checked.
 * Replaces: the per-call dequantisation of opMatMulNBits
 * (onnx_qlinear_ops.dart:127-149); the pack is what the Dart binding caches
 * per `bQ` Tensor (Expando keyed on the initializer). */
int mmnb_pack_nbits(mmnb_ctx *ctx, const uint8_t *b_q, int64_t b_q_len,
                    const float *scales, int64_t scales_len,
                    const uint8_t *zero_points, int64_t zero_points_len,
                    int64_t k, int64_t n, int64_t bits, int64_t block_size,
                    mmnb_pack **out);

/* y[m, n] = a[m, k] * dequant(B)^T, fp32 in and out, host buffers,
 * synchronous.  m = len(a) / k as in the reference (:152).
 * Replaces: opMatMulNBits (lib/src/onnx_qlinear_ops.dart:114-156), called
 * from the _dispatch arm 'MatMulNBits' (lib/src/onnx_graph.dart:1584-1596). */
int mmnb_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *pack, const float *a,
                      int64_t m, float *y);

/* Device-buffer form of mmnb_matmul_nbits (asynchronous on the context
 * stream): d_a fp32 [m, k] row-major, d_y fp32 [m, n].
 * Replaces: the same op, for callers that keep activations in HBM
 * (a decoder loop feeding one node's output to the next). */
int mmnb_matmul_nbits_dev(mmnb_ctx *ctx, const mmnb_pack *pack,
                          const float *d_a, int64_t m, float *d_y);

/* Allocation-free form of mmnb_matmul_nbits_dev.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture that has not run the call before, serving loops
 * and harnesses that forbid hipMalloc).  Same kernels and result bits as
 * mmnb_matmul_nbits_dev for packs from mmnb_pack_nbits; the prefill GEMM's
 * scratch (prepared activations, row exponents, K-slice partials and
 * counters) comes from a fixed device array of
 * mmnb_noalloc_workspace_bytes() bytes per GPU (64 MiB, held from library
 * load until the process ends) instead of the context's grow-only buffers.
 * Calls whose scratch would exceed it return MMNB_ERR_UNSUPPORTED (M x K up
 * to 2048 x 4096 fits); packs from mmnb_pack_nbits_ex with g_idx, bias,
 * bits 8 or float zero points return MMNB_ERR_UNSUPPORTED.  All calls on one
 * GPU share the array: calls that overlap on one GPU (two streams or two
 * contexts at once) race. */
int mmnb_matmul_nbits_dev_noalloc(mmnb_ctx *ctx, const mmnb_pack *pack,
                                  const float *d_a, int64_t m, float *d_y);
/* Bytes of the fixed workspace behind mmnb_matmul_nbits_dev_noalloc. */
int64_t mmnb_noalloc_workspace_bytes(void);

/* ---- MatMulNBits beyond the reference's 4-bit form -----------------------
 * The reference accepts bits = 4, uint8 zero points in its flat layout and
 * fp32 scales, and throws UnsupportedError for g_idx / bias inputs
 * (onnx_graph.dart:1585-1588, onnx_qlinear_ops.dart:117-119).  ORT-exported
 * models also use bits = 8, act-order g_idx, a bias, floating-point zero
 * points, fp16 scales / bias (widened exactly, as the reference's loader
 * widens fp16 initializers, onnx_proto_loader.dart:29-47, :217-227) and the
 * per-column zero-point layout [N, ceil(n_blocks * bits / 8)].  This entry
 * point packs all of them for mmnb_matmul_nbits / _dev (same semantics:
 * W[k, n] = (q - zp[n, g]) * scale[n, g], g = g_idx[k] or k / block_size,
 * y = A W + bias).  No reference counterpart: it extends the drop-in to
 * what the reference rejects. */
#define MMNB_DT_F32 1
#define MMNB_DT_U8 2
#define MMNB_DT_F16 10
#define MMNB_ZP_FLAT 0        /* nibble i = n * n_blocks + blk (the reference, :133-137) */
#define MMNB_ZP_PER_COLUMN 1  /* byte row of ceil(n_blocks / 2) per column (ORT) */

typedef struct mmnb_nbits_desc {
  int64_t k, n, bits, block_size;      /* bits 4 or 8 */
  const uint8_t *b_q;                  /* [n, ceil(k/bs), bs*bits/8] */
  int64_t b_q_len;
  const void *scales;                  /* [n * ceil(k/bs)] */
  int64_t scales_len;
  int scales_type;                     /* MMNB_DT_F32 | MMNB_DT_F16 */
  const void *zero_points;             /* NULL: 8 (bits 4) / 128 (bits 8) */
  int64_t zero_points_len;
  int zero_points_type;                /* MMNB_DT_U8 (packed by bits) | F32 | F16 */
  int zero_points_layout;              /* MMNB_ZP_FLAT | MMNB_ZP_PER_COLUMN (4-bit U8) */
  const int32_t *g_idx;                /* NULL or [k]; groups of block_size rows */
  int64_t g_idx_len;
  const void *bias;                    /* NULL or [n] */
  int64_t bias_len;
  int bias_type;                       /* MMNB_DT_F32 | MMNB_DT_F16 */
} mmnb_nbits_desc;

int mmnb_pack_nbits_ex(mmnb_ctx *ctx, const mmnb_nbits_desc *desc, mmnb_pack **out);

/* ---- DynamicQuantizeLinear --------------------------------------------- */

/* y = saturate(roundEven(x / scale) + zp), scale = fl32((max(0,x) -
 * min(0,x)) / 255.0) in double, zp = roundEven(clamp(fl32(-min/scale))).
 * Host buffers, synchronous; zero_point is returned as int64 like
 * Tensor.scalarInt.  Input the reference rejects -- scale != 0 and some x
 * NaN or infinite, where its _roundEven calls toInt() on a non-finite
 * quotient (onnx_ops.dart:2490-2497, :2574-2576) -- returns
 * MMNB_ERR_UNSUPPORTED (outputs unspecified).  NaN among zeros (scale 0)
 * rounds nothing and returns zp everywhere, as the reference does.
 * Replaces: opDynamicQuantizeLinear (lib/src/onnx_ops.dart:2556-2583),
 * _dispatch arm 'DynamicQuantizeLinear' (lib/src/onnx_graph.dart:1561-1562). */
int mmnb_dynamic_quantize_linear(mmnb_ctx *ctx, const float *x, int64_t n,
                                 uint8_t *y, float *scale,
                                 int64_t *zero_point);

/* Device-buffer form: d_scale (1 float) and d_zero_point (1 int32) are
 * written on the device, so a following MatMulInteger can consume them
 * without a host round trip.  It runs asynchronously and cannot report the
 * input the host form rejects: for that input it writes a NaN scale (never
 * produced otherwise) and defined bytes (NaN quantises to 0), so a NaN
 * *d_scale is the device-side error marker.  mmnb_dynamic_matmul_dev passes
 * that NaN scale on: its fp32 results are then NaN. */
int mmnb_dynamic_quantize_linear_dev(mmnb_ctx *ctx, const float *d_x,
                                     int64_t n, uint8_t *d_y, float *d_scale,
                                     int32_t *d_zero_point);

/* ---- MatMulInteger ----------------------------------------------------- */

/* Upload a MatMulInteger right-hand operand B [b_batch, k, n] (int8 when
 * b_is_signed, else uint8) with its zero point: NULL/0 (none), 1 (scalar)
 * or n (per column, only when n != 1); other lengths are
 * MMNB_ERR_UNSUPPORTED (onnx_qlinear_ops.dart:35-43).
 * Replaces: the B side of opMatMulInteger; the Dart binding caches the pack
 * per `b` Tensor. */
int mmnb_pack_integer(mmnb_ctx *ctx, const void *b, int b_is_signed,
                      int64_t b_batch, int64_t k, int64_t n,
                      const int64_t *b_zero_point, int64_t b_zero_point_len,
                      mmnb_pack **out);

/* y[batch, m, n] = (A - a_zp) (B - b_zp), exact int32.  A is
 * [a_batch, m, k] (int8 when a_is_signed, else uint8); a_zero_point NULL/0,
 * scalar (len 1) or per row (len m, m != 1).  batch = max(a_batch, b_batch);
 * each must equal batch or 1 (:44-47).  Host buffers, synchronous.  The
 * Dart binding widens y to Int64List (the reference returns Tensor.int64,
 * :75-78).
 * Replaces: opMatMulInteger (lib/src/onnx_qlinear_ops.dart:30-79),
 * _dispatch arm 'MatMulInteger' (lib/src/onnx_graph.dart:1563-1567). */
int mmnb_matmul_integer(mmnb_ctx *ctx, const mmnb_pack *pack, const void *a,
                        int a_is_signed, int64_t a_batch, int64_t m,
                        const int64_t *a_zero_point, int64_t a_zero_point_len,
                        int32_t *y);

/* Device-buffer form.  d_a_zero_point is a device int32 array of length
 * a_zero_point_len (0, 1 or m), e.g. the output of
 * mmnb_dynamic_quantize_linear_dev. */
int mmnb_matmul_integer_dev(mmnb_ctx *ctx, const mmnb_pack *pack,
                            const void *d_a, int a_is_signed, int64_t a_batch,
                            int64_t m, const int32_t *d_a_zero_point,
                            int64_t a_zero_point_len, int32_t *d_y);

/* The dynamic-quantisation chain of an ORT-exported MatMul, on the device:
 *   (a_u8, a_scale, a_zp) = DynamicQuantizeLinear(x)     x fp32 [m, k]
 *   acc = MatMulInteger(a_u8, B, a_zp, b_zp)             exact int32
 *   y   = fl32(fl32(acc) * fl32(a_scale * b_scale[j]))  Cast -> Mul -> Mul
 * b_scale is a device fp32 array of length 1 or n.  d_acc (int32 [m, n]) may
 * be NULL; when given it receives the exact accumulator.  d_a_q (uint8
 * [m, k]), d_a_scale (1 float) and d_a_zero_point (1 int32) are required
 * outputs of the quantisation step.
 * Replaces: the node sequence DynamicQuantizeLinear -> MatMulInteger ->
 * Cast -> Mul (onnx_graph.dart:1561-1567 dispatching onnx_ops.dart:2556-2583,
 * onnx_qlinear_ops.dart:30-79, onnx_ops.dart:579-606, :399-401). */
int mmnb_dynamic_matmul_dev(mmnb_ctx *ctx, const mmnb_pack *pack,
                            const float *d_x, int64_t m,
                            const float *d_b_scale, int64_t b_scale_len,
                            uint8_t *d_a_q, float *d_a_scale,
                            int32_t *d_a_zero_point, int32_t *d_acc,
                            float *d_y);

/* ---- QLinearMatMul, ConvInteger, QLinearConv ----------------------------
 * The integer products run on the MatMulInteger kernels (exact int32);
 * 8-bit outputs are int8 when *_is_signed, else uint8.  The reference
 * returns these as Tensor.int64 (the Dart binding widens). */

/* QLinearMatMul: acc = MatMulInteger(A, B, a_zp, b_zp) with B from
 * mmnb_pack_integer (its zero point is b_zp); mult = fl32(fl32(a_scale *
 * b_scale) / y_scale); y = clamp(roundEven(fl32(acc * mult)) + y_zp) to the
 * output type's range.  Per-tensor scales only (the Dart binding throws
 * UnsupportedError for others, onnx_qlinear_ops.dart:86-88).  Host buffers, synchronous.
 * Replaces: opQLinearMatMul (lib/src/onnx_qlinear_ops.dart:83-106),
 * _dispatch arm 'QLinearMatMul' (lib/src/onnx_graph.dart:1577-1583). */
int mmnb_qlinear_matmul(mmnb_ctx *ctx, const mmnb_pack *b_pack, const void *a,
                        int a_is_signed, int64_t a_batch, int64_t m,
                        const int64_t *a_zero_point, int64_t a_zero_point_len,
                        float a_scale, float b_scale, float y_scale,
                        int64_t y_zero_point, int y_is_signed, void *y);
/* Device-buffer form (d_a_zero_point: device int32, length 0, 1 or m). */
int mmnb_qlinear_matmul_dev(mmnb_ctx *ctx, const mmnb_pack *b_pack,
                            const void *d_a, int a_is_signed, int64_t a_batch,
                            int64_t m, const int32_t *d_a_zero_point,
                            int64_t a_zero_point_len, float a_scale,
                            float b_scale, float y_scale, int64_t y_zero_point,
                            int y_is_signed, void *d_y);

/* 2-D convolution geometry: strides [sh, sw], pads [top, left, bottom,
 * right], dilations [dh, dw] (ONNX attribute order).  A 1-D convolution is
 * the 2-D one with height 1 (the reference's reshape, onnx_qlinear_ops.dart:238-252). */
typedef struct mmnb_conv_params {
  int64_t strides[2];
  int64_t pads[4];
  int64_t dilations[2];
} mmnb_conv_params;

/* Upload a convolution weight w [m, c_per_group, kh, kw] (int8 when
 * w_is_signed, else uint8) with its zero point: NULL/0, scalar or per output
 * channel (length m); other lengths are MMNB_ERR_UNSUPPORTED
 * (onnx_qlinear_ops.dart:254-257).
 * Replaces: the weight side of opConvInteger / opQLinearConv; the Dart
 * binding caches the pack per `w` Tensor. */
int mmnb_pack_conv(mmnb_ctx *ctx, const void *w, int w_is_signed, int64_t m,
                   int64_t c_per_group, int64_t kh, int64_t kw, int64_t group,
                   const int64_t *w_zero_point, int64_t w_zero_point_len,
                   mmnb_pack **out);

/* Output height and width for an input [n, c, h, wd] (validates the
 * geometry: c = c_per_group * group, window within the padded input). */
int mmnb_conv_output_shape(const mmnb_pack *w, int64_t n, int64_t c, int64_t h,
                           int64_t wd, const mmnb_conv_params *prm,
                           int64_t *oh, int64_t *ow);

/* ConvInteger: y[n, m, oh, ow] = sum (x - x_zp)(w - w_zp[m]), exact int32;
 * x [n, c, h, wd] (int8 when x_is_signed, else uint8), x_zp scalar.  Host
 * buffers, synchronous.
 * Replaces: opConvInteger (lib/src/onnx_qlinear_ops.dart:235-267, accumulator :160-220), _dispatch
 * arm 'ConvInteger' (lib/src/onnx_graph.dart:1568-1576). */
int mmnb_conv_integer(mmnb_ctx *ctx, const mmnb_pack *w, const void *x,
                      int x_is_signed, int64_t n, int64_t c, int64_t h, int64_t wd,
                      int64_t x_zero_point, const mmnb_conv_params *prm,
                      int32_t *y);
int mmnb_conv_integer_dev(mmnb_ctx *ctx, const mmnb_pack *w, const void *d_x,
                          int x_is_signed, int64_t n, int64_t c, int64_t h,
                          int64_t wd, int64_t x_zero_point,
                          const mmnb_conv_params *prm, int32_t *d_y);

/* QLinearConv: acc as ConvInteger; per output channel c,
 * mult = x_scale * w_scale[c] / y_scale and y = clamp(roundEven((acc +
 * bias[c]) * mult) + y_zp), in double as the reference.  w_scale has 1 or m
 * values (host), bias m int32 values or NULL (host).
 * Replaces: opQLinearConv (lib/src/onnx_qlinear_ops.dart:270-308), _dispatch
 * arm 'QLinearConv' (lib/src/onnx_graph.dart:1597-1609). */
int mmnb_qlinear_conv(mmnb_ctx *ctx, const mmnb_pack *w, const void *x,
                      int x_is_signed, int64_t n, int64_t c, int64_t h, int64_t wd,
                      int64_t x_zero_point, float x_scale, const float *w_scale,
                      int64_t w_scale_len, float y_scale, int64_t y_zero_point,
                      int y_is_signed, const int32_t *bias,
                      const mmnb_conv_params *prm, void *y);
/* Device form: d_x / d_y device buffers; w_scale and bias stay host arrays
 * (uploaded per call, so this call is not capturable). */
int mmnb_qlinear_conv_dev(mmnb_ctx *ctx, const mmnb_pack *w, const void *d_x,
                          int x_is_signed, int64_t n, int64_t c, int64_t h,
                          int64_t wd, int64_t x_zero_point, float x_scale,
                          const float *w_scale, int64_t w_scale_len,
                          float y_scale, int64_t y_zero_point, int y_is_signed,
                          const int32_t *bias, const mmnb_conv_params *prm,
                          void *d_y);

/* ---- weight-pack loader -------------------------------------------------
 * Loads the quantized weights of an ONNX model file into resident packs:
 * every MatMulNBits (any input form mmnb_pack_nbits_ex accepts),
 * MatMulInteger / QLinearMatMul (constant B) and ConvInteger / QLinearConv
 * (constant W) node whose weight inputs are initializers.  Bytes go from the
 * file to the device: inline raw_data is read in place from the
 * memory-mapped model, external data (location / offset / length, relative
 * to the model's directory) from the memory-mapped companion file, so a
 * multi-GB weight file is never read into host memory whole.  Packs stay
 * resident until mmnb_model_free.
 * Replaces: loadOnnxModel (lib/onnx_runtime_dart_io.dart:19-42) and the
 * weight decoding of tensorFromProto (lib/src/onnx_proto_loader.dart:80-243)
 * for these nodes' weights; the Dart binding looks packs up by node name
 * instead of packing host tensors on first use. */
typedef struct mmnb_model mmnb_model;
int mmnb_model_load(mmnb_ctx *ctx, const char *path, mmnb_model **out);
int64_t mmnb_model_pack_count(const mmnb_model *model);
/* i-th packed node: op type, node name (its first output when unnamed) and
 * pack; the strings live as long as the model. */
int mmnb_model_pack_info(const mmnb_model *model, int64_t i, const char **op_type,
                         const char **node_name, const mmnb_pack **pack);
int mmnb_model_find(const mmnb_model *model, const char *node_name,
                    const mmnb_pack **pack);
int mmnb_model_free(mmnb_model *model);

/* The external-data guard: location a plain relative path inside the model's
 * directory (no "..", no absolute path, no drive), [offset, offset+length)
 * within the file's file_len bytes; MMNB_OK or MMNB_ERR_ARG.
 * Replaces: checkExternalRef (lib/onnx_runtime_dart_io.dart:44-69). */
int mmnb_check_external_ref(const char *location, int64_t offset, int64_t length,
                            int64_t file_len);

/* ---- decoder ops around MatMulNBits -------------------------------------
 * Device buffers, asynchronous on the context stream (like the _dev entry
 * points above).  fp32 throughout. */

/* RMSNorm over the last axis: y[r] = x[r] * gamma / sqrt(mean(x[r]^2) + eps)
 * for rows x dim row-major x and y, gamma [dim].  Sum of squares, the
 * normaliser and the products in double, one binary32 rounding per output.
 * Replaces: opRMSNorm (lib/src/onnx_ops.dart:1436-1461, last-axis case), as
 * dispatched for the fused RMSNorm pattern and SimplifiedLayerNormalization
 * (lib/src/onnx_graph.dart:973-977, :1008-1013). */
int mmnb_rmsnorm_dev(mmnb_ctx *ctx, const float *d_x, int64_t rows, int64_t dim,
                     const float *d_gamma, float eps, float *d_y);

/* RotaryEmbedding of x [batch, seq, hidden] (heads = num_heads, or
 * hidden / (2 half_rot) when num_heads is 0) at positions d_pos (int64,
 * [seq] when pos_rank is 1, [batch, seq] when 2); cos/sin caches
 * [max_pos, half_rot].  Rotation in double as the reference.
 * Replaces: opRotaryEmbedding (lib/src/onnx_ops.dart:2121-2181), dispatch
 * arm 'RotaryEmbedding' (lib/src/onnx_graph.dart:1001-1007). */
int mmnb_rotary_dev(mmnb_ctx *ctx, const float *d_x, int64_t batch, int64_t seq,
                    int64_t hidden, int64_t num_heads, const int64_t *d_pos,
                    int64_t pos_rank, const float *d_cos, const float *d_sin,
                    int64_t half_rot, int interleaved, float *d_y);

/* GroupQueryAttention: q [batch, seq, num_heads*head_size], k/v [batch, seq,
 * kv_heads*head_size], optional past [batch, kv_heads, past_len, head_size],
 * optional rotary (cos/sin [max_pos, half_rot], positions past_len..),
 * optional additive bias [batch, bias_heads, seq, past_len+seq]; scale <= 0
 * means 1/sqrt(head_size).  Writes out [batch, seq, num_heads*head_size] and
 * present_k/present_v [batch, kv_heads, past_len+seq, head_size].
 * head_size <= 128.  Rotary with batch > 1 is rejected (MMNB_ERR_ARG), as
 * the reference's position ids [1, seq] are indexed per batch and throw.
 * Replaces: opGroupQueryAttention (lib/src/onnx_ops.dart:1508-1640), dispatch
 * arm 'GroupQueryAttention' (lib/src/onnx_graph.dart:978-993). */
int mmnb_gqa_dev(mmnb_ctx *ctx, const float *d_q, const float *d_k, const float *d_v,
                 int64_t batch, int64_t seq, int64_t num_heads, int64_t kv_heads,
                 int64_t head_size, float scale, const float *d_past_k,
                 const float *d_past_v, int64_t past_len, const float *d_cos,
                 const float *d_sin, int64_t half_rot, int do_rotary, int interleaved,
                 const float *d_bias, int64_t bias_heads, float *d_out,
                 float *d_present_k, float *d_present_v);

/* ---- decoder session ----------------------------------------------------
 * A Qwen3-shaped int4 decoder (per layer: RMSNorm, MatMulNBits q/k/v,
 * per-head q/k RMSNorm, GroupQueryAttention with rotary and KV cache,
 * MatMulNBits o + residual, RMSNorm, MatMulNBits gate/up, SiLU * up,
 * MatMulNBits down + residual; final RMSNorm, MatMulNBits lm_head, greedy
 * argmax) with every weight, the KV cache and the step state in HBM.
 * Packs (mmnb_pack_nbits, block >= 64, no zero points) are the caller's and
 * must outlive the session: q/k/v concatenated along N (q | k | v), gate/up
 * interleaved along N (column 2j = gate j, 2j+1 = up j).  A decode step is
 * recorded once as a HIP graph and replayed per token.
 * Replaces: the node sequence an int4 export runs through the reference's
 * executor for one forward pass (OnnxModel.run, lib/onnx_runtime_dart.dart
 * :45-141) and the greedy loop around it (tool/smollm2_generate.dart:48-83);
 * MatMulNBits nodes use the kernels of mmnb_matmul_nbits. */
typedef struct mmnb_decoder mmnb_decoder;
typedef struct mmnb_decoder_config {
  int64_t layers, hidden, heads, kv_heads, head_dim, intermediate, vocab, max_len;
  float eps;        /* RMSNorm epsilon */
  float rope_theta; /* rotary base: angle = pos * theta^(-2i/head_dim) */
} mmnb_decoder_config;

/* embed fp32 [vocab, hidden] and final_norm [hidden] are copied to HBM. */
int mmnb_decoder_create(mmnb_ctx *ctx, const mmnb_decoder_config *cfg,
                        const float *embed, const float *final_norm,
                        const mmnb_pack *lm_head, mmnb_decoder **out);
/* Norm weights are copied; packs are referenced. */
int mmnb_decoder_set_layer(mmnb_decoder *dec, int64_t layer, const float *ln1,
                           const float *ln2, const float *q_norm, const float *k_norm,
                           const mmnb_pack *qkv, const mmnb_pack *o,
                           const mmnb_pack *gate_up, const mmnb_pack *down);
/* Prompt tokens through the model (KV cache grows by n); *next_token is the
 * greedy token of the last row. */
int mmnb_decoder_prefill(mmnb_decoder *dec, const int64_t *tokens, int64_t n,
                         int32_t *next_token);
/* `steps` greedy decode steps, each feeding the previous step's token;
 * tokens[i] (may be NULL) receives step i's token. */
int mmnb_decoder_decode(mmnb_decoder *dec, int64_t steps, int32_t *tokens);
/* Logits [vocab] of the last position computed. */
int mmnb_decoder_logits(mmnb_decoder *dec, float *logits);
/* Tokens held in the KV cache. */
int mmnb_decoder_position(mmnb_decoder *dec, int64_t *pos);
/* Decode steps replay the recorded HIP graph (use_graph != 0, the default)
 * or launch the step's kernels one by one.  While kernel timing is on
 * (mmnb_kernel_timing) steps always launch one by one, so that no timing
 * event is recorded into the graph. */
int mmnb_decoder_set_graph(mmnb_decoder *dec, int use_graph);
/* Empty the KV cache (weights stay). */
int mmnb_decoder_reset(mmnb_decoder *dec);
int mmnb_decoder_free(mmnb_decoder *dec);

/* ---- packs ------------------------------------------------------------- */

/* Free a pack's device memory.  Mirrors dropping the initializer Tensor
 * (OnnxModel.dispose / a NativeFinalizer on the Dart side). */
int mmnb_pack_free(mmnb_pack *pack);

/* Device bytes held by a pack. */
int64_t mmnb_pack_device_bytes(const mmnb_pack *pack);

/* The operator shape a pack serves: k = A's last dimension (MatMulNBits,
 * MatMulInteger) or c_per_group*kh*kw (convolution), n = output columns or
 * channels, batch = B's batch (MatMulInteger) or the group count (conv). */
int mmnb_pack_dims(const mmnb_pack *pack, int64_t *k, int64_t *n, int64_t *batch);

/* ---- device memory and timing (harness utilities; no reference
 *      counterpart: the reference has no device) ------------------------- */
int mmnb_device_alloc(mmnb_ctx *ctx, size_t bytes, void **d_ptr);
int mmnb_device_free(mmnb_ctx *ctx, void *d_ptr);
int mmnb_memcpy_h2d(mmnb_ctx *ctx, void *d_dst, const void *src, size_t bytes);
int mmnb_memcpy_d2h(mmnb_ctx *ctx, void *dst, const void *d_src, size_t bytes);
int mmnb_memset_dev(mmnb_ctx *ctx, void *d_dst, int value, size_t bytes);
int mmnb_memcpy_d2d(mmnb_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);
int mmnb_synchronize(mmnb_ctx *ctx);

/* Record timing event `slot` (0..15) on the context stream; read the
 * elapsed milliseconds between two recorded slots after they complete. */
int mmnb_event_record(mmnb_ctx *ctx, int slot);
int mmnb_event_elapsed_ms(mmnb_ctx *ctx, int slot_start, int slot_end,
                          float *ms);

/* Kernel timing mode.  While enabled, every kernel libmmnb launches records
 * start/stop events taken from its own dispatch (hipExtLaunchKernelGGL), so
 * the durations are the kernels' execution times, the quantity a
 * kernel-trace profiler reports.  Enabling (again) resets the record; at
 * most max_launches launches are recorded. */
int mmnb_kernel_timing(mmnb_ctx *ctx, int enable, int max_launches);

/* Sum, count, min and max of the recorded durations of kernel `kernel_id`
 * (see mmnb_kernel_name); waits for the recorded launches to finish. */
int mmnb_kernel_timing_read(mmnb_ctx *ctx, int kernel_id, int64_t *count,
                            double *total_ms, double *min_ms, double *max_ms);

/* Each recorded duration (ms) of kernel `kernel_id`, in launch order: up to
 * `cap` of them into ms_out, and the number recorded into *count (which may
 * exceed cap).  These are the dispatch's own start/end timestamps, the
 * per-kernel durations a kernel tracer reports, so medians taken from them
 * can be checked against a rocprofv3 kernel trace.  Waits for the recorded
 * launches to finish. */
int mmnb_kernel_timing_samples(mmnb_ctx *ctx, int kernel_id, float *ms_out, int64_t cap,
                               int64_t *count);

/* Name of kernel id 0.. (NULL past the last id). */
const char *mmnb_kernel_name(int kernel_id);

/* Platform calibration kernels (timed through the kernel timing mode):
 * an empty kernel (grid of `blocks` x 256 threads) and a streaming read of
 * `bytes` (multiple of 16) from d_buf with 16-byte loads, four per thread.
 * They measure the per-dispatch floor and the achievable HBM read rate that
 * the operator kernels are judged against. */
int mmnb_probe_empty(mmnb_ctx *ctx, int blocks);
int mmnb_probe_stream_read(mmnb_ctx *ctx, const void *d_buf, size_t bytes);

/* HIP graph capture of the context stream: between begin and end, the
 * "_dev" entry points are recorded instead of run (host entry points are
 * rejected).  Device scratch must already be large enough, i.e. each
 * captured call must have run once before.  The returned executable graph
 * replays the recorded work with one launch. */
int mmnb_graph_begin(mmnb_ctx *ctx);
int mmnb_graph_end(mmnb_ctx *ctx, void **graph_exec);
int mmnb_graph_launch(mmnb_ctx *ctx, void *graph_exec);
int mmnb_graph_destroy(mmnb_ctx *ctx, void *graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* MMNB_H */
