// Internal declarations shared by the libmmnb translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>
#include <mutex>
#include <string>

#include "../../include/mmnb.h"

namespace mmnb {

// ---------------------------------------------------------------------------
// Weight-pack layout for MatMulNBits (device).
//
// The reference hands over B as uint8 [N, n_blocks, block/2]: per output
// column n a contiguous run of n_blocks*block/2 bytes, two k per byte, low
// nibble = even k.  The pack keeps that column-major-by-n layout (one
// contiguous run per column, so a column streams with 16-byte loads) but pads
// every column to a multiple of 64 k (32 bytes) and permutes the eight dwords
// inside each 32-byte segment:
//
//     original dword i (k = 8i .. 8i+7 of the segment), i = 0..7
//     packed order:  d0 d2 d4 d6 | d1 d3 d5 d7
//
// so the first 16 bytes of a segment hold k = 16j + e and the second 16 bytes
// k = 16j + 8 + e (j = 0..3, e = 0..7).  A lane that loads 16 bytes therefore
// owns one 8-k half of each of four consecutive 16-k steps, which is the
// operand shape of the 32x32x16 f16 MFMA (lane group g = lane/32 holds
// k = 8g..8g+7 of each 16-k step).  Padding nibbles are zero.
//
// Scales stay fp32 [N, n_blocks]; zero points stay packed uint4 with the
// reference's flat nibble index n*n_blocks + blk (or absent: 8).
// ---------------------------------------------------------------------------
constexpr int kSegK = 64;        // k per 32-byte segment
constexpr int kSegBytes = 32;
constexpr size_t kTailPad = 1024;  // bytes of slack after every device buffer
constexpr int kGemmMaxSplitTiles = 1024;  // tiles of a K-sliced prefill GEMM

enum PackKind { kPackNBits = 1, kPackInteger = 2, kPackConv = 3 };

struct Scratch {
  void *ptr = nullptr;
  size_t cap = 0;
};

}  // namespace mmnb

struct mmnb_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  hipEvent_t events[16] = {};
  int cu_count = 0;
  // Largest dynamic LDS allocation one workgroup may take (bytes).
  int lds_max = 65536;
  // Device staging/scratch buffers, grown on demand and kept for reuse:
  //  0: activations in (fp32 / uint8), 1: outputs, 2: prepared activations
  //  (fp16 hi/lo), 3: small reductions, 4: raw weights while packing,
  //  5: small uploads (zero points), 6: convolution im2col rows, 7: block
  //  sums / the convolution's input zero point, 8: QLinearConv per-channel
  //  parameters, 9: gathered activations of an extended MatMulNBits pack,
  //  10: the prefill GEMM's K-slice partial tiles.
  mmnb::Scratch scratch[11];
  int live_packs = 0;
  // Kernel timing mode: launches go through hipExtLaunchKernelGGL with a
  // start/stop event pair taken from the dispatch itself.
  bool timing = false;
  std::vector<hipEvent_t> tev;   // 2 per slot
  std::vector<int> tkid;         // kernel id per used slot
  size_t tused = 0;
  // 4 KB device page: 1 KB of 0x00 and 1 KB of 0x80 (int8 padding), then a
  // 2 KB sink for the calibration kernels.
  void *d_pad = nullptr;
  // Per-tile arrival counters of the prefill GEMM's K slices (kGemmMaxSplitTiles
  // ints, zero at rest: the last slice of a tile resets its counter).
  int *d_gemm_cnt = nullptr;
  // Tuning override of the GEMV columns-per-lane R (MMNB_GEMV_R; 0 = auto).
  int gemv_r = 0;
  // Tuning override of the multi-row GEMV column groups per workgroup
  // (MMNB_GEMV_CG; 0 = auto).
  int gemv_cg = 0;
  // Prefill attention on the matrix cores (MMNB_ATTN_MFMA: 0 selects the
  // vector-ALU kernel; on by default).
  int attn_mfma = 1;
  // Decoder prefill: norms / SwiGLU write the GEMM's prepared activations
  // (MMNB_PREP_FUSE: 0 keeps fp32 rows + k_prep_a; on by default).
  int prep_fuse = 1;
  // Decode step: the o projection merges the attention's split partials
  // (MMNB_DEC_ATTN_DEFER: 0 keeps the attention launch's own count and
  // merge; on by default where the merge fits).
  int dec_attn_defer = 1;
  // Prefill GEMM LDS stages (2 or 3; MMNB_GEMM_STAGES tuning override).
  int gemm_stages = 2;
  // Prefill GEMM 128-column blocks per tile (MMNB_GEMM_CB: 1 or 2; 0 = auto).
  int gemm_cb = 0;
  // Prefill GEMM K slices per tile (MMNB_GEMM_KSPLIT: 1, 2, 4 or 8; 0 = auto).
  int gemm_ksplit = 0;
  // Stream capture in progress (no synchronisation or allocation allowed).
  bool capturing = false;
  // MatMulInteger row tile (32 or 64; 0 = by shape), from MMNB_MMI_TM.
  int mmi_tm = 0;
  // Device address of this device's fixed workspace for
  // mmnb_matmul_nbits_dev_noalloc (set by noalloc_setup at init), and why it
  // is null if the lookup failed.
  void *noalloc_ws = nullptr;
  std::string noalloc_err;
};

struct mmnb_pack {
  mmnb_ctx *ctx = nullptr;
  int kind = 0;
  int64_t bytes = 0;
  // --- MatMulNBits
  int64_t k = 0, n = 0, block = 0, n_blocks = 0;
  int64_t k64 = 0;        // k padded to a multiple of 64 (and >= n_blocks*block)
  int64_t col_bytes = 0;  // bytes per column in d_w (= k64 / 2)
  uint8_t *d_w = nullptr;
  float *d_scales = nullptr;
  uint8_t *d_zp = nullptr;  // packed uint4; 0x88 filler when the op has none
  // block-major copies for the prefill GEMM, one allocation of rows
  // [nb][2][ldsz] (scales, then the zero points as dwords), ldsz = n rounded
  // up to 4 (padding zero): d_st is the allocation, d_zt = d_st + ldsz inside
  // it (both with row stride 2 ldsz)
  float *d_st = nullptr;
  uint32_t *d_zt = nullptr;
  int64_t ldsz = 0;
  bool has_zp = false;
  // Block size the fast kernels cannot take (even, not a multiple of 16): the
  // reference's bytes [n][n_blocks][block/2] (col_bytes per column), scales
  // and flat zero points as they are, for k_nbits_generic; k64 = k.
  bool generic = false;
  // --- MatMulNBits beyond the reference's 4-bit form (mmnb_pack_nbits_ex):
  // the kernels run on a 4-bit "virtual" weight of k rows (k, n_blocks, d_w,
  // d_scales, d_zp above); A is first gathered into [m, k64] when d_asrc is
  // set, and afterwards y += bias[n] + sum_b corr[b][n] * asum[m][b] with
  // asum the block sums (block `block`) of the (gathered) A over corr_nb
  // blocks.
  bool ext = false;
  int64_t k_in = 0;           // the operator's K (A's last dimension)
  int32_t *d_asrc = nullptr;  // [k] column of A feeding each virtual row, -1 = zero
  float *d_corr = nullptr;    // [corr_nb, n]
  int64_t corr_nb = 0;
  float *d_bias = nullptr;    // [n]
  // --- MatMulInteger
  int64_t batch = 0;
  int64_t kpad = 0;          // k padded to a multiple of 64
  int b_signed = 0;
  int8_t *d_bt = nullptr;    // [batch, n, kpad] signed bytes (uint8 B xor 0x80)
  int32_t *d_colsum = nullptr;  // [batch, n] sum_k B'
  int32_t *d_ecol = nullptr;    // [n] or [batch, n]: (uint8 ? 128 : 0) - b_zp
  int64_t ecol_bstride = 0;     // n when the zero points differ per batch
  // --- convolution weight (kPackConv): the MatMulInteger fields above hold
  // w as B^T per group (batch = group, n = m / group, k = c_per_group*kh*kw)
  int64_t conv_m = 0, conv_cg = 0, conv_kh = 0, conv_kw = 0, conv_group = 0;
};

namespace mmnb {

// Error state (thread-local message) ---------------------------------------
int fail(int code, const std::string &msg);
int check_hip(hipError_t e, const char *what);
#define MMNB_HIP(call)                                        \
  do {                                                        \
    hipError_t _e = (call);                                   \
    if (_e != hipSuccess) return ::mmnb::check_hip(_e, #call); \
  } while (0)

// Kernel ids reported by the timing mode (see mmnb_kernel_name).
enum KernelId {
  kKernGemv = 0,
  kKernPrep = 1,
  kKernGemm = 2,
  kKernDqlMinmax = 3,
  kKernDqlQuant = 4,
  kKernMmi = 5,
  kKernRepack = 6,
  kKernPrepIntB = 7,
  kKernProbeEmpty = 8,
  kKernProbeRead = 9,
  kKernDecGemv = 10,     // decode MatMulNBits, RMSNorm prologue (q/k/v)
  kKernDecAttn = 11,     // attention (decode step and prompt rows)
  kKernDecOps = 12,      // norms, rotary, embedding, SwiGLU rows, step state
  kKernDecGemvRes = 13,  // decode MatMulNBits + residual (o, down)
  kKernDecGemvGlu = 14,  // decode MatMulNBits, RMSNorm + SwiGLU (gate/up)
  kKernDecGemvLm = 15,   // decode MatMulNBits, RMSNorm + argmax (lm_head)
  kKernIm2col = 16,      // convolution input rows for the MatMulInteger kernels
  kKernNbitsEx = 17,     // extended MatMulNBits: A gather, block sums, correction
  kKernNbitsAny = 18,    // MatMulNBits of a block size the fast kernels do not take
  kKernCount = 19
};

// Launch `kern` on the context stream; in timing mode the dispatch records
// its own start/stop events.
template <typename... KArgs, typename... Args>
int launch(mmnb_ctx *ctx, int kid, void (*kern)(KArgs...), dim3 grid, dim3 block,
           size_t shmem, Args... args) {
  if (ctx->timing && ctx->tused < ctx->tkid.size()) {
    const size_t i = ctx->tused++;
    ctx->tkid[i] = kid;
    hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)shmem, ctx->stream, ctx->tev[2 * i],
                          ctx->tev[2 * i + 1], 0, static_cast<KArgs>(args)...);
  } else {
    hipLaunchKernelGGL(kern, grid, block, shmem, ctx->stream, static_cast<KArgs>(args)...);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return check_hip(e, "kernel launch");
  return 0;
}

// Grow-only device scratch owned by the context.
int scratch_get(mmnb_ctx *ctx, int slot, size_t bytes, void **out);

// hipMalloc with kTailPad bytes of slack.
int device_alloc(size_t bytes, void **p);

// Serialises calls on one context.
struct CtxLock {
  explicit CtxLock(mmnb_ctx *c) : ctx(c) { ctx->mu.lock(); }
  ~CtxLock() { ctx->mu.unlock(); }
  mmnb_ctx *ctx;
};

inline int set_device(mmnb_ctx *ctx) {
  MMNB_HIP(hipSetDevice(ctx->device));
  return MMNB_OK;
}

#define MMNB_GUARD_CTX(ctx)                                          \
  do {                                                               \
    if (!(ctx)) return ::mmnb::fail(MMNB_ERR_ARG, "null context");  \
  } while (0)

// Fused M = 1 MatMulNBits for the decoder step (a pack without zero points,
// block >= 64):  y = W * a with optional RMSNorm prologue and epilogue.
//   norm_gamma != null: a = x * rsqrt(mean(x^2) + eps) * gamma (x = d_x)
//   epi kDecPlain:  y[n] = v;   kDecResidual: y[n] = resid[n] + v;
//   kDecSwiglu:  columns are gate/up interleaved, y[j] = silu(v[2j]) * v[2j+1];
//   kDecArgmax:  y[n] = v and workgroup b stores d_argmax[b] = the greatest
//                (orderable value << 32 | ~index) key of its columns, for
//                dec_gemv_blocks(ctx, n, k) workgroups.
enum DecEpilogue { kDecPlain = 0, kDecResidual = 1, kDecSwiglu = 2, kDecArgmax = 3 };
int launch_dec_gemv(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_x,
                    const float *norm_gamma, float eps, int epi, const float *resid,
                    float *d_y, unsigned long long *d_argmax);
int64_t dec_gemv_blocks(const mmnb_ctx *ctx, int64_t n, int64_t k);

// The decode attention's split partials, merged by the o projection's
// prologue instead of by the attention launch itself.  Query head qh's
// partial over split s: o[hd] at o + (qh * nsmax + s) * hd, (max, sum) at
// ml + 2 * (qh * nsmax + s); all nsmax splits are merged (a split past the
// position holds max -inf, sum 0, o 0).
struct DecAttnPartials {
  const float *o;
  const float *ml;
  int nsmax, hd;
};
constexpr int kDecAttnMaxSplits = 16;  // splits one merge holds in registers
constexpr int kDecAttnMaxK = 2048;     // heads * head_dim: two float4 per thread
constexpr int kDecAttnMergeThreads = 256;
// y[n] = resid[n] + (W * a)[n], a the merged attention output (p->k = heads
// * hd <= kDecAttnMaxK, nsmax <= kDecAttnMaxSplits, heads * G <=
// kDecAttnMergeThreads with G = 8 lanes per head for nsmax <= 8, else 16).
int launch_dec_gemv_attn(mmnb_ctx *ctx, const mmnb_pack *p, const DecAttnPartials &pa,
                         const float *resid, float *d_y);

// Builds a 4-bit MatMulNBits pack (lock held): b_q [n, ceil(k/bs), bs/2]
// bytes, scales fp32 [n * ceil(k/bs)], zp packed uint4 with the flat index
// (or null: every byte zp_fill).
// bs is a power of two >= 16; src_col (0: ceil(k/bs) * bs/2) is the byte
// stride of b_q's columns.
int pack_nbits_core(mmnb_ctx *ctx, const uint8_t *b_q, const float *scales,
                    const uint8_t *zp, int zp_fill, int64_t k, int64_t n, int64_t bs,
                    mmnb_pack **out, int64_t src_col = 0);
// The same for any even block size (lock held): power-of-two blocks >= 16
// as above, other multiples of 16 re-blocked to their largest power-of-two
// divisor, the rest as a generic pack; odd sizes MMNB_ERR_UNSUPPORTED.
int pack_nbits_any(mmnb_ctx *ctx, const uint8_t *b_q, const float *scales,
                   const uint8_t *zp, int zp_fill, int64_t k, int64_t n, int64_t bs,
                   mmnb_pack **out);
// Block sizes the fast kernels take as they are (powers of two >= 16).
bool nbits_block_native(int64_t bs);
// MatMulNBits on a generic pack (no scratch; the reference's order and bits).
int launch_nbits_generic(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                         int64_t m, float *d_y);

// MatMulNBits for any pack (plain or extended): gathers A, runs the kernels
// and the correction pass as the pack requires.  lda = row stride of A.
int run_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                     int64_t m, float *d_y);

// Kernel launchers (return MMNB_OK or an error code) -------------------------
// MatMulNBits: y[m, n] = a[m, k] * W;  lda = row stride of a (elements).
int launch_matmul_nbits(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a,
                        int64_t lda, int64_t m, float *d_y);
// The prefill GEMM (M > 8) with its activations prepared by the caller's own
// kernel instead of k_prep_a: gemm_prepared_a returns where to write them
// (scratch: the hi/lo fp16 units, [mpad / 32][segsp][4][2] x 1 KB, and the
// int row exponents [mpad]; rows >= M and k >= K zero) for this pack and M;
// launch_matmul_nbits_prepared then runs the GEMM on them.  Nothing that
// takes the same scratch may run in between.
int gemm_prepared_a(mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, int64_t *segsp,
                    int64_t *mpad, void **d_ap, int **d_exp);
int launch_matmul_nbits_prepared(mmnb_ctx *ctx, const mmnb_pack *p, int64_t m, float *d_y);
// MatMulNBits (plain packs) with all scratch carved from ws (ws_bytes,
// 256-byte aligned); MMNB_ERR_UNSUPPORTED if the call needs more.  Calls no
// allocator.
int launch_matmul_nbits_ws(mmnb_ctx *ctx, const mmnb_pack *p, const float *d_a, int64_t lda,
                           int64_t m, float *d_y, void *ws, size_t ws_bytes);
// Finds this device's fixed no-alloc workspace (once per context, with the
// context's device current).
int noalloc_setup(mmnb_ctx *ctx);

// DynamicQuantizeLinear on device.
int launch_dql(mmnb_ctx *ctx, const float *d_x, int64_t n, uint8_t *d_y,
               float *d_scale, int32_t *d_zp);

// Output stage of the MatMulInteger kernels.  Any of y / yf / yq may be
// set; the exact accumulator acc feeds each.
//   y:  int32 acc.
//   yf: fl32(fl32(acc) * fl32(a_scale * b_scale[j])), a_scale read from the
//       device (the dynamic-quantisation chain's Cast -> Mul -> Mul).
//   yq: 8-bit requantisation, clamp(rint(x) + yzp, lo, hi) stored as a byte:
//       rq_mode 1: x = fl32(acc * rq_mult) (QLinearMatMul's binary32 steps);
//       rq_mode 2: x = (acc + rq_bias[c]) * rq_mult_ch[c] in double
//                  (QLinearConv, c = output channel).
// Output element (batch bz, row, col) goes to (bz*M + row)*N + col, or with
// trans to (bz*N + col)*M + row (channel-major: a convolution's output with
// rows = positions, columns = channels of group bz, channel = bz*N + col).
// ecol_bstride: the pack's zero-point offsets per batch (0 = shared).
struct MmiEpi {
  int32_t *y = nullptr;
  float *yf = nullptr;
  const float *a_scale = nullptr;
  const float *b_scale = nullptr;
  int64_t b_scale_len = 0;
  uint8_t *yq = nullptr;
  int rq_mode = 0;
  float rq_mult = 0.0f;
  const double *rq_mult_ch = nullptr;
  const int32_t *rq_bias = nullptr;
  int32_t yzp = 0, lo = 0, hi = 255;
  int trans = 0;
  int64_t ecol_bstride = 0;
  // A's zero point as a constant (azp_len must be 1; the pointer is unused)
  int azp_is_const = 0;
  int32_t azp_const = 0;
};

// MatMulInteger on the device.  d_azp: device int32 of length azp_len (0, 1
// or m).
int launch_matmul_integer(mmnb_ctx *ctx, const mmnb_pack *p, const void *d_a,
                          int a_signed, int64_t a_batch, int64_t m,
                          const int32_t *d_azp, int64_t azp_len, const MmiEpi &out);

// Platform calibration kernels.
int launch_probe_empty(mmnb_ctx *ctx, int blocks);
int launch_probe_read(mmnb_ctx *ctx, const void *d_buf, size_t bytes);

// Pack construction helpers (device-side repack kernels).
// Allocates and fills p->d_st / p->d_zt from p->d_scales / p->d_zp.
int build_gemm_sz(mmnb_ctx *ctx, mmnb_pack *p);
int repack_nbits_weights(mmnb_ctx *ctx, const uint8_t *d_src, int64_t n,
                         int64_t k, int64_t src_col_bytes,
                         int64_t dst_col_bytes, uint8_t *d_dst);
// B [batch, k, n] row-major, or [batch, n, k] with b_trans (a convolution
// weight, output channel major).  Zero points: bzp_len 0, 1, n (per column,
// shared by the batches) or batch*n (per column of each batch; d_ecol then
// holds batch*n entries).
int prepare_integer_b(mmnb_ctx *ctx, const uint8_t *d_src, int b_signed, int b_trans,
                      int64_t batch, int64_t k, int64_t n, int64_t kpad,
                      const int32_t *d_bzp, int64_t bzp_len, int8_t *d_bt,
                      int32_t *d_colsum, int32_t *d_ecol);

}  // namespace mmnb
