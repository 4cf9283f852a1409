// MatMulNBits for callers that cannot allocate device memory: code under
// HIP graph capture, serving loops and harnesses that forbid hipMalloc.
//
// mmnb_matmul_nbits_dev takes its prefill-GEMM scratch (prepared
// activations, row exponents, K-slice partial tiles) from the context's
// grow-only buffers, which call hipMalloc the first time a shape needs more.
// mmnb_matmul_nbits_dev_noalloc runs the same kernels on a fixed workspace
// instead: the file-scope device array `scratch` below, kNoAllocBytes per
// GPU, held from module load until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, taken once per context at
// mmnb_init with the context's device current (each GPU holds its own copy
// of the array at its own address), and only that address is ever passed to
// kernels.  Every call on one GPU shares the array and leaves its contents
// behind; the K-slice counters that must start at zero are cleared by the
// activation-prep kernel of each call.  Calls that overlap on one GPU (two
// streams or two contexts at once) race on the array.
#include <hip/hip_runtime.h>

#include <string>

#include "mmnb_internal.h"

namespace mmnb {

// 64 MiB: a prefill of M x K <= 2048 x 4096 (the largest prefill shape
// benchmarked) with its K-slice partials fits.
constexpr size_t kNoAllocBytes = size_t(64) << 20;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

int noalloc_setup(mmnb_ctx *ctx) {
  void *ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return check_hip(e, "hipGetSymbolAddress(no-alloc workspace)");
  if (!ptr) return fail(MMNB_ERR_DEVICE, "no-alloc workspace has no device address");
  ctx->noalloc_ws = ptr;
  return MMNB_OK;
}

}  // namespace mmnb

using namespace mmnb;

extern "C" {

int64_t mmnb_noalloc_workspace_bytes(void) { return (int64_t)kNoAllocBytes; }

int mmnb_matmul_nbits_dev_noalloc(mmnb_ctx *ctx, const mmnb_pack *pack, const float *d_a,
                                  int64_t m, float *d_y) {
  MMNB_GUARD_CTX(ctx);
  if (!pack || pack->kind != kPackNBits || pack->ctx != ctx)
    return fail(MMNB_ERR_ARG, "MatMulNBits: not a MatMulNBits pack of this context");
  if (pack->ext)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits (no-alloc): packs with g_idx, bias, bits 8 or float zero points "
                "need per-call buffers; use mmnb_matmul_nbits_dev");
  if (m < 0) return fail(MMNB_ERR_ARG, "MatMulNBits: negative M");
  if (m == 0) return MMNB_OK;
  if (!d_a || !d_y) return fail(MMNB_ERR_ARG, "MatMulNBits: null buffer");
  if (!ctx->noalloc_ws)
    return fail(MMNB_ERR_DEVICE, "no-alloc workspace not set up: " + ctx->noalloc_err);
  CtxLock lk(ctx);
  int rc = set_device(ctx);
  if (rc) return rc;
  return launch_matmul_nbits_ws(ctx, pack, d_a, pack->k_in, m, d_y, ctx->noalloc_ws,
                                kNoAllocBytes);
}

}  // extern "C"
