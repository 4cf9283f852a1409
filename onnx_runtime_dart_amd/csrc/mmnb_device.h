// Device helpers shared by the libmmnb kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mmnb {

// s_waitcnt immediate that waits for vmcnt <= n (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima, i.e. no wait).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Makes every value given (kernel arguments, the block size) live in SGPRs
// at this point, so the compiler issues all their scalar loads at once,
// ahead of the kernel's first memory access, and waits for them once: left
// to itself it fetched a kernel's arguments in dependent rounds, each a
// memory round trip, when control flow or the hidden block size split them.
template <typename T>
__device__ __forceinline__ void kernarg_fence(const T &v) {
  asm volatile("" ::"s"(v));
}
template <typename T, typename... R>
__device__ __forceinline__ void kernarg_fence(const T &v, const R &...rest) {
  asm volatile("" ::"s"(v));
  kernarg_fence(rest...);
}

// Buffer resource over raw bytes at base (no range limit: callers clamp
// their offsets; 32-bit data format, so loads return the bytes as stored).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, -1, 0x00020000);
}

// 16-byte global->LDS DMA through a buffer resource (buffer_load_dwordx4
// ... lds): lane l's 16 bytes at base + voff + soff land at lds + 16 l (lds
// wave-uniform).  The compiler counts it on vmcnt only, so LDS reads issued
// after it keep in-order lgkmcnt waits; after the FLAT form
// (global_load_lds) it waits for every outstanding LDS read (lgkmcnt(0))
// before their first use.  Read the staged bytes through vector-type
// pointers (ext_vector_type): a read through a HIP struct type (uint4) makes
// the compiler wait for every outstanding LDS DMA (vmcnt(0)) first, the
// prefetched stages' too.  The callers order their reads after the DMA they
// need with their own vmcnt waits and barriers.  A plain function, so that
// template kernels can use it (a DMA builtin written directly in a template
// kernel's body made the host pass drop that kernel's launch stub).
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          void *lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, 0);
}

// v + (v moved by the DPP control CTRL), every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                false);
  return v + __builtin_bit_cast(float, moved);
}

// max(v, v moved by the DPP control CTRL), every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                false);
  return fmaxf(v, __builtin_bit_cast(float, moved));
}

// Sum / maximum over each aligned group of G = 8 or 16 lanes, in every lane
// of the group (quad butterflies, then the half-row and row mirrors).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  if constexpr (G == 16) v = dpp_add<0x140>(v);  // row_mirror
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
  v = dpp_max<0xB1>(v);
  v = dpp_max<0x4E>(v);
  v = dpp_max<0x141>(v);
  if constexpr (G == 16) v = dpp_max<0x140>(v);
  return v;
}

// Sum over each group of 32 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float half_wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  // xor 16 inside each 32-lane group (ds_swizzle bit mode, xor_mask = 16)
  const int o = __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F);
  return v + __builtin_bit_cast(float, o);
}

// The 32 activations of a GEMV chunk -- k = base + 16 j + e, j = 0..3,
// e = 0..7, ar pointing at k = base -- into every lane of a wave whose two
// halves (lanes l and l + 32, h = l / 32) work on the same chunk: each half
// loads two of the four 8-float runs (h = 0 runs 0 and 1, h = 1 runs 2 and 3)
// and v_permlane32_swap hands each half the other's, so the wave issues half
// the load instructions for the same values.  Every lane must take part
// (full exec mask).
__device__ __forceinline__ void load_chunk32_paired(const float *ar, int h, float *av) {
  float part[16];
  const float *ah = ar + 32 * h;
#pragma unroll
  for (int jj = 0; jj < 2; jj++) {
    const float4 x0 = *(const float4 *)(ah + 16 * jj);
    const float4 x1 = *(const float4 *)(ah + 16 * jj + 4);
    part[8 * jj + 0] = x0.x; part[8 * jj + 1] = x0.y; part[8 * jj + 2] = x0.z;
    part[8 * jj + 3] = x0.w; part[8 * jj + 4] = x1.x; part[8 * jj + 5] = x1.y;
    part[8 * jj + 6] = x1.z; part[8 * jj + 7] = x1.w;
  }
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const unsigned u = __builtin_bit_cast(unsigned, part[e]);
    // [0]: lanes 0-31's value in every lane, [1]: lanes 32-63's
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    av[e] = __builtin_bit_cast(float, (unsigned)sw[0]);
    av[16 + e] = __builtin_bit_cast(float, (unsigned)sw[1]);
  }
}

// ---- Exact weight dequantisation for the fp32 FMA kernels.
//
// A weight dword w holds 8 nibbles q_e (e = 0..7; byte b holds e = 2b in its
// low and e = 2b+1 in its high nibble).  The kernels need (q - zp) exactly:
// the reference forms fl32((q - zp) * scale) per weight
// (onnx_qlinear_ops.dart:146), so a block whose nibbles all equal its zero
// point contributes exactly zero.  Folding the zero point in afterwards
// (scale * sum a q - scale * zp * sum a) cancels catastrophically there.
//
// Each nibble becomes the exact (q - zp) times a power of two with one SDWA
// convert:
//   zero point 8 (no zero-point input): q ^ 8 is the 4-bit two's complement
//     of q - 8.  v_cvt_off_f32_i4 converts the signed 4-bit value in bits
//     3:0 of its (byte-selected) operand to value / 16, so the low nibbles
//     of w ^ 0x88888888 and of (w ^ 0x88888888) >> 4 give (q - 8) / 16
//     directly: two bit operations per dword;
//   any zero point z: 8q + (128 - 8z) lies in [8, 248] (no carry between
//     bytes), and xor 0x80 turns that excess-128 byte into 8 (q - z), read
//     by a sign-extending byte convert.
// The products a * (q - 8) / 16 and a * 8(q - z) are the exact products
// scaled by a power of two; the kernels undo it once on the accumulated
// value (dq_unscale).

// Signed byte B of v as float (v_cvt_f32_i32 with an SDWA sign-extended
// byte select: one instruction).
template <int B>
__device__ __forceinline__ float sbyte_f32(uint32_t v) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(r) : "v"(v));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(r) : "v"(v));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(r) : "v"(v));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(r) : "v"(v));
  return r;
}

// The signed 4-bit value in bits 3:0 of byte B of v, divided by 16
// (v_cvt_off_f32_i4 with an SDWA byte select: one instruction).
template <int B>
__device__ __forceinline__ float snib16_f32(uint32_t v) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(r) : "v"(v));
  else if constexpr (B == 1)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(r) : "v"(v));
  else if constexpr (B == 2)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(r) : "v"(v));
  else
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(r) : "v"(v));
  return r;
}

// The byte-offset constant of zero point z for the explicit-zero-point form.
__device__ __forceinline__ uint32_t dq8_const(int z) { return (uint32_t)(128 - 8 * z) * 0x01010101u; }

// Scale S of the dequantised values: 1/16 (zero point 8) or 8 (explicit
// zero points); the kernels multiply each block's scale by 1 / S (exact for
// normal scales), so no sum is S times larger or smaller than the result.
template <bool HAS_ZP>
constexpr float dq_unscale() { return HAS_ZP ? 0.125f : 16.0f; }

// Nibbles of w as 8 floats f[e] = S * (q_e - z), S = 1/16 (HAS_ZP false,
// z = 8) or 8 (HAS_ZP true, zc = dq8_const(z)); exact.
template <bool HAS_ZP>
__device__ __forceinline__ void dq_nibbles(uint32_t w, uint32_t zc, float *f) {
  if constexpr (HAS_ZP) {
    const uint32_t lo = (((w << 3) & 0x78787878u) + zc) ^ 0x80808080u;
    const uint32_t hi = (((w >> 1) & 0x78787878u) + zc) ^ 0x80808080u;
    f[0] = sbyte_f32<0>(lo);
    f[1] = sbyte_f32<0>(hi);
    f[2] = sbyte_f32<1>(lo);
    f[3] = sbyte_f32<1>(hi);
    f[4] = sbyte_f32<2>(lo);
    f[5] = sbyte_f32<2>(hi);
    f[6] = sbyte_f32<3>(lo);
    f[7] = sbyte_f32<3>(hi);
  } else {
    const uint32_t x = w ^ 0x88888888u, xh = x >> 4;
    f[0] = snib16_f32<0>(x);
    f[1] = snib16_f32<0>(xh);
    f[2] = snib16_f32<1>(x);
    f[3] = snib16_f32<1>(xh);
    f[4] = snib16_f32<2>(x);
    f[5] = snib16_f32<2>(xh);
    f[6] = snib16_f32<3>(x);
    f[7] = snib16_f32<3>(xh);
  }
}

// Greedy-decoding key of a logit: orderable bits of v above ~col, so the
// largest key is the largest logit with ties going to the lowest column.
__device__ __forceinline__ unsigned long long argmax_key(float v, int col) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)col);
}

// Loads and stores of data that another workgroup of the same launch writes
// or reads (COH): agent-scope relaxed atomics, which bypass the per-XCD L2
// and so are coherent across XCDs without a cache flush.  Completion of such
// stores (s_waitcnt vmcnt(0)) before a grid-wide signal publishes them.
template <bool COH>
__device__ __forceinline__ float ld_act(const float *p) {
  if constexpr (COH)
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

template <bool COH>
__device__ __forceinline__ void st_act(float *p, float v) {
  if constexpr (COH)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}

// ---- The prefill GEMM's prepared activations (written by k_prep_a, or by a
// producer kernel that owns whole rows).  Row m is scaled by 2^e_m, e_m
// chosen from the row's largest magnitude so that it lands in [2^13, 2^14),
// and split into two fp16 terms hi = fp16(a'), lo = fp16(a' - hi).  Layout:
// one 1 KB unit per (32-row block, 64-k segment s, 16-k step j, part hi|lo),
// lane l holding row l%32, k = 64s + 16j + 8(l/32) + {0,4,1,5,2,6,3,7}.

// |v| for finite v, 0 for NaN and infinities: rows are scaled by their
// largest FINITE magnitude, so the finite elements of a row that also holds
// an infinity or a NaN keep their precision and stay within fp16's range.
__device__ __forceinline__ float finite_abs(float v) {
  const float a = fabsf(v);
  return a < INFINITY ? a : 0.0f;
}

// The row exponent e_m for a row whose largest finite magnitude is mx (0 for
// an all-zero row).
__device__ __forceinline__ int prep_a_exponent(float mx) {
  return (mx > 0.0f && mx < INFINITY) ? 13 - ilogbf(mx) : 0;
}

typedef _Float16 prep_h8 __attribute__((ext_vector_type(8)));

// Stores half g (k = k0 + 8g .. k0 + 8g + 7; k0 a multiple of 16) of row
// `row`, values v[0..7], exponent ex, into the units of a layout with segsp
// segments per row block.
__device__ __forceinline__ void prep_a_store8(uint4 *__restrict__ out, int64_t segsp,
                                              int64_t row, int64_t k0, int g, const float *v,
                                              int ex) {
  const int64_t rb = row >> 5;
  const int rl = (int)(row & 31);
  const int64_t s = k0 >> 6;
  const int j = (int)((k0 >> 4) & 3);
  const int64_t base = ((rb * segsp + s) * 4 + j) * 2;  // unit index of part 0
  _Float16 hi[8], lo[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float x = ldexpf(v[e], ex);
    const _Float16 h = (_Float16)x;
    hi[e] = h;
    // a NaN or infinite element keeps hi = x and lo = 0 (x - hi would be
    // NaN for an infinity): each product hi * w is then the reference's
    // a * w, +-inf, or NaN where w == 0, and the sums follow IEEE as its do
    const float d = x - (float)h;
    lo[e] = (_Float16)(d == d ? d : 0.0f);
  }
  const prep_h8 hv = {hi[0], hi[4], hi[1], hi[5], hi[2], hi[6], hi[3], hi[7]};
  const prep_h8 lv = {lo[0], lo[4], lo[1], lo[5], lo[2], lo[6], lo[3], lo[7]};
  out[(base + 0) * 64 + 32 * g + rl] = __builtin_bit_cast(uint4, hv);
  out[(base + 1) * 64 + 32 * g + rl] = __builtin_bit_cast(uint4, lv);
}

// Both halves: k = k0 .. k0+15 of row `row`, values v[0..15].
__device__ __forceinline__ void prep_a_store16(uint4 *__restrict__ out, int64_t segsp,
                                               int64_t row, int64_t k0, const float *v,
                                               int ex) {
  prep_a_store8(out, segsp, row, k0, 0, v, ex);
  prep_a_store8(out, segsp, row, k0, 1, v + 8, ex);
}

}  // namespace mmnb
