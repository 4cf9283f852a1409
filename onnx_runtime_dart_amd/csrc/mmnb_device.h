// Device helpers shared by the libmmnb kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mmnb {

// s_waitcnt immediate that waits for vmcnt <= n (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima, i.e. no wait).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// v + (v moved by the DPP control CTRL), every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                false);
  return v + __builtin_bit_cast(float, moved);
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

}  // namespace mmnb
