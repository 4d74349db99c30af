// Device helpers shared by the GDN decode and prefill kernels (gfx950 / CDNA4).
//
// bf16 values travel as raw uint16_t bit patterns so that no vendor bf16 type
// appears in any signature.  Reductions use DPP row operations and ds_swizzle,
// which stay inside the wave and touch no LDS memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int kHeadDim = 128;  // dk == dv == 128 for every kernel in this library

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Round-to-nearest-even float -> bf16 bits; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// Two bf16 values packed into one dword (lo element in the low half).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}

// softplus with the torch default threshold: x > 20 -> x.
__device__ __forceinline__ float softplus20(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// Log-space decay of one token/head: -exp(A_log) * softplus(a + dt_bias).
__device__ __forceinline__ float log_gate(float A_log, float a, float dt_bias) {
  return -expf(A_log) * softplus20(a + dt_bias);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// Cross-lane moves.  DPP controls (GCN/CDNA encoding):
//   quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_ror:4 = 0x124, row_ror:8 = 0x128
// ds_swizzle bitmask mode: offset = xor_mask<<10 | or_mask<<5 | and_mask.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

template <int PATTERN>
__device__ __forceinline__ float swizzle(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), PATTERN));
}

// Sum over each aligned group of 16 lanes; every lane receives the group sum.
__device__ __forceinline__ float sum16(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x124>(x);
  x += dpp_mov<0x128>(x);
  return x;
}

// Sum over each aligned group of 32 lanes (half wave); every lane gets the sum.
__device__ __forceinline__ float sum32(float x) {
  x = sum16(x);
  x += swizzle<(0x10 << 10) | 0x1F>(x);  // lane ^ 16 inside the 32-lane group
  return x;
}

__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

}  // namespace gdn
