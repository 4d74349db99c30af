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

typedef __bf16 gdn_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float gdn_f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even float -> bf16 bits (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two bf16 values packed into one dword (lo element in the low half), one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const gdn_f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, gdn_bf16x2_t));
}

// The two floats a packed bf16 pair represents.
__device__ __forceinline__ float bf16lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

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
