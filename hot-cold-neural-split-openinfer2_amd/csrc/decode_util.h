// Token arithmetic shared by the decode kernels: fp16/bf16 rounding, the one
// canonical RMSNorm factor (so every kernel agrees bit for bit) and the
// normalised-token value the predictor query uses.
#pragma once
#include "oi2_device.h"

namespace oi2 {

// ── small helpers ──────────────────────────────────────────────────────────

__device__ __forceinline__ float half_lo(uint32_t d) { return half_bits_to_float((uint16_t)(d & 0xFFFFu)); }
__device__ __forceinline__ float half_hi(uint32_t d) { return half_bits_to_float((uint16_t)(d >> 16)); }

__device__ __forceinline__ float round_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __builtin_bit_cast(float, u & 0xFFFF0000u);
}

__device__ __forceinline__ float round_f16(float f) { return (float)(_Float16)f; }

// The one RMSNorm factor every kernel uses, so all of them agree bit for bit:
// partial t = sequential fma of x[16t .. 16t+16)^2; total = DPP tree over
// lanes of (p[4l] + p[4l+1]) + (p[4l+2] + p[4l+3]); r = rsqrt(total/H + eps).
__device__ __forceinline__ float ssq16(const float v[16]) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s = fmaf(v[e], v[e], s);
  return s;
}

// r from this lane's four partials (loaded early by the caller; all 64 lanes
// of the wave take part).
__device__ __forceinline__ float r_from_part(f32x4 p, float eps) {
  const float s = wave_sum((p.x + p.y) + (p.z + p.w));
  return rsqrtf(s * (1.0f / kH) + eps);
}

__device__ __forceinline__ f32x4 load_part(const float* parts) {
  return reinterpret_cast<const f32x4*>(parts)[lane_id()];
}

__device__ __forceinline__ float r_from_parts(const float* parts, float eps) {
  return r_from_part(load_part(parts), eps);
}

__device__ __forceinline__ void load_h16(const uint16_t* x, int e0, float v[16]) {
  const u32x4* px = reinterpret_cast<const u32x4*>(x + e0);
  const u32x4 a = px[0], b = px[1];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    v[2 * d] = half_lo(a[d]);
    v[2 * d + 1] = half_hi(a[d]);
    v[8 + 2 * d] = half_lo(b[d]);
    v[8 + 2 * d + 1] = half_hi(b[d]);
  }
}

// Block-wide canonical r for one H-row of x (every thread must call it).
__device__ float block_rnorm(const uint16_t* x, float eps, float* s_parts) {
  float v[16];
  load_h16(x, 16 * threadIdx.x, v);
  s_parts[threadIdx.x] = ssq16(v);
  __syncthreads();
  const float r = r_from_parts(s_parts, eps);
  __syncthreads();
  return r;
}

// x_n = fp16((x * r) * w): the normalised hidden state as nn.RMSNorm's fp16
// output (engine.py:247-249); the predictor query, oi2_rmsnorm and the
// kernels that normalise their own input use it.  The fp32 product passes
// through an empty asm before the fp16 rounding: otherwise instruction
// selection fuses the last product with the rounding (v_fma_mixlo_f16, one
// rounding instead of fp32 then fp16) in some kernels and not in others,
// whatever the contraction setting, and the kernels' x_n then differ in rare
// elements by one fp16 ulp - enough to move a predictor logit across the
// threshold.
__device__ __forceinline__ float xn_exact(float x, float r, float w) {
  float u = x * r * w;
  asm("" : "+v"(u));
  return round_f16(u);
}

}  // namespace oi2
