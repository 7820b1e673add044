// Device-side helpers shared by the gfx950 kernels: record layout, INT4 / FP8
// decode, wave-64 reductions.
//
// Cold record layout (splitter.py:23-39, 55-76, 239-246): 6400 bytes =
//   u16 nid | gate 2048 B | up 2048 B | down 2048 B | 3 x 32 fp16 scales | pad
// Records sit at 16 + 6400 k past a 4096-aligned section start, so record
// bases are 16-byte aligned and every payload vector starts 2 bytes past a
// 16-byte boundary.  gfx950 under amdhsa runs global memory in unaligned
// mode, so the kernels read payload chunks with plain 16-byte loads at
// base + 2 + 16 c.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oi2 {

constexpr int kH = 4096;                 // hidden size the record format is sized for
constexpr int kGroup = 128;              // INT4 group size
constexpr int kGroups = kH / kGroup;     // 32 scales per vector
constexpr int kVecBytes = kH / 2;        // 2048 nibble bytes per vector
constexpr int kRecBytes = 6400;          // NEURON_RECORD_BYTES
constexpr int kOffGate = 2;
constexpr int kOffUp = kOffGate + kVecBytes;        // 2050
constexpr int kOffDown = kOffUp + kVecBytes;        // 4098
constexpr int kOffScales = kOffDown + kVecBytes;    // 6146
constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Bit reinterpretation of one dword.  Take the dword by value: clang's
// __builtin_bit_cast applied directly to an ext-vector element expression
// (v.y, v[k]) reads element 0 instead.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }

// 16 payload bytes at a 2-byte aligned address (one global_load_dwordx4).
__device__ __forceinline__ u32x4 load16_a2(const uint8_t* p) {
  return *reinterpret_cast<const u32x4_a2*>(p);
}

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// The same loads with the non-temporal hint, for weights that one launch
// reads once: a plain 2 GB read streams at ~6.0 TB/s on this GPU, a
// non-temporal one at ~7.3 TB/s.
__device__ __forceinline__ u32x4 load16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16_a2_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_a2*>(p));
}

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// Signed INT4 nibbles of one dword as exact fp16 pairs, splitter.py:111-124:
// byte b holds element 2k in bits 0-3 and 2k+1 in bits 4-7, two's complement.
// Output pairs: p[0] = (e0, e4), p[1] = (e1, e5), p[2] = (e2, e6), p[3] = (e3, e7),
// nibble k & 1 of each 16-bit half of d >> (8 (k >> 1)).
// A nibble at bits 0-3 of a half, its top bit flipped (n + 8, 0..15), in the
// mantissa of 1024.0 (0x6400) reads 1024 + n + 8: one and-xor,
// ((d & 0x000F000F) ^ 0x64086408), then - 1032.  A nibble at bits 4-7 reads
// 1024 + 16 (n + 8) the same way ((d & 0x00F000F0) ^ 0x64806480); times
// 1/16 minus 72 it is n.  Every step is exact in fp16.
__device__ __forceinline__ void int4x8_to_f16x2x4(uint32_t d, f16x2 p[4]) {
  const f16x2 b0 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const f16x2 s1 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const f16x2 b1 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const uint32_t d8 = d >> 8;
  p[0] = __builtin_bit_cast(f16x2, (d & 0x000F000Fu) ^ 0x64086408u) + b0;
  p[1] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (d & 0x00F000F0u) ^ 0x64806480u), s1, b1);
  p[2] = __builtin_bit_cast(f16x2, (d8 & 0x000F000Fu) ^ 0x64086408u) + b0;
  p[3] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (d8 & 0x00F000F0u) ^ 0x64806480u), s1, b1);
}

__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

// Two fp8 e4m3fn (bytes 0,1 or 2,3 of d) -> fp16 pair, exact (every e4m3 value
// is an fp16 normal).
__device__ __forceinline__ f16x2 fp8x2_to_f16x2(uint32_t d, bool hi) {
  return hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d, 1.0f, true)
            : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d, 1.0f, false);
}

__device__ __forceinline__ f32x2 fp8x2_to_f32x2(uint32_t d, bool hi) {
  return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(d, true) : __builtin_amdgcn_cvt_pk_f32_fp8(d, false);
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a wave with DPP (quad swaps, row mirrors, then
// row_bcast:15 / row_bcast:31 to carry row sums up to lane 63); every lane
// receives the total.  Fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);       // row_half_mirror
  v += dpp_f<0x140>(v);       // row_mirror
  v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return readlane_f(v, 63);
}

// The same DPP steps on a double, each step moving the two 32-bit halves.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xF,
                                                            false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// wave_sum in double precision (the predictor's sums, whose logits decide
// the active set against a threshold and must stay within a small fraction
// of 1e-6 of exact arithmetic).
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_d<0xB1>(v);
  v += dpp_d<0x4E>(v);
  v += dpp_d<0x141>(v);
  v += dpp_d<0x140>(v);
  v += dpp_d<0x142, 0xA>(v);
  v += dpp_d<0x143, 0xC>(v);
  return readlane_d(v, 63);
}

// N wave_sum reductions at once, one DPP step at a time for all N values, so
// the steps of different values overlap instead of waiting on each other.
// Each value goes through exactly wave_sum's additions; its total ends in
// lane 63.
template <int N>
__device__ __forceinline__ void wave_sums_to_last(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0x141>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0x140>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0x142, 0xA>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<0x143, 0xC>(v[i]);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Sums of 16 values over the 64 lanes of a wave, transposed: lane l returns
// the total of value l & 15.  Within each row of 16 lanes four steps halve the
// values a lane carries: the lane and its partner (row_mirror, then
// row_half_mirror, lane ^ 2, lane ^ 1) both add their copies of each half,
// and the lane keeps the half that its lane bit (3, 2, 1, 0) names.  Two lane
// exchanges then add the four rows.  About 50 instructions against 96 for 16
// separate reductions.
__device__ __forceinline__ float wave_sums16_transposed(const float (&v)[16]) {
  const int l = lane_id();
  float w[8], x[4], y[2];
  const bool b3 = (l >> 3) & 1, b2 = (l >> 2) & 1, b1 = (l >> 1) & 1, b0 = l & 1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float a = v[k] + dpp_f<0x140>(v[k]), b = v[k + 8] + dpp_f<0x140>(v[k + 8]);
    w[k] = b3 ? b : a;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = w[k] + dpp_f<0x141>(w[k]), b = w[k + 4] + dpp_f<0x141>(w[k + 4]);
    x[k] = b2 ? b : a;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float a = x[k] + dpp_f<0x4E>(x[k]), b = x[k + 2] + dpp_f<0x4E>(x[k + 2]);
    y[k] = b1 ? b : a;
  }
  const float a = y[0] + dpp_f<0xB1>(y[0]), b = y[1] + dpp_f<0xB1>(y[1]);
  float z = b0 ? b : a;
  z += __shfl_xor(z, 16);
  z += __shfl_xor(z, 32);
  return z;
}


// ── raw buffer access ─────────────────────────────────────────────────────

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
constexpr uint32_t kNoOff = 0x80000000u;       // an offset past every range: reads zero

// A buffer descriptor over [p, p + bytes).  p and bytes must be wave-uniform
// (lane 0's are taken for the whole wave); lane-dependent parts go in the
// access offset.  readfirstlane lets the compiler see the uniformity
// (otherwise it wraps each access in a loop over the wave's descriptors).
__device__ __forceinline__ rsrc_t rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  // readfirstlane returns int: widen each half as uint32_t, or a low half
  // >= 2^31 would sign-extend over the high half
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
// Plain buffer loads: a lane whose offset is past the range reads zero, so
// masked loads stay unconditional and the compiler never has to wait for one
// before issuing the next.
__device__ __forceinline__ u32x4 bld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2v bld8(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bld4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint16_t bld2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
// 16 bytes per lane straight into LDS: lane l lands at dst + 16 l (a lane past
// the range writes zero).  dst is the wave's 1 KB destination.
__device__ __forceinline__ void bld16_lds(rsrc_t r, void* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, off, 0, 0, 0);
}
// The same loads with the non-temporal hint, for weights that one launch
// reads once: a plain 2 GB read streams at ~6.0 TB/s on this GPU, a
// non-temporal one at ~7.3 TB/s.
constexpr int kNt = 2;
__device__ __forceinline__ u32x4 wld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNt);
}
__device__ __forceinline__ u32x2v wld8(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNt);
}
__device__ __forceinline__ void wld16_lds(rsrc_t r, void* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, off, 0, 0, kNt);
}
__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// engine.py:163-170: act = relu if activation == "relu" else silu;
// act(g) * act(u) when act_on_both, else act(g) * u.
__device__ __forceinline__ float gated_act(float g, float u, int relu, int both) {
  float ag = relu ? fmaxf(g, 0.0f) : silu(g);
  float au = both ? (relu ? fmaxf(u, 0.0f) : silu(u)) : u;
  return ag * au;
}

}  // namespace oi2
