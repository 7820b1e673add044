// Grouped-query attention for decode on gfx950: GroupedQueryAttention.forward
// (engine.py:90-125) with the KV cache kept in place.
//
// One call runs three kernels on its stream:
//   k_attn_gemv (qkv)  RMSNorm of the token rows (input_layernorm,
//                      engine.py:93), then q, k, v = fp16(x_n W^T) from the
//                      fp8 e4m3fn weights (the reference keeps them fp8 at
//                      rest and widens to fp16, engine.py:80-83), RoPE on q
//                      and k (engine.py:102-103, 140-157), q to a buffer and
//                      k, v appended to the cache at past + t (engine.py:105-109)
//   k_attn_sdpa1       attention of every query row over its visible cache
//                      positions (engine.py:114-121) for spans of at most
//                      1024 positions: one workgroup per (row, query head)
//                      reads the whole span and writes the output
//   k_attn_sdpa        the same for longer spans: split over the sequence,
//                      every K / V row read once for the group's query heads;
//                      the last workgroup of a (row, kv head) merges the splits
//   k_attn_gemv (out)  out = fp16(attn W_o^T) (engine.py:122-123), and
//                      optionally x + out in the same pass
//
// Rounding follows the reference's fp16 tensors: x_n, q, k, v, the RoPE
// products, sums and differences, the attention output and out are each
// rounded to fp16 where the reference's fp16 ops round them; dot products
// accumulate in fp32.
//
// Cache layout: k_cache, v_cache (batch, n_kv, cap, 128) fp16, the
// reference's (B, n_kv, S, D) tensors with room for cap positions.
#include "capi_util.h"
#include "decode_util.h"

namespace oi2 {
namespace {

constexpr int kHd = 128;                 // head_dim (engine.py:72: hidden / n_q)
constexpr int kHalf = kHd / 2;
constexpr int kThreads = 256;
constexpr int kMaxRows = 8;              // token rows per GEMV launch
constexpr int kMinPosPerWg = 32;         // 4 waves x 2 steps of 4 positions
constexpr int kMaxTabBytes = 64 << 10;   // the merge's m / l table in LDS

struct GemvArgs {
  const uint16_t* x;          // this launch's first input row (rows, H)
  int row0;                   // call-wide index of that row (b * seq + t)
  const uint16_t* norm_w;     // RMSNorm weight, or null: the rows are used as they are
  float eps;
  const uint8_t* w0;          // weight blocks of 128 rows (.., H), fp8 e4m3fn
  const uint8_t* w1;
  const uint8_t* w2;
  int blocks0, blocks1;       // 128-row blocks in w0 and w1; the rest are w2's
  int mode;                   // 0: q / k / v epilogue, 1: output epilogue
  // mode 0
  uint16_t* q;                // (rows, n_q * 128)
  int q_width;                // n_q * 128
  uint16_t* k_cache;
  uint16_t* v_cache;
  int n_kv, cap, past, seq;
  const float* cos;           // (seq, 64)
  const float* sin;
  uint32_t* counters;         // cleared here (once per call) for k_attn_sdpa
  int n_counters;
  // mode 1
  uint16_t* out;              // (rows, H)
  const uint16_t* residual;   // (rows, H) or null
  uint16_t* x_out;
};

struct SdpaArgs {
  const uint16_t* q;          // (rows, n_kv * G * 128)
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int n_kv, cap, past, seq, causal, n_split, part_stride;
  float scale;
  float* part;                // (rows, n_kv, n_split, part_stride)
  uint32_t* counters;         // (rows, n_kv)
  uint16_t* out;              // (rows, n_kv * G * 128)
};

// Workgroup barrier on LDS traffic only: the weight loads stay in flight.
__device__ __forceinline__ void lds_bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16 fp16 (two dwords x 4, natural order) -> float.
__device__ __forceinline__ void unpack16(const u32x4 (&x)[2], float v[16]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    v[2 * d] = half_lo(x[0][d]);
    v[2 * d + 1] = half_hi(x[0][d]);
    v[8 + 2 * d] = half_lo(x[1][d]);
    v[8 + 2 * d + 1] = half_hi(x[1][d]);
  }
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return (uint32_t)float_to_half_bits(a) | ((uint32_t)float_to_half_bits(b) << 16);
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kSc1 = 16;                 // cache-policy operand: agent-coherent access

// A buffer descriptor over [p, p + bytes); p and bytes must be uniform over
// the wave (lane 0's are taken).  Offsets past the range read zero.
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

template <typename T>
__device__ __forceinline__ void st_coherent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T ld_coh(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp8 GEMV over R token rows.  Wave w of workgroup b takes the row pair
// (128 blk + j, 128 blk + j + 64) of block blk, task = 4 b + w, j = task & 63:
// the two rows RoPE rotates together sit in one wave.  Lane l reads 16 weight
// bytes at 16 l + 1024 i (i < 4) of each row; the inputs it multiplies them
// with were staged in LDS in that order, so its LDS reads are consecutive
// 16-byte pieces across the wave.
template <int R>
__global__ __launch_bounds__(kThreads) void k_attn_gemv(GemvArgs a) {
  __shared__ __align__(16) uint16_t s_x[R * kH];
  __shared__ __align__(16) float s_parts[R][kThreads];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int task = blockIdx.x * 4 + wave;
  const int hb = task >> 6, j = task & 63;

  if (a.counters && blockIdx.x == 0)
    for (int i = tid; i < a.n_counters; i += kThreads) a.counters[i] = 0u;

  // this thread's 16 input elements of every row, then the weights
  u32x4 xin[R][2];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const u32x4* px = reinterpret_cast<const u32x4*>(a.x + (size_t)r * kH + 16 * tid);
    xin[r][0] = px[0];
    xin[r][1] = px[1];
  }
  u32x4 wn[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
  if (a.norm_w) {
    const u32x4* pw = reinterpret_cast<const u32x4*>(a.norm_w + 16 * tid);
    wn[0] = pw[0];
    wn[1] = pw[1];
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint8_t* W;
  int blk;
  if (hb < a.blocks0) {
    W = a.w0;
    blk = hb;
  } else if (hb < a.blocks0 + a.blocks1) {
    W = a.w1;
    blk = hb - a.blocks0;
  } else {
    W = a.w2;
    blk = hb - a.blocks0 - a.blocks1;
  }
  const uint8_t* row0 = W + (size_t)(blk * kHd + j) * kH + 16 * lane;
  const uint8_t* row1 = row0 + (size_t)kHalf * kH;
  u32x4 w0[4], w1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w0[i] = load16_nt(row0 + 1024 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) w1[i] = load16_nt(row1 + 1024 * i);
  __builtin_amdgcn_sched_barrier(0);

  // x_n = fp16((x r) w) (nn.RMSNorm on fp16, engine.py:93), staged in LDS:
  // thread t holds elements [16 t, 16 t + 16), which GEMV lane t & 63 needs
  // for its piece i = t >> 6; its two halves go to pieces 2 i and 2 i + 1 of
  // 64 consecutive 16-byte slots.  One row at a time, from the packed
  // inputs, so that only one row's floats are live.
  if (a.norm_w) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v[16];
      unpack16(xin[r], v);
      s_parts[r][tid] = ssq16(v);
    }
    lds_bar();
  }
  float wf[16];
  unpack16(wn, wf);
  {
    const int i = tid >> 6, l = tid & 63;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v[16];
      unpack16(xin[r], v);
      if (a.norm_w) {
        const float rr = r_from_parts(&s_parts[r][0], a.eps);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = xn_exact(v[e], rr, wf[e]);
      }
      u32x4 lo, hi;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        lo[d] = pack_f16x2(v[2 * d], v[2 * d + 1]);
        hi[d] = pack_f16x2(v[8 + 2 * d], v[8 + 2 * d + 1]);
      }
      u32x4* sx = reinterpret_cast<u32x4*>(s_x + (size_t)r * kH);
      sx[(2 * i) * 64 + l] = lo;
      sx[(2 * i + 1) * 64 + l] = hi;
    }
  }
  lds_bar();

  float acc[2 * R];
#pragma unroll
  for (int e = 0; e < 2 * R; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x2 p0[8], p1[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      p0[2 * d] = fp8x2_to_f16x2(w0[i][d], false);
      p0[2 * d + 1] = fp8x2_to_f16x2(w0[i][d], true);
      p1[2 * d] = fp8x2_to_f16x2(w1[i][d], false);
      p1[2 * d + 1] = fp8x2_to_f16x2(w1[i][d], true);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4* sx = reinterpret_cast<const u32x4*>(s_x + (size_t)r * kH);
      const u32x4 xa = sx[(2 * i) * 64 + lane], xb = sx[(2 * i + 1) * 64 + lane];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        acc[2 * r] = dot2(p0[m], as_f16x2(xa[m]), acc[2 * r]);
        acc[2 * r + 1] = dot2(p1[m], as_f16x2(xa[m]), acc[2 * r + 1]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        acc[2 * r] = dot2(p0[4 + m], as_f16x2(xb[m]), acc[2 * r]);
        acc[2 * r + 1] = dot2(p1[4 + m], as_f16x2(xb[m]), acc[2 * r + 1]);
      }
    }
  }
  wave_sums_to_last<2 * R>(acc);
  float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s0 = readlane_f(acc[2 * r], 63), s1 = readlane_f(acc[2 * r + 1], 63);
    if (lane == r) {
      t0 = s0;
      t1 = s1;
    }
  }
  if (lane >= R) return;
  const int row = a.row0 + lane;
  const float y0 = round_f16(t0), y1 = round_f16(t1);
  if (a.mode == 1) {
    uint16_t* o = a.out + (size_t)row * kH + hb * kHd + j;
    o[0] = float_to_half_bits(y0);
    o[kHalf] = float_to_half_bits(y1);
    if (a.residual) {
      const uint16_t* rs = a.residual + (size_t)row * kH + hb * kHd + j;
      uint16_t* xo = a.x_out + (size_t)row * kH + hb * kHd + j;
      xo[0] = float_to_half_bits(half_bits_to_float(rs[0]) + y0);
      xo[kHalf] = float_to_half_bits(half_bits_to_float(rs[kHalf]) + y1);
    }
    return;
  }
  const int b = row / a.seq, t = row - b * a.seq;
  float o0 = y0, o1 = y1;
  if (hb < a.blocks0 + a.blocks1) {
    // engine.py:150-157: cat(x1 cos - x2 sin, x1 sin + x2 cos), the tables
    // cast to fp16 and every product and sum an fp16 op
    const float c = round_f16(a.cos[t * kHalf + j]), s = round_f16(a.sin[t * kHalf + j]);
    o0 = round_f16(round_f16(y0 * c) - round_f16(y1 * s));
    o1 = round_f16(round_f16(y0 * s) + round_f16(y1 * c));
  }
  uint16_t* dst;
  if (hb < a.blocks0) {
    dst = a.q + (size_t)row * a.q_width + blk * kHd + j;
  } else {
    uint16_t* cache = hb < a.blocks0 + a.blocks1 ? a.k_cache : a.v_cache;
    dst = cache + (((size_t)b * a.n_kv + blk) * a.cap + (a.past + t)) * kHd + j;
  }
  dst[0] = float_to_half_bits(o0);
  dst[kHalf] = float_to_half_bits(o1);
}

// Attention of query row r (batch b, position past + t) against kv head g's
// cache positions [0, n_r), n_r = past + t + 1 when causal, else past + seq
// (engine.py:118-121: causal only without a cache).  Workgroup (split, g, r)
// takes 4 STEPS positions per wave, 16 STEPS per workgroup.  Lane
// (k = lane >> 4, jj = lane & 15) holds dims [8 jj, 8 jj + 8) of position
// 4 step + k, so one 16-byte load per lane reads 4 whole K (or V) rows, and
// the 16-lane row sums give each of the G query heads its score.  Each wave
// keeps its own max, exp-sum and weighted V sum; the workgroup merges its 4
// waves and stores one partial; the workgroup that completes the set of
// partials of (r, g) merges them into the fp16 output, its loads all
// independent of each other (the m / l table first, then 16-byte pieces of
// the partial sums, several in flight per thread).
template <int G, int STEPS>
__global__ __launch_bounds__(kThreads) void k_attn_sdpa(SdpaArgs a) {
  extern __shared__ float s_tab[];                 // merge: m then l, (n_split, G) each
  // the waves' partial sums; later the merge's per-group sums (1024 floats)
  constexpr int kRedFloats = 4 * G * kHd > 1024 ? 4 * G * kHd : 1024;
  __shared__ __align__(16) float s_red[kRedFloats];
  float (*s_o)[G][kHd] = reinterpret_cast<float (*)[G][kHd]>(s_red);
  __shared__ float s_m[4][G], s_l[4][G];
  __shared__ uint32_t s_last;
  constexpr int kPW = 4 * STEPS;
  const int split = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6, k = lane >> 4, jj = lane & 15;
  const int b = r / a.seq, t = r - b * a.seq;
  const int n_r = a.causal ? a.past + t + 1 : a.past + a.seq;
  const int width = a.n_kv * G * kHd;
  const int base = split * 4 * kPW + wave * kPW;

  u32x4 qv[G];
#pragma unroll
  for (int h = 0; h < G; ++h)
    qv[h] = *reinterpret_cast<const u32x4*>(a.q + (size_t)r * width + (g * G + h) * kHd + 8 * jj);
  const size_t head = ((size_t)b * a.n_kv + g) * a.cap;
  u32x4 kr[STEPS], vr[STEPS];
#pragma unroll
  for (int it = 0; it < STEPS; ++it) {
    const int p = base + 4 * it + k;
    const int pc = p < n_r ? p : n_r - 1;
    kr[it] = *reinterpret_cast<const u32x4*>(a.k_cache + (head + pc) * kHd + 8 * jj);
  }
#pragma unroll
  for (int it = 0; it < STEPS; ++it) {
    const int p = base + 4 * it + k;
    const int pc = p < n_r ? p : n_r - 1;
    vr[it] = *reinterpret_cast<const u32x4*>(a.v_cache + (head + pc) * kHd + 8 * jj);
  }

  float s[STEPS * G];
#pragma unroll
  for (int it = 0; it < STEPS; ++it)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float d = 0.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m) d = dot2(as_f16x2(kr[it][m]), as_f16x2(qv[h][m]), d);
      s[it * G + h] = d;
    }
  // sums over the 16 lanes of each row: every lane of the row gets the total
#pragma unroll
  for (int e = 0; e < STEPS * G; ++e) s[e] += dpp_f<0xB1>(s[e]);
#pragma unroll
  for (int e = 0; e < STEPS * G; ++e) s[e] += dpp_f<0x4E>(s[e]);
#pragma unroll
  for (int e = 0; e < STEPS * G; ++e) s[e] += dpp_f<0x141>(s[e]);
#pragma unroll
  for (int e = 0; e < STEPS * G; ++e) s[e] += dpp_f<0x140>(s[e]);

  const float ninf = -__builtin_inff();
  float mx[G];
#pragma unroll
  for (int h = 0; h < G; ++h) mx[h] = ninf;
#pragma unroll
  for (int it = 0; it < STEPS; ++it) {
    const bool ok = base + 4 * it + k < n_r;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s[it * G + h] = ok ? s[it * G + h] * a.scale : ninf;
      mx[h] = fmaxf(mx[h], s[it * G + h]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    mx[h] = fmaxf(mx[h], __shfl_xor(mx[h], 16));
    mx[h] = fmaxf(mx[h], __shfl_xor(mx[h], 32));
  }
  float l[G], o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
  }
#pragma unroll
  for (int it = 0; it < STEPS; ++it) {
    float vf[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      vf[2 * d] = half_lo(vr[it][d]);
      vf[2 * d + 1] = half_hi(vr[it][d]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float sv = s[it * G + h];
      const float p = sv == ninf ? 0.0f : __expf(sv - mx[h]);
      l[h] += p;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = fmaf(p, vf[e], o[h][e]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] += __shfl_xor(l[h], 16);
    l[h] += __shfl_xor(l[h], 32);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[h][e] += __shfl_xor(o[h][e], 16);
      o[h][e] += __shfl_xor(o[h][e], 32);
    }
  }
  if (k == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wave][h][8 * jj + e] = o[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_m[wave][h] = mx[h];
      s_l[wave][h] = l[h];
    }
  }
  __syncthreads();

  float* part_rg = a.part + (size_t)(r * a.n_kv + g) * a.n_split * a.part_stride;
  float* mine = part_rg + (size_t)split * a.part_stride;
  for (int idx = tid; idx < G * kHd; idx += kThreads) {
    const int h = idx / kHd, d = idx - h * kHd;
    float M = ninf;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][h]);
    float ow = 0.0f, lw = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = s_m[w][h] == ninf ? 0.0f : __expf(s_m[w][h] - M);
      ow = fmaf(sc, s_o[w][h][d], ow);
      lw = fmaf(sc, s_l[w][h], lw);
    }
    st_coherent(mine + h * kHd + d, ow);
    if (d == 0) {
      st_coherent(mine + G * kHd + h, M);
      st_coherent(mine + G * kHd + G + h, lw);
    }
  }
  // publish: every store acknowledged, then one arrival; the arrival that
  // completes the set merges it
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(a.counters + r * a.n_kv + g, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    s_last = old + 1 == (uint32_t)a.n_split ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;

  // thread (grp, h, q): 4 dims [4 q, 4 q + 4) of head h over splits
  // grp, grp + kGrp, ...: its 16-byte agent-coherent loads of the partial
  // sums (up to 8 at once) go out first, then the m / l table of every
  // split (one agent-coherent load per entry), so both are in flight
  // together
  const int n_split = a.n_split;
  float* s_pm = s_tab;
  float* s_pl = s_tab + n_split * G;
  constexpr int kGrp = kThreads / (32 * G);
  constexpr int kBatch = 8;
  const int q = tid & 31, h = (tid >> 5) % G, grp = tid / (32 * G);
  const rsrc_t rs = make_rsrc(part_rg, (uint32_t)((size_t)n_split * a.part_stride * 4));
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  u32x4 pv[kBatch];
  auto load_batch = [&](int sp0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int sp = sp0 + u * kGrp;
      // a split past the end reads zero through the descriptor's range
      const uint32_t off = sp < n_split ? (uint32_t)(((size_t)sp * a.part_stride + h * kHd + 4 * q) * 4)
                                        : 0xFFFFFFF0u;
      pv[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kSc1);
    }
  };
  load_batch(grp);
  for (int i = tid; i < n_split * G; i += kThreads) {
    const int sp = i / G, hh = i - sp * G;
    const float* P = part_rg + (size_t)sp * a.part_stride + G * kHd;
    s_pm[i] = ld_coh(P + hh);
    s_pl[i] = ld_coh(P + G + hh);
  }
  __syncthreads();
  float M = ninf;
  for (int sp = 0; sp < n_split; ++sp) M = fmaxf(M, s_pm[sp * G + h]);
  for (int sp0 = grp;;) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int sp = sp0 + u * kGrp;
      const float m = sp < n_split ? s_pm[sp * G + h] : ninf;
      const float w = m == ninf ? 0.0f : __expf(m - M);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(w, as_f32(pv[u][e]), acc[e]);
    }
    sp0 += kBatch * kGrp;
    if (sp0 >= n_split) break;
    load_batch(sp0);
  }
  __syncthreads();
  float* red = s_red;                               // kGrp x G x 128 = 1024 floats
#pragma unroll
  for (int e = 0; e < 4; ++e) red[(grp * G + h) * kHd + 4 * q + e] = acc[e];
  __syncthreads();
  if (grp != 0) return;
  float L = 0.0f;
  for (int sp = 0; sp < n_split; ++sp) {
    const float m = s_pm[sp * G + h];
    L = fmaf(m == ninf ? 0.0f : __expf(m - M), s_pl[sp * G + h], L);
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float O = 0.0f;
#pragma unroll
    for (int gg = 0; gg < kGrp; ++gg) O += red[(gg * G + h) * kHd + 4 * q + e];
    a.out[(size_t)r * width + (g * G + h) * kHd + 4 * q + e] = float_to_half_bits(O * inv);
  }
}

// Attention of query row r, query head hq, against its kv head's positions
// [0, n_r) in one workgroup, for spans of at most kOneWgMax positions: no
// partial sum leaves the workgroup, so there is no store to acknowledge, no
// arrival and no second pass over partial sums.  Workgroup x takes kv head
// g = x mod n_kv and query head hq = g G + x / n_kv, so that with 8 kv heads
// the G workgroups reading one kv head's cache share an XCD (and its L2).
// The 16 waves take chunks of 8 positions in turn (chunk c goes to wave
// c mod 16: at 513 positions 65 chunks, 4 or 5 per wave, against 2 or 3 for
// chunks of 16, 1.4 % slower); each wave keeps a running max, exp-sum and
// weighted V sum, rescaled when a chunk raises the max, with its next
// chunk's K / V loads in flight while it computes the current one.  The waves meet in LDS at the
// end.  Lane (k = lane >> 4, jj = lane & 15) holds dims [8 jj, 8 jj + 8) of
// position 8 c + 4 step + k, as in k_attn_sdpa; positions past n_r read zero
// through the descriptors' range and score -inf.
constexpr int kOneWgThreads = 1024;
constexpr int kOneWgMax = 1024;

__global__ __launch_bounds__(kOneWgThreads) void k_attn_sdpa1(SdpaArgs a, int G) {
  constexpr int kW = kOneWgThreads / kWave;
  constexpr int ST = 2;                           // steps of 4 positions per chunk
  constexpr int kChunk = 4 * ST;
  __shared__ __align__(16) float s_o[kW][kHd];
  __shared__ float s_m[kW], s_l[kW];
  const int g = blockIdx.x % a.n_kv, hq = g * G + blockIdx.x / a.n_kv, r = blockIdx.y;
  const int tid = threadIdx.x, lane = lane_id(), k = lane >> 4, jj = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = r / a.seq, t = r - b * a.seq;
  const int n_r = a.causal ? a.past + t + 1 : a.past + a.seq;
  const int width = a.n_kv * G * kHd;
  const float ninf = -__builtin_inff();

  const u32x4 qv = *reinterpret_cast<const u32x4*>(a.q + (size_t)r * width + hq * kHd + 8 * jj);
  const size_t head = ((size_t)b * a.n_kv + g) * a.cap * kHd;
  const rsrc_t rk = make_rsrc(a.k_cache + head, (uint32_t)n_r * kHd * 2);
  const rsrc_t rv = make_rsrc(a.v_cache + head, (uint32_t)n_r * kHd * 2);
  const int n_ch = (n_r + kChunk - 1) / kChunk;

  auto issue = [&](int c, u32x4 (&kr)[ST], u32x4 (&vr)[ST]) {
#pragma unroll
    for (int it = 0; it < ST; ++it)
      kr[it] = __builtin_amdgcn_raw_buffer_load_b128(
          rk, (uint32_t)(kChunk * c + 4 * it + k) * (kHd * 2) + 16 * jj, 0, 0);
#pragma unroll
    for (int it = 0; it < ST; ++it)
      vr[it] = __builtin_amdgcn_raw_buffer_load_b128(
          rv, (uint32_t)(kChunk * c + 4 * it + k) * (kHd * 2) + 16 * jj, 0, 0);
  };

  float m = ninf, l = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  auto chunk = [&](int c, const u32x4 (&kr)[ST], const u32x4 (&vr)[ST]) {
    float s[ST];
#pragma unroll
    for (int it = 0; it < ST; ++it) {
      float d = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) d = dot2(as_f16x2(kr[it][q]), as_f16x2(qv[q]), d);
      s[it] = d;
    }
#pragma unroll
    for (int e = 0; e < ST; ++e) s[e] += dpp_f<0xB1>(s[e]);
#pragma unroll
    for (int e = 0; e < ST; ++e) s[e] += dpp_f<0x4E>(s[e]);
#pragma unroll
    for (int e = 0; e < ST; ++e) s[e] += dpp_f<0x141>(s[e]);
#pragma unroll
    for (int e = 0; e < ST; ++e) s[e] += dpp_f<0x140>(s[e]);
    float cm = ninf;
#pragma unroll
    for (int it = 0; it < ST; ++it) {
      s[it] = kChunk * c + 4 * it + k < n_r ? s[it] * a.scale : ninf;
      cm = fmaxf(cm, s[it]);
    }
    cm = fmaxf(cm, __shfl_xor(cm, 16));
    cm = fmaxf(cm, __shfl_xor(cm, 32));
    const float mn = fmaxf(m, cm);
    // the running sums were taken against m; a chunk with a larger score
    // rescales them (exp(-inf) = 0 before the first valid score)
    const float alpha = mn == ninf ? 1.0f : __expf(m - mn);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= alpha;
    m = mn;
#pragma unroll
    for (int it = 0; it < ST; ++it) {
      const float p = s[it] == ninf ? 0.0f : __expf(s[it] - m);
      l += p;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        o[2 * d] = fmaf(p, half_lo(vr[it][d]), o[2 * d]);
        o[2 * d + 1] = fmaf(p, half_hi(vr[it][d]), o[2 * d + 1]);
      }
    }
  };

  // two register sets in turn: the next chunk's loads go out before the
  // current chunk's arithmetic (past the last chunk they read zero and
  // move no data)
  if (wave < n_ch) {
    u32x4 ka[ST], va[ST], kb[ST], vb[ST];
    int c = wave;
    issue(c, ka, va);
    for (;;) {
      issue(c + kW, kb, vb);
      __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the arithmetic
      chunk(c, ka, va);
      c += kW;
      if (c >= n_ch) break;
      issue(c + kW, ka, va);
      __builtin_amdgcn_sched_barrier(0);
      chunk(c, kb, vb);
      c += kW;
      if (c >= n_ch) break;
    }
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += __shfl_xor(o[e], 16);
    o[e] += __shfl_xor(o[e], 32);
  }
  if (k == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_o[wave][8 * jj + e] = o[e];
  }
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
  __syncthreads();
  if (tid < kHd) {
    float M = ninf;
#pragma unroll
    for (int w = 0; w < kW; ++w) M = fmaxf(M, s_m[w]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float sc = s_m[w] == ninf ? 0.0f : __expf(s_m[w] - M);
      O = fmaf(sc, s_o[w][tid], O);
      L = fmaf(sc, s_l[w], L);
    }
    a.out[(size_t)r * width + hq * kHd + tid] = float_to_half_bits(O * (1.0f / L));
  }
}

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline int part_stride_floats(int G) { return ((G * kHd + 2 * G) + 31) & ~31; }

template <int R>
void launch_gemv_r(const GemvArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL(k_attn_gemv<R>, dim3(blocks * 16), dim3(kThreads), 0, st, a);
}

void launch_gemv(const GemvArgs& a, int rows, int blocks, hipStream_t st) {
  switch (rows) {
    case 1: launch_gemv_r<1>(a, blocks, st); break;
    case 2: launch_gemv_r<2>(a, blocks, st); break;
    case 3: launch_gemv_r<3>(a, blocks, st); break;
    case 4: launch_gemv_r<4>(a, blocks, st); break;
    case 5: launch_gemv_r<5>(a, blocks, st); break;
    case 6: launch_gemv_r<6>(a, blocks, st); break;
    case 7: launch_gemv_r<7>(a, blocks, st); break;
    default: launch_gemv_r<8>(a, blocks, st); break;
  }
}

template <int G>
void launch_sdpa_g(const SdpaArgs& a, int steps, int rows, size_t lds, hipStream_t st) {
  const dim3 grid(a.n_split, a.n_kv, rows);
  switch (steps) {
    case 2: hipLaunchKernelGGL((k_attn_sdpa<G, 2>), grid, dim3(kThreads), lds, st, a); break;
    case 4: hipLaunchKernelGGL((k_attn_sdpa<G, 4>), grid, dim3(kThreads), lds, st, a); break;
    default: hipLaunchKernelGGL((k_attn_sdpa<G, 8>), grid, dim3(kThreads), lds, st, a); break;
  }
}

void launch_sdpa1(const SdpaArgs& a, int G, int rows, hipStream_t st) {
  hipLaunchKernelGGL(k_attn_sdpa1, dim3(a.n_kv * G, rows), dim3(kOneWgThreads), 0, st, a, G);
}

void launch_sdpa(const SdpaArgs& a, int G, int steps, int rows, size_t lds, hipStream_t st) {
  switch (G) {
    case 1: launch_sdpa_g<1>(a, steps, rows, lds, st); break;
    case 2: launch_sdpa_g<2>(a, steps, rows, lds, st); break;
    case 4: launch_sdpa_g<4>(a, steps, rows, lds, st); break;
    default: launch_sdpa_g<8>(a, steps, rows, lds, st); break;
  }
}

// Positions per wave step count: the longest span (8 steps, 128 positions
// per workgroup) that still gives at least 256 workgroups, else shorter
// spans for more of them (2 steps, 32 positions per workgroup at least).
int choose_steps(int rows, int n_kv, int n_max) {
  for (int steps = 8; steps > 2; steps /= 2) {
    const int64_t wgs = (int64_t)rows * n_kv * ((n_max + 16 * steps - 1) / (16 * steps));
    if (wgs >= 256) return steps;
  }
  return 2;
}

struct WsLayout {
  size_t q, attn, counters, part, total;
};

// The split partial sums are sized for the launch the call makes: none when
// the span (past + seq positions) fits one workgroup per query head, else
// the splits choose_steps picks for that span.
WsLayout ws_layout(int rows, int n_q, int n_kv, int span) {
  const int G = n_q / n_kv;
  const int per_split = span <= kOneWgMax ? 0 : 16 * choose_steps(rows, n_kv, span);
  const size_t n_split = per_split ? (size_t)(span + per_split - 1) / per_split : 0;
  WsLayout w;
  w.q = 0;
  w.attn = w.q + align256((size_t)rows * n_q * kHd * 2);
  w.counters = w.attn + align256((size_t)rows * kH * 2);
  w.part = w.counters + align256((size_t)rows * n_kv * 4);
  w.total = w.part + align256((size_t)rows * n_kv * n_split * part_stride_floats(G) * 4);
  return w;
}

}  // namespace
}  // namespace oi2

using namespace oi2;

extern "C" {

size_t oi2_attn_workspace_bytes(int32_t batch, int32_t seq, int32_t n_q, int32_t n_kv, int32_t past) {
  if (batch <= 0 || seq <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv || past < 0 ||
      (int64_t)past + seq > INT32_MAX)
    return 0;
  return ws_layout(batch * seq, n_q, n_kv, past + seq).total;
}

int oi2_attn_forward(const uint16_t* x, int32_t batch, int32_t seq, const oi2_attn* w, float eps,
                     const float* cos, const float* sin, uint16_t* k_cache, uint16_t* v_cache,
                     int32_t cache_cap, int32_t past, int32_t causal, uint16_t* out, uint16_t* x_out,
                     void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(w, "null attention weights");
  OI2_CHECK_ARG(batch >= 1 && seq >= 1, "batch %d, seq %d", batch, seq);
  const int n_q = w->n_q, n_kv = w->n_kv;
  OI2_CHECK_ARG(n_q * kHd == kH, "n_q %d: head_dim = %d / n_q must be %d", n_q, kH, kHd);
  OI2_CHECK_ARG(n_kv >= 1 && n_q % n_kv == 0, "n_kv %d does not divide n_q %d", n_kv, n_q);
  const int G = n_q / n_kv;
  OI2_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8, "query heads per kv head %d: 1, 2, 4 or 8", G);
  OI2_CHECK_ARG(past >= 0 && cache_cap >= 1 && (int64_t)past + seq <= cache_cap,
                "past %d + seq %d exceeds the cache capacity %d", past, seq, cache_cap);
  OI2_CHECK_ARG(x && (uintptr_t)x % 16 == 0, "x must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(w->wq && w->wk && w->wv && w->wo, "null weight");
  OI2_CHECK_ARG((uintptr_t)w->wq % 16 == 0 && (uintptr_t)w->wk % 16 == 0 && (uintptr_t)w->wv % 16 == 0 &&
                    (uintptr_t)w->wo % 16 == 0,
                "weights must be 16-byte aligned");
  OI2_CHECK_ARG(w->norm_w && (uintptr_t)w->norm_w % 16 == 0,
                "norm weight must be non-null (ones for nn.RMSNorm's default) and 16-byte aligned");
  OI2_CHECK_ARG(k_cache && v_cache && (uintptr_t)k_cache % 16 == 0 && (uintptr_t)v_cache % 16 == 0,
                "caches must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(cos && sin, "null RoPE tables");
  OI2_CHECK_ARG(out, "null output");
  OI2_CHECK_ARG((size_t)batch * n_kv * cache_cap * kHd < ((size_t)1 << 40), "cache too large");
  const int rows = batch * seq;
  const WsLayout L = ws_layout(rows, n_q, n_kv, past + seq);
  OI2_CHECK_ARG(workspace && workspace_bytes >= L.total, "workspace of %zu bytes, %zu needed",
                workspace_bytes, L.total);
  hipStream_t st = (hipStream_t)stream;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  uint16_t* qb = reinterpret_cast<uint16_t*>(ws + L.q);
  uint16_t* attn = reinterpret_cast<uint16_t*>(ws + L.attn);
  uint32_t* counters = reinterpret_cast<uint32_t*>(ws + L.counters);
  float* part = reinterpret_cast<float*>(ws + L.part);

  GemvArgs g{};
  g.norm_w = w->norm_w;
  g.eps = eps;
  g.w0 = w->wq;
  g.w1 = w->wk;
  g.w2 = w->wv;
  g.blocks0 = n_q;
  g.blocks1 = n_kv;
  g.mode = 0;
  g.q = qb;
  g.q_width = n_q * kHd;
  g.k_cache = k_cache;
  g.v_cache = v_cache;
  g.n_kv = n_kv;
  g.cap = cache_cap;
  g.past = past;
  g.seq = seq;
  g.cos = cos;
  g.sin = sin;
  g.n_counters = rows * n_kv;
  for (int r0 = 0; r0 < rows; r0 += kMaxRows) {
    const int rc = rows - r0 < kMaxRows ? rows - r0 : kMaxRows;
    g.x = x + (size_t)r0 * kH;
    g.row0 = r0;
    g.counters = r0 == 0 ? counters : nullptr;
    launch_gemv(g, rc, n_q + 2 * n_kv, st);
    OI2_CHECK_LAUNCH();
  }

  SdpaArgs s{};
  s.q = qb;
  s.k_cache = k_cache;
  s.v_cache = v_cache;
  s.n_kv = n_kv;
  s.cap = cache_cap;
  s.past = past;
  s.seq = seq;
  s.causal = causal ? 1 : 0;
  s.scale = 1.0f / sqrtf((float)kHd);
  s.out = attn;
  if (past + seq <= kOneWgMax) {
    // short spans: the whole span in one workgroup per (row, query head)
    s.n_split = 1;
    launch_sdpa1(s, G, rows, st);
    OI2_CHECK_LAUNCH();
  } else {
    const int steps = choose_steps(rows, n_kv, past + seq);
    s.n_split = (past + seq + 16 * steps - 1) / (16 * steps);
    s.part_stride = part_stride_floats(G);
    const size_t tab = (size_t)2 * s.n_split * G * sizeof(float);
    if (tab > (size_t)kMaxTabBytes) {
      set_error("%d positions need %d sequence splits; the merge table holds %d", past + seq, s.n_split,
                kMaxTabBytes / (int)(2 * G * sizeof(float)));
      return OI2_EUNSUPPORTED;
    }
    s.part = part;
    s.counters = counters;
    launch_sdpa(s, G, steps, rows, tab, st);
    OI2_CHECK_LAUNCH();
  }

  GemvArgs o{};
  o.norm_w = nullptr;
  o.w0 = w->wo;
  o.blocks0 = kH / kHd;
  o.blocks1 = 0;
  o.mode = 1;
  o.out = out;
  o.residual = x_out ? x : nullptr;
  o.x_out = x_out;
  for (int r0 = 0; r0 < rows; r0 += kMaxRows) {
    const int rc = rows - r0 < kMaxRows ? rows - r0 : kMaxRows;
    o.x = attn + (size_t)r0 * kH;
    o.row0 = r0;
    launch_gemv(o, rc, kH / kHd, st);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

}  // extern "C"
