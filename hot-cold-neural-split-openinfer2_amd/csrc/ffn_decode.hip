// Decode-path kernels for gfx950: cold-record dequant, RMSNorm, the fused
// hot/cold FFN (two launches: gate/up phase, down phase) and the low-rank
// predictor with on-device index compaction.
//
// Launch shapes: 256 threads (4 wave64s) per workgroup everywhere.
//
// ffn_up   : workgroup roles by blockIdx range
//   cold   - wave gw takes chunk gw / wpc of the active list and every wpc-th
//            item of it: 16-byte loads of each record, gate and up dots
//            against the normalised token, activation, and the record's down
//            column times h into 64 accumulators per lane; one fp32 partial
//            row of y per workgroup, which ffn_down sums.
//   pred   - one wave per predictor down row (the lookahead layer's z).
//   hot    - two neurons per wave: fp8 gate/up rows -> fp16 pairs -> v_dot2.
// ffn_down : roles
//   pred   - 256 neurons per workgroup: logits = U z + b, threshold, LUT
//            filter, ballot/prefix compaction into an ascending chunk.
//   down   - 16 output rows per workgroup: fp8 down rows x h_hot (h staged in
//            LDS once per workgroup), plus the cold partial rows, plus the
//            residual; it also emits x * w_next and the sum-of-squares
//            partial the next layer's RMSNorm needs.
//
// Every load a role needs is issued up front and unconditionally (a lane
// whose data is absent reads zero through the buffer descriptor's range), the
// token first, so the barriers wait only for LDS (lds_barrier) and each
// compute step waits only for the loads it uses.  (__syncthreads() would wait
// for every outstanding global load on gfx950; loads under a condition make
// the compiler wait for all of them where the branches join.)
#include "capi_util.h"
#include "ffn_kernels.h"
#include "decode_util.h"

namespace oi2 {

// Device-side signals between the staging copy and the kernels around it.
// The data a signal publishes (an active list, a layer's staged records) is
// written with agent-coherent write-through stores; each wave waits for its
// stores' acknowledgements, the workgroup meets at a barrier, and one lane
// adds 1 to the signal word.  A waiting wave polls that word with relaxed
// agent-scope loads and then reads the data with ordinary loads: every
// published address is read at most once per launch after its signal, and
// each launch starts with clean caches, so no stale line can be hit.  No L2
// writeback or invalidate is issued (either stalls every in-flight load of
// the XCD).  Past `spin` polls a wait sets the error word and gives up, so
// every wait ends; once the error word is set (until the host reports and
// clears it) every wait gives up at once, so a token whose streams did not
// run side by side costs one bound, not one per layer.  Returns whether the
// signal was seen (the same value in every lane).
__device__ __forceinline__ bool stage_wait(const uint32_t* word, uint32_t target, uint32_t* err,
                                           uint32_t spin) {
  if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
  uint32_t n = 0;
  bool seen = true;
  while ((uint32_t)__builtin_amdgcn_readfirstlane(
             (int)__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < target) {
    __builtin_amdgcn_s_sleep(2);
    if (++n >= spin) {
      __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      seen = false;
      break;
    }
    if ((n & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
      seen = false;
      break;
    }
  }
  return __builtin_amdgcn_readfirstlane((int)seen) != 0;
}

__device__ __forceinline__ void stage_signal_wg(uint32_t* word) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ void st_wt(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T ld_coherent(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix of the clamped chunk counts, per wave: lane k holds the
// prefix of chunks k, k+64, k+128, k+192.  Returns the total.
template <bool kCoherent = false>
__device__ __forceinline__ int wave_chunk_prefix(const ActiveList& al, int excl[4]) {
  const int lane = lane_id();
  int total = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    excl[m] = total;
    if (64 * m < al.n_chunks) {
      const int k = lane + 64 * m;
      int c = 0;
      if (k < al.n_chunks) {
        c = kCoherent ? ld_coherent(al.counts + k) : al.counts[k];
        c = c < 0 ? 0 : (c > al.chunk ? al.chunk : c);
      }
      int v = c;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off, kWave);
        if (lane >= off) v += t;
      }
      excl[m] = total + v - c;
      total += __shfl(v, 63, kWave);
    }
  }
  return total;
}

// Position (chunk * chunk_size + index in chunk) of active item i
// (0 <= i < total) in the chunked list, wave-uniform.
__device__ __forceinline__ int item_pos(const ActiveList& al, const int excl[4], int i) {
  const int lane = lane_id();
  int c = -1;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const bool in = (lane + 64 * m) < al.n_chunks && excl[m] <= i;
    c += __popcll(__ballot(in));
  }
  const int sel = c >> 6;
  const int e = sel == 0 ? excl[0] : sel == 1 ? excl[1] : sel == 2 ? excl[2] : excl[3];
  const int base = __shfl(e, c & 63, kWave);
  return c * al.chunk + (i - base);
}

// A barrier over LDS only: the waves' LDS stores are complete, their global
// loads may still be in flight (__syncthreads() would wait for those too).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// r = rsqrt(mean(x^2) + eps) from this lane's four sum-of-squares partials
// (loaded as raw 16 bytes early on), or 1 without a norm.  All 64 lanes take part.
__device__ __forceinline__ float token_r(const TokenIn& tk, u32x4 pq) {
  return tk.use_norm ? r_from_part(f32x4{as_f32(pq.x), as_f32(pq.y), as_f32(pq.z), as_f32(pq.w)}, tk.eps)
                     : 1.0f;
}

// The token as the up roles read it, thread t of 256 taking elements
// [16 t, 16 t + 16): its xw halves (xa, xb) and the lane's four partials
// (pq).  With tk.norm_w the thread forms them from x and the weight with
// k_prep's arithmetic (xw = fp16(x w), partial t = ssq16 of x) and puts its
// partial in s_ssq[t]: finish_partials() then reads the lane's four after
// the role's first LDS barrier.  Otherwise xw and the partials are loaded.
struct TokenLoads {
  u32x4 xa, xb, pq, wa, wb;
};

// Issued first in a role (every load unconditional: absent data reads zero).
__device__ __forceinline__ TokenLoads token_loads(const TokenIn& tk, int t) {
  TokenLoads r;
  const bool fold = tk.norm_w != nullptr;
  const rsrc_t rx = rsrc(fold ? tk.x : tk.xw, kH * 2);
  r.xa = bld16(rx, 32 * t);
  r.xb = bld16(rx, 32 * t + 16);
  r.pq = bld16(rsrc(tk.ssq, (tk.use_norm && !fold) ? 256 * 4 : 0u), 16 * lane_id());
  const rsrc_t rw = rsrc(tk.norm_w, fold ? kH * 2 : 0u);
  r.wa = bld16(rw, 32 * t);
  r.wb = bld16(rw, 32 * t + 16);
  return r;
}

__device__ __forceinline__ void token_fold(const TokenIn& tk, int t, TokenLoads& r, float* s_ssq) {
  if (!tk.norm_w) return;
  const u32x4 wa = r.wa, wb = r.wb;
  float v[16], w[16];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    v[2 * d] = half_lo(r.xa[d]);
    v[2 * d + 1] = half_hi(r.xa[d]);
    v[8 + 2 * d] = half_lo(r.xb[d]);
    v[8 + 2 * d + 1] = half_hi(r.xb[d]);
    w[2 * d] = half_lo(wa[d]);
    w[2 * d + 1] = half_hi(wa[d]);
    w[8 + 2 * d] = half_lo(wb[d]);
    w[8 + 2 * d + 1] = half_hi(wb[d]);
  }
  s_ssq[t] = ssq16(v);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    r.xa[d] = (uint32_t)float_to_half_bits(v[2 * d] * w[2 * d]) |
              ((uint32_t)float_to_half_bits(v[2 * d + 1] * w[2 * d + 1]) << 16);
    r.xb[d] = (uint32_t)float_to_half_bits(v[8 + 2 * d] * w[8 + 2 * d]) |
              ((uint32_t)float_to_half_bits(v[8 + 2 * d + 1] * w[8 + 2 * d + 1]) << 16);
  }
}

// After the first LDS barrier: the lane's four partials from s_ssq when the
// role formed them.
__device__ __forceinline__ void finish_partials(const TokenIn& tk, TokenLoads& r, const float* s_ssq) {
  if (!tk.norm_w) return;
  const f32x4 p = reinterpret_cast<const f32x4*>(s_ssq)[lane_id()];
  r.pq = u32x4{as_u32(p.x), as_u32(p.y), as_u32(p.z), as_u32(p.w)};
}

// ── ffn_up roles ────────────────────────────────────────────────────────────

// ── cold gate/up/act/down ───────────────────────────────────────────────────

// Wave gw takes chunk gw / wpc of the active list and that chunk's items
// j = gw % wpc, + wpc, + 2 wpc, ... (cold_split sizes wpc for about two items
// per wave).  So a wave finds its records from its own chunk's count and
// slots, loaded together first thing, with no prefix over the other chunks.
// Per item: gate and up against the paired
// x (fp16 dot2 over the exact INT4 decode), h = act(...), and h * s * q over
// the item's down column into 64 accumulators per lane.  The four waves sum
// in LDS and every cold workgroup writes one fp32 partial row of y (zeros
// without items), which ffn_down sums.
// Record buffers per cold wave (measured: 2, 3 and 4 run alike; 2 needs the
// fewest registers).
constexpr int kColdRing = 2;

// A wave-uniform int32 through the constant address space: a scalar load,
// which neither queues behind nor waits for the wave's vector loads.
__device__ __forceinline__ int32_t sload_i32(const int32_t* p) {
  typedef const __attribute__((address_space(4))) int32_t ci32;
  return *reinterpret_cast<ci32*>(reinterpret_cast<uintptr_t>(p));
}

__device__ void cold_role(const UpArgs& a, int wg, uint32_t* s_pair, float* s_red, float* s_ssq) {
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = lane_id();
  const ActiveList& al = a.act;
  const int wpc = a.cold_wpc;
  const int c = (wg * 4 + w) / wpc, j0 = wg * 4 + w - c * wpc;
  const bool in_list = c < al.n_chunks;
  const int cc = in_list ? c : 0;
  // 1. this wave's chunk count and slots (lane k: item j0 + k wpc), then the token
  int cnt = sload_i32(al.counts + cc);
  cnt = !in_list || cnt < 0 ? 0 : (cnt > al.chunk ? al.chunk : cnt);
  const uint32_t list_bytes = (uint32_t)al.n_chunks * (uint32_t)al.chunk * 4;
  const rsrc_t rsl = rsrc(al.slots, al.slots ? list_bytes : 0);
  auto slot_off = [&](int k) {
    const int j = j0 + k * wpc;
    return j < al.chunk ? 4 * (uint32_t)(cc * al.chunk + j) : kNoOff;
  };
  const int lane_slot = (int)bld4(rsl, slot_off(lane));
  TokenLoads tl = token_loads(a.tok, t);
  // staged records wait for the copy (records staged in list order: item j of
  // chunk c is record c * chunk + j); a wait that gives up reads the records
  // from the copy's source through the slot list instead
  const uint8_t* rec_base = a.records;
  int n_rec = a.n_records;
  const int32_t* slot_list = al.slots;
  int lane_slot_v = lane_slot;
  if (a.stage_ready && !stage_wait(a.stage_ready, a.stage_target, a.stage_err, a.stage_spin)) {
    rec_base = a.stage_src;
    n_rec = a.stage_src_n;
    slot_list = a.stage_slots;
    lane_slot_v = (int)bld4(rsrc(a.stage_slots, list_bytes), slot_off(lane));
  }
  const bool by_slot = slot_list != nullptr;
  const int n_items = cnt > j0 ? (cnt - j0 + wpc - 1) / wpc : 0;

  // 2. records through a descriptor over the record array: an absent item
  //    reads zero, so every load is unconditional
  const rsrc_t rrec = rsrc(rec_base, (uint32_t)n_rec * kRecBytes);
  const rsrc_t rgb = rsrc(a.cold_gbias, a.cold_gbias ? (uint32_t)n_rec * 4 : 0);
  struct Rec {
    u32x4 q[6];
    uint32_t sdw;       // lane l < 48: halves 2l, 2l + 1 of the record's 96 group scales
    float gbias;
    bool valid;
  };
  const int g0 = lane >> 2;
  auto load_slot = [&](int sl, bool valid, Rec& R) {
    R.valid = valid && sl >= 0 && sl < n_rec;
    const uint32_t ro = R.valid ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
    for (int it = 0; it < 6; ++it) R.q[it] = wld16(rrec, ro + kOffGate + 16 * (lane + 64 * it));
    R.sdw = bld4(rrec, lane < 48 ? ro + kOffScales + 4 * lane : kNoOff);
    R.gbias = as_f32(bld4(rgb, R.valid ? 4 * (uint32_t)sl : kNoOff));
  };
  // items k < 64 take their slot from lane k of lane_slot; every refill is
  // issued (past the last item it reads zeros), so the compiler sees the same
  // loads in flight on every pass and waits for exactly the record in use
  const int n_main = n_items < 64 ? n_items : 64;
  auto load_rec = [&](int k, Rec& R) {
    const int sl = by_slot ? __builtin_amdgcn_readlane(lane_slot_v, k & 63) : cc * al.chunk + j0 + k * wpc;
    load_slot(sl, k < n_main, R);
  };
  Rec R[kColdRing];
#pragma unroll
  for (int k = 0; k < kColdRing; ++k) load_rec(k, R[k]);

  // 3. the token's (e0,e4) (e1,e5) (e2,e6) (e3,e7) pairs, the order the INT4
  //    unpack produces, into LDS
  token_fold(a.tok, t, tl, s_ssq);
  {
    const u32x4 xa = tl.xa, xb = tl.xb;
    u32x4 pa, pb;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // element k is half (k & 1) of dword k >> 1; element k + 4 the same half
      // of dword 2 + (k >> 1); v_perm picks the two halves into one dword
      const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
      pa[k] = __builtin_amdgcn_perm(xa[2 + (k >> 1)], xa[k >> 1], sel);
      pb[k] = __builtin_amdgcn_perm(xb[2 + (k >> 1)], xb[k >> 1], sel);
    }
    reinterpret_cast<u32x4*>(s_pair)[2 * t] = pa;
    reinterpret_cast<u32x4*>(s_pair)[2 * t + 1] = pb;
  }
  lds_barrier();
  finish_partials(a.tok, tl, s_ssq);
  const float r = token_r(a.tok, tl.pq);
  float acc[64];
#pragma unroll
  for (int k = 0; k < 64; ++k) acc[k] = 0.0f;
  auto compute = [&](const Rec& R) {
    if (!R.valid) return;
    float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      // token pairs for elements [32 lane + 2048 it, +32)
      const u32x4* px = reinterpret_cast<const u32x4*>(s_pair) + (32 * lane + 2048 * it) / 8;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const u32x4 xv = px[d];
        f16x2 tg[4], tu[4];
        int4x8_to_f16x2x4(R.q[it][d], tg);
        int4x8_to_f16x2x4(R.q[2 + it][d], tu);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          pg[it] = dot2(tg[k], as_f16x2(xv[k]), pg[it]);
          pu[it] = dot2(tu[k], as_f16x2(xv[k]), pu[it]);
        }
      }
    }
    // this lane's group scales: gate, up, down of groups g0 and g0 + 16
    float s[6];
#pragma unroll
    for (int v = 0; v < 6; ++v) {
      const int hf = 32 * (v >> 1) + 16 * (v & 1) + g0;
      const uint32_t d = __shfl(R.sdw, hf >> 1, kWave);
      s[v] = (hf & 1) ? half_hi(d) : half_lo(d);
    }
    float g = r * wave_sum(pg[0] * s[0] + pg[1] * s[1]);
    const float u = r * wave_sum(pu[0] * s[2] + pu[1] * s[3]);
    g += R.gbias;
    const float h = gated_act(g, u, a.relu, a.both);
    const float hs[2] = {h * s[4], h * s[5]};
    // the record's down column, elements [32 lane + 2048 it, +32)
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        f16x2 tq[4];
        int4x8_to_f16x2x4(R.q[4 + it][d], tq);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[32 * it + 8 * d + k] = fmaf(hs[it], (float)tq[k].x, acc[32 * it + 8 * d + k]);
          acc[32 * it + 8 * d + k + 4] = fmaf(hs[it], (float)tq[k].y, acc[32 * it + 8 * d + k + 4]);
        }
      }
  };
  for (int k = 0; k < n_main; k += kColdRing) {
#pragma unroll
    for (int m = 0; m < kColdRing; ++m) {
      compute(R[m]);                       // item k + m (skipped past the last)
      load_rec(k + m + kColdRing, R[m]);   // refill: kColdRing items ahead
    }
  }
  // items past 64 (a chunk longer than 64 of this wave's strides): one at a time
  for (int k = 64; k < n_items; ++k) {
    const int j = j0 + k * wpc;
    load_slot(by_slot ? sload_i32(slot_list + cc * al.chunk + j) : cc * al.chunk + j, true, R[0]);
    compute(R[0]);
  }
  // 4. sum the four waves in LDS (fixed order, padded against bank
  //    conflicts), then one coalesced 16 KB partial row
  for (int st = 0; st < 4; ++st) {
    if (w == st) {
#pragma unroll
      for (int idx = 0; idx < 64; ++idx) {
        const int j = 32 * lane + 2048 * (idx >> 5) + (idx & 31);
        const int pj = j + (j >> 5);
        s_red[pj] = (st == 0) ? acc[idx] : s_red[pj] + acc[idx];
      }
    }
    lds_barrier();
  }
  float* dst = a.cold_part + (size_t)wg * kH;
#pragma unroll
  for (int m = 0; m < kH / kThreads / 4; ++m) {
    const int j = 4 * (t + kThreads * m);
    f32x4 v;
    v.x = s_red[j + (j >> 5)];
    v.y = s_red[j + 1 + ((j + 1) >> 5)];
    v.z = s_red[j + 2 + ((j + 2) >> 5)];
    v.w = s_red[j + 3 + ((j + 3) >> 5)];
    *reinterpret_cast<f32x4*>(dst + j) = v;
  }
}

// bf16 weights of one predictor down row for this lane (elements
// 8 (lane + 64 it) .. +8, it < 8), loaded before anything else.
struct PredRowBf16 {
  u32x4 v[8];
};

template <bool BF16>
__device__ void pred_d_role_t(const UpArgs& a, int row) {
  const int lane = lane_id();
  PredRowBf16 dw;
  if constexpr (BF16) {
    const uint16_t* drow = reinterpret_cast<const uint16_t*>(a.pd_w) + (size_t)row * kH;
#pragma unroll
    for (int it = 0; it < 8; ++it) dw.v[it] = load16_nt(reinterpret_cast<const uint8_t*>(drow + 8 * (lane + 64 * it)));
  }
  const bool norm = a.pd_norm_w && !a.pd_q;
  // every input of the row issued before the first use
  u32x4 xv[8], wv[8];
  if (!a.pd_q) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int e0 = 8 * (lane + 64 * it);
      xv[it] = *reinterpret_cast<const u32x4*>(a.tok.x + e0);
      wv[it] = norm ? *reinterpret_cast<const u32x4*>(a.pd_norm_w + e0) : u32x4{0, 0, 0, 0};
    }
  }
  const f32x4 part = norm ? load_part(a.tok.ssq) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float r = norm ? r_from_part(part, a.tok.eps) : 1.0f;
  // four partial sums, one per quarter of the row (elements [1024 q, 1024 q +
  // 1024)), combined as (p0 + p1) + (p2 + p3): the persistent token kernel
  // splits a row over four workgroups in exactly this order.  Double
  // precision: each product of two floats is exact in a double, and the
  // logits built from z stay within ~1e-15 of exact arithmetic, far inside
  // the 1e-6 band the active-set contract exempts.
  double accq[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    double& acc = accq[it >> 1];
    const int e0 = 8 * (lane + 64 * it);
    float q[8];
    if (a.pd_q) {
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = a.pd_q[e0 + k];
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float v0 = half_lo(xv[it][d]), v1 = half_hi(xv[it][d]);
        if (norm) {
          v0 = xn_exact(v0, r, half_lo(wv[it][d]));
          v1 = xn_exact(v1, r, half_hi(wv[it][d]));
        }
        q[2 * d] = BF16 ? round_bf16(v0) : v0;
        q[2 * d + 1] = BF16 ? round_bf16(v1) : v1;
      }
    }
    if constexpr (BF16) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc = fma((double)bf16_bits_to_float((uint16_t)(dw.v[it][d] & 0xFFFFu)), (double)q[2 * d], acc);
        acc = fma((double)bf16_bits_to_float((uint16_t)(dw.v[it][d] >> 16)), (double)q[2 * d + 1], acc);
      }
    } else {
      const float* drow = reinterpret_cast<const float*>(a.pd_w) + (size_t)row * kH;
      const f32x4 d0 = *reinterpret_cast<const f32x4*>(drow + e0);
      const f32x4 d1 = *reinterpret_cast<const f32x4*>(drow + e0 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = fma((double)d0[k], (double)q[k], acc);
        acc = fma((double)d1[k], (double)q[4 + k], acc);
      }
    }
  }
  const double z = (wave_sum_d(accq[0]) + wave_sum_d(accq[1])) + (wave_sum_d(accq[2]) + wave_sum_d(accq[3]));
  if (lane == 0) a.pd_z[row] = z;
}

__device__ void pred_d_role(const UpArgs& a, int wg) {
  const int row = wg * 4 + (threadIdx.x >> 6);
  if (row >= a.pd_rank) return;
  if (a.pd_bf16)
    pred_d_role_t<true>(a, row);
  else
    pred_d_role_t<false>(a, row);
}

// Two neurons per wave.  The token goes out first and the weights behind it,
// every load unconditional (rows past n_hot read zero through the
// descriptor's range), so the LDS copy of the token waits only for the
// token, the barrier waits for no global load, and each step of the dot
// products waits only for the weight chunk it uses: the products run while
// the later chunks are still arriving.
__device__ void hot_up_role(const UpArgs& a, int wg, uint32_t* s_nat, float* s_ssq) {
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = lane_id();
  const int k0 = (wg * 4 + w) * 2;
  TokenLoads tl = token_loads(a.tok, t);
  const uint32_t hot_bytes = (uint32_t)a.n_hot * kH;
  const rsrc_t rg = rsrc(a.gate_q, hot_bytes), ru = rsrc(a.up_q, hot_bytes);
  u32x4 qg[2][4], qu[2][4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const uint32_t off = (uint32_t)k0 * kH + 1024 * it + 16 * lane;
    qg[0][it] = wld16(rg, off);
    qu[0][it] = wld16(ru, off);
    qg[1][it] = wld16(rg, off + kH);
    qu[1][it] = wld16(ru, off + kH);
  }
  // scales (and gate bias) of neuron k0 + lane for lanes 0 and 1
  const int kl = k0 + (lane & 1);
  const uint32_t so = (lane < 2 && kl < a.n_hot) ? 4 * (uint32_t)kl : kNoOff;
  const uint32_t sb = (uint32_t)a.n_hot * 4;
  const float gsc = as_f32(bld4(rsrc(a.gate_s, sb), so));
  const float usc = as_f32(bld4(rsrc(a.up_s, sb), so));
  const float gbi = as_f32(bld4(rsrc(a.hot_gbias, a.hot_gbias ? sb : 0), so));
  token_fold(a.tok, t, tl, s_ssq);
  reinterpret_cast<u32x4*>(s_nat)[2 * t] = tl.xa;
  reinterpret_cast<u32x4*>(s_nat)[2 * t + 1] = tl.xb;
  lds_barrier();
  if (k0 >= a.n_hot) return;
  finish_partials(a.tok, tl, s_ssq);
  const float r = token_r(a.tok, tl.pq);
  float g[2] = {0.0f, 0.0f}, u[2] = {0.0f, 0.0f};
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const u32x4* p = reinterpret_cast<const u32x4*>(s_nat) + (1024 * it + 16 * lane) / 8;
    const u32x4 x0 = p[0], x1 = p[1];
    const f16x2 xp[8] = {as_f16x2(x0.x), as_f16x2(x0.y), as_f16x2(x0.z), as_f16x2(x0.w),
                         as_f16x2(x1.x), as_f16x2(x1.y), as_f16x2(x1.z), as_f16x2(x1.w)};
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        g[n] = dot2(fp8x2_to_f16x2(qg[n][it][d], false), xp[2 * d], g[n]);
        g[n] = dot2(fp8x2_to_f16x2(qg[n][it][d], true), xp[2 * d + 1], g[n]);
        u[n] = dot2(fp8x2_to_f16x2(qu[n][it][d], false), xp[2 * d], u[n]);
        u[n] = dot2(fp8x2_to_f16x2(qu[n][it][d], true), xp[2 * d + 1], u[n]);
      }
  }
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    g[n] = wave_sum(g[n]);
    u[n] = wave_sum(u[n]);
  }
  if (lane < 2 && kl < a.n_hot) {
    const float gg = r * (lane ? g[1] : g[0]) * gsc + gbi;
    const float uu = r * (lane ? u[1] : u[0]) * usc;
    a.h_hot[kl] = gated_act(gg, uu, a.relu, a.both);
  }
}

__global__ __launch_bounds__(kThreads, 3) void k_ffn_up(UpArgs a) {
  // hot: natural xw (8 KB); cold: paired xw (8 KB) + padded reduction (16.5 KB)
  __shared__ u32x4 s_xw4[kH / 8];
  __shared__ float s_red[kH + kH / 32];
  __shared__ __attribute__((aligned(16))) float s_ssq[256];   // the partials a role formed itself
  uint32_t* s_xw = reinterpret_cast<uint32_t*>(s_xw4);
  int b = blockIdx.x;
  if (b < a.wg_cold) {
    cold_role(a, b, s_xw, s_red, s_ssq);
    return;
  }
  b -= a.wg_cold;
  if (b < a.wg_pred) {
    pred_d_role(a, b);
    return;
  }
  b -= a.wg_pred;
  hot_up_role(a, b, s_xw, s_ssq);
}

// Predictor-only launches (layer 0's lookahead, the standalone predictor
// entry points) use their own symbols so per-kernel statistics of k_ffn_up /
// k_ffn_down cover whole FFN layers only.
__global__ __launch_bounds__(kThreads) void k_pred_up(UpArgs a) { pred_d_role(a, blockIdx.x); }

// x -> (xw = fp16(x * w) or x, 256 canonical sum-of-squares partials).  One
// workgroup; 16 elements per thread.
__global__ __launch_bounds__(kThreads) void k_prep(const uint16_t* x, const uint16_t* w, uint16_t* xw,
                                                   float* ssq) {
  const int t = threadIdx.x;
  float v[16];
  load_h16(x, 16 * t, v);
  ssq[t] = ssq16(v);
  if (xw) {
    float wv[16];
    if (w) load_h16(w, 16 * t, wv);
    uint16_t* o = xw + 16 * t;
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] = float_to_half_bits(w ? v[e] * wv[e] : v[e]);
  }
}

// ── ffn_down roles ──────────────────────────────────────────────────────────

__device__ void pred_u_role(const DownArgs& a, int c, int* s_wcnt) {
  const int t = threadIdx.x, w = t >> 6, lane = lane_id();
  const int n = c * kSelChunk + t;
  bool keep = false;
  const int lutv = (n < a.inter && a.lut) ? a.lut[n] : n;
  if (n < a.inter) {
    // the row in batches of 64 rank entries, each batch's loads issued
    // together; the sum and the threshold test in double precision
    double logit;
    double acc = 0.0;
    if (a.pu_bf16) {
      const uint16_t* urow = reinterpret_cast<const uint16_t*>(a.pu_w) + (size_t)n * a.pu_rank;
      const double bias = bf16_bits_to_float(reinterpret_cast<const uint16_t*>(a.pu_b)[n]);
      for (int rb = 0; rb < a.pu_rank; rb += 64) {
        u32x4 uv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          uv[k] = rb + 8 * k < a.pu_rank ? *reinterpret_cast<const u32x4*>(urow + rb + 8 * k)
                                         : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (rb + 8 * k >= a.pu_rank) break;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const int r = rb + 8 * k + 2 * d;
            acc = fma((double)bf16_bits_to_float((uint16_t)(uv[k][d] & 0xFFFFu)), a.pd_z[r], acc);
            acc = fma((double)bf16_bits_to_float((uint16_t)(uv[k][d] >> 16)), a.pd_z[r + 1], acc);
          }
        }
      }
      logit = acc + bias;
    } else {
      const float* urow = reinterpret_cast<const float*>(a.pu_w) + (size_t)n * a.pu_rank;
      const double bias = reinterpret_cast<const float*>(a.pu_b)[n];
      for (int rb = 0; rb < a.pu_rank; rb += 64) {
        f32x4 uv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
          uv[k] = rb + 4 * k < a.pu_rank ? *reinterpret_cast<const f32x4*>(urow + rb + 4 * k)
                                         : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          if (rb + 4 * k >= a.pu_rank) break;
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = fma((double)uv[k][e], a.pd_z[rb + 4 * k + e], acc);
        }
      }
      logit = acc + bias;
    }
    const float logit32 = (float)logit;
    if (a.logits_out) a.logits_out[n] = logit32;
    if (a.probs_out) a.probs_out[n] = 1.0f / (1.0f + __expf(-logit32));
    const bool fire = logit >= (double)a.thr;
    if (a.mask_out) a.mask_out[n] = fire ? 1 : 0;
    keep = fire && lutv >= 0;
  }
  if (a.sel_counts == nullptr) return;
  const uint64_t bal = __ballot(keep);
  const int wpos = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) s_wcnt[w] = __popcll(bal);
  __syncthreads();
  int base = 0;
  for (int ww = 0; ww < w; ++ww) base += s_wcnt[ww];
  if (keep) {
    const size_t pos = (size_t)c * kSelChunk + base + wpos;
    if (a.sel_flag) {
      st_wt(a.sel_slots + pos, lutv);
      st_wt(a.sel_ids + pos, n);
    } else {
      a.sel_slots[pos] = lutv;
      a.sel_ids[pos] = n;
    }
  }
  if (t == 0) {
    const int cnt = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
    if (a.sel_flag)
      st_wt(a.sel_counts + c, cnt);
    else
      a.sel_counts[c] = cnt;
  }
}

struct DownShared {
  float h[kH + kH / 4];              // h_hot, element j at j + 4 (j >> 4)
  float cold[4][kRowsPerDownWG];     // per-wave cold sums
  float yhot[kRowsPerDownWG];
  float out[kRowsPerDownWG];
};

// Accumulate the 16 down nibbles at rows [j0, j0+16) of one record, times hs.
__device__ __forceinline__ void cold_down16(uint32_t n0, uint32_t n1, float hs, float acc[16]) {
  f16x2 t[4];
  int4x8_to_f16x2x4(n0, t);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc[k] = fmaf(hs, (float)t[k].x, acc[k]);
    acc[k + 4] = fmaf(hs, (float)t[k].y, acc[k + 4]);
  }
  int4x8_to_f16x2x4(n1, t);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc[8 + k] = fmaf(hs, (float)t[k].x, acc[8 + k]);
    acc[12 + k] = fmaf(hs, (float)t[k].y, acc[12 + k]);
  }
}

__device__ void down_role(const DownArgs& a, int b, DownShared& sh) {
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = lane_id();
  // XCD-aware tiling: consecutive blockIdx go to different XCDs (b % 8), so
  // give each XCD a contiguous 512-row band; its 32 tiles then share the L2
  // lines holding those rows' nibbles of every cold record.
  const int tile = (b & 7) * (kDownWG / 8) + (b >> 3);
  const int j0 = tile * kRowsPerDownWG;
  // Loads in the order they are used, all unconditional (past a range reads
  // zero): h_hot once per workgroup (thread t: elements [16t, 16t+16)), the
  // cold partial rows, the hot down rows, the epilogue operands.
  const uint32_t hb = a.n_hot > 0 ? (uint32_t)a.n_hot * 4 : 0;
  const rsrc_t rh = rsrc(a.h_hot, hb);
  u32x4 hl[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) hl[m] = bld16(rh, 64 * t + 16 * m);
  // cold: thread t sums rows [j0 + 4 (t & 3), +4) of partial rows p = t/4 + 64 m
  const int n_part = a.cold_part ? a.cold_wg : 0;
  const rsrc_t rcp = rsrc(a.cold_part, (uint32_t)n_part * kH * 4);
  auto part_off = [&](int p) { return p < n_part ? 4 * (uint32_t)(p * kH + j0 + 4 * (t & 3)) : kNoOff; };
  constexpr int kPre = 4;
  u32x4 pv[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) pv[k] = bld16(rcp, part_off((t >> 2) + 64 * k));
  // hot down rows: 4 per wave, chunk c = lane + 64 it of each (chunks past the
  // row stride read zero)
  const int nch = a.down_stride >> 4;
  const rsrc_t rd = rsrc(a.down_q, a.n_hot > 0 ? (uint32_t)kH * a.down_stride : 0);
  u32x4 q[4][4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const uint32_t row = (uint32_t)(j0 + 4 * w + rr) * a.down_stride;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = lane + 64 * it;
      q[rr][it] = wld16(rd, c < nch ? row + 16 * c : kNoOff);
    }
  }
  float dsc[4];
  const rsrc_t rds = rsrc(a.down_s, a.n_hot > 0 ? kH * 4 : 0);
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) dsc[rr] = as_f32(bld4(rds, 4 * (j0 + 4 * w + rr)));
  const int je = j0 + (t & (kRowsPerDownWG - 1));
  const float res_v = half_bits_to_float(bld2(rsrc(a.res, a.res ? kH * 2 : 0), 2 * je));
  const uint16_t nwb = bld2(rsrc(a.next_norm_w, a.next_norm_w ? kH * 2 : 0), 2 * je);
  const float nw_v = a.next_norm_w ? half_bits_to_float(nwb) : 1.0f;
  // every load above is issued before any of them is used
  __builtin_amdgcn_sched_barrier(0);

  // 1. h into LDS (padded so that lanes 64 bytes apart hit different banks)
#pragma unroll
  for (int m = 0; m < 4; ++m) *reinterpret_cast<u32x4*>(sh.h + 20 * t + 4 * m) = hl[m];
  lds_barrier();
  // 2. cold partial sums; more than 256 rows: the rest now
  f32x4 cp = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < kPre; ++k) cp += f32x4{as_f32(pv[k].x), as_f32(pv[k].y), as_f32(pv[k].z), as_f32(pv[k].w)};
  // (four loads in flight per pass, rows past n_part reading zero; the sum
  // keeps the row order)
  for (int p0 = (t >> 2) + 64 * kPre; p0 < n_part; p0 += 4 * (kThreads / 4)) {
    u32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = bld16(rcp, part_off(p0 + k * (kThreads / 4)));
#pragma unroll
    for (int k = 0; k < 4; ++k) cp += f32x4{as_f32(v[k].x), as_f32(v[k].y), as_f32(v[k].z), as_f32(v[k].w)};
  }
  // h values of this lane's chunks
  float hv[4][16];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const float* ph = sh.h + 20 * (lane + 64 * it);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(ph + 4 * m);
      hv[it][4 * m] = v[0];
      hv[it][4 * m + 1] = v[1];
      hv[it][4 * m + 2] = v[2];
      hv[it][4 * m + 3] = v[3];
    }
  }
  // 3. hot rows
  float yh[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (a.n_hot > 0) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float acc = 0.0f;
#pragma unroll
      for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const f32x2 lo = fp8x2_to_f32x2(q[rr][it][d], false);
          const f32x2 hi = fp8x2_to_f32x2(q[rr][it][d], true);
          acc = fmaf(lo.x, hv[it][4 * d], acc);
          acc = fmaf(lo.y, hv[it][4 * d + 1], acc);
          acc = fmaf(hi.x, hv[it][4 * d + 2], acc);
          acc = fmaf(hi.y, hv[it][4 * d + 3], acc);
        }
      yh[rr] = wave_sum(acc);
    }
  }
  // 4. cold sums: lanes with the same (t & 3) hold the same 4 rows
  {
    f32x4 v = cp;
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
      v.x += __shfl_xor(v.x, off, kWave);
      v.y += __shfl_xor(v.y, off, kWave);
      v.z += __shfl_xor(v.z, off, kWave);
      v.w += __shfl_xor(v.w, off, kWave);
    }
    if (lane < 4) {
      sh.cold[w][4 * lane] = v.x;
      sh.cold[w][4 * lane + 1] = v.y;
      sh.cold[w][4 * lane + 2] = v.z;
      sh.cold[w][4 * lane + 3] = v.w;
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sh.yhot[4 * w + rr] = (a.n_hot > 0) ? yh[rr] * dsc[rr] : 0.0f;
  }
  __syncthreads();
  if (t < kRowsPerDownWG) {
    const float yc = (sh.cold[0][t] + sh.cold[1][t]) + (sh.cold[2][t] + sh.cold[3][t]);
    const float y = sh.yhot[t] + yc;
    const int j = j0 + t;
    if (a.y32) a.y32[j] = y;
    const uint16_t ob = float_to_half_bits(res_v + y);
    if (a.out) a.out[j] = ob;
    if (a.out2) a.out2[j] = ob;
    const float o = half_bits_to_float(ob);
    sh.out[t] = o;
    if (a.xw_out) a.xw_out[j] = float_to_half_bits(a.next_norm_w ? o * nw_v : o);
  }
  if (a.ssq_out) {
    __syncthreads();
    if (t == 0) a.ssq_out[tile] = ssq16(sh.out);
  }
}

__global__ __launch_bounds__(kThreads) void k_ffn_down(DownArgs a) {
  __shared__ DownShared sh;
  __shared__ int s_wcnt[4];
  int b = blockIdx.x;
  if (b < a.wg_pred) {
    pred_u_role(a, b, s_wcnt);
    return;
  }
  b -= a.wg_pred;
  down_role(a, b, sh);
}

__global__ __launch_bounds__(kThreads) void k_pred_down(DownArgs a) {
  __shared__ int s_wcnt[4];
  pred_u_role(a, blockIdx.x, s_wcnt);
  if (a.sel_flag) stage_signal_wg(a.sel_flag);   // this chunk of the list is written
}

// ── standalone kernels ──────────────────────────────────────────────────────

// Cold-record staging: copy every active record of one layer from its source
// (HBM, or pinned host memory read over PCIe) to the staging buffer, record p
// of the chunked list to dst + 6400 p, so the FFN reads the staged records
// through a slot-less list.  One wave per record: 400 16-byte chunks, all
// loads issued before the stores.  Invalid slots stage an all-zero record,
// which contributes exactly zero to the FFN.
//
// The copy's loads wait on PCIe for microseconds; a CU that hosts one of its
// waves serves the FFN's HBM loads behind them.  The kernel therefore holds
// the whole 160 KB of its CU's LDS, so no FFN workgroup lands on a CU that
// is copying.
constexpr int kStageLdsWords = 160 * 1024 / 4;


// Copy one layer's active records (items of the chunked list, list position
// p to dst + 6400 p), wave `first` of `n_waves` taking every n_waves-th item.
// kPublish: the list is read with coherent loads and the records stored
// write-through, for the persistent copy kernel that runs beside the kernels
// publishing the list and reading the records.
template <bool kPublish>
__device__ void stage_copy_layer(const uint8_t* src_base, int n_records, const ActiveList& act, int cap,
                                 uint8_t* dst_base, int first, int n_waves) {
  int excl[4];
  int total = wave_chunk_prefix<kPublish>(act, excl);
  total = total < cap ? total : cap;
  const int lane = lane_id();
  constexpr int kChunks = kRecBytes / 16;   // 400
  // the destination and its size as scalars (they come from a table in
  // memory; a per-lane descriptor would make the compiler loop every store
  // over the distinct values)
  const uint64_t dv = reinterpret_cast<uint64_t>(dst_base);
  uint8_t* dst_u = reinterpret_cast<uint8_t*>(
      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(dv >> 32)) << 32) |
      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)dv));
  const __amdgpu_buffer_rsrc_t rdst = __builtin_amdgcn_make_buffer_rsrc(
      dst_u, (short)0, __builtin_amdgcn_readfirstlane((int)((uint32_t)cap * kRecBytes)), 0x00020000);
  // two records per wave in flight, both loaded before either is stored
  // (measured: one leaves the PCIe link short of requests; three or four
  // gain nothing over two)
  constexpr int kInFlight = 2;
  for (int i = first; i < total; i += kInFlight * n_waves) {
    int p[kInFlight];
    u32x4 v[kInFlight][7];
#pragma unroll
    for (int r = 0; r < kInFlight; ++r) {
      const int ii = i + r * n_waves;
      p[r] = ii < total ? item_pos(act, excl, ii) : -1;
      const int slot = p[r] < 0 ? -1 : act.slots ? (kPublish ? ld_coherent(act.slots + p[r]) : act.slots[p[r]])
                                                 : p[r];
      const bool valid = slot >= 0 && slot < n_records;
      const u32x4* src = reinterpret_cast<const u32x4*>(src_base + (size_t)(valid ? slot : 0) * kRecBytes);
#pragma unroll
      for (int it = 0; it < 7; ++it) {
        const int c = lane + 64 * it;
        v[r][it] = (valid && c < kChunks) ? __builtin_nontemporal_load(src + c) : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int r = 0; r < kInFlight; ++r) {
      if (p[r] < 0) continue;
#pragma unroll
      for (int it = 0; it < 7; ++it) {
        const int c = lane + 64 * it;
        if (c < kChunks) {
          if constexpr (kPublish)
            __builtin_amdgcn_raw_buffer_store_b128(v[r][it], rdst,
                                                   (uint32_t)p[r] * kRecBytes + 16u * (uint32_t)c, 0,
                                                   16 /* sc1: agent-coherent write-through */);
          else
            reinterpret_cast<u32x4*>(dst_base + (size_t)p[r] * kRecBytes)[c] = v[r][it];
        }
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void k_stage_gather(StageArgs a) {
  __shared__ uint32_t s_reserve[kStageLdsWords];
  if (a.cap < 0) reinterpret_cast<volatile uint32_t*>(s_reserve)[threadIdx.x] = 0;  // never runs
  stage_copy_layer<false>(a.src, a.n_records, a.act, a.cap, a.dst,
                          blockIdx.x * (kThreads / kWave) + (int)(threadIdx.x >> 6),
                          gridDim.x * (kThreads / kWave));
}

// The whole token's staging in one launch on the side stream: for each layer
// in turn, wait until its active list is complete (sel[L]), copy its records
// as k_stage_gather does, and signal ready[L] per workgroup (measured faster
// than a signal per wave, which lets the waves drift apart).  Its workgroups
// reserve their CUs' LDS like k_stage_gather.  The buffer a layer's records
// go to was last read by the FFN two layers back, which the main stream
// finishes before it signals this layer's selection.
__global__ __launch_bounds__(kThreads) void k_stage_copy(StageCopyArgs a) {
  __shared__ uint32_t s_reserve[kStageLdsWords - kThreads / kWave];
  __shared__ bool s_ok[kThreads / kWave];
  if (a.cap < 0) reinterpret_cast<volatile uint32_t*>(s_reserve)[threadIdx.x] = 0;  // never runs
  uint32_t* err = a.sync + stage_err_word(a.n_layers);
  for (int L = 0; L < a.n_layers; ++L) {
    const StageLayer T = a.layers[L];
    if (T.n_records == 0) continue;
    // a wave whose wait for the list gives up copies nothing, and its
    // workgroup never signals the layer ready: the FFN's wait then gives up
    // too and reads the records from the source
    const bool listed = stage_wait(a.sync + stage_sel_word(L), T.sel_target, err, a.spin);
    if (listed)
      stage_copy_layer<true>(T.src, T.n_records, T.act, a.cap, T.dst,
                             blockIdx.x * (kThreads / kWave) + (int)(threadIdx.x >> 6),
                             gridDim.x * (kThreads / kWave));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    s_ok[threadIdx.x >> 6] = listed;
    __syncthreads();
    bool all = true;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) all = all && s_ok[w];
    __syncthreads();
    if (all && threadIdx.x == 0)
      __hip_atomic_fetch_add(a.sync + stage_ready_word(L), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Main-stream signal of a layer whose list needs no selection kernel.
__global__ void k_stage_signal(uint32_t* word) {
  if (threadIdx.x == 0) __hip_atomic_fetch_add(word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(kThreads) void k_fill_u32(uint32_t* p, int n, uint32_t v) {
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) p[i] = v;
}


// Records [32 bx, 32 bx + 32) of the request, elements [256 by, 256 by + 256)
// of each of their three vectors, so every store is coalesced:
// - gate and up rows: wave w takes records w, w + 4, ..., lane l elements
//   4 l .. 4 l + 3 (one 16-byte store per lane, 1 KB per wave);
// - down_t (H, n): lane l takes record l % 32 and elements 32 (l / 32) .. +31
//   of the wave's 64, and each store writes two rows' 32 consecutive records
//   (a 128-byte line each).
// A value is (float)nibble * fp16 scale, exact in fp32; an invalid slot
// gives NaN (0 times a NaN scale).  (Non-temporal stores measured slower:
// 0.36 against 0.43 of the HBM peak for 1147 records.)
constexpr int kDqRecs = 32, kDqElems = 256;

__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* records, int n_records,
                                                      const int32_t* slots, int n, float* gate,
                                                      float* up, float* down_t) {
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = lane_id();
  const int r0 = blockIdx.x * kDqRecs, e0 = blockIdx.y * kDqElems;
  auto nib = [](uint32_t v, int k) { return (float)((int)(((v >> (4 * k)) & 0xFu) ^ 8u) - 8); };
  const rsrc_t rrec = rsrc(records, (uint32_t)n_records * kRecBytes);
  // this lane's record for the down rows; lanes 0-7 also hold the slots of
  // the wave's 8 gate/up records
  const int rl = r0 + (lane & (kDqRecs - 1));
  const int slot_l = rl < n ? slots[rl] : -1;
  const int rg = r0 + w + 4 * (lane & 7);
  const int slot_g = rg < n ? slots[rg] : -1;

  // gate and up rows
  constexpr int kG = kDqRecs / 4;
  uint32_t qg[kG][2];
  uint32_t sg[kG][2];
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    const int sl = __builtin_amdgcn_readlane(slot_g, i);
    const bool valid = sl >= 0 && sl < n_records;
    const uint32_t ro = valid ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int e = e0 + 4 * lane;
      qg[i][v] = bld2(rrec, ro + kOffGate + v * kVecBytes + e / 2);
      sg[i][v] = bld2(rrec, ro + kOffScales + 2 * (32 * v + e / 128));
      if (!valid) sg[i][v] = 0x7E00u;      // fp16 NaN
    }
  }
  // down rows: this lane's 32 elements in one 16-byte load
  const bool valid_l = slot_l >= 0 && slot_l < n_records;
  const uint32_t rol = valid_l ? (uint32_t)slot_l * kRecBytes : kNoOff;
  const int eb = e0 + 64 * w + 32 * (lane / kDqRecs);
  const u32x4 qd = bld16(rrec, rol + kOffDown + eb / 2);
  uint32_t sd = bld2(rrec, rol + kOffScales + 2 * (64 + eb / 128));
  if (!valid_l) sd = 0x7E00u;
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    const int ri = r0 + w + 4 * i;
    if (ri >= n) break;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const float sc = half_bits_to_float((uint16_t)sg[i][v]);
      const f32x4 o = {nib(qg[i][v], 0) * sc, nib(qg[i][v], 1) * sc, nib(qg[i][v], 2) * sc,
                       nib(qg[i][v], 3) * sc};
      float* dst = (v == 0 ? gate : up) + (size_t)ri * kH + e0 + 4 * lane;
      *reinterpret_cast<f32x4*>(dst) = o;
    }
  }
  if (rl < n) {
    const float sc = half_bits_to_float((uint16_t)sd);
#pragma unroll
    for (int k = 0; k < 32; ++k) down_t[(size_t)(eb + k) * n + rl] = nib(qd[k >> 3], k & 7) * sc;
  }
}

// One row per workgroup; thread t holds elements 16 t .. 16 t + 15 of the row
// and of the weight (both loaded up front), and writes its 16 outputs as two
// 16-byte stores.
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const uint16_t* x, const uint16_t* w,
                                                      float eps, uint16_t* out) {
  __shared__ float s_parts[kThreads];
  const uint16_t* xr = x + (size_t)blockIdx.x * kH;
  float v[16], wv[16];
  load_h16(xr, 16 * threadIdx.x, v);
  load_h16(w, 16 * threadIdx.x, wv);
  s_parts[threadIdx.x] = ssq16(v);
  __syncthreads();
  const float r = r_from_parts(s_parts, eps);
  u32x4 o[2];
#pragma unroll
  for (int e = 0; e < 16; e += 2)
    o[e >> 3][(e & 7) >> 1] = (uint32_t)float_to_half_bits(xn_exact(v[e], r, wv[e])) |
                              ((uint32_t)float_to_half_bits(xn_exact(v[e + 1], r, wv[e + 1])) << 16);
  u32x4* dst = reinterpret_cast<u32x4*>(out + (size_t)blockIdx.x * kH + 16 * threadIdx.x);
  dst[0] = o[0];
  dst[1] = o[1];
}

// Query for batch > 1 (engine.py:277): mean over rows of RMSNorm(x), fp16
// rounded, then cast to the predictor dtype.  One workgroup.
__global__ __launch_bounds__(kThreads) void k_query(const uint16_t* x, int rows, const uint16_t* w,
                                                    float eps, int to_bf16, float* q) {
  __shared__ float s_parts[kThreads];
  float sum[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) sum[e] = 0.0f;
  float wv[16];
  if (w) load_h16(w, 16 * threadIdx.x, wv);
  for (int b = 0; b < rows; ++b) {
    const uint16_t* xr = x + (size_t)b * kH;
    const float r = w ? block_rnorm(xr, eps, s_parts) : 1.0f;
    float v[16];
    load_h16(xr, 16 * threadIdx.x, v);
#pragma unroll
    for (int e = 0; e < 16; ++e) sum[e] += w ? xn_exact(v[e], r, wv[e]) : v[e];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float m = round_f16(sum[e] / (float)rows);
    q[16 * threadIdx.x + e] = to_bf16 ? round_bf16(m) : m;
  }
}

// One hidden-state row of any supported dtype cast to the predictor dtype
// (predictor.py:455: hidden_state.to(parameter dtype)), as fp32 values: fp16
// and bf16 widen exactly; fp32 is kept, or rounded to bf16 for a bf16
// predictor.  One workgroup, 16 elements per thread.
__global__ __launch_bounds__(kThreads) void k_cast_query(const void* h, int h_dtype, int to_bf16,
                                                         float* q) {
  const int e0 = 16 * threadIdx.x;
  float v[16];
  if (h_dtype == OI2_DTYPE_F32) {
    const f32x4* p = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(h) + e0);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x4 t = p[m];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * m + k] = t[k];
    }
  } else if (h_dtype == OI2_DTYPE_BF16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(h) + e0);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const u32x4 t = p[m];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        v[8 * m + 2 * d] = bf16_bits_to_float((uint16_t)(t[d] & 0xFFFFu));
        v[8 * m + 2 * d + 1] = bf16_bits_to_float((uint16_t)(t[d] >> 16));
      }
    }
  } else {
    load_h16(reinterpret_cast<const uint16_t*>(h), e0, v);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) q[e0 + e] = to_bf16 ? round_bf16(v[e]) : v[e];
}

// Chunked selection -> dense ascending list + total.  One workgroup.
__global__ __launch_bounds__(kThreads) void k_compact_dense(const int32_t* slots, const int32_t* ids,
                                                            const int32_t* counts, int n_chunks,
                                                            int32_t* dslots, int32_t* dids,
                                                            int32_t* total) {
  __shared__ int s_prefix[kMaxChunks + 1];
  ActiveList al{slots, counts, n_chunks, kSelChunk};
  chunk_prefix(al, s_prefix);
  for (int c = 0; c < n_chunks; ++c) {
    const int cnt = s_prefix[c + 1] - s_prefix[c];
    for (int k = threadIdx.x; k < cnt; k += kThreads) {
      dslots[s_prefix[c] + k] = slots[(size_t)c * kSelChunk + k];
      dids[s_prefix[c] + k] = ids[(size_t)c * kSelChunk + k];
    }
  }
  if (threadIdx.x == 0) *total = s_prefix[n_chunks];
}

// ── host side ───────────────────────────────────────────────────────────────

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}

void clear_error() { g_err.clear(); }

static int n_chunks_for(int inter) { return (inter + kSelChunk - 1) / kSelChunk; }

ColdSplit cold_split(int n_chunks, int expected) {
  int waves = (expected + kColdItemsPerWave - 1) / kColdItemsPerWave;
  waves = waves < 1 ? 1 : (waves > kMaxColdWaves ? kMaxColdWaves : waves);
  const int nc = n_chunks < 1 ? 1 : n_chunks;
  const int wpc = (waves + nc - 1) / nc;
  return ColdSplit{wpc, (nc * wpc + 3) / 4};
}

static int validate_hot(const oi2_hot* hot) {
  if (!hot || hot->n_hot == 0) return OI2_OK;
  OI2_CHECK_ARG(hot->n_hot > 0 && hot->n_hot <= kH, "n_hot %d must be in 0..%d", hot->n_hot, kH);
  OI2_CHECK_ARG(hot->down_stride >= hot->n_hot && hot->down_stride % 16 == 0 &&
                    hot->down_stride <= 4096,
                "down_stride %d must be >= n_hot %d, a multiple of 16 and <= 4096",
                hot->down_stride, hot->n_hot);
  OI2_CHECK_ARG(hot->gate_q && hot->up_q && hot->down_q && hot->gate_scale && hot->up_scale &&
                    hot->down_scale,
                "hot weight pointers must be non-null");
  OI2_CHECK_ARG(((uintptr_t)hot->gate_q | (uintptr_t)hot->up_q | (uintptr_t)hot->down_q) % 16 == 0,
                "hot weights must be 16-byte aligned");
  return OI2_OK;
}

static int validate_pred(const oi2_predictor* p) {
  OI2_CHECK_ARG(p && p->down_w && p->up_w && p->up_b, "predictor pointers must be non-null");
  OI2_CHECK_ARG(p->inter > 0 && p->inter <= 65536, "predictor inter %d out of range", p->inter);
  OI2_CHECK_ARG(p->rank > 0 && p->rank <= 256 && p->rank % 8 == 0,
                "predictor rank %d must be a multiple of 8 in 1..256", p->rank);
  OI2_CHECK_ARG(p->dtype == OI2_DTYPE_F32 || p->dtype == OI2_DTYPE_BF16, "predictor dtype %d",
                p->dtype);
  return OI2_OK;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

FfnWs ffn_ws(void* base, int n_hot, int cold_wg) {
  char* p = reinterpret_cast<char*>(base);
  FfnWs w;
  w.h_hot = reinterpret_cast<float*>(p);
  p += align256((size_t)(n_hot > 0 ? n_hot : 0) * 4 + 64);
  w.cold_part = reinterpret_cast<float*>(p);
  p += align256((size_t)cold_wg * kH * 4);
  w.xw = reinterpret_cast<uint16_t*>(p);
  p += align256(kH * 2);
  w.ssq = reinterpret_cast<float*>(p);
  return w;
}

}  // namespace oi2

using namespace oi2;

extern "C" {

const char* oi2_last_error(void) { return g_err.c_str(); }
int oi2_abi_version(void) { return OI2_ABI_VERSION; }
int oi2_record_bytes(void) { return kRecBytes; }

int oi2_dequant_records(const uint8_t* records, int32_t n_records, const int32_t* slots, int32_t n,
                        float* gate, float* up, float* down_t, void* stream) {
  clear_error();
  OI2_CHECK_ARG(n >= 0, "n must be >= 0");
  if (n == 0) return OI2_OK;
  OI2_CHECK_ARG(records && slots && gate && up && down_t, "null pointer");
  OI2_CHECK_ARG(n_records > 0 && n_records <= INT32_MAX / kRecBytes, "n_records %d must be in 1..%d",
                n_records, INT32_MAX / kRecBytes);
  OI2_CHECK_ARG((uintptr_t)records % 16 == 0, "records must be 16-byte aligned");
  hipLaunchKernelGGL(k_dequant, dim3((n + kDqRecs - 1) / kDqRecs, kH / kDqElems), dim3(kThreads), 0,
                     (hipStream_t)stream, records, n_records, slots, n, gate, up, down_t);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

int oi2_rmsnorm(const uint16_t* x, const uint16_t* w, int32_t rows, float eps, uint16_t* out,
                void* stream) {
  clear_error();
  OI2_CHECK_ARG(rows >= 0, "rows must be >= 0");
  if (rows == 0) return OI2_OK;
  OI2_CHECK_ARG(x && w && out, "null pointer");
  OI2_CHECK_ARG(((uintptr_t)x | (uintptr_t)w) % 16 == 0, "x and w must be 16-byte aligned");
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, x, w, eps, out);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

size_t oi2_ffn_workspace_bytes(int32_t batch, int32_t n_hot, int32_t cold_capacity) {
  if (batch >= 2) return batch_ws_bytes(batch, n_hot, cold_capacity > 0 ? cold_capacity : 0);
  return ffn_ws_bytes(n_hot, cold_capacity > 0 ? cold_rows_bound(cold_capacity) : 0);
}

int oi2_ffn_forward(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                    const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active,
                    int32_t act, int32_t act_on_both, int32_t add_residual, uint16_t* out,
                    float* y32, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  FfnCall c;
  int rc = ffn_validate(x, batch, norm_w, hot, cold, active, act, &c);
  if (rc || batch == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (batch >= 2)
    return batch_ffn(x, batch, norm_w, eps, hot, c.has_cold ? cold : nullptr,
                     c.has_cold ? active : nullptr, act == OI2_ACT_RELU, act_on_both != 0,
                     add_residual, out, y32, workspace, workspace_bytes, st);
  const int ws_wg = c.has_cold ? cold_rows_bound(c.cap) : 0;
  OI2_CHECK_ARG(workspace && workspace_bytes >= ffn_ws_bytes(c.n_hot, ws_wg),
                "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                ffn_ws_bytes(c.n_hot, ws_wg));
  return ffn_decode_tokens(x, batch, norm_w, eps, hot, cold, active, act, act_on_both, add_residual,
                           out, y32, c, ffn_ws(workspace, c.n_hot, ws_wg), st);
}

int oi2_ffn_forward_chain(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                          const uint16_t* xn_in, const oi2_hot* hot, const oi2_cold* cold,
                          const oi2_active* active, int32_t act, int32_t act_on_both, int32_t add_residual,
                          uint16_t* out, float* y32, const uint16_t* next_norm_w, float next_eps,
                          uint16_t* xn_next, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(batch >= 2, "batch %d: the chained call runs batches of 2 and more", batch);
  FfnCall c;
  int rc = ffn_validate(x, batch, norm_w, hot, cold, active, act, &c);
  if (rc) return rc;
  OI2_CHECK_ARG((uintptr_t)xn_in % 16 == 0 && (uintptr_t)next_norm_w % 16 == 0 && (uintptr_t)xn_next % 16 == 0 &&
                    (uintptr_t)out % 16 == 0,
                "xn_in, next_norm_w, xn_next and out must be 16-byte aligned");
  OI2_CHECK_ARG(!next_norm_w || (xn_next && out), "next_norm_w needs xn_next and out");
  return batch_ffn(x, batch, norm_w, eps, hot, c.has_cold ? cold : nullptr, c.has_cold ? active : nullptr,
                   act == OI2_ACT_RELU, act_on_both != 0, add_residual, out, y32, workspace, workspace_bytes,
                   (hipStream_t)stream, xn_in, next_norm_w, next_eps, next_norm_w ? xn_next : nullptr);
}

}  // extern "C"

namespace oi2 {

int ffn_validate(const uint16_t* x, int batch, const uint16_t* norm_w, const oi2_hot* hot,
                 const oi2_cold* cold, const oi2_active* active, int act, FfnCall* c) {
  OI2_CHECK_ARG(batch >= 0, "batch must be >= 0");
  *c = FfnCall{};
  if (batch == 0) return OI2_OK;
  OI2_CHECK_ARG(x, "x is null");
  OI2_CHECK_ARG((uintptr_t)x % 16 == 0 && (!norm_w || (uintptr_t)norm_w % 16 == 0),
                "x and norm_w must be 16-byte aligned");
  OI2_CHECK_ARG(act == OI2_ACT_SILU || act == OI2_ACT_RELU, "act %d", act);
  int rc = validate_hot(hot);
  if (rc) return rc;
  c->n_hot = hot ? hot->n_hot : 0;
  c->has_cold = cold && active && cold->n_records > 0 && active->n_chunks > 0;
  if (c->has_cold) {
    OI2_CHECK_ARG(cold->records && (uintptr_t)cold->records % 16 == 0,
                  "cold records must be non-null and 16-byte aligned");
    OI2_CHECK_ARG(active->slots && active->counts, "active list pointers are null");
    OI2_CHECK_ARG(active->n_chunks <= kMaxChunks && active->chunk > 0,
                  "active list: n_chunks %d (max %d), chunk %d", active->n_chunks, kMaxChunks,
                  active->chunk);
    c->cap = active->n_chunks * active->chunk;
    const int expected = active->expected > 0 && active->expected < c->cap ? active->expected : c->cap;
    const ColdSplit cs = cold_split(active->n_chunks, expected);
    c->wg_cold = cs.wg;
    c->cold_wpc = cs.wpc;
  }
  return OI2_OK;
}

// The decode kernels for `batch` tokens one after another (k_prep, k_ffn_up,
// k_ffn_down per token), every token reusing the scratch buffers in `ws`,
// whose cold partial rows must hold c.wg_cold rows.  Nothing in `ws` needs
// to be cleared first: every buffer is written before it is read.
int ffn_decode_tokens(const uint16_t* x, int batch, const uint16_t* norm_w, float eps,
                      const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active, int act,
                      int act_on_both, int add_residual, uint16_t* out, float* y32,
                      const FfnCall& c, const FfnWs& ws, hipStream_t st) {
  const int n_hot = c.n_hot;
  const bool has_cold = c.has_cold;
  const int cap = c.cap;
  const int wg_cold = c.wg_cold;
  for (int b = 0; b < batch; ++b) {
    const uint16_t* xb = x + (size_t)b * kH;
    // with a norm, every up workgroup forms x * w and the norm's partials
    // itself (no separate prep launch)
    UpArgs ua{};
    ua.tok = TokenIn{xb, xb, nullptr, eps, norm_w ? 1 : 0, norm_w};
    ua.relu = act == OI2_ACT_RELU;
    ua.both = act_on_both != 0;
    ua.n_hot = n_hot;
    if (n_hot) {
      ua.gate_q = hot->gate_q;
      ua.up_q = hot->up_q;
      ua.gate_s = hot->gate_scale;
      ua.up_s = hot->up_scale;
      ua.hot_gbias = hot->gate_bias;
    }
    ua.h_hot = ws.h_hot;
    if (has_cold) {
      ua.records = cold->records;
      ua.n_records = cold->n_records;
      ua.cold_gbias = cold->gate_bias;
      ua.act = ActiveList{active->slots, active->counts, active->n_chunks, active->chunk};
      ua.cold_part = ws.cold_part;
      ua.cold_wpc = c.cold_wpc;
    }
    ua.wg_cold = wg_cold;
    ua.wg_pred = 0;
    ua.wg_hot = (n_hot + 7) / 8;
    const int grid_up = ua.wg_cold + ua.wg_hot;
    if (grid_up > 0) {
      hipLaunchKernelGGL(k_ffn_up, dim3(grid_up), dim3(kThreads), 0, st, ua);
      OI2_CHECK_LAUNCH();
    }
    DownArgs da{};
    da.res = add_residual ? xb : nullptr;
    da.h_hot = ws.h_hot;
    da.n_hot = n_hot;
    if (n_hot) {
      da.down_stride = hot->down_stride;
      da.down_q = hot->down_q;
      da.down_s = hot->down_scale;
    }
    if (has_cold) {
      da.cold_part = ws.cold_part;
      da.cold_wg = wg_cold;
    }
    da.out = out ? out + (size_t)b * kH : nullptr;
    da.y32 = y32 ? y32 + (size_t)b * kH : nullptr;
    da.wg_pred = 0;
    da.wg_down = kDownWG;
    hipLaunchKernelGGL(k_ffn_down, dim3(da.wg_down), dim3(kThreads), 0, st, da);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}


}  // namespace oi2

extern "C" {

// Predictor workspace: the query q (H floats), z (rank + 64 doubles), the
// norm's sum-of-squares partials (kDownWG floats).
static size_t pred_ws_z_off() { return (size_t)kH * sizeof(float); }
static size_t pred_ws_ssq_off(int rank) { return pred_ws_z_off() + (size_t)(rank + 64) * sizeof(double); }

size_t oi2_predict_workspace_bytes(const oi2_predictor* p) {
  const int rank = p ? p->rank : 256;
  return pred_ws_ssq_off(rank) + (size_t)kDownWG * sizeof(float);
}

int launch_predictor(const TokenIn& tok, const uint16_t* norm_w, const float* q,
                     const oi2_predictor* p, float thr, const int32_t* lut, int32_t* slots,
                     int32_t* ids, int32_t* counts, float* logits, float* probs, uint8_t* mask,
                     double* z, hipStream_t st) {
  UpArgs ua{};
  ua.tok = tok;
  ua.pd_w = p->down_w;
  ua.pd_rank = p->rank;
  ua.pd_bf16 = p->dtype == OI2_DTYPE_BF16;
  ua.pd_norm_w = norm_w;
  ua.pd_q = q;
  ua.pd_z = z;
  ua.wg_pred = (p->rank + 3) / 4;
  hipLaunchKernelGGL(k_pred_up, dim3(ua.wg_pred), dim3(kThreads), 0, st, ua);
  OI2_CHECK_LAUNCH();
  DownArgs da{};
  da.pu_w = p->up_w;
  da.pu_b = p->up_b;
  da.pu_rank = p->rank;
  da.pu_bf16 = p->dtype == OI2_DTYPE_BF16;
  da.inter = p->inter;
  da.pd_z = z;
  da.thr = thr;
  da.lut = lut;
  da.sel_slots = slots;
  da.sel_ids = ids;
  da.sel_counts = counts;
  da.logits_out = logits;
  da.probs_out = probs;
  da.mask_out = mask;
  da.wg_pred = n_chunks_for(p->inter);
  da.wg_down = 0;
  hipLaunchKernelGGL(k_pred_down, dim3(da.wg_pred), dim3(kThreads), 0, st, da);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

int oi2_predict(const void* h, int32_t h_dtype, int32_t rows, const oi2_predictor* p,
                float threshold_logit, float* logits, float* probs, uint8_t* mask,
                void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(rows >= 0, "rows must be >= 0");
  OI2_CHECK_ARG(h_dtype == OI2_DTYPE_F16 || h_dtype == OI2_DTYPE_F32 || h_dtype == OI2_DTYPE_BF16,
                "h_dtype %d is not OI2_DTYPE_F16, _F32 or _BF16", h_dtype);
  int rc = validate_pred(p);
  if (rc) return rc;
  if (rows == 0) return OI2_OK;
  OI2_CHECK_ARG(h && (uintptr_t)h % 16 == 0, "h must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(workspace && workspace_bytes >= oi2_predict_workspace_bytes(p),
                "predict workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* q = reinterpret_cast<float*>(workspace);
  double* z = reinterpret_cast<double*>(reinterpret_cast<uint8_t*>(workspace) + pred_ws_z_off());
  const size_t row_bytes = (size_t)kH * (h_dtype == OI2_DTYPE_F32 ? 4 : 2);
  for (int b = 0; b < rows; ++b) {
    const void* hb = reinterpret_cast<const uint8_t*>(h) + (size_t)b * row_bytes;
    hipLaunchKernelGGL(k_cast_query, dim3(1), dim3(kThreads), 0, st, hb, (int)h_dtype,
                       p->dtype == OI2_DTYPE_BF16 ? 1 : 0, q);
    OI2_CHECK_LAUNCH();
    rc = launch_predictor(TokenIn{nullptr, nullptr, nullptr, 0.0f, 0}, nullptr, q, p,
                          threshold_logit, nullptr, nullptr, nullptr, nullptr,
                          logits ? logits + (size_t)b * p->inter : nullptr,
                          probs ? probs + (size_t)b * p->inter : nullptr,
                          mask ? mask + (size_t)b * p->inter : nullptr, z, st);
    if (rc) return rc;
  }
  return OI2_OK;
}

int oi2_predict_select(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                       const oi2_predictor* p, float threshold_logit, const int32_t* lut,
                       int32_t* slots, int32_t* ids, int32_t* counts, int32_t* dense_slots,
                       int32_t* dense_ids, int32_t* total, void* workspace,
                       size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_pred(p);
  if (rc) return rc;
  OI2_CHECK_ARG(batch >= 1, "batch must be >= 1");
  OI2_CHECK_ARG(x && (uintptr_t)x % 16 == 0, "x must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(!norm_w || (uintptr_t)norm_w % 16 == 0, "norm_w must be 16-byte aligned");
  OI2_CHECK_ARG(slots && ids && counts, "selection outputs are null");
  OI2_CHECK_ARG(!total || (dense_slots && dense_ids), "dense outputs are null");
  OI2_CHECK_ARG(workspace && workspace_bytes >= oi2_predict_workspace_bytes(p),
                "predict workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* q = reinterpret_cast<float*>(workspace);
  double* z = reinterpret_cast<double*>(reinterpret_cast<uint8_t*>(workspace) + pred_ws_z_off());
  float* ssq = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + pred_ws_ssq_off(p->rank));
  const float* qp = nullptr;
  if (batch > 1) {
    hipLaunchKernelGGL(k_query, dim3(1), dim3(kThreads), 0, st, x, batch, norm_w, eps,
                       p->dtype == OI2_DTYPE_BF16 ? 1 : 0, q);
    OI2_CHECK_LAUNCH();
    qp = q;
  } else if (norm_w) {
    hipLaunchKernelGGL(k_prep, dim3(1), dim3(kThreads), 0, st, x, nullptr, nullptr, ssq);
    OI2_CHECK_LAUNCH();
  }
  rc = launch_predictor(TokenIn{x, nullptr, ssq, eps, norm_w ? 1 : 0}, norm_w, qp,
                        p, threshold_logit, lut, slots, ids, counts, nullptr, nullptr, nullptr, z, st);
  if (rc) return rc;
  if (total) {
    hipLaunchKernelGGL(k_compact_dense, dim3(1), dim3(kThreads), 0, st, slots, ids, counts,
                       n_chunks_for(p->inter), dense_slots, dense_ids, total);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

}  // extern "C"
