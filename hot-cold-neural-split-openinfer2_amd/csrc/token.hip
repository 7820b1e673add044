// Persistent decode kernel: every FFN layer of one token (batch 1) in one
// launch -- DesdemonaEngine.forward's FFN loop (engine.py:421-438), each
// layer's active set predicted one layer ahead (engine.py:432-436).
//
// 512 workgroups of 256 threads, all resident together (two per CU):
//   256 U groups  gate/up of 4 hot neurons per wave (fp8 rows), the cold
//                 records of one active-list chunk (INT4 gate/up -> h_cold),
//                 and one row of the next layer's predictor z = D q
//   256 D groups  one 16-row output tile: fp8 down rows x h_hot plus the 16
//                 down nibbles of every active cold record x h_cold, the
//                 residual, the next layer's x * w and sum-of-squares
//                 partial; and one chunk of the next layer's logits,
//                 threshold and ascending compaction
// Per layer the U groups run, then the D groups.  A group signals the end of
// its phase on a device-wide counter and only then issues the loads of its
// weights for the next layer, before it waits for the other role: the weight
// stream stays in flight across every phase boundary.
//
// Signals: per-XCD arrival counters (32 groups each), then one counter per
// role, whose last arrival writes a per-XCD release flag that the groups of
// that XCD poll; the signal words are accessed agent-coherently (sc1).
// Data that crosses workgroups inside the launch (h, h_cold, z, x, x * w, the
// partials, the active lists) is stored write-through (sc1), and a group
// signals only after s_waitcnt vmcnt(0) on its stores.  Every such buffer has
// one slice per layer, so each address is written at most once per launch
// and read only after the signal that completes its writes: no L2 or L1 can
// hold a stale copy of it (the launch starts with the caches invalidated),
// and readers use ordinary cached loads -- the 32 groups of an XCD share the
// lines in L2.  No L2 writeback or invalidate is issued inside the launch: on
// this part those stall every in-flight weight load of the XCD.
//
// Every wait is bounded: past kSpinLimit polls a group sets the error word and
// goes on (the token is then garbage and the host reports it), so every wave
// reaches the end of the kernel.
#include "capi_util.h"
#include "decode_util.h"
#include "ffn_kernels.h"

namespace oi2 {
namespace {

constexpr int kPerXcd = kTokGroups / 8;
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr int kSyncGo = 0, kSyncXcd = 1024, kSyncAll = 2048, kSyncErr = kTokSyncErr;
constexpr int kSc1 = 16;             // cache-policy operand: agent-coherent access
constexpr int kColdPerRound = 2;     // cold records in flight per U wave
constexpr int kGather = 4;           // cold items per D thread per batch (the first before the U signal)

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// A buffer descriptor over [p, p + bytes).  Every call site passes
// wave-uniform values; readfirstlane lets the compiler see that (otherwise it
// wraps each load in a loop over the distinct descriptors of the wave).
__device__ __forceinline__ rsrc_t rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  // readfirstlane returns int: widen each half as uint32_t, or a low half
  // >= 2^31 would sign-extend over the high half
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
// Plain buffer loads.  A lane whose offset is past the descriptor's range
// (kNoOff, or any offset of a zero-size descriptor) reads zero: masked loads
// stay unconditional, so the compiler never has to wait for one before
// issuing the next.
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
constexpr uint32_t kNoOff = 0x80000000u;
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
__device__ __forceinline__ void cst2(rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kSc1);
}
template <typename T>
__device__ __forceinline__ T cld(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void cst(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// End of a phase for group g of role r (0 U, 1 D): epoch e.
__device__ __forceinline__ void tok_arrive(uint32_t* sync, int r, int g, uint32_t e) {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (threadIdx.x == 0) {
    const uint32_t o1 = __hip_atomic_fetch_add(sync + kSyncXcd + 64 * (8 * r + (g & 7)), 1u,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (o1 + 1 == (uint32_t)kPerXcd * e) {
      const uint32_t o2 = __hip_atomic_fetch_add(sync + kSyncAll + 64 * r, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
      if (o2 + 1 == 8u * e)
        for (int x = 0; x < 8; ++x) cst(sync + kSyncGo + 64 * (8 * r + x), e);
    }
  }
}

// Wait until every group of role r has ended epoch e.
__device__ __forceinline__ void tok_wait(uint32_t* sync, int r, int g, uint32_t e) {
  if (threadIdx.x < kWave) {
    const uint32_t* go = sync + kSyncGo + 64 * (8 * r + (g & 7));
    uint32_t n = 0;
    while (cld(go) < e) {
      __builtin_amdgcn_s_sleep(1);
      if (++n >= kSpinLimit) {
        cst(sync + kSyncErr, 1u);
        break;
      }
      if ((n & 63) == 0 && cld(sync + kSyncErr)) break;
    }
  }
  lds_sync();
}

struct TokShared {
  union {
    struct {
      uint32_t nat[kH / 2];     // x * w, natural order
      uint32_t pair[kH / 2];    // x * w, the (e0,e4) (e1,e5).. pairs of the INT4 decode
      uint32_t q[kH / 2];       // the next layer's predictor query, bf16 pairs
    } u;
    struct {
      float h[kTokMaxHot];
      float z[kTokMaxRank];
      float cold[4][16];
      float yhot[16];
      float out[16];
      int wcnt[4];
      int wsum[4];
      int pfx[kTokChunks + 1];  // exclusive prefix of the list's chunk counts
    } d;
    uint8_t pad[64 * 1024];     // two groups per CU: one U, one D on most CUs
  };
};

// ── U groups ────────────────────────────────────────────────────────────────

template <int NPW>
__device__ void u_group(const TokArgs& a, int g, TokShared& sh) {
  const int t = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform, and known to be
  const int gw = 4 * g + w;                       // U wave 0..1023
  const int prow = 4 * kTokGroups - 1 - gw;       // predictor row of this wave
  const int n = a.n_layers;
  // this iteration's weights: hot gate (0..3) and up (4..7) chunks of
  // neurons gw * NPW + j, or in W[0] the next layer's predictor row
  u32x4 W[NPW][8];
  float gsc = 0.0f, usc = 0.0f, gbi = 0.0f;       // lane j < NPW: neuron gw * NPW + j
  auto hot_of = [&](int L) { return L >= 0 ? a.layers[L].n_hot : 0; };
  // wave v runs row 1023 - v of layer L+1's predictor (waves without hot rows)
  auto pred_row_of = [&](int L, int v) {
    if (L + 1 >= n) return false;
    const TokLayer& P = a.layers[L + 1];
    return P.pd_w != nullptr && 4 * kTokGroups - 1 - v < P.rank && v * NPW >= hot_of(L);
  };
  auto pred_row = [&](int L) { return pred_row_of(L, gw); };
  auto prefetch = [&](int L) {
    const bool pr = pred_row(L);
    rsrc_t ra = rsrc(nullptr, 0), rb = ra, rgs = ra, rus = ra, rgb = ra;
    if (pr) {
      const TokLayer& P = a.layers[L + 1];
      ra = rb = rsrc(P.pd_w, (uint32_t)P.rank * kH * 2);
    } else if (L >= 0) {
      const TokLayer& T = a.layers[L];
      const uint32_t nh = (uint32_t)T.n_hot;
      ra = rsrc(T.gate_q, nh * kH);
      rb = rsrc(T.up_q, nh * kH);
      rgs = rsrc(T.gate_s, nh * 4);
      rus = rsrc(T.up_s, nh * 4);
      rgb = rsrc(T.hot_gbias, T.hot_gbias ? nh * 4 : 0u);
    }
#pragma unroll
    for (int j = 0; j < NPW; ++j)
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        uint32_t oa, ob;
        if (pr) {     // slot 0 holds the row; the other slots read zero
          oa = j == 0 ? (uint32_t)prow * kH * 2 + 16 * (lane + 64 * it) : kNoOff;
          ob = j == 0 ? (uint32_t)prow * kH * 2 + 16 * (lane + 64 * (4 + it)) : kNoOff;
        } else {      // neurons past n_hot are past the range: zero
          oa = ob = (uint32_t)(gw * NPW + j) * kH + 1024 * it + 16 * lane;
        }
        W[j][it] = bld16(ra, oa);
        W[j][4 + it] = bld16(rb, ob);
      }
    const uint32_t so = lane < NPW ? (uint32_t)(gw * NPW + lane) * 4 : kNoOff;
    gsc = as_f32(bld4(rgs, so));
    usc = as_f32(bld4(rus, so));
    gbi = as_f32(bld4(rgb, so));
  };

  // Each iteration first issues its own weight loads, then waits for the
  // other role: for L >= 0 that is right after this group's previous signal.
  // (Loads issued in one iteration and consumed in the next would be copied
  // between registers at the loop edge, and each copy waits for its load.)
  for (int L = -1; L < n; ++L) {
    prefetch(L);
    if (L >= 0) tok_wait(a.sync, 1, g, (uint32_t)(L + 1));
    const uint16_t* xl = L <= 0 ? a.x_in : a.xbuf + (size_t)(L - 1) * kH;   // input of layer max(L, 0)
    const bool prd = pred_row(L);
    const int nh = hot_of(L);
    // 1. this group's chunk of layer L's active list: count and first slots together
    int act_chunk = 0, n_records = 0;
    const uint8_t* records = nullptr;
    const float* cgb = nullptr;
    rsrc_t rcnt = rsrc(nullptr, 0), rslt = rcnt, rrec = rcnt;
    if (L >= 0 && a.layers[L].n_records > 0 && a.layers[L].act_counts) {
      const TokLayer& T = a.layers[L];
      act_chunk = T.act_chunk;
      n_records = T.n_records;
      records = T.records;
      cgb = T.cold_gbias;
      rcnt = rsrc(T.act_counts, kTokChunks * 4);
      rslt = rsrc(T.act_slots, (uint32_t)kTokChunks * act_chunk * 4);
      rrec = rsrc(T.records, (uint32_t)n_records * kRecBytes);
    }
    const uint32_t c_raw = bld4(rcnt, 4 * g);
    int s_raw[kColdPerRound];
#pragma unroll
    for (int i = 0; i < kColdPerRound; ++i) {
      const int k = w + 4 * i;
      s_raw[i] = (int)bld4(rslt, k < act_chunk ? 4 * (uint32_t)(g * act_chunk + k) : kNoOff);
    }
    // 2. the token: x * w (hot, cold) and the sum-of-squares partials
    const u32x4* pxw = reinterpret_cast<const u32x4*>(a.xw + (size_t)(L < 0 ? 0 : L) * kH) + 2 * t;
    const u32x4 xa = pxw[0], xb = pxw[1];
    const u32x4 pr = reinterpret_cast<const u32x4*>(a.ssq + (size_t)(L < 0 ? 0 : L) * kTokGroups)[lane];
    // 3. cold records of the chunk: gate and up halves, their scales
    const int cnt = act_chunk ? (int)min(c_raw, (uint32_t)act_chunk) : 0;
    u32x4 q[kColdPerRound][4];
    float s[kColdPerRound][4];
    int slot[kColdPerRound];
    const int g0 = lane >> 2;
    auto load_records = [&](int base, bool first) {
#pragma unroll
      for (int i = 0; i < kColdPerRound; ++i) {
        const int k = base + w + 4 * i;
        const int sl = first ? s_raw[i] : (int)bld4(rslt, k < act_chunk ? 4 * (uint32_t)(g * act_chunk + k) : kNoOff);
        const bool v = k < cnt && sl >= 0 && sl < n_records;
        slot[i] = v ? sl : -1;
        const uint32_t ro = v ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          q[i][it] = bld16(rrec, ro + kOffGate + 16 * (lane + 64 * it));
          q[i][2 + it] = bld16(rrec, ro + kOffUp + 16 * (lane + 64 * it));
        }
#pragma unroll
        for (int vv = 0; vv < 2; ++vv) {
          s[i][2 * vv] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * vv + g0)));
          s[i][2 * vv + 1] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * vv + 16 + g0)));
        }
      }
    };
    // 4. x * w into LDS; in workgroups with predictor rows, the query
    //    q = bf16(fp16(x r w')) with the next layer's norm weight w'
    //    (pred_d_role's arithmetic)
    const float r = r_from_part(f32x4{as_f32(pr.x), as_f32(pr.y), as_f32(pr.z), as_f32(pr.w)}, a.eps);
    const bool pred_wg = pred_row_of(L, 4 * g + 3);
    if (pred_wg) {
      const u32x4* px = reinterpret_cast<const u32x4*>(xl) + 2 * t;
      const uint8_t* nw = reinterpret_cast<const uint8_t*>(a.layers[L + 1].norm_w);
      const u32x4 x0 = px[0], x1 = px[1];
      const u32x4 w0 = load16(nw + 32 * t), w1 = load16(nw + 32 * t + 16);
      u32x4 q0, q1;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        q0[d] = (__builtin_bit_cast(uint32_t, round_bf16(xn_exact(half_lo(x0[d]), r, half_lo(w0[d])))) >> 16) |
                (__builtin_bit_cast(uint32_t, round_bf16(xn_exact(half_hi(x0[d]), r, half_hi(w0[d])))) & 0xFFFF0000u);
        q1[d] = (__builtin_bit_cast(uint32_t, round_bf16(xn_exact(half_lo(x1[d]), r, half_lo(w1[d])))) >> 16) |
                (__builtin_bit_cast(uint32_t, round_bf16(xn_exact(half_hi(x1[d]), r, half_hi(w1[d])))) & 0xFFFF0000u);
      }
      reinterpret_cast<u32x4*>(sh.u.q)[2 * t] = q0;
      reinterpret_cast<u32x4*>(sh.u.q)[2 * t + 1] = q1;
    }
    if (L >= 0) {
      reinterpret_cast<u32x4*>(sh.u.nat)[2 * t] = xa;
      reinterpret_cast<u32x4*>(sh.u.nat)[2 * t + 1] = xb;
      u32x4 pa, pb;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
        pa[k] = __builtin_amdgcn_perm(xa[2 + (k >> 1)], xa[k >> 1], sel);
        pb[k] = __builtin_amdgcn_perm(xb[2 + (k >> 1)], xb[k >> 1], sel);
      }
      reinterpret_cast<u32x4*>(sh.u.pair)[2 * t] = pa;
      reinterpret_cast<u32x4*>(sh.u.pair)[2 * t + 1] = pb;
    }
    lds_sync();
    // 5. hot neurons (same accumulation order as the two-launch path)
    if (gw * NPW < nh) {
      float gg[NPW], uu[NPW];
#pragma unroll
      for (int j = 0; j < NPW; ++j) gg[j] = uu[j] = 0.0f;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const u32x4* p = reinterpret_cast<const u32x4*>(sh.u.nat) + (1024 * it + 16 * lane) / 8;
        const u32x4 x0 = p[0], x1 = p[1];
        const f16x2 xp[8] = {as_f16x2(x0.x), as_f16x2(x0.y), as_f16x2(x0.z), as_f16x2(x0.w),
                             as_f16x2(x1.x), as_f16x2(x1.y), as_f16x2(x1.z), as_f16x2(x1.w)};
#pragma unroll
        for (int j = 0; j < NPW; ++j)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            gg[j] = dot2(fp8x2_to_f16x2(W[j][it][d], false), xp[2 * d], gg[j]);
            gg[j] = dot2(fp8x2_to_f16x2(W[j][it][d], true), xp[2 * d + 1], gg[j]);
            uu[j] = dot2(fp8x2_to_f16x2(W[j][4 + it][d], false), xp[2 * d], uu[j]);
            uu[j] = dot2(fp8x2_to_f16x2(W[j][4 + it][d], true), xp[2 * d + 1], uu[j]);
          }
      }
      float hg = 0.0f, hu = 0.0f;
#pragma unroll
      for (int j = 0; j < NPW; ++j) {
        const float sg = wave_sum(gg[j]), su = wave_sum(uu[j]);
        if (lane == j) {
          hg = sg;
          hu = su;
        }
      }
      const int k = gw * NPW + lane;
      if (lane < NPW && k < nh) cst(a.h + (size_t)L * a.hstride + k, gated_act(r * hg * gsc + gbi, r * hu * usc, a.relu, a.both));
    }
    // the chunk's first cold records, issued once the hot rows are consumed
    // (both sets together do not fit the register budget)
    if (cnt > 0) load_records(0, true);
    // 6. the next layer's predictor row: z = D q
    if (prd) {
      float acc = 0.0f;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const u32x4 qv = reinterpret_cast<const u32x4*>(sh.u.q)[lane + 64 * it];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          acc = fmaf(bf16_bits_to_float((uint16_t)(W[0][it][d] & 0xFFFFu)),
                     bf16_bits_to_float((uint16_t)(qv[d] & 0xFFFFu)), acc);
          acc = fmaf(bf16_bits_to_float((uint16_t)(W[0][it][d] >> 16)),
                     bf16_bits_to_float((uint16_t)(qv[d] >> 16)), acc);
        }
      }
      acc = wave_sum(acc);
      if (lane == 0) cst(a.z + (size_t)(L + 1) * kTokMaxRank + prow, acc);
    }
    // 7. cold records of the chunk: h = act(gate, up) in list order
    for (int base = 0; base < cnt; base += 4 * kColdPerRound) {
      if (base > 0) load_records(base, false);
#pragma unroll
      for (int i = 0; i < kColdPerRound; ++i) {
        if (slot[i] < 0) continue;
        float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const u32x4* p = reinterpret_cast<const u32x4*>(sh.u.pair) + (32 * lane + 2048 * it) / 8;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const u32x4 xq = p[d];
            f16x2 tq[4];
            int4x8_to_f16x2x4(q[i][it][d], tq);
#pragma unroll
            for (int k = 0; k < 4; ++k) pg[it] = dot2(tq[k], as_f16x2(xq[k]), pg[it]);
            int4x8_to_f16x2x4(q[i][2 + it][d], tq);
#pragma unroll
            for (int k = 0; k < 4; ++k) pu[it] = dot2(tq[k], as_f16x2(xq[k]), pu[it]);
          }
        }
        float gv = r * wave_sum(pg[0] * s[i][0] + pg[1] * s[i][1]);
        const float uv = r * wave_sum(pu[0] * s[i][2] + pu[1] * s[i][3]);
        gv += cgb ? cgb[slot[i]] : 0.0f;
        const float h = gated_act(gv, uv, a.relu, a.both);
        if (lane == 0) cst(a.hc + (size_t)L * kTokChunks * kTokMaxChunk + (size_t)g * act_chunk + base + w + 4 * i, h);
      }
    }
    tok_arrive(a.sync, 0, g, (uint32_t)(L + 2));
  }
}

// ── D groups ────────────────────────────────────────────────────────────────

__device__ void d_group(const TokArgs& a, int g, TokShared& sh) {
  const int t = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform, and known to be
  const int n = a.n_layers;
  // XCD-aware tiling: the 32 groups of an XCD (g & 7) own one contiguous
  // 512-row band, so they share the L2 lines of every cold record's down nibbles
  const int tile = (g & 7) * (kTokGroups / 8) + (g >> 3);
  const int j0 = tile * 16;
  const int je = j0 + (t & 15);
  // this iteration's weights: the wave's 4 down rows (chunks lane + 64 it),
  // and for lanes < 16 one predictor-up row of the next layer (chunk g)
  u32x4 Q[4][4];
  float dsc[4];
  uint16_t nwv_bits = 0, pbias_bits = 0;
  u32x4 P[8];
  int plut_raw = 0;
  auto pred_n = [&](int L) {            // predictor-up neuron of this lane, or -1
    if (L + 1 >= n || lane >= 16) return -1;
    const TokLayer& P1 = a.layers[L + 1];
    const int kk = 16 * w + lane;
    const int nn = g * P1.sel_chunk + kk;
    return (P1.pd_w && kk < P1.sel_chunk && nn < P1.inter) ? nn : -1;
  };
  auto prefetch = [&](int L) {
    rsrc_t rq = rsrc(nullptr, 0), rds = rq, rnw = rq, rpu = rq, rpb = rq, rlut = rq;
    int stride = 0, nch = 0;
    if (L >= 0) {
      const TokLayer& T = a.layers[L];
      stride = T.down_stride;
      nch = T.n_hot > 0 ? stride >> 4 : 0;
      rq = rsrc(T.down_q, T.n_hot > 0 ? (uint32_t)kH * stride : 0u);
      rds = rsrc(T.down_s, T.n_hot > 0 ? kH * 4 : 0u);
      rnw = rsrc(a.layers[L + 1 < n ? L + 1 : L].norm_w, kH * 2);
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int row = j0 + 4 * w + rr;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int c = lane + 64 * it;
        Q[rr][it] = bld16(rq, c < nch ? (uint32_t)(row * stride + 16 * c) : kNoOff);
      }
      dsc[rr] = as_f32(bld4(rds, 4 * row));
    }
    nwv_bits = bld2(rnw, 2 * je);
    const int nn = pred_n(L);
    int rank = 0;
    if (L + 1 < n && a.layers[L + 1].pd_w) {
      const TokLayer& P1 = a.layers[L + 1];
      rank = P1.rank;
      rpu = rsrc(P1.pu_w, (uint32_t)P1.inter * P1.rank * 2);
      rpb = rsrc(P1.pu_b, (uint32_t)P1.inter * 2);
      if (P1.lut) rlut = rsrc(P1.lut, (uint32_t)P1.inter * 4);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      P[k] = bld16(rpu, (nn >= 0 && 8 * k < rank) ? (uint32_t)(nn * rank + 8 * k) * 2 : kNoOff);
    pbias_bits = bld2(rpb, nn >= 0 ? 2 * (uint32_t)nn : kNoOff);
    plut_raw = (int)bld4(rlut, nn >= 0 ? 4 * (uint32_t)nn : kNoOff);
  };

  for (int L = -1; L < n; ++L) {
    prefetch(L);   // issued right after the previous signal (see u_group)
    // cold items of layer L's list, spread evenly: item i (list order) goes
    // to thread i mod 256, a batch of kGather at a time.  The first batch's
    // slots, down nibbles of rows [j0, j0 + 16) and their scales load while
    // the U groups run; only the cold activations wait for them.
    int total = 0, act_chunk = 0, n_records = 0;
    const uint8_t* records = nullptr;
    const int32_t* act_slots = nullptr;
    int gpos[kGather], gslot[kGather];
    u32x2v gnib[kGather];
    rsrc_t rgs = rsrc(nullptr, 0), rgr = rgs;
    float gsc[kGather];
    // list position and record data of items t + 256 (b + m), m < kGather
    auto gather = [&](int b) {
#pragma unroll
      for (int m = 0; m < kGather; ++m) {
        const int i = t + kThreads * (b + m);
        gpos[m] = -1;
        if (i < total) {
          int lo = 0, hi = kTokChunks;            // pfx[lo] <= i < pfx[hi]
          while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (sh.d.pfx[mid] <= i) lo = mid;
            else hi = mid;
          }
          gpos[m] = lo * act_chunk + (i - sh.d.pfx[lo]);
        }
      }
      int sl[kGather];
#pragma unroll
      for (int m = 0; m < kGather; ++m) sl[m] = (int)bld4(rgs, gpos[m] >= 0 ? 4 * (uint32_t)gpos[m] : kNoOff);
#pragma unroll
      for (int m = 0; m < kGather; ++m) {
        const bool v = gpos[m] >= 0 && sl[m] >= 0 && sl[m] < n_records;
        gslot[m] = v ? sl[m] : -1;
        const uint32_t ro = v ? (uint32_t)sl[m] * kRecBytes : kNoOff;
        gnib[m] = bld8(rgr, ro + kOffDown + j0 / 2);
        gsc[m] = half_bits_to_float(bld2(rgr, ro + kOffScales + 2 * (64 + j0 / kGroup)));
      }
    };
#pragma unroll
    for (int m = 0; m < kGather; ++m) {
      gpos[m] = gslot[m] = -1;
      gnib[m] = u32x2v{0, 0};
      gsc[m] = 0.0f;
    }
    if (L >= 0) {
      tok_wait(a.sync, 1, g, (uint32_t)(L + 1));     // layer L's list is complete
      const TokLayer& T = a.layers[L];
      if (T.n_records > 0 && T.act_counts) {
        act_chunk = T.act_chunk;
        n_records = T.n_records;
        records = T.records;
        act_slots = T.act_slots;
        rgs = rsrc(act_slots, (uint32_t)kTokChunks * act_chunk * 4);
        rgr = rsrc(records, (uint32_t)n_records * kRecBytes);
        const int c = (int)min((uint32_t)T.act_counts[t], (uint32_t)act_chunk);
        int v = c;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const int u = __shfl_up(v, off, kWave);
          if (lane >= off) v += u;
        }
        if (lane == kWave - 1) sh.d.wsum[w] = v;
        lds_sync();
        int base = 0;
        for (int ww = 0; ww < w; ++ww) base += sh.d.wsum[ww];
        total = sh.d.wsum[0] + sh.d.wsum[1] + sh.d.wsum[2] + sh.d.wsum[3];
        sh.d.pfx[t] = base + v - c;
        if (t == 0) sh.d.pfx[kTokChunks] = total;
        lds_sync();
        gather(0);
      }
    }
    tok_wait(a.sync, 0, g, (uint32_t)(L + 2));       // U(L) done: h, h_cold, z
    const TokLayer* T = L >= 0 ? &a.layers[L] : nullptr;
    const int nh = T ? T->n_hot : 0;
    // h and z into LDS; this thread's cold activations; the residual
    {
      // the slice is zero past n_hot up to the next multiple of 4 (never
      // written), and the range ends there: quads past it read zero
      const rsrc_t rh = rsrc(a.h + (size_t)(L < 0 ? 0 : L) * a.hstride, (uint32_t)(nh + 3) / 4 * 16);
#pragma unroll
      for (int m = 0; m < kTokMaxHot / 4 / kThreads; ++m)
        reinterpret_cast<u32x4*>(sh.d.h)[t + kThreads * m] = bld16(rh, 16 * (t + kThreads * m));
    }
    const int pn = pred_n(L);
    const int rank = (L + 1 < n) ? a.layers[L + 1].rank : 0;
    if (t < kTokMaxRank / 4 && 4 * t < rank) {
      const u32x4 v = reinterpret_cast<const u32x4*>(a.z + (size_t)(L + 1) * kTokMaxRank)[t];
      reinterpret_cast<u32x4*>(sh.d.z)[t] = v;
    }
    const rsrc_t rhc = rsrc(a.hc + (size_t)(L < 0 ? 0 : L) * kTokChunks * kTokMaxChunk,
                            kTokChunks * kTokMaxChunk * 4);
    float ghc[kGather];
#pragma unroll
    for (int m = 0; m < kGather; ++m) ghc[m] = as_f32(bld4(rhc, gslot[m] >= 0 ? 4 * (uint32_t)gpos[m] : kNoOff));
    float res_v = 0.0f;
    if (L >= 0 && t < 16) {
      const uint16_t* xl = L == 0 ? a.x_in : a.xbuf + (size_t)(L - 1) * kH;
      res_v = half_bits_to_float(xl[je]);
    }
    lds_sync();
    // 1. next layer's logits, threshold, LUT hot filter, ascending compaction
    //    (the fma order of the two-launch path)
    if (L + 1 < n && a.layers[L + 1].pd_w) {
      const TokLayer& P1 = a.layers[L + 1];
      bool keep = false;
      const int nn = pn;
      const int plut = P1.lut ? plut_raw : nn;
      if (nn >= 0) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (8 * k >= rank) break;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const int rr = 8 * k + 2 * d;
            acc = fmaf(bf16_bits_to_float((uint16_t)(P[k][d] & 0xFFFFu)), sh.d.z[rr], acc);
            acc = fmaf(bf16_bits_to_float((uint16_t)(P[k][d] >> 16)), sh.d.z[rr + 1], acc);
          }
        }
        const float logit = acc + bf16_bits_to_float(pbias_bits);
        keep = logit >= a.thr && plut >= 0;
      }
      const uint64_t bal = __ballot(keep);
      if (lane == 0) sh.d.wcnt[w] = __popcll(bal);
      lds_sync();
      int base = 0;
      for (int ww = 0; ww < w; ++ww) base += sh.d.wcnt[ww];
      if (keep) {
        const int pos = g * P1.sel_chunk + base + __popcll(bal & ((1ull << lane) - 1ull));
        cst(P1.sel_slots + pos, plut);
        cst(P1.sel_ids + pos, nn);
      }
      if (t == 0) cst(P1.sel_counts + g, sh.d.wcnt[0] + sh.d.wcnt[1] + sh.d.wcnt[2] + sh.d.wcnt[3]);
    }
    if (L >= 0) {
      // 2. hot down rows: 4 per wave
      float yh[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (nh > 0) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const f32x4* ph = reinterpret_cast<const f32x4*>(sh.d.h) + 4 * (lane + 64 * it);
          float hv[16];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f32x4 v = ph[m];
            hv[4 * m] = v[0];
            hv[4 * m + 1] = v[1];
            hv[4 * m + 2] = v[2];
            hv[4 * m + 3] = v[3];
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const f32x2 lo = fp8x2_to_f32x2(Q[rr][it][d], false);
              const f32x2 hi = fp8x2_to_f32x2(Q[rr][it][d], true);
              acc[rr] = fmaf(lo.x, hv[4 * d], acc[rr]);
              acc[rr] = fmaf(lo.y, hv[4 * d + 1], acc[rr]);
              acc[rr] = fmaf(hi.x, hv[4 * d + 2], acc[rr]);
              acc[rr] = fmaf(hi.y, hv[4 * d + 3], acc[rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) yh[rr] = wave_sum(acc[rr]);
      }
      // 3. cold: this thread's items (chunk t) x their 16 down nibbles
      float yc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) yc[e] = 0.0f;
      auto cold_item = [&](u32x2v nib, float hs) {
        f16x2 tq[4];
        int4x8_to_f16x2x4(nib.x, tq);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          yc[k] = fmaf(hs, (float)tq[k].x, yc[k]);
          yc[k + 4] = fmaf(hs, (float)tq[k].y, yc[k + 4]);
        }
        int4x8_to_f16x2x4(nib.y, tq);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          yc[8 + k] = fmaf(hs, (float)tq[k].x, yc[8 + k]);
          yc[12 + k] = fmaf(hs, (float)tq[k].y, yc[12 + k]);
        }
      };
#pragma unroll
      for (int m = 0; m < kGather; ++m)
        if (gslot[m] >= 0) cold_item(gnib[m], ghc[m] * gsc[m]);
      // lists longer than 256 kGather items: further batches, loaded now
      for (int b = kGather; t + kThreads * b < total; b += kGather) {
        gather(b);
#pragma unroll
        for (int m = 0; m < kGather; ++m) ghc[m] = as_f32(bld4(rhc, gslot[m] >= 0 ? 4 * (uint32_t)gpos[m] : kNoOff));
#pragma unroll
        for (int m = 0; m < kGather; ++m)
          if (gslot[m] >= 0) cold_item(gnib[m], ghc[m] * gsc[m]);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) yc[e] = wave_sum(yc[e]);
      if (lane == 0) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sh.d.cold[w][e] = yc[e];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sh.d.yhot[4 * w + rr] = nh > 0 ? yh[rr] * dsc[rr] : 0.0f;
      }
      lds_sync();
      // 4. x_{L+1} = x_L + y; the next layer's x * w and sum-of-squares partial
      if (t < 16) {
        const float yct = (sh.d.cold[0][t] + sh.d.cold[1][t]) + (sh.d.cold[2][t] + sh.d.cold[3][t]);
        const float y = sh.d.yhot[t] + yct;
        const uint16_t ob = float_to_half_bits(res_v + y);
        cst2(rsrc(a.xbuf + (size_t)L * kH, kH * 2), 2 * je, ob);
        if (L == n - 1) a.x_out[je] = ob;
        const float o = half_bits_to_float(ob);
        sh.d.out[t] = o;
        if (L + 1 < n) cst2(rsrc(a.xw + (size_t)(L + 1) * kH, kH * 2), 2 * je, float_to_half_bits(o * half_bits_to_float(nwv_bits)));
      }
      if (L + 1 < n) {
        lds_sync();
        if (t == 0) cst(a.ssq + (size_t)(L + 1) * kTokGroups + tile, ssq16(sh.d.out));
      }
    }
    tok_arrive(a.sync, 1, g, (uint32_t)(L + 2));
  }
}

template <int NPW>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_token(TokArgs a) {
  __shared__ TokShared sh;
  const int b = blockIdx.x;
  const int g = (b >> 4) * 8 + (b & 7);      // index within the role; g & 7 = b & 7 (the XCD)
  if (((b >> 3) & 1) == 0)
    u_group<NPW>(a, g, sh);
  else
    d_group(a, g, sh);
}

}  // namespace

// x -> x * w of layer 0 and its 256 sum-of-squares partials (k_prep's
// arithmetic), and a zeroed signal area for the token kernel that follows.
__global__ __launch_bounds__(kThreads) void k_tok_prep(const uint16_t* x, const uint16_t* w, uint16_t* xw,
                                                       float* ssq, uint32_t* sync) {
  const int t = threadIdx.x;
  float v[16], wv[16];
  load_h16(x, 16 * t, v);
  ssq[t] = ssq16(v);
  load_h16(w, 16 * t, wv);
#pragma unroll
  for (int e = 0; e < 16; ++e) xw[16 * t + e] = float_to_half_bits(v[e] * wv[e]);
  for (int i = t; i < kTokSyncWords; i += kThreads) sync[i] = 0u;
}

int tok_launch(const TokArgs& a, int npw, hipStream_t st) {
  if (npw == 2)
    hipLaunchKernelGGL(k_token<2>, dim3(kTokGrid), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(k_token<4>, dim3(kTokGrid), dim3(kThreads), 0, st, a);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

// Number of token-kernel workgroups the device holds at once (the launch
// needs all kTokGrid of them resident).
int tok_resident(int npw, int* resident) {
  int dev = 0, cus = 0, per_cu = 0;
  OI2_CHECK_HIP(hipGetDevice(&dev));
  OI2_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (npw == 2)
    OI2_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_token<2>, kThreads, 0));
  else
    OI2_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_token<4>, kThreads, 0));
  *resident = per_cu * cus;
  return OI2_OK;
}

}  // namespace oi2
