// Persistent decode kernel: every FFN layer of one token (batch 1) in one
// launch -- DesdemonaEngine.forward's FFN loop (engine.py:421-438), each
// layer's active set predicted one layer ahead (engine.py:432-436).
//
// 256 workgroups of 512 threads, one per CU, all resident together.  Group g
// owns, in every layer:
//   hot      neurons [14 g, 14 g + 14) of the gate/up half (fp8 rows)
//   cold     chunk g of the layer's active list: the INT4 gate/up of its
//            records -> h_cold, and their down columns x h_cold summed over
//            the chunk's items into a partial of all 4096 outputs
//   down     output tile g: 16 rows (fp8 down rows x h_hot, plus the tile's
//            rows of every chunk's cold partial), the residual and the next
//            layer's x * w and sum-of-squares partial
//   predictor row g of the next layer's z = D q (g < rank), and chunk g of the
//            next layer's logits, threshold and ascending compaction
// Each layer is a U phase (gate/up) and a D phase (down), and each phase ends
// with a device-wide signal.
//
// Wave 0 is the control wave: it polls the signals, loads the phase's
// cross-group inputs (mostly straight into LDS), runs the predictor, stores
// every cross-group output and signals.  Waves 1..7 are workers: they hold
// the phase's weights in registers, loaded one phase ahead, and compute from
// LDS.  The split matters because a wave's loads complete in order: the
// control wave never has weight loads in flight ahead of the loads the
// phase waits on, and the workers never wait on a cross-group input.
// Worker loads, in issue order per layer: half the next gate/up rows (end of
// U, after the control wave's stores are acknowledged and its arrival is
// issued: B3), the other half (D1a, once the phase's inputs are in), then at
// the end of D (D2, once the control wave has computed the next list, which
// overlaps the workers' down products, and issued the phase's stores) the
// next chunk's records and the next layer's first down rows, and the other
// down rows after the U products (issued earlier they would stall those
// products while the CU's memory queue is full).  Each phase's compute needs
// only loads older than the ones still streaming, and the halves issued at
// B1 / D1 go out after the phase's cross-group inputs: a CU's memory pipeline
// is in order, and a backlog of weight loads ahead of those inputs would
// delay the whole phase.
//
// The cold down projection is done where the records are: after the U
// products every wave of a group with items takes 512 output rows and sums
// its chunk's items' down nibbles x activation x scale over them, in list
// order; the control wave stores the 16 KB partial, and in the D phase each
// output tile adds its 16 rows of every chunk's partial (chunks without items
// are skipped), in chunk order.  (The alternative, each tile gathering the 8
// bytes of its rows from every active record, costs ~540 scattered loads per
// group per layer; they queue ahead of the U signal's polls, and the groups
// whose rows share a cache line across XCDs see the signal ~2.5 us late.)
//
// Signals: per-XCD arrival counters (32 groups each); the last arrival of an
// XCD writes that XCD's flag for the phase, and a waiting group polls all 8
// flags with one load (lane l reads XCD l & 7's).  No signal takes a second,
// cross-XCD atomic.  The signal words are accessed agent-coherently (sc1).  Data
// that crosses groups inside the launch (h, h_cold, z, x, x * w, the
// partials, the active lists) is stored write-through (sc1), and a control
// wave signals only after s_waitcnt vmcnt(0) on its stores.  Every such
// buffer has one slice per layer, so each address is written at most once per
// launch and read only after the signal that completes its writes: no L2 or
// L1 can hold a stale copy (the launch starts with the caches invalidated)
// and readers use ordinary cached loads.  No L2 writeback or invalidate is
// issued inside the launch: on this part those stall every in-flight weight
// load of the XCD.
//
// Every wait is bounded: past a host-set number of polls a group sets the
// error word and goes on (the token is then garbage and the host reports it,
// clearing the signal words), so every wave reaches the end of the kernel.
#include "capi_util.h"
#include "decode_util.h"
#include "ffn_kernels.h"

namespace oi2 {
namespace {

constexpr int kPerXcd = kTokGroups / 8;
constexpr int kSyncGo = 0, kSyncXcd = 1024, kSyncErr = kTokSyncErr;
static_assert(kTokSyncGoD == kSyncGo + 64 * 8, "the host reads the D flag of XCD 0");
constexpr int kSc1 = 16;                       // cache-policy operand: agent-coherent access
constexpr int kWorkers = kTokThreads / kWave - 1;
constexpr int kColdR = 1;                      // cold records per worker (items wi + 7 i)
constexpr int kCtlCold = 2;                    // the control wave's items, right after the workers'
constexpr int kRows = kH / kTokGroups;         // 16 output rows per group
constexpr int kSlice = kH / (kWorkers + 1);    // cold partial rows per wave: 512, 8 per lane
constexpr int kPre = 16;                       // items whose slice nibbles are in LDS before the U phase
static_assert(kWorkers == 7, "the row split and the epilogue's sum assume 7 workers");
static_assert(kTokWorkers == kWorkers, "host and kernel agree on the worker count");

// The layer table through the constant address space: its fields load with
// scalar loads, which wait on their own counter, so reading them never makes
// a wave wait for its vector loads (the weights in flight).
typedef const __attribute__((address_space(4))) TokLayer CLayer;
__device__ __forceinline__ CLayer* layer_table(const TokArgs& a) {
  return reinterpret_cast<CLayer*>(reinterpret_cast<uintptr_t>(a.layers));
}

// Agent-coherent (write-through) stores at a descriptor + lane offset: one
// offset register per lane rather than a 64-bit address.
__device__ __forceinline__ void cst2(rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kSc1);
}
__device__ __forceinline__ void cst4(rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kSc1);
}
__device__ __forceinline__ void cst16(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kSc1);
}
__device__ __forceinline__ void cst8(rsrc_t r, uint32_t off, double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  u32x2v w;
  w.x = (uint32_t)u;
  w.y = (uint32_t)(u >> 32);
  __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, kSc1);
}
__device__ __forceinline__ double as_f64(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
template <typename T>
__device__ __forceinline__ T cld(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void cst(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 8 halves e0..e7 (natural order) as the pairs (e0,e4) (e1,e5) (e2,e6)
// (e3,e7) the INT4 decode produces.
__device__ __forceinline__ u32x4 pair_layout(u32x4 x) {
  u32x4 p;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    p[k] = __builtin_amdgcn_perm(x[2 + (k >> 1)], x[k >> 1], (k & 1) ? 0x07060302u : 0x05040100u);
  return p;
}

// Workgroup barrier that waits for LDS traffic only (never for vector memory
// loads: the workers' weight loads stay in flight across it).
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// vmcnt(0), issued both as asm (a fence the compiler cannot move) and as the
// builtin, which tells the compiler's counter model that every load has
// landed: otherwise, once stores are in flight too, it waits for those
// stores before the next use of any earlier load's register.
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0) expcnt(7) lgkmcnt(15)
}

// Signal epochs count on across launches, so the signal words are never
// cleared: a launch's epoch e of a phase is E = base + e, base being the D
// flag of the group's XCD when the launch starts (a group reads it before its
// own first arrival, so before that flag can move; the launch leaves every
// flag at base + n + 1).
// Counter and flag comparisons are modulo 2^32.

// Control wave: end of phase r (0 U, 1 D) for group g, epoch E.  With
// `release_workers` the workgroup barrier that lets the worker waves issue
// their next loads comes right after the first atomic is issued, so that the
// atomic is ahead of those loads in the CU's memory pipeline.
__device__ __forceinline__ void tok_arrive(uint32_t* sync, int r, int g, uint32_t e, bool release_workers = false) {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  // a zero the compiler takes for a per-lane value: with a per-lane address
  // it leaves the one-lane atomic alone instead of broadcasting its result
  // to the wave, which would wait for the result before the barrier
  uint32_t zo;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zo));
  uint32_t o1 = 0u;
  if (lane_id() == 0)
    o1 = __hip_atomic_fetch_add(sync + kSyncXcd + 64 * (8 * r + (g & 7)) + zo, 1u, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
  if (release_workers) bar();
  asm volatile("" : "+v"(o1));   // the result is first touched here, past the barrier
  if (lane_id() == 0 && o1 + 1 == (uint32_t)kPerXcd * e)   // the XCD's last arrival
    cst(sync + kSyncGo + 64 * (8 * r + (g & 7)), e);
}

// Control wave: wait until every group has ended epoch E of phase r.  Past
// `spin` polls it records the launch (base + 1) in the error word and goes
// on; so do the waits of other groups once they see that record.
__device__ __forceinline__ void tok_wait(uint32_t* sync, int r, int g, uint32_t e, uint32_t base, uint32_t spin) {
  (void)g;
  const uint32_t* xf = sync + kSyncGo + 64 * (8 * r + (lane_id() & 7));   // lane l: XCD l & 7
  uint32_t n = 0;
  while (__builtin_amdgcn_ballot_w64((int32_t)(cld(xf) - e) < 0) != 0) {
    __builtin_amdgcn_s_sleep(1);
    if (++n >= spin) {
      cst(sync + kSyncErr, base + 1u);
      break;
    }
    if ((n & 63) == 0 && cld(sync + kSyncErr) == base + 1u) break;
  }
}

// The epoch base of this launch (see above).
__device__ __forceinline__ uint32_t tok_base(const uint32_t* sync, int g) {
  return cld(sync + kSyncGo + 64 * (8 + (g & 7)));
}

// A trace stamp of the control wave (kept in LDS, copied out at the end, so
// tracing adds no memory traffic inside the launch).
#define TOK_TRACE(L, k)                                                              \
  do {                                                                               \
    if (TR && (L) >= 0 && (L) < kTokTraceLayers && lane_id() == 0)                   \
      sh.trace[(L)][(k)] = __builtin_amdgcn_s_memrealtime();                         \
  } while (0)

struct alignas(16) TokShared {
  uint32_t nat[kH / 2];       // x * w of the layer
  uint32_t xq[kH / 8];        // predictor group: a quarter of x_L,
  uint32_t wq[kH / 8];        //   of the next layer's norm weight,
  uint32_t pd[kH / 8];        //   and of its predictor down row (bf16)
  float h[kTokMaxHot];        // the layer's hot activations
  uint32_t pu[8 * kWave * 4]; // predictor up rows of chunk g: 16-byte piece m of neuron l at 64 m + l
  float ycp[kH];              // this group's cold down partial (its chunk's items), all rows
  uint32_t snib[kWorkers + 1][kPre][kWave];   // the first items' down nibbles: wave w's slice, lane l
  uint16_t sdsc[kPre][kGroups];               // and their down scales
  float cpin[kTokGroups * kRows];   // every chunk's cold partial, the tile's 16 rows (chunk-major)
  float dsc[kRows];           // the tile's down row scales
  int cnt[kTokChunks];        // the layer's chunk counts
  int lst_slot[kTokMaxChunk]; // chunk g of the next layer's list
  int lst_id[kTokMaxChunk];
  float h_out[kWorkers * 3];  // this group's hot activations
  float hc_out[kTokMaxChunk]; // this group's cold activations (chunk order)
  float cpart[kWorkers][kRows];
  float out[kRows];
  double z[kTokMaxRank];
  uint64_t trace[kTokTraceLayers][kTokTracePoints];   // the control wave's stamps, when traced
  float r;
  int lst_cnt;
};
static_assert(offsetof(TokShared, nat) % 16 == 0 && offsetof(TokShared, xq) % 16 == 0 &&
              offsetof(TokShared, wq) % 16 == 0 && offsetof(TokShared, pd) % 16 == 0 &&
              offsetof(TokShared, h) % 16 == 0 && offsetof(TokShared, pu) % 16 == 0 &&
              offsetof(TokShared, ycp) % 16 == 0 && offsetof(TokShared, cpin) % 16 == 0 &&
              offsetof(TokShared, dsc) % 16 == 0,
              "LDS DMA targets and 16-byte reads are 16-byte aligned");

// The cold down partial of this group's chunk for rows 512 w + 8 l .. + 8
// (wave w, lane l): every item of the chunk in list order, its down nibbles
// times its activation times the rows' group scale (the two-launch path's
// arithmetic: activation x scale in fp32, then the fma with the nibble).
// Items k < kPre come from LDS (loaded by the control wave before the phase);
// the rest are loaded here, four at a time.  Result to ycp.
__device__ __forceinline__ void cold_slice(const TokShared& sh, float* ycp, int w, int cnt, rsrc_t rrec,
                                           int n_records) {
  const int l = lane_id();
  const uint32_t nb_off = kOffDown + (uint32_t)(kSlice / 2 * w + 4 * l);
  const uint32_t sc_off = kOffScales + 2 * (uint32_t)(2 * kGroups + kSlice / kGroup * w + (8 * l) / kGroup);
  float y8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y8[e] = 0.0f;
  auto add = [&](uint32_t nib, float sc, float hv) {
    const float hs = hv * sc;
    f16x2 tq[4];
    int4x8_to_f16x2x4(nib, tq);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      y8[k] = fmaf(hs, (float)tq[k].x, y8[k]);
      y8[k + 4] = fmaf(hs, (float)tq[k].y, y8[k + 4]);
    }
  };
  const int kp = cnt < kPre ? cnt : kPre;
  for (int k = 0; k < kp; ++k)
    add(sh.snib[w][k][l], half_bits_to_float(sh.sdsc[k][kSlice / kGroup * w + (8 * l) / kGroup]), sh.hc_out[k]);
  for (int k0 = kPre; k0 < cnt; k0 += 4) {
    uint32_t nb[4];
    float sc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int k = k0 + q;
      const int sl = k < cnt ? sh.lst_slot[k] : -1;
      const uint32_t ro = (sl >= 0 && sl < n_records) ? (uint32_t)sl * kRecBytes : kNoOff;
      nb[q] = bld4(rrec, ro == kNoOff ? kNoOff : ro + nb_off);
      sc[q] = half_bits_to_float(bld2(rrec, ro == kNoOff ? kNoOff : ro + sc_off));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (k0 + q < cnt) add(nb[q], sc[q], sh.hc_out[k0 + q]);
  }
  reinterpret_cast<f32x4*>(ycp)[2 * l] = f32x4{y8[0], y8[1], y8[2], y8[3]};
  reinterpret_cast<f32x4*>(ycp)[2 * l + 1] = f32x4{y8[4], y8[5], y8[6], y8[7]};
}

// Control wave, before the U phase's wait: the down nibbles of every wave's
// slice and the down scales of the chunk's first kPre items into LDS (their
// completion is covered by the wave's vmcnt(0) before B1).
__device__ __forceinline__ void slice_preload(TokShared& sh, int cnt, rsrc_t rrec, int n_records) {
  const int l = lane_id();
  const int kp = cnt < kPre ? cnt : kPre;
  for (int k = 0; k < kp; ++k) {
    const int sl = sh.lst_slot[k];
    const bool ok = sl >= 0 && sl < n_records;
    const uint32_t ro = (uint32_t)sl * kRecBytes;
#pragma unroll
    for (int w = 0; w <= kWorkers; ++w)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rrec, (lds_void*)sh.snib[w][k], 4, ok ? ro + kOffDown + (uint32_t)(kSlice / 2 * w + 4 * l) : kNoOff, 0, 0, 0);
  }
  // scales: lane l takes 16 bytes l & 3 of item l >> 2's 64-byte down scale array
  const int k = l >> 2;
  const int sl = k < kp ? sh.lst_slot[k] : -1;
  const bool ok = sl >= 0 && sl < n_records;
  bld16_lds(rrec, sh.sdsc, ok ? (uint32_t)sl * kRecBytes + kOffScales + 4 * kGroups + 16 * (uint32_t)(l & 3) : kNoOff);
}

// ── the control wave ────────────────────────────────────────────────────────

template <int NPW, bool TR>
__device__ void control(const TokArgs& a, int g, TokShared& sh) {
  const int l = lane_id();
  const int n = a.n_layers;
  const int tile = (g & 7) * (kTokGroups / 8) + (g >> 3);   // XCD-aware: an XCD owns 512 rows
  const int j0 = tile * kRows;
  const int g0 = l >> 2;
  CLayer* LT = layer_table(a);
  const uint32_t base = tok_base(a.sync, g);
  for (int L = -1; L < n; ++L) {
    CLayer* T = L >= 0 ? LT + L : nullptr;
    CLayer* N = L + 1 < n ? LT + L + 1 : nullptr;
    // ================= U phase of layer L (L = -1: only layer 0's predictor)
    const bool has_cold = T && T->n_records > 0 && T->act_counts;
    const int chunk = has_cold ? T->act_chunk : 0;
    // the next layer's predictor: group g sums quarter g & 3 of row g >> 2
    const bool pred = N && N->pd_w && g < 4 * N->rank;
    // loaded ahead of the wait (weights, and the records of this group's own
    // list, computed by this wave in the previous D phase): a predictor
    // group's quarter of the next norm weight and D row, and the chunk's
    // items past the workers' share
    if (pred) {
      const rsrc_t rw = rsrc(N->norm_w, kH * 2);
      const rsrc_t rd = rsrc(N->pd_w + (size_t)(g >> 2) * kH, kH * 2);
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const uint32_t off = 16 * (uint32_t)(l + 64 * (2 * (g & 3) + it));
        bld16_lds(rw, sh.wq + 256 * it, off);
        wld16_lds(rd, sh.pd + 256 * it, off);
      }
    }
    const int ccnt = has_cold ? sh.lst_cnt : 0;
    const rsrc_t rrec = rsrc(has_cold ? T->records : nullptr, has_cold ? (uint32_t)T->n_records * kRecBytes : 0u);
    const rsrc_t rcgb = rsrc(has_cold ? T->cold_gbias : nullptr,
                             (has_cold && T->cold_gbias) ? (uint32_t)T->n_records * 4 : 0u);
    u32x4 CQ[kCtlCold][4];
    float CS[kCtlCold][4], CG[kCtlCold];
    int CSL[kCtlCold];
#pragma unroll
    for (int i = 0; i < kCtlCold; ++i) {
      const int k = kWorkers * kColdR + i;
      const int sl = k < ccnt ? sh.lst_slot[k] : -1;
      const bool vv = has_cold && sl >= 0 && sl < T->n_records;
      CSL[i] = vv ? sl : -1;
      const uint32_t ro = vv ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        CQ[i][it] = wld16(rrec, ro + kOffGate + 16 * (l + 64 * it));
        CQ[i][2 + it] = wld16(rrec, ro + kOffUp + 16 * (l + 64 * it));
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        CS[i][2 * q] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * q + g0)));
        CS[i][2 * q + 1] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * q + 16 + g0)));
      }
      CG[i] = as_f32(bld4(rcgb, vv ? 4 * (uint32_t)sl : kNoOff));
    }
    // the slices of the chunk's cold down partial: the first items' nibbles
    // and scales
    const int nrec = has_cold ? T->n_records : 0;
    if (has_cold) slice_preload(sh, ccnt, rrec, nrec);
    if (L >= 0) tok_wait(a.sync, 1, g, base + (uint32_t)(L + 1), base, a.spin);
    TOK_TRACE(L, 0);
    // inputs the previous phase produced: x * w into LDS, the sum-of-squares
    // partials, the list's counts, and for a predictor group x_L
    if (T) {
      const rsrc_t rx = rsrc(a.xw + (size_t)L * kH, kH * 2);
#pragma unroll
      for (int it = 0; it < 8; ++it) bld16_lds(rx, sh.nat + 256 * it, 16 * (l + 64 * it));
    }
    // the layer's 256 sum-of-squares partials, this lane's four (layer 0's
    // come from x_in itself, k_prep's arithmetic: partial t sums x[16 t ..
    // 16 t + 16))
    u32x4 pp;
    if (L >= 0) {
      pp = bld16(rsrc(a.ssq + (size_t)L * kTokGroups, kTokGroups * 4), 16 * l);
    } else {
      const rsrc_t rx0 = rsrc(a.x_in, kH * 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v0 = bld16(rx0, 16 * (uint32_t)(8 * l + 2 * q)), v1 = bld16(rx0, 16 * (uint32_t)(8 * l + 2 * q + 1));
        float v[16];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          v[2 * d] = half_lo(v0[d]);
          v[2 * d + 1] = half_hi(v0[d]);
          v[8 + 2 * d] = half_lo(v1[d]);
          v[8 + 2 * d + 1] = half_hi(v1[d]);
        }
        pp[q] = as_u32(ssq16(v));
      }
    }
    const rsrc_t rcnt = rsrc(has_cold ? T->act_counts : nullptr, has_cold ? kTokChunks * 4 : 0u);
    int cnt4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) cnt4[q] = (int)bld4(rcnt, 4 * (4 * l + q));
    if (pred) {
      const uint16_t* xl = L <= 0 ? a.x_in : a.xbuf + (size_t)(L - 1) * kH;
      const rsrc_t rx = rsrc(xl, kH * 2);
#pragma unroll
      for (int it = 0; it < 2; ++it)
        bld16_lds(rx, sh.xq + 256 * it, 16 * (uint32_t)(l + 64 * (2 * (g & 3) + it)));
    }
    const float r = r_from_part(f32x4{as_f32(pp.x), as_f32(pp.y), as_f32(pp.z), as_f32(pp.w)}, a.eps);
    // the chunk counts (lane l: chunks 4 l .. 4 l + 3): which chunks' cold
    // partials the D phase reads
#pragma unroll
    for (int q = 0; q < 4; ++q) sh.cnt[4 * l + q] = min(max(cnt4[q], 0), chunk);
    if (l == 0) sh.r = r;
    wait_vm();
    bar();   // B1: x * w, r and the chunk counts are in LDS
    TOK_TRACE(L, 1);
    // a quarter of the next layer's predictor row: z = D q, q =
    // bf16(fp16(x r w')) (pred_d_role's arithmetic and partial sums);
    // stored with the phase's other outputs
    double zrow = 0.0;
    if (pred) {
      double acc = 0.0;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const u32x4 xv = reinterpret_cast<const u32x4*>(sh.xq)[l + 64 * it];
        const u32x4 wv = reinterpret_cast<const u32x4*>(sh.wq)[l + 64 * it];
        const u32x4 dv = reinterpret_cast<const u32x4*>(sh.pd)[l + 64 * it];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float q0 = round_bf16(xn_exact(half_lo(xv[d]), r, half_lo(wv[d])));
          const float q1 = round_bf16(xn_exact(half_hi(xv[d]), r, half_hi(wv[d])));
          acc = fma((double)bf16_bits_to_float((uint16_t)(dv[d] & 0xFFFFu)), (double)q0, acc);
          acc = fma((double)bf16_bits_to_float((uint16_t)(dv[d] >> 16)), (double)q1, acc);
        }
      }
      zrow = wave_sum_d(acc);
    }
    // the chunk's items past the workers' share (cold_role's arithmetic);
    // past kCtlCold more, one at a time
    for (int k = kWorkers * kColdR; k < ccnt; ++k) {
      const int i = k - kWorkers * kColdR;
      if (i >= kCtlCold) {   // rare: load this record now into slot 0
        const int sl = sh.lst_slot[k];
        const bool vv = sl >= 0 && sl < T->n_records;
        CSL[0] = vv ? sl : -1;
        const uint32_t ro = vv ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          CQ[0][it] = wld16(rrec, ro + kOffGate + 16 * (l + 64 * it));
          CQ[0][2 + it] = wld16(rrec, ro + kOffUp + 16 * (l + 64 * it));
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          CS[0][2 * q] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * q + g0)));
          CS[0][2 * q + 1] = half_bits_to_float(bld2(rrec, ro + kOffScales + 2 * (32 * q + 16 + g0)));
        }
        CG[0] = as_f32(bld4(rcgb, vv ? 4 * (uint32_t)sl : kNoOff));
      }
      const int c = i >= kCtlCold ? 0 : i;
      float hv = 0.0f;
#pragma unroll
      for (int cc = 0; cc < kCtlCold; ++cc) {
        if (cc != c) continue;
        if (CSL[cc] < 0) break;
        float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const u32x4* p = reinterpret_cast<const u32x4*>(sh.nat) + (32 * l + 2048 * it) / 8;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const u32x4 xq = pair_layout(p[d]);
            f16x2 tq[4];
            int4x8_to_f16x2x4(CQ[cc][it][d], tq);
#pragma unroll
            for (int e = 0; e < 4; ++e) pg[it] = dot2(tq[e], as_f16x2(xq[e]), pg[it]);
            int4x8_to_f16x2x4(CQ[cc][2 + it][d], tq);
#pragma unroll
            for (int e = 0; e < 4; ++e) pu[it] = dot2(tq[e], as_f16x2(xq[e]), pu[it]);
          }
        }
        const float gv = r * wave_sum(pg[0] * CS[cc][0] + pg[1] * CS[cc][1]) + CG[cc];
        const float uv = r * wave_sum(pu[0] * CS[cc][2] + pu[1] * CS[cc][3]);
        hv = gated_act(gv, uv, a.relu, a.both);
      }
      if (l == 0) sh.hc_out[k] = hv;
    }
    bar();   // B2: the workers' activations are in LDS
    TOK_TRACE(L, 2);
    // this wave's rows of the cold down partial, then every wave's in LDS
    if (has_cold && ccnt > 0) cold_slice(sh, sh.ycp, 0, ccnt, rrec, nrec);
    bar();
    if (pred && l == 0)
      cst8(rsrc(a.z + (size_t)(L + 1) * 4 * kTokMaxRank, 4 * kTokMaxRank * 8), 8 * (uint32_t)g, zrow);
    if (T) {
      const int k = g * kWorkers * NPW + l;
      if (l < kWorkers * NPW && k < T->n_hot)
        cst4(rsrc(a.h + (size_t)L * kTokMaxHot, kTokMaxHot * 4), 4 * (uint32_t)k, as_u32(sh.h_out[l]));
      // the chunk's cold down partial (chunks without items store none;
      // the D phase skips them by their count)
      if (has_cold && ccnt > 0) {
        const rsrc_t rc = rsrc(a.cpart + ((size_t)L * kTokGroups + g) * kH, kH * 4);
#pragma unroll
        for (int i = 0; i < kH / 4 / kWave; ++i)
          cst16(rc, 16 * (uint32_t)(l + kWave * i), reinterpret_cast<const u32x4*>(sh.ycp)[l + kWave * i]);
      }
    }
    // B3 (inside): the stores are acknowledged and the arrival is issued,
    // ahead of the workers' next loads
    tok_arrive(a.sync, 0, g, base + (uint32_t)(L + 2), true);
    TOK_TRACE(L, 3);

    // ================= D phase of layer L (L = -1: only layer 0's selection)
    const bool psel = N && N->pd_w;                      // the next layer's list is predicted
    const bool pstat = N && !N->pd_w && N->n_records > 0 && N->act_counts;   // or fixed
    // loaded ahead of the wait (weights, and x_L, which the U phase's wait
    // already covers): the tile's residual, next norm weight and down row
    // scales, and the next layer's predictor up rows, bias and LUT entries
    // of chunk g (lane l = neuron g * chunk + l) or its fixed list
    float res_v = 0.0f, nwv = 1.0f;
    u32x4 dsv = {0u, 0u, 0u, 0u};                        // the tile's down row scales (lanes < 4)
    if (T || N) {
      const uint16_t* xl = L <= 0 ? a.x_in : a.xbuf + (size_t)(L - 1) * kH;
      const uint32_t ro = l < kRows ? 2 * (uint32_t)(j0 + l) : kNoOff;
      res_v = half_bits_to_float(bld2(rsrc(xl, kH * 2), ro));
      nwv = N ? half_bits_to_float(bld2(rsrc(N->norm_w, kH * 2), ro)) : 1.0f;
    }
    if (T) dsv = bld16(rsrc(T->down_s + j0, T->n_hot > 0 ? kRows * 4 : 0u), l < kRows / 4 ? 16 * (uint32_t)l : kNoOff);
    int ch_n = 0, nn = -1;
    uint16_t pbits = 0;
    int plut = -1;
    if (psel) {
      ch_n = N->sel_chunk;
      const int rank = N->rank;
      nn = (l < ch_n && g * ch_n + l < N->inter) ? g * ch_n + l : -1;
      const rsrc_t ru = rsrc(N->pu_w, (uint32_t)N->inter * rank * 2);
#pragma unroll
      for (int m = 0; m < 8; ++m)
        wld16_lds(ru, sh.pu + 256 * m, (nn >= 0 && 8 * m < rank) ? (uint32_t)(nn * rank + 8 * m) * 2 : kNoOff);
      pbits = bld2(rsrc(N->pu_b, (uint32_t)N->inter * 2), nn >= 0 ? 2 * (uint32_t)nn : kNoOff);
      plut = N->lut ? (int)bld4(rsrc(N->lut, (uint32_t)N->inter * 4), nn >= 0 ? 4 * (uint32_t)nn : kNoOff) : nn;
    }
    int scnt = 0, sslot = -1;
    if (pstat) {   // a layer without a predictor: chunk g of its fixed list
      ch_n = N->act_chunk;
      scnt = (int)bld4(rsrc(N->act_counts, kTokChunks * 4), 4 * (uint32_t)g);
      sslot = (int)bld4(rsrc(N->act_slots, (uint32_t)kTokChunks * ch_n * 4),
                        l < ch_n ? 4 * (uint32_t)(g * ch_n + l) : kNoOff);
    }
    tok_wait(a.sync, 0, g, base + (uint32_t)(L + 2), base, a.spin);
    TOK_TRACE(L, 4);
    // inputs the U phase produced: h, the batch's activations x the tile
    // group's down scale (list order), and the next layer's z
    if (T) {
      const rsrc_t rh = rsrc(a.h + (size_t)L * kTokMaxHot, kTokMaxHot * 4);
#pragma unroll
      for (int it = 0; it < kTokMaxHot * 4 / 1024; ++it) bld16_lds(rh, sh.h + 256 * it, 16 * (l + 64 * it));
      // the tile's 16 rows of every chunk's cold partial (chunk-major; a
      // chunk without items reads zero)
      if (has_cold) {
        const rsrc_t rc = rsrc(a.cpart + (size_t)L * kTokGroups * kH, kTokGroups * kH * 4);
#pragma unroll
        for (int m = 0; m < kTokGroups * kRows / 4 / kWave; ++m) {
          const int cg = 16 * m + (l >> 2);
          const uint32_t off = sh.cnt[cg] > 0 ? 4 * (uint32_t)(cg * kH + j0) + 16 * (uint32_t)(l & 3) : kNoOff;
          bld16_lds(rc, sh.cpin + 256 * m, off);
        }
      }
    }
    double zl = 0.0;
    if (psel) {
      const rsrc_t rz = rsrc(a.z + (size_t)(L + 1) * 4 * kTokMaxRank, (uint32_t)N->rank * 32);
      const u32x4 za = bld16(rz, 32 * (uint32_t)l), zb = bld16(rz, 32 * (uint32_t)l + 16);
      zl = (as_f64(za.x, za.y) + as_f64(za.z, za.w)) + (as_f64(zb.x, zb.y) + as_f64(zb.z, zb.w));
    }
    if (l < kTokMaxRank) sh.z[l] = zl;
    wait_vm();
    if (l < kRows / 4) reinterpret_cast<u32x4*>(sh.dsc)[l] = dsv;
    // take the loaded values into plain registers now, before any store
    asm volatile("" : "+v"(res_v), "+v"(nwv));
    bar();   // D1a: h and the gather activations are in LDS (the workers start)
    TOK_TRACE(L, 5);
    // the next layer's logits in the fma order of the two-launch path,
    // threshold, LUT hot filter and ascending compaction
    if (psel) {
      const int rank = N->rank;
      bool keep = false;
      if (nn >= 0) {
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          if (8 * m >= rank) break;
          const u32x4 pv = reinterpret_cast<const u32x4*>(sh.pu)[64 * m + l];
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            acc = fma((double)bf16_bits_to_float((uint16_t)(pv[d] & 0xFFFFu)), sh.z[8 * m + 2 * d], acc);
            acc = fma((double)bf16_bits_to_float((uint16_t)(pv[d] >> 16)), sh.z[8 * m + 2 * d + 1], acc);
          }
        }
        keep = acc + (double)bf16_bits_to_float(pbits) >= (double)a.thr && plut >= 0;
      }
      const uint64_t bal = __ballot(keep);
      if (keep) {
        const int pos = __popcll(bal & ((1ull << l) - 1ull));
        sh.lst_slot[pos] = plut;
        sh.lst_id[pos] = nn;
      }
      if (l == 0) sh.lst_cnt = __popcll(bal);
    } else if (pstat) {
      const int c = min(max(scnt, 0), ch_n);
      if (l < c) sh.lst_slot[l] = sslot;
      if (l == 0) sh.lst_cnt = c;
    } else if (l == 0) {
      sh.lst_cnt = 0;
    }
    bar();   // D1b: the next chunk's list is in LDS
    TOK_TRACE(L, 6);
    // the next layer's list, after every use of a loaded value: the compiler
    // makes a wave wait for its outstanding stores before it uses a load
    // issued ahead of them
    if (psel) {
      const int c = sh.lst_cnt;
      if (l < c) {
        cst4(rsrc(N->sel_slots + (size_t)g * ch_n, (uint32_t)ch_n * 4), 4 * (uint32_t)l, (uint32_t)sh.lst_slot[l]);
        cst4(rsrc(N->sel_ids + (size_t)g * ch_n, (uint32_t)ch_n * 4), 4 * (uint32_t)l, (uint32_t)sh.lst_id[l]);
      }
      if (l == 0) cst4(rsrc(N->sel_counts, kTokChunks * 4), 4 * (uint32_t)g, (uint32_t)c);
    }
    // the epilogue: the workers' row sums were in LDS at D1b
    if (T) {
      if (l < kRows) {
        const float y = ((sh.cpart[0][l] + sh.cpart[1][l]) + (sh.cpart[2][l] + sh.cpart[3][l])) +
                        ((sh.cpart[4][l] + sh.cpart[5][l]) + sh.cpart[6][l]);
        const uint16_t ob = float_to_half_bits(res_v + y);
        cst2(rsrc(a.xbuf + (size_t)L * kH, kH * 2), 2 * (uint32_t)(j0 + l), ob);
        if (L == n - 1) __builtin_amdgcn_raw_buffer_store_b16(ob, rsrc(a.x_out, kH * 2), 2 * (uint32_t)(j0 + l), 0, 0);
        const float o = half_bits_to_float(ob);
        sh.out[l] = o;
        if (N) cst2(rsrc(a.xw + (size_t)(L + 1) * kH, kH * 2), 2 * (uint32_t)(j0 + l), float_to_half_bits(o * nwv));
      }
      if (N) {
        __builtin_amdgcn_wave_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (l == 0) cst4(rsrc(a.ssq + (size_t)(L + 1) * kTokGroups, kTokGroups * 4), 4 * (uint32_t)tile, as_u32(ssq16(sh.out)));
      }
    } else if (N) {   // layer 0's x * w and sum-of-squares partial of the tile (k_prep's arithmetic)
      if (l < kRows) {
        sh.out[l] = res_v;
        cst2(rsrc(a.xw, kH * 2), 2 * (uint32_t)(j0 + l), float_to_half_bits(res_v * nwv));
      }
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (l == 0) cst4(rsrc(a.ssq, kTokGroups * 4), 4 * (uint32_t)tile, as_u32(ssq16(sh.out)));
    }
    bar();   // D2: the phase's stores are issued, ahead of the workers' next loads
    tok_arrive(a.sync, 1, g, base + (uint32_t)(L + 2));
    TOK_TRACE(L, 7);
  }
  if (TR) {   // the stamps out, once every layer is done
    const int nl = n < kTokTraceLayers ? n : kTokTraceLayers;
    for (int i = l; i < nl * kTokTracePoints; i += kWave) {
      const int L = i / kTokTracePoints, k = i % kTokTracePoints;
      a.trace[((size_t)L * kTokGroups + g) * kTokTracePoints + k] = sh.trace[L][k];
    }
  }
}

// ── the worker waves ────────────────────────────────────────────────────────

// Every worker load is unconditional (absent data reads as zero through an
// empty or short descriptor) and issued in the same order each layer --
// gather nibbles, next gate/up rows (end of U and D1a), next chunk's records
// and down rows (end of D) -- so the compiler can wait for exactly
// the loads a compute step needs and leave the younger ones streaming.
template <int NPW>
__device__ void worker(const TokArgs& a, int g, int wi, TokShared& sh) {
  const int l = lane_id();
  const int n = a.n_layers;
  const int tile = (g & 7) * (kTokGroups / 8) + (g >> 3);
  const int j0 = tile * kRows;
  // down rows: every worker lane takes kpl columns of all 16 rows of the tile
  // (columns k0 .. k0 + kpl), so the h reads and the products are split
  // evenly; its per-row sums take one chunk's cold partial (lane slot
  // wi 64 + l < 256) before one reduction
  constexpr int kpl = NPW == 2 ? 8 : 16;
  static_assert(kWorkers * kWave * kpl >= (NPW == 2 ? NPW * kWorkers * kTokGroups : kTokMaxHot),
                "the worker columns cover every hot neuron");
  const int kc = (wi * kWave + l) * kpl;
  const int k0 = (g * kWorkers + wi) * NPW;       // hot neurons [k0, k0 + NPW)
  const int g0 = l >> 2;
  CLayer* LT = layer_table(a);
  // weights, each loaded one phase ahead of its use
  u32x4 WU[NPW][8];           // gate (0..3) and up (4..7) chunks of the hot neurons
  float gsc = 0.0f, usc = 0.0f, gbi = 0.0f;       // lane j < NPW: neuron k0 + j
  typedef typename std::conditional<NPW == 2, u32x2v, u32x4>::type dcol_t;
  dcol_t WD[kRows];           // down rows: this lane's columns of each row
  u32x4 RQ[kColdR][4];        // cold records of the chunk: gate and up halves,
  float RS[kColdR][4];        //   their group scales,
  float RG[kColdR];           //   gate bias
  int RSL[kColdR];            //   and slots
  // neurons [j0h, j1h) of the gate/up rows (and, with the first, the scales)
  auto load_hot = [&](int L, int j0h, int j1h) {          // L may be n: reads zero
    const bool v = L < n;
    CLayer& T = LT[v ? L : n - 1];
    const uint32_t nh = v ? (uint32_t)T.n_hot : 0u;
    const rsrc_t ra = rsrc(T.gate_q, nh * kH), rb = rsrc(T.up_q, nh * kH);
#pragma unroll
    for (int j = 0; j < NPW; ++j) {
      if (j < j0h || j >= j1h) continue;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const uint32_t o = (uint32_t)(k0 + j) * kH + 1024 * it + 16 * l;   // past n_hot: zero
        WU[j][it] = wld16(ra, o);
        WU[j][4 + it] = wld16(rb, o);
      }
    }
    if (j0h == 0) {
      const uint32_t so = l < NPW ? 4 * (uint32_t)(k0 + l) : kNoOff;
      gsc = as_f32(bld4(rsrc(T.gate_s, nh * 4), so));
      usc = as_f32(bld4(rsrc(T.up_s, nh * 4), so));
      gbi = as_f32(bld4(rsrc(T.hot_gbias, T.hot_gbias ? nh * 4 : 0u), so));
    }
  };
  // down rows [r0, r1) of the tile: this lane's columns (stride is a multiple
  // of 16, so a run that starts inside the row ends inside it)
  auto load_down = [&](int L, int r0, int r1) {         // L may be n (or -1): reads zero
    const bool v = L >= 0 && L < n;
    CLayer& T = LT[v ? L : 0];
    const int stride = T.down_stride;
    const bool hv = v && T.n_hot > 0;
    const rsrc_t rq = rsrc(T.down_q, hv ? (uint32_t)kH * stride : 0u);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      if (r < r0 || r >= r1) continue;
      const uint32_t o = kc < stride ? (uint32_t)((j0 + r) * stride + kc) : kNoOff;
      if constexpr (NPW == 2) WD[r] = wld8(rq, o);
      else WD[r] = wld16(rq, o);
    }
  };
  // records of chunk items k = wi + kWorkers i of layer L (the list in LDS)
  auto load_records = [&](int L) {      // L may be n: reads zero
    const bool v = L < n;
    CLayer& T = LT[v ? L : n - 1];
    const int cnt = v ? sh.lst_cnt : 0;
    const uint32_t nr = v ? (uint32_t)T.n_records : 0u;
    const rsrc_t rr = rsrc(T.records, nr * kRecBytes);
    const rsrc_t rb = rsrc(T.cold_gbias, T.cold_gbias ? nr * 4 : 0u);
#pragma unroll
    for (int i = 0; i < kColdR; ++i) {
      const int k = wi + kWorkers * i;
      const int sl = k < cnt ? sh.lst_slot[k] : -1;
      const bool ok = sl >= 0 && (uint32_t)sl < nr;
      RSL[i] = ok ? sl : -1;
      const uint32_t ro = ok ? (uint32_t)sl * kRecBytes : kNoOff;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        RQ[i][it] = bld16(rr, ro + kOffGate + 16 * (l + 64 * it));
        RQ[i][2 + it] = bld16(rr, ro + kOffUp + 16 * (l + 64 * it));
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        RS[i][2 * q] = half_bits_to_float(bld2(rr, ro + kOffScales + 2 * (32 * q + g0)));
        RS[i][2 * q + 1] = half_bits_to_float(bld2(rr, ro + kOffScales + 2 * (32 * q + 16 + g0)));
      }
      RG[i] = as_f32(bld4(rb, ok ? 4 * (uint32_t)sl : kNoOff));
    }
  };
  for (int L = -1; L < n; ++L) {
    CLayer* T = L >= 0 ? LT + L : nullptr;
    const bool has_cold = T && T->n_records > 0 && T->act_counts;
    // ================= U phase
    bar();   // B1: the control's inputs have landed
    if (T) {
      const float r = sh.r;
      // hot neurons (the accumulation order of the two-launch path)
      if (k0 < T->n_hot) {
        float gg[NPW], uu[NPW];
#pragma unroll
        for (int j = 0; j < NPW; ++j) gg[j] = uu[j] = 0.0f;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const u32x4* p = reinterpret_cast<const u32x4*>(sh.nat) + (1024 * it + 16 * l) / 8;
          const u32x4 x0 = p[0], x1 = p[1];
          const f16x2 xp[8] = {as_f16x2(x0.x), as_f16x2(x0.y), as_f16x2(x0.z), as_f16x2(x0.w),
                               as_f16x2(x1.x), as_f16x2(x1.y), as_f16x2(x1.z), as_f16x2(x1.w)};
#pragma unroll
          for (int j = 0; j < NPW; ++j)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              gg[j] = dot2(fp8x2_to_f16x2(WU[j][it][d], false), xp[2 * d], gg[j]);
              gg[j] = dot2(fp8x2_to_f16x2(WU[j][it][d], true), xp[2 * d + 1], gg[j]);
              uu[j] = dot2(fp8x2_to_f16x2(WU[j][4 + it][d], false), xp[2 * d], uu[j]);
              uu[j] = dot2(fp8x2_to_f16x2(WU[j][4 + it][d], true), xp[2 * d + 1], uu[j]);
            }
        }
        float gu[2 * NPW];
#pragma unroll
        for (int j = 0; j < NPW; ++j) {
          gu[j] = gg[j];
          gu[NPW + j] = uu[j];
        }
        wave_sums_to_last(gu);
        float hg = 0.0f, hu = 0.0f;
#pragma unroll
        for (int j = 0; j < NPW; ++j) {
          const float sg = readlane_f(gu[j], kWave - 1), su = readlane_f(gu[NPW + j], kWave - 1);
          if (l == j) {
            hg = sg;
            hu = su;
          }
        }
        if (l < NPW) sh.h_out[wi * NPW + l] = gated_act(r * hg * gsc + gbi, r * hu * usc, a.relu, a.both);
      }
      // this worker's cold items of chunk g: h = act(gate, up) (cold_role's arithmetic)
      if (has_cold) {
#pragma unroll
        for (int i = 0; i < kColdR; ++i) {
          if (RSL[i] < 0) {   // an invalid slot contributes zero to the partial
            if (l == 0 && wi + kWorkers * i < sh.lst_cnt) sh.hc_out[wi + kWorkers * i] = 0.0f;
            continue;
          }
          float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
#pragma unroll
          for (int it = 0; it < 2; ++it) {
            const u32x4* p = reinterpret_cast<const u32x4*>(sh.nat) + (32 * l + 2048 * it) / 8;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const u32x4 xq = pair_layout(p[d]);
              f16x2 tq[4];
              int4x8_to_f16x2x4(RQ[i][it][d], tq);
#pragma unroll
              for (int k = 0; k < 4; ++k) pg[it] = dot2(tq[k], as_f16x2(xq[k]), pg[it]);
              int4x8_to_f16x2x4(RQ[i][2 + it][d], tq);
#pragma unroll
              for (int k = 0; k < 4; ++k) pu[it] = dot2(tq[k], as_f16x2(xq[k]), pu[it]);
            }
          }
          float su[2] = {pg[0] * RS[i][0] + pg[1] * RS[i][1], pu[0] * RS[i][2] + pu[1] * RS[i][3]};
          wave_sums_to_last(su);
          const float gv = r * readlane_f(su[0], kWave - 1) + RG[i];
          const float uv = r * readlane_f(su[1], kWave - 1);
          const float hv = gated_act(gv, uv, a.relu, a.both);
          if (l == 0) sh.hc_out[wi + kWorkers * i] = hv;
        }
      }
    }
    load_down(L, 6, kRows);      // the rest of this layer's down rows
    bar();   // B2: every item's activation is in LDS
    // this wave's rows of the chunk's cold down partial
    if (has_cold && sh.lst_cnt > 0)
      cold_slice(sh, sh.ycp + kSlice * (wi + 1), wi + 1, sh.lst_cnt, rsrc(T->records, (uint32_t)T->n_records * kRecBytes),
                 T->n_records);
    bar();   // every wave's slice is in LDS
    bar();   // B3
    load_hot(L + 1, 0, 1);       // half the next gate/up rows now ...
    // ================= D phase
    bar();   // D1a: the control's inputs have landed
    load_hot(L + 1, 1, NPW);     // ... the rest once the phase's inputs are in
    float yc[kRows];
#pragma unroll
    for (int e = 0; e < kRows; ++e) yc[e] = 0.0f;
    if (T) {
      // hot: this lane's columns of the tile's 16 down rows, each row's sum
      // times its scale (the cold terms join these sums)
      float hv[kpl];
#pragma unroll
      for (int m = 0; m < kpl / 4; ++m) {
        const f32x4 v = kc < kTokMaxHot ? reinterpret_cast<const f32x4*>(sh.h + kc)[m] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        hv[4 * m] = v[0];
        hv[4 * m + 1] = v[1];
        hv[4 * m + 2] = v[2];
        hv[4 * m + 3] = v[3];
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float p = 0.0f;
#pragma unroll
        for (int w = 0; w < kpl / 4; ++w) {
          const f32x2 lo = fp8x2_to_f32x2(WD[r][w], false);
          const f32x2 hi = fp8x2_to_f32x2(WD[r][w], true);
          p = fmaf(lo.x, hv[4 * w], p);
          p = fmaf(lo.y, hv[4 * w + 1], p);
          p = fmaf(hi.x, hv[4 * w + 2], p);
          p = fmaf(hi.y, hv[4 * w + 3], p);
        }
        yc[r] = p * sh.dsc[r];
      }
      // cold: chunk wi 64 + l's partial of the tile's 16 rows (zero for a
      // chunk without items)
      if (has_cold && wi * kWave + l < kTokGroups) {
        const f32x4* cp = reinterpret_cast<const f32x4*>(sh.cpin + (wi * kWave + l) * kRows);
#pragma unroll
        for (int q = 0; q < kRows / 4; ++q) {
          const f32x4 v = cp[q];
#pragma unroll
          for (int e = 0; e < 4; ++e) yc[4 * q + e] += v[e];
        }
      }
      const float yt = wave_sums16_transposed(yc);   // lane l: row l & 15
      if (l < kRows) sh.cpart[wi][l] = yt;
    }
    bar();   // D1b: the next chunk's list (computed meanwhile) is in LDS
    bar();   // D2: the control wave's stores of the phase are issued
    load_records(L + 1);
    load_down(L + 1, 0, 6);      // the next layer's first down rows (the rest after the U products)
  }
}

template <int NPW, bool TR = false>
__global__ __launch_bounds__(kTokThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_token(TokArgs a) {
  __shared__ TokShared sh;
  const int g = blockIdx.x;   // consecutive groups run on different XCDs (g & 7)
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (w == 0)
    control<NPW, TR>(a, g, sh);
  else
    worker<NPW>(a, g, w - 1, sh);
}

}  // namespace

int tok_launch(const TokArgs& a, int npw, hipStream_t st) {
  // a traced launch runs its own instantiation: the untraced kernel carries
  // no trace code at all
  if (a.trace) {
    if (npw == 2)
      hipLaunchKernelGGL((k_token<2, true>), dim3(kTokGroups), dim3(kTokThreads), 0, st, a);
    else
      hipLaunchKernelGGL((k_token<3, true>), dim3(kTokGroups), dim3(kTokThreads), 0, st, a);
  } else if (npw == 2) {
    hipLaunchKernelGGL(k_token<2>, dim3(kTokGroups), dim3(kTokThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(k_token<3>, dim3(kTokGroups), dim3(kTokThreads), 0, st, a);
  }
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

// Number of token-kernel workgroups the device holds at once (the launch
// needs all kTokGroups of them resident).
int tok_resident(int npw, int* resident) {
  int dev = 0, cus = 0, per_cu = 0;
  OI2_CHECK_HIP(hipGetDevice(&dev));
  OI2_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (npw == 2)
    OI2_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_token<2>, kTokThreads, 0));
  else
    OI2_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_token<3>, kTokThreads, 0));
  *resident = per_cu * cus;
  return OI2_OK;
}

}  // namespace oi2
