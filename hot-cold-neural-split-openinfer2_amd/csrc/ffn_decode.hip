// Decode-path kernels for gfx950: cold-record dequant, RMSNorm, the fused
// hot/cold FFN (two launches: gate/up phase, down phase) and the low-rank
// predictor with on-device index compaction.
//
// Launch shapes: 256 threads (4 wave64s) per workgroup everywhere.
//
// ffn_up   : workgroup roles by blockIdx range, cold first so the gather
//            workgroups are dispatched ahead of the bulk hot stream:
//   cold   - one wave per active record (round robin): 16-byte loads of the
//            gate/up/down nibbles + scales, gate/up dots against the
//            normalised token, activation, then the record's down column
//            scaled by h into 64 per-lane accumulators; the workgroup sums its
//            4 waves in LDS and writes one fp32 partial y (16 KB).
//   pred   - one wave per predictor down row (the lookahead layer's z).
//   hot    - two neurons per wave: fp8 gate/up rows -> fp16 pairs ->
//            v_dot2 against the fp16 normalised token, activation, h_hot.
// ffn_down : roles
//   pred   - 256 neurons per workgroup: logits = U z + b, threshold, LUT
//            filter, ballot/prefix compaction into an ascending chunk.
//   down   - 16 output rows per workgroup: fp8 down rows x h_hot, plus the
//            sum of the cold partials, plus the residual.
#include "capi_util.h"
#include "ffn_kernels.h"

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

// rsqrt(mean(x^2) + eps) over the H fp16 values of x; every thread of the
// block must call it.
__device__ float block_rnorm(const uint16_t* x, float eps, float* s_red) {
  const int t = threadIdx.x;
  const u32x4* p = reinterpret_cast<const u32x4*>(x + 16 * t);
  u32x4 a = p[0], b = p[1];
  float s = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float v0 = half_lo(a[d]), v1 = half_hi(a[d]), v2 = half_lo(b[d]), v3 = half_hi(b[d]);
    s += v0 * v0 + v1 * v1 + v2 * v2 + v3 * v3;
  }
  s = wave_sum(s);
  if (lane_id() == 0) s_red[t >> 6] = s;
  __syncthreads();
  float tot = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  __syncthreads();
  return rsqrtf(tot * (1.0f / kH) + eps);
}

// 16 normalised elements x_n[e0 .. e0+16) as floats holding fp16 values:
// fp16(x * r * w), or x itself when w is null.
__device__ __forceinline__ void load_xn16(const uint16_t* x, const uint16_t* w, float r, int e0,
                                          float v[16]) {
  const u32x4* px = reinterpret_cast<const u32x4*>(x + e0);
  u32x4 xa = px[0], xb = px[1];
  if (w) {
    const u32x4* pw = reinterpret_cast<const u32x4*>(w + e0);
    u32x4 wa = pw[0], wb = pw[1];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v[2 * d] = round_f16(half_lo(xa[d]) * r * half_lo(wa[d]));
      v[2 * d + 1] = round_f16(half_hi(xa[d]) * r * half_hi(wa[d]));
      v[8 + 2 * d] = round_f16(half_lo(xb[d]) * r * half_lo(wb[d]));
      v[8 + 2 * d + 1] = round_f16(half_hi(xb[d]) * r * half_hi(wb[d]));
    }
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v[2 * d] = half_lo(xa[d]);
      v[2 * d + 1] = half_hi(xa[d]);
      v[8 + 2 * d] = half_lo(xb[d]);
      v[8 + 2 * d + 1] = half_hi(xb[d]);
    }
  }
}

// Exclusive prefix of the (clamped) chunk counts into s_prefix[0..n_chunks].
__device__ void chunk_prefix(const ActiveList& al, int* s_prefix) {
  const int t = threadIdx.x;
  int c = 0;
  if (t < al.n_chunks) {
    c = al.counts[t];
    c = c < 0 ? 0 : (c > al.chunk ? al.chunk : c);
  }
  s_prefix[t + 1] = c;
  if (t == 0) s_prefix[0] = 0;
  __syncthreads();
  // Hillis-Steele inclusive scan over s_prefix[1..256]
  for (int off = 1; off < kThreads; off <<= 1) {
    int v = (t >= off) ? s_prefix[t + 1 - off] : 0;
    __syncthreads();
    s_prefix[t + 1] += v;
    __syncthreads();
  }
}

// ── ffn_up roles ────────────────────────────────────────────────────────────

__device__ void cold_role(const UpArgs& a, int wg, float r, float* s_lds, int* s_prefix) {
  const int w = threadIdx.x >> 6, lane = lane_id();
  chunk_prefix(a.act, s_prefix);
  const int n_chunks = a.act.n_chunks;
  const int total = s_prefix[n_chunks];
  // workgroups actually used: about kRecordsPerColdWG records each, so the
  // number of 16 KB partial rows follows the active count, not the capacity
  int n_eff = (total + kRecordsPerColdWG - 1) / kRecordsPerColdWG;
  n_eff = n_eff < 1 ? 1 : (n_eff > a.wg_cold ? a.wg_cold : n_eff);
  if (wg == 0 && threadIdx.x == 0 && a.n_part_out) *a.n_part_out = n_eff;
  if (wg >= n_eff) return;

  // token values for elements [32 lane + 2048 it, +32), in nibble-pair order
  f16x2 xc[2][16];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    float v[32];
    const int e0 = 32 * lane + 2048 * it;
    load_xn16(a.x, a.norm_w, r, e0, v);
    load_xn16(a.x, a.norm_w, r, e0 + 16, v + 16);
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        xc[it][4 * d + k].x = (_Float16)v[8 * d + k];
        xc[it][4 * d + k].y = (_Float16)v[8 * d + k + 4];
      }
  }

  float acc[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) acc[i] = 0.0f;

  const int n_waves = n_eff * 4;
  for (int i = wg * 4 + w; i < total; i += n_waves) {
    int lo = 0, hi = n_chunks;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_prefix[mid] <= i) lo = mid; else hi = mid;
    }
    const int slot = a.act.slots[(size_t)lo * a.act.chunk + (i - s_prefix[lo])];
    if (slot < 0 || slot >= a.n_records) continue;
    const uint8_t* rec = a.records + (size_t)slot * kRecBytes;
    u32x4 q[6];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      q[it] = load16_a2(rec + kOffGate + 16 * (lane + 64 * it));
      q[2 + it] = load16_a2(rec + kOffUp + 16 * (lane + 64 * it));
      q[4 + it] = load16_a2(rec + kOffDown + 16 * (lane + 64 * it));
    }
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(rec + kOffScales);
    const int g0 = lane >> 2;
    const float sg0 = half_bits_to_float(sc[g0]), sg1 = half_bits_to_float(sc[16 + g0]);
    const float su0 = half_bits_to_float(sc[32 + g0]), su1 = half_bits_to_float(sc[48 + g0]);
    const float sd0 = half_bits_to_float(sc[64 + g0]), sd1 = half_bits_to_float(sc[80 + g0]);

    float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        f16x2 p[4];
        int4x8_to_f16x2x4(q[it][d], p);
#pragma unroll
        for (int k = 0; k < 4; ++k) pg[it] = dot2(p[k], xc[it][4 * d + k], pg[it]);
        int4x8_to_f16x2x4(q[2 + it][d], p);
#pragma unroll
        for (int k = 0; k < 4; ++k) pu[it] = dot2(p[k], xc[it][4 * d + k], pu[it]);
      }
    float g = wave_sum(pg[0] * sg0 + pg[1] * sg1);
    const float u = wave_sum(pu[0] * su0 + pu[1] * su1);
    if (a.cold_gbias) g += a.cold_gbias[slot];
    const float h = gated_act(g, u, a.relu, a.both);
    const float hs[2] = {h * sd0, h * sd1};
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        f16x2 p[4];
        int4x8_to_f16x2x4(q[4 + it][d], p);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[32 * it + 8 * d + k] += hs[it] * (float)p[k].x;
          acc[32 * it + 8 * d + k + 4] += hs[it] * (float)p[k].y;
        }
      }
  }

  // sum the four waves in LDS (fixed order), then one coalesced partial row
  for (int s = 0; s < 4; ++s) {
    if (w == s) {
#pragma unroll
      for (int idx = 0; idx < 64; ++idx) {
        const int j = 32 * lane + 2048 * (idx >> 5) + (idx & 31);
        const int pj = j + (j >> 5);
        s_lds[pj] = (s == 0) ? acc[idx] : s_lds[pj] + acc[idx];
      }
    }
    __syncthreads();
  }
  float* dst = a.partials + (size_t)wg * kH;
#pragma unroll
  for (int m = 0; m < kH / kThreads; ++m) {
    const int j = threadIdx.x + kThreads * m;
    dst[j] = s_lds[j + (j >> 5)];
  }
}

__device__ void pred_d_role(const UpArgs& a, int wg, float r) {
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int row = wg * 4 + w;
  if (row >= a.pd_rank) return;
  float acc = 0.0f;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int e0 = 8 * (lane + 64 * it);
    float q[8];
    if (a.pd_q) {
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = a.pd_q[e0 + k];
    } else {
      const u32x4 xv = *reinterpret_cast<const u32x4*>(a.x + e0);
      u32x4 wv = {0, 0, 0, 0};
      if (a.pd_norm_w) wv = *reinterpret_cast<const u32x4*>(a.pd_norm_w + e0);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float v0 = half_lo(xv[d]), v1 = half_hi(xv[d]);
        if (a.pd_norm_w) {
          v0 = round_f16(v0 * r * half_lo(wv[d]));
          v1 = round_f16(v1 * r * half_hi(wv[d]));
        }
        q[2 * d] = a.pd_bf16 ? round_bf16(v0) : v0;
        q[2 * d + 1] = a.pd_bf16 ? round_bf16(v1) : v1;
      }
    }
    if (a.pd_bf16) {
      const uint16_t* drow = reinterpret_cast<const uint16_t*>(a.pd_w) + (size_t)row * kH;
      const u32x4 dv = *reinterpret_cast<const u32x4*>(drow + e0);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc = fmaf(bf16_bits_to_float((uint16_t)(dv[d] & 0xFFFFu)), q[2 * d], acc);
        acc = fmaf(bf16_bits_to_float((uint16_t)(dv[d] >> 16)), q[2 * d + 1], acc);
      }
    } else {
      const float* drow = reinterpret_cast<const float*>(a.pd_w) + (size_t)row * kH;
      const f32x4 d0 = *reinterpret_cast<const f32x4*>(drow + e0);
      const f32x4 d1 = *reinterpret_cast<const f32x4*>(drow + e0 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = fmaf(d0[k], q[k], acc);
        acc = fmaf(d1[k], q[4 + k], acc);
      }
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) a.pd_z[row] = acc;
}

__device__ void hot_up_role(const UpArgs& a, int wg, float r) {
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int k0 = (wg * 4 + w) * 2;
  if (k0 >= a.n_hot) return;
  const bool two = (k0 + 1) < a.n_hot;
  u32x4 qg[2][4], qu[2][4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const size_t off = (size_t)k0 * kH + 1024 * it + 16 * lane;
    qg[0][it] = load16(a.gate_q + off);
    qu[0][it] = load16(a.up_q + off);
    if (two) {
      qg[1][it] = load16(a.gate_q + off + kH);
      qu[1][it] = load16(a.up_q + off + kH);
    } else {
      qg[1][it] = u32x4{0, 0, 0, 0};
      qu[1][it] = u32x4{0, 0, 0, 0};
    }
  }
  f16x2 xp[4][8];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    float v[16];
    load_xn16(a.x, a.norm_w, r, 1024 * it + 16 * lane, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xp[it][k].x = (_Float16)v[2 * k];
      xp[it][k].y = (_Float16)v[2 * k + 1];
    }
  }
  float g[2] = {0.0f, 0.0f}, u[2] = {0.0f, 0.0f};
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        g[n] = dot2(fp8x2_to_f16x2(qg[n][it][d], false), xp[it][2 * d], g[n]);
        g[n] = dot2(fp8x2_to_f16x2(qg[n][it][d], true), xp[it][2 * d + 1], g[n]);
        u[n] = dot2(fp8x2_to_f16x2(qu[n][it][d], false), xp[it][2 * d], u[n]);
        u[n] = dot2(fp8x2_to_f16x2(qu[n][it][d], true), xp[it][2 * d + 1], u[n]);
      }
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    g[n] = wave_sum(g[n]);
    u[n] = wave_sum(u[n]);
  }
  if (lane < 2 && (lane == 0 || two)) {
    const int k = k0 + lane;
    float gg = (lane ? g[1] : g[0]) * a.gate_s[k];
    const float uu = (lane ? u[1] : u[0]) * a.up_s[k];
    if (a.hot_gbias) gg += a.hot_gbias[k];
    a.h_hot[k] = gated_act(gg, uu, a.relu, a.both);
  }
}

__global__ __launch_bounds__(kThreads) void k_ffn_up(UpArgs a) {
  __shared__ float s_lds[kLdsRed];
  __shared__ int s_prefix[kMaxChunks + 1];
  __shared__ float s_red[4];
  const bool need_r = (a.norm_w != nullptr) || (a.wg_pred > 0 && a.pd_norm_w != nullptr && a.pd_q == nullptr);
  float r = 1.0f;
  if (need_r) r = block_rnorm(a.x, a.eps, s_red);
  int b = blockIdx.x;
  if (b < a.wg_cold) {
    cold_role(a, b, r, s_lds, s_prefix);
    return;
  }
  b -= a.wg_cold;
  if (b < a.wg_pred) {
    pred_d_role(a, b, r);
    return;
  }
  b -= a.wg_pred;
  hot_up_role(a, b, r);
}

// Predictor-only launches (layer 0's lookahead, the standalone predictor
// entry points) use their own symbols so per-kernel statistics of k_ffn_up /
// k_ffn_down cover whole FFN layers only.
__global__ __launch_bounds__(kThreads) void k_pred_up(UpArgs a) {
  __shared__ float s_red[4];
  float r = 1.0f;
  if (a.pd_norm_w != nullptr && a.pd_q == nullptr) r = block_rnorm(a.x, a.eps, s_red);
  pred_d_role(a, blockIdx.x, r);
}

// ── ffn_down roles ──────────────────────────────────────────────────────────

__device__ void pred_u_role(const DownArgs& a, int c, int* s_wcnt) {
  const int t = threadIdx.x, w = t >> 6, lane = lane_id();
  const int n = c * kSelChunk + t;
  bool keep = false;
  if (n < a.inter) {
    float logit;
    if (a.pu_bf16) {
      const uint16_t* urow = reinterpret_cast<const uint16_t*>(a.pu_w) + (size_t)n * a.pu_rank;
      float acc = 0.0f;
      for (int r0 = 0; r0 < a.pu_rank; r0 += 8) {
        const u32x4 uv = *reinterpret_cast<const u32x4*>(urow + r0);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          acc = fmaf(bf16_bits_to_float((uint16_t)(uv[d] & 0xFFFFu)), a.pd_z[r0 + 2 * d], acc);
          acc = fmaf(bf16_bits_to_float((uint16_t)(uv[d] >> 16)), a.pd_z[r0 + 2 * d + 1], acc);
        }
      }
      logit = acc + bf16_bits_to_float(reinterpret_cast<const uint16_t*>(a.pu_b)[n]);
    } else {
      const float* urow = reinterpret_cast<const float*>(a.pu_w) + (size_t)n * a.pu_rank;
      float acc = 0.0f;
      for (int r0 = 0; r0 < a.pu_rank; r0 += 4) {
        const f32x4 uv = *reinterpret_cast<const f32x4*>(urow + r0);
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = fmaf(uv[k], a.pd_z[r0 + k], acc);
      }
      logit = acc + reinterpret_cast<const float*>(a.pu_b)[n];
    }
    if (a.logits_out) a.logits_out[n] = logit;
    if (a.probs_out) a.probs_out[n] = 1.0f / (1.0f + __expf(-logit));
    const bool fire = logit >= a.thr;
    if (a.mask_out) a.mask_out[n] = fire ? 1 : 0;
    keep = fire && (a.lut == nullptr || a.lut[n] >= 0);
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
    a.sel_slots[pos] = a.lut ? a.lut[n] : n;
    a.sel_ids[pos] = n;
  }
  if (t == 0) a.sel_counts[c] = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
}

__device__ void down_role(const DownArgs& a, int wg, float* s_part, float* s_yhot) {
  const int t = threadIdx.x, w = t >> 6, lane = lane_id();
  const int j0 = wg * kRowsPerDownWG;
  float yh[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (a.n_hot > 0) {
    const int nch = a.down_stride >> 4;
    u32x4 q[4][4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const uint8_t* row = a.down_q + (size_t)(j0 + 4 * w + rr) * a.down_stride;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int c = lane + 64 * it;
        q[rr][it] = (c < nch) ? load16(row + 16 * c) : u32x4{0, 0, 0, 0};
      }
    }
    float hv[4][16];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int k0 = 16 * (lane + 64 * it);
      if (k0 + 16 <= a.n_hot) {
        const f32x4* ph = reinterpret_cast<const f32x4*>(a.h_hot + k0);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const f32x4 v = ph[m];
          hv[it][4 * m] = v[0];
          hv[it][4 * m + 1] = v[1];
          hv[it][4 * m + 2] = v[2];
          hv[it][4 * m + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) hv[it][e] = (k0 + e < a.n_hot) ? a.h_hot[k0 + e] : 0.0f;
      }
    }
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
  if (lane == 0) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int j = j0 + 4 * w + rr;
      s_yhot[4 * w + rr] = (a.n_hot > 0) ? yh[rr] * a.down_s[j] : 0.0f;
    }
  }
  const int row = t & 15, ps = t >> 4;
  float s = 0.0f;
  const int n_part = a.n_part_in ? *a.n_part_in : a.n_partials;
  for (int p = ps; p < n_part; p += 16) s += a.partials[(size_t)p * kH + j0 + row];
  s_part[t] = s;
  __syncthreads();
  if (t < 16) {
    float yc = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; ++m) yc += s_part[16 * m + t];
    const float y = s_yhot[t] + yc;
    const int j = j0 + t;
    if (a.y32) a.y32[j] = y;
    const float o = (a.res ? half_bits_to_float(a.res[j]) : 0.0f) + y;
    const uint16_t ob = float_to_half_bits(o);
    if (a.out) a.out[j] = ob;
    if (a.out2) a.out2[j] = ob;
  }
}

__global__ __launch_bounds__(kThreads) void k_ffn_down(DownArgs a) {
  __shared__ float s_part[kThreads];
  __shared__ float s_yhot[kRowsPerDownWG];
  __shared__ int s_wcnt[4];
  int b = blockIdx.x;
  if (b < a.wg_pred) {
    pred_u_role(a, b, s_wcnt);
    return;
  }
  b -= a.wg_pred;
  down_role(a, b, s_part, s_yhot);
}

__global__ __launch_bounds__(kThreads) void k_pred_down(DownArgs a) {
  __shared__ int s_wcnt[4];
  pred_u_role(a, blockIdx.x, s_wcnt);
}

// ── standalone kernels ──────────────────────────────────────────────────────

// One workgroup per record: 384 16-byte payload chunks (gate 0-127, up
// 128-255, down 256-383), 32 elements each, times the group's fp16 scale.
__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* records, int n_records,
                                                      const int32_t* slots, int n, float* gate,
                                                      float* up, float* down_t) {
  const int ri = blockIdx.x;
  const int slot = slots[ri];
  const bool valid = slot >= 0 && slot < n_records;
  const uint8_t* rec = records + (size_t)(valid ? slot : 0) * kRecBytes;
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(rec + kOffScales);
  for (int c = threadIdx.x; c < 384; c += kThreads) {
    const int v = c >> 7, cc = c & 127;
    const u32x4 q = valid ? load16_a2(rec + kOffGate + 16 * c) : u32x4{0, 0, 0, 0};
    const float s = valid ? half_bits_to_float(sc[32 * v + (cc >> 2)]) : __builtin_nanf("");
    const int e0 = 32 * cc;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const uint32_t byte = (q[d] >> (8 * bb)) & 0xFFu;
        const int lo = (int)((byte & 0xFu) ^ 8u) - 8;
        const int hi = (int)((byte >> 4) ^ 8u) - 8;
        const int e = e0 + 8 * d + 2 * bb;
        const float f0 = (float)lo * s, f1 = (float)hi * s;
        if (v == 0) {
          gate[(size_t)ri * kH + e] = f0;
          gate[(size_t)ri * kH + e + 1] = f1;
        } else if (v == 1) {
          up[(size_t)ri * kH + e] = f0;
          up[(size_t)ri * kH + e + 1] = f1;
        } else {
          down_t[(size_t)e * n + ri] = f0;
          down_t[(size_t)(e + 1) * n + ri] = f1;
        }
      }
  }
}

__global__ __launch_bounds__(kThreads) void k_rmsnorm(const uint16_t* x, const uint16_t* w,
                                                      float eps, uint16_t* out) {
  __shared__ float s_red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * kH;
  const float r = block_rnorm(xr, eps, s_red);
  float v[16];
  load_xn16(xr, w, r, 16 * threadIdx.x, v);
  uint16_t* o = out + (size_t)blockIdx.x * kH + 16 * threadIdx.x;
#pragma unroll
  for (int e = 0; e < 16; ++e) o[e] = float_to_half_bits(v[e]);
}

// Query for batch > 1 (engine.py:277): mean over rows of RMSNorm(x), fp16
// rounded, then cast to the predictor dtype.  One workgroup.
__global__ __launch_bounds__(kThreads) void k_query(const uint16_t* x, int rows, const uint16_t* w,
                                                    float eps, int to_bf16, float* q) {
  __shared__ float s_red[4];
  float sum[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) sum[e] = 0.0f;
  for (int b = 0; b < rows; ++b) {
    const uint16_t* xr = x + (size_t)b * kH;
    const float r = w ? block_rnorm(xr, eps, s_red) : 1.0f;
    float v[16];
    load_xn16(xr, w, r, 16 * threadIdx.x, v);
#pragma unroll
    for (int e = 0; e < 16; ++e) sum[e] += v[e];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float m = round_f16(sum[e] / (float)rows);
    q[16 * threadIdx.x + e] = to_bf16 ? round_bf16(m) : m;
  }
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

static int cold_wg_for(int capacity) {
  int wg = (capacity + kRecordsPerColdWG - 1) / kRecordsPerColdWG;
  return wg < 1 ? 1 : (wg > kMaxColdWG ? kMaxColdWG : wg);
}

static int validate_hot(const oi2_hot* hot) {
  if (!hot || hot->n_hot == 0) return OI2_OK;
  OI2_CHECK_ARG(hot->n_hot > 0, "n_hot must be >= 0");
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
  OI2_CHECK_ARG(n_records > 0, "n_records must be > 0");
  OI2_CHECK_ARG((uintptr_t)records % 16 == 0, "records must be 16-byte aligned");
  hipLaunchKernelGGL(k_dequant, dim3(n), dim3(kThreads), 0, (hipStream_t)stream, records,
                     n_records, slots, n, gate, up, down_t);
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

size_t oi2_ffn_workspace_bytes(int32_t batch, int32_t n_hot) {
  (void)batch;
  const size_t hot = (size_t)((n_hot > 0 ? n_hot : 0) + 64) * sizeof(float);
  return hot + (size_t)kMaxColdWG * kH * sizeof(float) + 256;
}

int oi2_ffn_forward(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                    const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active,
                    int32_t act, int32_t act_on_both, int32_t add_residual, uint16_t* out,
                    float* y32, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(batch >= 0, "batch must be >= 0");
  if (batch == 0) return OI2_OK;
  OI2_CHECK_ARG(x, "x is null");
  OI2_CHECK_ARG((uintptr_t)x % 16 == 0 && (!norm_w || (uintptr_t)norm_w % 16 == 0),
                "x and norm_w must be 16-byte aligned");
  OI2_CHECK_ARG(act == OI2_ACT_SILU || act == OI2_ACT_RELU, "act %d", act);
  int rc = validate_hot(hot);
  if (rc) return rc;
  const int n_hot = hot ? hot->n_hot : 0;
  const bool has_cold = cold && active && cold->n_records > 0 && active->n_chunks > 0;
  if (has_cold) {
    OI2_CHECK_ARG(cold->records && (uintptr_t)cold->records % 16 == 0,
                  "cold records must be non-null and 16-byte aligned");
    OI2_CHECK_ARG(active->slots && active->counts, "active list pointers are null");
    OI2_CHECK_ARG(active->n_chunks <= kMaxChunks && active->chunk > 0,
                  "active list: n_chunks %d (max %d), chunk %d", active->n_chunks, kMaxChunks,
                  active->chunk);
  }
  OI2_CHECK_ARG(workspace && workspace_bytes >= oi2_ffn_workspace_bytes(batch, n_hot),
                "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                oi2_ffn_workspace_bytes(batch, n_hot));
  float* h_hot = reinterpret_cast<float*>(workspace);
  float* partials = h_hot + ((n_hot + 64) & ~63);
  int* n_part = reinterpret_cast<int*>(partials + (size_t)kMaxColdWG * kH);
  const int wg_cold = has_cold ? cold_wg_for(active->n_chunks * active->chunk < cold->n_records
                                                 ? active->n_chunks * active->chunk
                                                 : cold->n_records)
                               : 0;
  hipStream_t st = (hipStream_t)stream;
  for (int b = 0; b < batch; ++b) {
    const uint16_t* xb = x + (size_t)b * kH;
    UpArgs ua{};
    ua.x = xb;
    ua.norm_w = norm_w;
    ua.eps = eps;
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
    ua.h_hot = h_hot;
    if (has_cold) {
      ua.records = cold->records;
      ua.n_records = cold->n_records;
      ua.cold_gbias = cold->gate_bias;
      ua.act = ActiveList{active->slots, active->counts, active->n_chunks, active->chunk};
    }
    ua.partials = partials;
    ua.n_part_out = n_part;
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
    da.h_hot = h_hot;
    da.n_hot = n_hot;
    if (n_hot) {
      da.down_stride = hot->down_stride;
      da.down_q = hot->down_q;
      da.down_s = hot->down_scale;
    }
    da.partials = partials;
    da.n_partials = 0;
    da.n_part_in = wg_cold ? n_part : nullptr;
    da.out = out ? out + (size_t)b * kH : nullptr;
    da.y32 = y32 ? y32 + (size_t)b * kH : nullptr;
    da.wg_pred = 0;
    da.wg_down = kH / kRowsPerDownWG;
    hipLaunchKernelGGL(k_ffn_down, dim3(da.wg_down), dim3(kThreads), 0, st, da);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

size_t oi2_predict_workspace_bytes(const oi2_predictor* p) {
  const int rank = p ? p->rank : 256;
  return (size_t)(kH + rank + 64) * sizeof(float);
}

static int launch_predictor(const uint16_t* x, const uint16_t* norm_w, float eps, const float* q,
                            const oi2_predictor* p, float thr, const int32_t* lut, int32_t* slots,
                            int32_t* ids, int32_t* counts, float* logits, float* probs,
                            uint8_t* mask, float* z, hipStream_t st) {
  UpArgs ua{};
  ua.x = x;
  ua.eps = eps;
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

int oi2_predict(const uint16_t* h, int32_t rows, const oi2_predictor* p, float threshold_logit,
                float* logits, float* probs, uint8_t* mask, void* workspace,
                size_t workspace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(rows >= 0, "rows must be >= 0");
  int rc = validate_pred(p);
  if (rc) return rc;
  if (rows == 0) return OI2_OK;
  OI2_CHECK_ARG(h && (uintptr_t)h % 16 == 0, "h must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(workspace && workspace_bytes >= oi2_predict_workspace_bytes(p),
                "predict workspace too small");
  float* z = reinterpret_cast<float*>(workspace) + kH;
  for (int b = 0; b < rows; ++b) {
    rc = launch_predictor(h + (size_t)b * kH, nullptr, 0.0f, nullptr, p, threshold_logit, nullptr,
                          nullptr, nullptr, nullptr, logits ? logits + (size_t)b * p->inter : nullptr,
                          probs ? probs + (size_t)b * p->inter : nullptr,
                          mask ? mask + (size_t)b * p->inter : nullptr, z, (hipStream_t)stream);
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
  float* z = q + kH;
  const float* qp = nullptr;
  if (batch > 1) {
    hipLaunchKernelGGL(k_query, dim3(1), dim3(kThreads), 0, st, x, batch, norm_w, eps,
                       p->dtype == OI2_DTYPE_BF16 ? 1 : 0, q);
    OI2_CHECK_LAUNCH();
    qp = q;
  }
  rc = launch_predictor(x, norm_w, eps, qp, p, threshold_logit, lut, slots, ids, counts, nullptr,
                        nullptr, nullptr, z, st);
  if (rc) return rc;
  if (total) {
    hipLaunchKernelGGL(k_compact_dense, dim3(1), dim3(kThreads), 0, st, slots, ids, counts,
                       n_chunks_for(p->inter), dense_slots, dense_ids, total);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

}  // extern "C"
