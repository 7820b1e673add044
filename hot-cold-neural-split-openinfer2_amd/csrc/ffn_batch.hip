// Multi-token hot/cold FFN on the matrix cores: batch decode with a shared
// active cold set and prefill chunks, sparse_ffn (engine.py:173-209) for
// x (M, H) with M >= 2.
//
// Three launches after the norm (and a compaction of the active list):
//   k_bup    H_hot  (M, n_hot) = act(s_g * X G^T + b, s_u * X U^T)   fp8 rows
//            H_cold (M, n_act) = act(sum_g s_g,g (X Q_g^T)_g + b, ...)  INT4 records
//   k_bdown  partial Y slabs: H_hot D_hot^T (fp8 rows, row scale) over K
//            splits, and H_cold D_cold over item splits (records decoded and
//            scaled into LDS, transposed for the MFMA B operand)
//   k_bfinal out = x + sum of slabs (fp16), y32
// Every product is v_mfma_f32_16x16x32_f16 with fp32 accumulation.  fp8 and
// INT4 weights convert to fp16 exactly; INT4 group scales (one per 128 K) are
// applied to each 128-wide K block's partial sums in fp32, so the gate/up
// products are exact up to fp32 accumulation.  Down weights of cold records
// are rounded once to fp16 (q * s needs 15 significant bits).
//
// MFMA 16x16x32 f16 operand layout (lane l, element i): A[l%16][8(l/16)+i],
// B[8(l/16)+i][l%16], D[4(l/16)+i][l%16].  Only the pairing of A and B
// elements along K matters, so each 128-wide K block is split among the four
// lane groups as 32 contiguous K per group, 8 per MFMA step.
#include "capi_util.h"
#include "ffn_kernels.h"

namespace oi2 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

constexpr int kBM = 64;          // token rows per tile
constexpr int kBN = 64;          // output columns per workgroup (4 waves x 16)
constexpr int kBK = 128;         // K block = INT4 scale group
constexpr int kLdA = kBK + 8;    // LDS row of the A tile, halves (272 B)
constexpr int kBKc = 32;         // items per step of the cold down product
constexpr int kLdT = kBKc + 8;   // LDS row of the decoded cold down tile, halves (80 B)

__device__ __forceinline__ h8 cat8(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
  const h4 lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const h4 hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// 8 fp8 e4m3 (two dwords, K order) -> 8 fp16 in K order, exact.
__device__ __forceinline__ h8 fp8x8_h8(uint32_t d0, uint32_t d1) {
  return cat8(fp8x2_to_f16x2(d0, false), fp8x2_to_f16x2(d0, true), fp8x2_to_f16x2(d1, false),
              fp8x2_to_f16x2(d1, true));
}

// 8 INT4 (one dword, K order) -> fp16 in the order (e0,e4,e1,e5,e2,e6,e3,e7), exact.
__device__ __forceinline__ h8 int4x8_h8(uint32_t d) {
  f16x2 p[4];
  int4x8_to_f16x2x4(d, p);
  return cat8(p[0], p[1], p[2], p[3]);
}

__device__ __forceinline__ f32x4 mfma16(h8 a, h8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t dword_of(const u32x4& a, const u32x4& b, int i) {
  return i < 4 ? a[i] : b[i - 4];
}

// Rows m0..m0+63, columns k0..k0+127 of the fp16 matrix A (row stride ld
// halves) into s[64][kLdA]; rows >= M and columns >= K read as zero.  PAIR
// stores each group of 8 as (x0,x4,x1,x5,x2,x6,x3,x7), the order the INT4
// decode produces.  Requires ld, K multiples of 8 and A 16-byte aligned.
template <bool PAIR>
__device__ __forceinline__ void stage_a(const uint16_t* A, int ld, int M, int K, int m0, int k0,
                                        uint16_t* s) {
  const int t = threadIdx.x;
  const int c = t & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = (t >> 4) + 16 * r;
    const int m = m0 + row, k = k0 + 8 * c;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < M && k < K) v = *reinterpret_cast<const u32x4*>(A + (size_t)m * ld + k);
    if (PAIR) {
      const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w;
      v.x = (d0 & 0xFFFFu) | (d2 << 16);
      v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
      v.z = (d1 & 0xFFFFu) | (d3 << 16);
      v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
    }
    *reinterpret_cast<u32x4*>(s + row * kLdA + 8 * c) = v;
  }
}

__device__ __forceinline__ h8 a_frag(const uint16_t* s, int ms, int step) {
  const int l = lane_id();
  return *reinterpret_cast<const h8*>(s + (16 * ms + (l & 15)) * kLdA + 32 * (l >> 4) + 8 * step);
}

// ── gate/up ─────────────────────────────────────────────────────────────────

__global__ __launch_bounds__(kThreads) void k_bup(BUpArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[kBM * kLdA];
  const int w = threadIdx.x >> 6, l = lane_id();
  const int m0 = blockIdx.y * kBM;
  f32x4 accg[4], accu[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) accg[ms] = accu[ms] = f32x4{0.f, 0.f, 0.f, 0.f};

  if ((int)blockIdx.x < a.hot_wg) {
    // hot: this lane's weight row n, 32 fp8 per 128-wide K block
    const int n = blockIdx.x * kBN + 16 * w + (l & 15);
    const bool nv = n < a.n_hot;
    const uint8_t* gr = a.gate_q + (size_t)(nv ? n : 0) * kH + 32 * (l >> 4);
    const uint8_t* ur = a.up_q + (size_t)(nv ? n : 0) * kH + 32 * (l >> 4);
    for (int kb = 0; kb < kH / kBK; ++kb) {
      u32x4 g0 = {0u, 0u, 0u, 0u}, g1 = g0, u0 = g0, u1 = g0;
      if (nv) {
        g0 = load16(gr + kb * kBK);
        g1 = load16(gr + kb * kBK + 16);
        u0 = load16(ur + kb * kBK);
        u1 = load16(ur + kb * kBK + 16);
      }
      __syncthreads();
      stage_a<false>(a.xn, kH, a.M, kH, m0, kb * kBK, sA);
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const h8 bg = fp8x8_h8(dword_of(g0, g1, 2 * s), dword_of(g0, g1, 2 * s + 1));
        const h8 bu = fp8x8_h8(dword_of(u0, u1, 2 * s), dword_of(u0, u1, 2 * s + 1));
#pragma unroll
        for (int ms = 0; ms < 4; ++ms) {
          const h8 av = a_frag(sA, ms, s);
          accg[ms] = mfma16(av, bg, accg[ms]);
          accu[ms] = mfma16(av, bu, accu[ms]);
        }
      }
    }
    const float sg = nv ? a.gate_s[n] : 0.f, su = nv ? a.up_s[n] : 0.f;
    const float gb = (nv && a.hot_gbias) ? a.hot_gbias[n] : 0.f;
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * ms + 4 * (l >> 4) + i;
        const float h = nv ? gated_act(fmaf(accg[ms][i], sg, gb), accu[ms][i] * su, a.relu, a.both)
                           : 0.f;
        a.hh[(size_t)m * a.ldh + n] = float_to_half_bits(h);
      }
    return;
  }

  // cold: this lane's item i of the dense active list
  const int total = min(*a.total, a.cap);
  const int i0 = ((int)blockIdx.x - a.hot_wg) * kBN;
  if (i0 >= total) return;
  const int i = i0 + 16 * w + (l & 15);
  int slot = i < total ? a.dslots[i] : -1;
  const bool iv = slot >= 0 && slot < a.n_records;
  const uint8_t* rec = a.records + (size_t)(iv ? slot : 0) * kRecBytes;
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(rec + kOffScales);
  for (int kb = 0; kb < kH / kBK; ++kb) {
    u32x4 qg = {0u, 0u, 0u, 0u}, qu = qg;
    float sg = 0.f, su = 0.f;
    if (iv) {
      qg = load16_a2(rec + kOffGate + 64 * kb + 16 * (l >> 4));
      qu = load16_a2(rec + kOffUp + 64 * kb + 16 * (l >> 4));
      sg = half_bits_to_float(sc[kb]);
      su = half_bits_to_float(sc[kGroups + kb]);
    }
    __syncthreads();
    stage_a<true>(a.xn, kH, a.M, kH, m0, kb * kBK, sA);
    __syncthreads();
    f32x4 tg[4], tu[4];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) tg[ms] = tu[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const h8 bg = int4x8_h8(qg[s]);
      const h8 bu = int4x8_h8(qu[s]);
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        const h8 av = a_frag(sA, ms, s);
        tg[ms] = mfma16(av, bg, tg[ms]);
        tu[ms] = mfma16(av, bu, tu[ms]);
      }
    }
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        accg[ms][e] = fmaf(sg, tg[ms][e], accg[ms][e]);
        accu[ms][e] = fmaf(su, tu[ms][e], accu[ms][e]);
      }
  }
  const float gb = (iv && a.cold_gbias) ? a.cold_gbias[slot] : 0.f;
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * ms + 4 * (l >> 4) + e;
      const float h = iv ? gated_act(accg[ms][e] + gb, accu[ms][e], a.relu, a.both) : 0.f;
      a.hc[(size_t)m * a.ldc + i] = float_to_half_bits(h);
    }
}

// ── down ────────────────────────────────────────────────────────────────────

__global__ __launch_bounds__(kThreads) void k_bdown(BDownArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[kBM * kLdA];
  __shared__ __attribute__((aligned(16))) uint16_t sT[kBN * kLdT];
  const int w = threadIdx.x >> 6, l = lane_id(), t = threadIdx.x;
  const int m0 = blockIdx.y * kBM;
  const int tile = blockIdx.x % (kH / kBN), split = blockIdx.x / (kH / kBN);
  const int h0 = tile * kBN;
  const int hcol = h0 + 16 * w + (l & 15);
  f32x4 acc[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) acc[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
  float out_scale = 1.f;

  if (split < a.hot_splits) {
    const int kb0 = split * a.hot_blocks / a.hot_splits;
    const int kb1 = (split + 1) * a.hot_blocks / a.hot_splits;
    const uint8_t* dr = a.down_q + (size_t)hcol * a.down_stride;
    for (int kb = kb0; kb < kb1; ++kb) {
      const int k = kb * kBK + 32 * (l >> 4);
      u32x4 q0 = {0u, 0u, 0u, 0u}, q1 = q0;
      if (k < a.down_stride) q0 = load16(dr + k);
      if (k + 16 < a.down_stride) q1 = load16(dr + k + 16);
      __syncthreads();
      stage_a<false>(a.hh, a.ldh, a.M, a.ldh, m0, kb * kBK, sA);
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const h8 b = fp8x8_h8(dword_of(q0, q1, 2 * s), dword_of(q0, q1, 2 * s + 1));
#pragma unroll
        for (int ms = 0; ms < 4; ++ms) acc[ms] = mfma16(a_frag(sA, ms, s), b, acc[ms]);
      }
    }
    if (a.hot_blocks > 0) out_scale = a.down_s[hcol];
  } else {
    const int cs = split - a.hot_splits;
    const int total = min(*a.total, a.cap);
    int per = (total + a.cold_splits - 1) / a.cold_splits;
    per = (per + kBKc - 1) / kBKc * kBKc;
    const int ib = cs * per, ie = min(total, ib + per);
    // staging role of this thread: item (t >> 3) of the step, h values 8 (t & 7) ..
    const int ti = t >> 3, th = 8 * (t & 7);
    for (int it0 = ib; it0 < ie; it0 += kBKc) {
      const int it = it0 + ti;
      const int slot = it < ie ? a.dslots[it] : -1;
      const bool v = slot >= 0 && slot < a.n_records;
      uint32_t d = 0;
      float s = 0.f;
      if (v) {
        const uint8_t* rec = a.records + (size_t)slot * kRecBytes;
        d = *reinterpret_cast<const u32_a2*>(rec + kOffDown + (h0 + th) / 2);
        s = half_bits_to_float(
            reinterpret_cast<const uint16_t*>(rec + kOffScales)[2 * kGroups + h0 / kGroup]);
      }
      // A: this lane's 8 items of rows m, zero past the end of the list
      h8 av[4];
      const int ka = it0 + 8 * (l >> 4);
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        const int m = m0 + 16 * ms + (l & 15);
        h8 x = {};
        if (m < a.M && ka < ie) {
          x = *reinterpret_cast<const h8*>(a.hc + (size_t)m * a.ldc + ka);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (ka + j >= ie) x[j] = (_Float16)0.f;
        }
        av[ms] = x;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int q = (int)((d >> (4 * j)) & 0xFu) ^ 8;
        const float wv = (float)(q - 8) * s;
        sT[(th + j) * kLdT + ti] = float_to_half_bits(wv);
      }
      __syncthreads();
      const h8 b = *reinterpret_cast<const h8*>(sT + (16 * w + (l & 15)) * kLdT + 8 * (l >> 4));
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) acc[ms] = mfma16(av[ms], b, acc[ms]);
    }
  }
  float* part = a.part + (size_t)split * a.Mpad * kH;
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * ms + 4 * (l >> 4) + e;
      part[(size_t)m * kH + hcol] = acc[ms][e] * out_scale;
    }
}

// out = res + sum of the partial slabs (fp16), y32 = the sum (fp32).
__global__ __launch_bounds__(kThreads) void k_bfinal(const float* part, int n_slabs, int Mpad, int M,
                                                    const uint16_t* res, uint16_t* out, float* y32) {
  const int n4 = M * (kH / 4);
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n4; q += gridDim.x * kThreads) {
    f32x4 y = reinterpret_cast<const f32x4*>(part)[q];
    for (int s = 1; s < n_slabs; ++s)
      y += reinterpret_cast<const f32x4*>(part + (size_t)s * Mpad * kH)[q];
    if (y32) reinterpret_cast<f32x4*>(y32)[q] = y;
    if (out) {
      float r[4] = {0.f, 0.f, 0.f, 0.f};
      if (res) {
        const uint2 rv = reinterpret_cast<const uint2*>(res)[q];
        r[0] = half_bits_to_float((uint16_t)(rv.x & 0xFFFFu));
        r[1] = half_bits_to_float((uint16_t)(rv.x >> 16));
        r[2] = half_bits_to_float((uint16_t)(rv.y & 0xFFFFu));
        r[3] = half_bits_to_float((uint16_t)(rv.y >> 16));
      }
      const uint32_t lo = (uint32_t)float_to_half_bits(r[0] + y.x) |
                          ((uint32_t)float_to_half_bits(r[1] + y.y) << 16);
      const uint32_t hi = (uint32_t)float_to_half_bits(r[2] + y.z) |
                          ((uint32_t)float_to_half_bits(r[3] + y.w) << 16);
      reinterpret_cast<uint2*>(out)[q] = make_uint2(lo, hi);
    }
  }
}

// Dense copy of a chunked active list (any chunk size): dslots[0 .. total).
__global__ __launch_bounds__(kThreads) void k_bcompact(ActiveList al, int cap, int32_t* dslots,
                                                      int32_t* total) {
  __shared__ int s_prefix[kMaxChunks + 1];
  chunk_prefix(al, s_prefix);
  for (int c = 0; c < al.n_chunks; ++c) {
    const int base = s_prefix[c];
    const int cnt = s_prefix[c + 1] - base;
    for (int k = threadIdx.x; k < cnt; k += kThreads)
      if (base + k < cap) dslots[base + k] = al.slots[(size_t)c * al.chunk + k];
  }
  if (threadIdx.x == 0) *total = min(s_prefix[al.n_chunks], cap);
}

// ── host ────────────────────────────────────────────────────────────────────

struct BatchPlan {
  int M, Mpad, mt, ldh, hot_blocks, cap, ldc, hot_splits, cold_splits;
  size_t off_xn, off_hh, off_hc, off_dslots, off_total, off_part, bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static BatchPlan batch_plan(int M, int n_hot, int cap) {
  BatchPlan p{};
  p.M = M;
  p.Mpad = (M + kBM - 1) / kBM * kBM;
  p.mt = p.Mpad / kBM;
  p.ldh = n_hot > 0 ? (n_hot + kBK - 1) / kBK * kBK : 0;
  p.hot_blocks = p.ldh / kBK;
  p.cap = cap;
  p.ldc = cap > 0 ? (cap + kBN - 1) / kBN * kBN : 0;
  // fill ~256 workgroups per launch: split K when there are few token tiles
  const int splits = p.mt >= 4 ? 1 : 4 / p.mt;
  p.hot_splits = n_hot > 0 ? splits : 0;
  p.cold_splits = cap > 0 ? splits : 0;
  if (p.hot_splits + p.cold_splits == 0) p.hot_splits = 1;   // a zero slab
  size_t o = 0;
  p.off_xn = o;
  o = align256(o + (size_t)M * kH * 2);
  p.off_hh = o;
  o = align256(o + (size_t)p.Mpad * p.ldh * 2);
  p.off_hc = o;
  o = align256(o + (size_t)p.Mpad * p.ldc * 2);
  p.off_dslots = o;
  o = align256(o + (size_t)cap * 4);
  p.off_total = o;
  o = align256(o + 16);
  p.off_part = o;
  o = align256(o + (size_t)(p.hot_splits + p.cold_splits) * p.Mpad * kH * 4);
  p.bytes = o;
  return p;
}

size_t batch_ws_bytes(int M, int n_hot, int cap) { return batch_plan(M, n_hot, cap).bytes; }

int batch_ffn(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const oi2_hot* hot,
              const oi2_cold* cold, const oi2_active* active, int relu, int both, int add_residual,
              uint16_t* out, float* y32, void* workspace, size_t workspace_bytes, hipStream_t st) {
  const int n_hot = hot ? hot->n_hot : 0;
  const bool has_cold = cold && active && cold->n_records > 0 && active->n_chunks > 0;
  const int cap = has_cold ? active->n_chunks * active->chunk : 0;
  const BatchPlan p = batch_plan(M, n_hot, cap);
  OI2_CHECK_ARG(workspace && workspace_bytes >= p.bytes,
                "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, p.bytes);
  OI2_CHECK_ARG((uintptr_t)workspace % 256 == 0, "workspace must be 256-byte aligned");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + p.off_xn);
  uint16_t* hh = reinterpret_cast<uint16_t*>(ws + p.off_hh);
  uint16_t* hc = reinterpret_cast<uint16_t*>(ws + p.off_hc);
  int32_t* dslots = reinterpret_cast<int32_t*>(ws + p.off_dslots);
  int32_t* total = reinterpret_cast<int32_t*>(ws + p.off_total);
  float* part = reinterpret_cast<float*>(ws + p.off_part);

  const uint16_t* xa = x;
  if (norm_w) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(kThreads), 0, st, x, norm_w, eps, xn);
    OI2_CHECK_LAUNCH();
    xa = xn;
  }
  if (has_cold) {
    ActiveList al{active->slots, active->counts, active->n_chunks, active->chunk};
    hipLaunchKernelGGL(k_bcompact, dim3(1), dim3(kThreads), 0, st, al, cap, dslots, total);
    OI2_CHECK_LAUNCH();
  }
  const int hot_wg = p.ldh / kBN;
  const int cold_wg = p.ldc / kBN;
  if (hot_wg + cold_wg > 0) {
    BUpArgs ua{};
    ua.xn = xa;
    ua.M = M;
    ua.relu = relu;
    ua.both = both;
    ua.n_hot = n_hot;
    if (n_hot) {
      ua.gate_q = hot->gate_q;
      ua.up_q = hot->up_q;
      ua.gate_s = hot->gate_scale;
      ua.up_s = hot->up_scale;
      ua.hot_gbias = hot->gate_bias;
    }
    ua.hh = hh;
    ua.ldh = p.ldh;
    ua.hot_wg = hot_wg;
    if (has_cold) {
      ua.records = cold->records;
      ua.n_records = cold->n_records;
      ua.cold_gbias = cold->gate_bias;
      ua.dslots = dslots;
      ua.total = total;
      ua.cap = cap;
    }
    ua.hc = hc;
    ua.ldc = p.ldc;
    hipLaunchKernelGGL(k_bup, dim3(hot_wg + cold_wg, p.mt), dim3(kThreads), 0, st, ua);
    OI2_CHECK_LAUNCH();
  }
  BDownArgs da{};
  da.M = M;
  da.Mpad = p.Mpad;
  da.hh = hh;
  da.ldh = p.ldh;
  da.hot_blocks = p.hot_blocks;
  da.hot_splits = p.hot_splits;
  if (n_hot) {
    da.down_q = hot->down_q;
    da.down_stride = hot->down_stride;
    da.down_s = hot->down_scale;
  } else {
    da.hot_blocks = 0;   // a zero slab
  }
  if (has_cold) {
    da.hc = hc;
    da.ldc = p.ldc;
    da.records = cold->records;
    da.n_records = cold->n_records;
    da.dslots = dslots;
    da.total = total;
    da.cap = cap;
  }
  da.cold_splits = p.cold_splits;
  da.part = part;
  const int slabs = p.hot_splits + p.cold_splits;
  hipLaunchKernelGGL(k_bdown, dim3((kH / kBN) * slabs, p.mt), dim3(kThreads), 0, st, da);
  OI2_CHECK_LAUNCH();
  const int n4 = M * (kH / 4);
  int grid = (n4 + kThreads - 1) / kThreads;
  grid = grid > 2048 ? 2048 : grid;
  hipLaunchKernelGGL(k_bfinal, dim3(grid), dim3(kThreads), 0, st, part, slabs, p.Mpad, M,
                     add_residual ? x : nullptr, out, y32);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

}  // namespace oi2
