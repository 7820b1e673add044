// Multi-token hot/cold FFN on the matrix cores: batch decode with a shared
// active cold set and prefill chunks, sparse_ffn (engine.py:173-209) for
// x (M, H) with M >= 2.
//
// After the norm and a compaction of the active list:
//   gate/up  H_hot  (M, n_hot) = act(s_g * X G^T + b, s_u * X U^T)   fp8 rows
//            H_cold (M, n_act) = act(sum_g s_g,g (X Q_g^T)_g + b, ...)  INT4 records
//            k_bup_s (M <= 64): 16 weight rows per workgroup, the 4 waves
//            split K and meet in LDS, A fragments straight from L2, every
//            weight load of a wave issued up front; k_bup (M > 64): 64 rows x
//            64 tokens per workgroup, A tiles shared through LDS
//   down     Y (M, H) fp32, zeroed, accumulated with fp32 atomics:
//            hot  H_hot D_hot^T (fp8 rows, row scale), k_bdown_hot_s / k_bdown_hot
//            cold H_cold D_cold: 128 outputs x 256 items per workgroup, the
//            items' down nibbles decoded and scaled into LDS, transposed for
//            the MFMA B operand (k_bdown_cold)
//   k_bfinal out = x + Y (fp16), y32 = Y
// Summation order across workgroups follows the atomics, so repeated runs
// can differ in the last bits (well inside the FFN tolerance).
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
#include <algorithm>

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
  // K blocks of this workgroup (blockIdx.z of ksplit)
  const int kbs = blockIdx.z * (kH / kBK) / a.ksplit, kbe = (blockIdx.z + 1) * (kH / kBK) / a.ksplit;
  f32x4 accg[4], accu[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) accg[ms] = accu[ms] = f32x4{0.f, 0.f, 0.f, 0.f};

  if ((int)blockIdx.x < a.hot_wg) {
    // hot: this lane's weight row n, 32 fp8 per 128-wide K block
    const int n = blockIdx.x * kBN + 16 * w + (l & 15);
    const bool nv = n < a.n_hot;
    const uint8_t* gr = a.gate_q + (size_t)(nv ? n : 0) * kH + 32 * (l >> 4);
    const uint8_t* ur = a.up_q + (size_t)(nv ? n : 0) * kH + 32 * (l >> 4);
    for (int kb = kbs; kb < kbe; ++kb) {
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
    if (a.ksplit > 1) {   // partial sums; k_bact finishes
      float* pg = a.pg + (size_t)blockIdx.z * a.Mpad * a.ldp;
      float* pu = a.pu + (size_t)blockIdx.z * a.Mpad * a.ldp;
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const size_t o = (size_t)(m0 + 16 * ms + 4 * (l >> 4) + i) * a.ldp + n;
          pg[o] = accg[ms][i];
          pu[o] = accu[ms][i];
        }
      return;
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
  for (int kb = kbs; kb < kbe; ++kb) {
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
  if (a.ksplit > 1) {
    float* pg = a.pg + (size_t)blockIdx.z * a.Mpad * a.ldp;
    float* pu = a.pu + (size_t)blockIdx.z * a.Mpad * a.ldp;
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const size_t o = (size_t)(m0 + 16 * ms + 4 * (l >> 4) + e) * a.ldp + a.ldh + i;
        pg[o] = accg[ms][e];
        pu[o] = accu[ms][e];
      }
    return;
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

// Sum of k_bup's ksplit partial gate/up sums, then scales, bias and the
// activation: H_hot and H_cold for rows < M.
__global__ __launch_bounds__(kThreads) void k_bact(BUpArgs a) {
  const int total = a.total ? min(*a.total, a.cap) : 0;
  const int n = a.M * a.ldp;
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n; q += gridDim.x * kThreads) {
    const int m = q / a.ldp, c = q - m * a.ldp;
    float g = 0.f, u = 0.f;
    for (int z = 0; z < a.ksplit; ++z) {
      const size_t o = (size_t)z * a.Mpad * a.ldp + (size_t)m * a.ldp + c;
      g += a.pg[o];
      u += a.pu[o];
    }
    if (c < a.ldh) {
      const bool nv = c < a.n_hot;
      float h = 0.f;
      if (nv) {
        const float gb = a.hot_gbias ? a.hot_gbias[c] : 0.f;
        h = gated_act(fmaf(g, a.gate_s[c], gb), u * a.up_s[c], a.relu, a.both);
      }
      a.hh[(size_t)m * a.ldh + c] = float_to_half_bits(h);
    } else {
      const int i = c - a.ldh;
      if (i >= total) continue;   // never read
      const int slot = a.dslots[i];
      float h = 0.f;
      if (slot >= 0 && slot < a.n_records) {
        const float gb = a.cold_gbias ? a.cold_gbias[slot] : 0.f;
        h = gated_act(g + gb, u, a.relu, a.both);
      }
      a.hc[(size_t)m * a.ldc + i] = float_to_half_bits(h);
    }
  }
}

// ── gate/up for at most 64 tokens ───────────────────────────────────────────

// Workgroup = 16 weight rows (hot rows, or items of the dense active list);
// wave w takes K blocks [8w, 8w+8).  MS = token subtiles of 16 (M <= 16 MS).
template <int MS>
__global__ __launch_bounds__(kThreads) void k_bup_s(BUpArgs a) {
  constexpr int NB = kH / kBK / 4;
  constexpr int PF = MS >= 4 ? 4 : 8;   // K blocks whose weight loads are in flight together
  __shared__ f32x4 s_red[3][2 * MS][kWave];
  const int w = threadIdx.x >> 6, l = lane_id();
  const int kb0 = w * NB;
  const uint16_t* xr[MS];
  bool av[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
    const int m = 16 * ms + (l & 15);
    av[ms] = m < a.M;
    xr[ms] = a.xn + (size_t)(av[ms] ? m : 0) * kH + 32 * (l >> 4);
  }
  f32x4 accg[MS], accu[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) accg[ms] = accu[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool hot = (int)blockIdx.x < a.hot_wg;
  int col;
  bool cv;
  int slot = -1;
  if (hot) {
    col = blockIdx.x * 16 + (l & 15);
    cv = col < a.n_hot;
    const uint8_t* gr = a.gate_q + (size_t)(cv ? col : 0) * kH + 32 * (l >> 4);
    const uint8_t* ur = a.up_q + (size_t)(cv ? col : 0) * kH + 32 * (l >> 4);
    for (int ph = 0; ph < NB; ph += PF) {
      u32x4 G[PF][2], U[PF][2];
#pragma unroll
      for (int b = 0; b < PF; ++b) {
        const int k = (kb0 + ph + b) * kBK;
        const u32x4 z = {0u, 0u, 0u, 0u};
        G[b][0] = cv ? load16(gr + k) : z;
        G[b][1] = cv ? load16(gr + k + 16) : z;
        U[b][0] = cv ? load16(ur + k) : z;
        U[b][1] = cv ? load16(ur + k + 16) : z;
      }
#pragma unroll
      for (int b = 0; b < PF; ++b) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          h8 A[MS];
#pragma unroll
          for (int ms = 0; ms < MS; ++ms)
            A[ms] = av[ms] ? *reinterpret_cast<const h8*>(xr[ms] + (kb0 + ph + b) * kBK + 8 * s) : h8{};
          const h8 bg = fp8x8_h8(dword_of(G[b][0], G[b][1], 2 * s), dword_of(G[b][0], G[b][1], 2 * s + 1));
          const h8 bu = fp8x8_h8(dword_of(U[b][0], U[b][1], 2 * s), dword_of(U[b][0], U[b][1], 2 * s + 1));
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) {
            accg[ms] = mfma16(A[ms], bg, accg[ms]);
            accu[ms] = mfma16(A[ms], bu, accu[ms]);
          }
        }
      }
    }
  } else {
    const int total = min(*a.total, a.cap);
    const int i0 = ((int)blockIdx.x - a.hot_wg) * 16;
    if (i0 >= total) return;   // the whole workgroup
    col = i0 + (l & 15);
    slot = col < total ? a.dslots[col] : -1;
    cv = slot >= 0 && slot < a.n_records;
    const uint8_t* rec = a.records + (size_t)(cv ? slot : 0) * kRecBytes;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(rec + kOffScales);
    for (int ph = 0; ph < NB; ph += PF) {
      u32x4 QG[PF], QU[PF];
      float SG[PF], SU[PF];
#pragma unroll
      for (int b = 0; b < PF; ++b) {
        const int kb = kb0 + ph + b;
        const u32x4 z = {0u, 0u, 0u, 0u};
        QG[b] = cv ? load16_a2(rec + kOffGate + 64 * kb + 16 * (l >> 4)) : z;
        QU[b] = cv ? load16_a2(rec + kOffUp + 64 * kb + 16 * (l >> 4)) : z;
        SG[b] = cv ? half_bits_to_float(sc[kb]) : 0.f;
        SU[b] = cv ? half_bits_to_float(sc[kGroups + kb]) : 0.f;
      }
#pragma unroll
      for (int b = 0; b < PF; ++b) {
        f32x4 tg[MS], tu[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) tg[ms] = tu[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          h8 A[MS];
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) {
            const h8 v = av[ms] ? *reinterpret_cast<const h8*>(xr[ms] + (kb0 + ph + b) * kBK + 8 * s)
                                : h8{};
            A[ms] = __builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7);
          }
          const h8 bg = int4x8_h8(QG[b][s]);
          const h8 bu = int4x8_h8(QU[b][s]);
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) {
            tg[ms] = mfma16(A[ms], bg, tg[ms]);
            tu[ms] = mfma16(A[ms], bu, tu[ms]);
          }
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            accg[ms][e] = fmaf(SG[b], tg[ms][e], accg[ms][e]);
            accu[ms][e] = fmaf(SU[b], tu[ms][e], accu[ms][e]);
          }
      }
    }
  }
  if (w > 0) {
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      s_red[w - 1][2 * ms][l] = accg[ms];
      s_red[w - 1][2 * ms + 1][l] = accu[ms];
    }
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int v = 0; v < 3; ++v)
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      accg[ms] += s_red[v][2 * ms][l];
      accu[ms] += s_red[v][2 * ms + 1][l];
    }
  float sg = 1.f, su = 1.f, gb = 0.f;
  if (hot) {
    sg = cv ? a.gate_s[col] : 0.f;
    su = cv ? a.up_s[col] : 0.f;
    gb = (cv && a.hot_gbias) ? a.hot_gbias[col] : 0.f;
  } else {
    gb = (cv && a.cold_gbias) ? a.cold_gbias[slot] : 0.f;
  }
  uint16_t* dst = hot ? a.hh : a.hc;
  const int ld = hot ? a.ldh : a.ldc;
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * ms + 4 * (l >> 4) + e;
      const float h = cv ? gated_act(fmaf(accg[ms][e], sg, gb), accu[ms][e] * su, a.relu, a.both) : 0.f;
      dst[(size_t)m * ld + col] = float_to_half_bits(h);
    }
}

// ── down ────────────────────────────────────────────────────────────────────

// Hot half for at most 64 tokens: workgroup = 16 output rows, the 4 waves
// split the K blocks and meet in LDS; adds into y.
template <int MS>
__global__ __launch_bounds__(kThreads) void k_bdown_hot_s(BDownArgs a) {
  constexpr int NBmax = 8;   // ldh <= 4096: at most 32 blocks, 8 per wave
  __shared__ f32x4 s_red[3][MS][kWave];
  const int w = threadIdx.x >> 6, l = lane_id();
  const int h = blockIdx.x * 16 + (l & 15);
  const int nb = a.hot_blocks;
  const int b0 = w * nb / 4, b1 = (w + 1) * nb / 4;
  const uint8_t* dr = a.down_q + (size_t)h * a.down_stride + 32 * (l >> 4);
  u32x4 D[NBmax][2];
#pragma unroll
  for (int b = 0; b < NBmax; ++b) {
    const int k = (b0 + b) * kBK + 32 * (l >> 4);
    const u32x4 z = {0u, 0u, 0u, 0u};
    const bool in = b0 + b < b1;
    D[b][0] = (in && k < a.down_stride) ? load16(dr + (b0 + b) * kBK) : z;
    D[b][1] = (in && k + 16 < a.down_stride) ? load16(dr + (b0 + b) * kBK + 16) : z;
  }
  const uint16_t* hr[MS];
  bool av[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
    const int m = 16 * ms + (l & 15);
    av[ms] = m < a.M;
    hr[ms] = a.hh + (size_t)(av[ms] ? m : 0) * a.ldh + 32 * (l >> 4);
  }
  f32x4 acc[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) acc[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < NBmax; ++b) {
    if (b0 + b >= b1) break;
    h8 A[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        A[ms][s] = av[ms] ? *reinterpret_cast<const h8*>(hr[ms] + (b0 + b) * kBK + 8 * s) : h8{};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const h8 bv = fp8x8_h8(dword_of(D[b][0], D[b][1], 2 * s), dword_of(D[b][0], D[b][1], 2 * s + 1));
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) acc[ms] = mfma16(A[ms][s], bv, acc[ms]);
    }
  }
  if (w > 0) {
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) s_red[w - 1][ms][l] = acc[ms];
  }
  __syncthreads();
  if (w != 0) return;
  const float sd = a.down_s[h];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
    const f32x4 v = acc[ms] + s_red[0][ms][l] + s_red[1][ms][l] + s_red[2][ms][l];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * ms + 4 * (l >> 4) + e;
      if (m < a.M) a.y[(size_t)m * kH + h] = v[e] * sd;   // the first and only hot writer
    }
  }
}

// Hot half for more than 64 tokens: 64 tokens x 64 outputs per workgroup, A
// tiles through LDS, K blocks split over hot_splits workgroups; adds into y.
__global__ __launch_bounds__(kThreads) void k_bdown_hot(BDownArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[kBM * kLdA];
  const int w = threadIdx.x >> 6, l = lane_id();
  const int m0 = blockIdx.y * kBM;
  const int tile = blockIdx.x % (kH / kBN), split = blockIdx.x / (kH / kBN);
  const int hcol = tile * kBN + 16 * w + (l & 15);
  f32x4 acc[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) acc[ms] = f32x4{0.f, 0.f, 0.f, 0.f};
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
  const float sd = a.down_s[hcol];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * ms + 4 * (l >> 4) + e;
      if (m >= a.M) continue;
      if (a.hot_splits == 1)
        a.y[(size_t)m * kH + hcol] = acc[ms][e] * sd;   // the first and only hot writer
      else
        unsafeAtomicAdd(a.y + (size_t)m * kH + hcol, acc[ms][e] * sd);
    }
}

// Cold half: workgroup = 128 outputs (4 waves x 32) x 64 tokens x a range of
// the dense active list, taken 256 items per step.  Per step each thread
// decodes 64 down values of two items (q * s rounded to fp16) into the LDS
// tile T[h][item], the A tile (64 tokens x 256 items of H_cold) is staged
// once for the 4 waves, and each wave runs 8 MFMA steps of 32 items.  The
// range's sum is added into y.
constexpr int kCT = 128;
constexpr int kCI = 256;
constexpr int kLdT2 = kCI + 8;   // 528-byte LDS rows

__global__ __launch_bounds__(kThreads) void k_bdown_cold(BDownArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sT[kCT * kLdT2];
  __shared__ __attribute__((aligned(16))) uint16_t sH[kBM * kLdT2];
  const int t = threadIdx.x, w = t >> 6, l = lane_id();
  const int h0 = blockIdx.x * kCT, m0 = blockIdx.z * kBM;
  const int total = min(*a.total, a.cap);
  const int n_steps = (total + kCI - 1) / kCI;
  const int st0 = blockIdx.y * n_steps / gridDim.y, st1 = (blockIdx.y + 1) * n_steps / gridDim.y;
  if (st0 >= st1) return;   // the whole workgroup
  const int ms_n = min(4, (a.M - m0 + 15) / 16);
  const int p = t & 127, q = t >> 7;
  f32x4 acc[4][2];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) acc[ms][0] = acc[ms][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int stp = st0; stp < st1; ++stp) {
    const int ig = stp * kCI;
    u32x4 raw[2][2];
    float sc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int it = ig + 2 * p + j;
      const int slot = it < total ? a.dslots[it] : -1;
      const bool v = slot >= 0 && slot < a.n_records;
      const uint8_t* rec = a.records + (size_t)(v ? slot : 0) * kRecBytes;
      const u32x4 z = {0u, 0u, 0u, 0u};
      raw[j][0] = v ? load16_a2(rec + kOffDown + (h0 + 64 * q) / 2) : z;
      raw[j][1] = v ? load16_a2(rec + kOffDown + (h0 + 64 * q) / 2 + 16) : z;
      sc[j] = v ? half_bits_to_float(
                      reinterpret_cast<const uint16_t*>(rec + kOffScales)[2 * kGroups + h0 / kGroup])
                : 0.f;
    }
    // A tile: thread t -> row t >> 2, items 64 (t & 3) .. +64 of the step
    u32x4 hv[8];
    {
      const int r = t >> 2, c0 = ig + 64 * (t & 3);
      const int m = m0 + r;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int ka = c0 + 8 * c;
        u32x4 x = {0u, 0u, 0u, 0u};
        if (m < a.M && ka < total) {
          x = *reinterpret_cast<const u32x4*>(a.hc + (size_t)m * a.ldc + ka);
          // items past the end of the list read as zero
          if (ka + 8 > total) {
            const int keep = total - ka;   // 1..7 halves
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint32_t lo_ok = (2 * d) < keep ? 0xFFFFu : 0u;
              const uint32_t hi_ok = (2 * d + 1) < keep ? 0xFFFF0000u : 0u;
              x[d] &= lo_ok | hi_ok;
            }
          }
        }
        hv[c] = x;
      }
    }
    __syncthreads();   // the previous step's MFMAs are done with sT / sH
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) {
      const uint32_t d0 = dword_of(raw[0][0], raw[0][1], jj >> 3);
      const uint32_t d1 = dword_of(raw[1][0], raw[1][1], jj >> 3);
      const int q0 = (int)((d0 >> (4 * (jj & 7))) & 0xFu) ^ 8;
      const int q1 = (int)((d1 >> (4 * (jj & 7))) & 0xFu) ^ 8;
      const uint32_t pr = (uint32_t)float_to_half_bits((float)(q0 - 8) * sc[0]) |
                          ((uint32_t)float_to_half_bits((float)(q1 - 8) * sc[1]) << 16);
      *reinterpret_cast<uint32_t*>(sT + (64 * q + jj) * kLdT2 + 2 * p) = pr;
    }
    {
      const int r = t >> 2, c0 = 64 * (t & 3);
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *reinterpret_cast<u32x4*>(sH + r * kLdT2 + c0 + 8 * c) = hv[c];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      h8 av[4];
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
        av[ms] = *reinterpret_cast<const h8*>(sH + (16 * ms + (l & 15)) * kLdT2 + 32 * s + 8 * (l >> 4));
#pragma unroll
      for (int ns = 0; ns < 2; ++ns) {
        const h8 b = *reinterpret_cast<const h8*>(sT + (32 * w + 16 * ns + (l & 15)) * kLdT2 +
                                                  32 * s + 8 * (l >> 4));
#pragma unroll
        for (int ms = 0; ms < 4; ++ms)
          if (ms < ms_n) acc[ms][ns] = mfma16(av[ms], b, acc[ms][ns]);
      }
    }
  }
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < 2; ++ns)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * ms + 4 * (l >> 4) + e;
        const int h = h0 + 32 * w + 16 * ns + (l & 15);
        if (ms < ms_n && m < a.M) unsafeAtomicAdd(a.y + (size_t)m * kH + h, acc[ms][ns][e]);
      }
}

// y = 0 over M rows.
__global__ __launch_bounds__(kThreads) void k_bfill(float* y, int n4) {
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n4; q += gridDim.x * kThreads)
    reinterpret_cast<f32x4*>(y)[q] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// out = res + y (fp16), y32 = y.
__global__ __launch_bounds__(kThreads) void k_bfinal(const float* yacc, int M, const uint16_t* res,
                                                    uint16_t* out, float* y32) {
  const int n4 = M * (kH / 4);
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n4; q += gridDim.x * kThreads) {
    const f32x4 y = reinterpret_cast<const f32x4*>(yacc)[q];
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
  int M, Mpad, mt, ldh, hot_blocks, cap, ldc, hot_splits, ksplit;
  size_t off_xn, off_hh, off_hc, off_dslots, off_total, off_y, off_pg, off_pu, bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kSkinnyMax = 16;   // token counts up to this use the one-tile split-K kernels

static BatchPlan batch_plan(int M, int n_hot, int cap) {
  BatchPlan p{};
  p.M = M;
  p.Mpad = (M + kBM - 1) / kBM * kBM;
  p.mt = p.Mpad / kBM;
  p.ldh = n_hot > 0 ? (n_hot + kBK - 1) / kBK * kBK : 0;
  p.hot_blocks = p.ldh / kBK;
  p.cap = cap;
  p.ldc = cap > 0 ? (cap + kBN - 1) / kBN * kBN : 0;
  p.hot_splits = p.mt >= 4 ? 1 : 4 / p.mt;
  // tiled gate/up with few token tiles: split K over workgroups
  p.ksplit = (M > kSkinnyMax && p.mt < 4) ? 4 / p.mt : 1;
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
  p.off_y = o;
  o = align256(o + (size_t)M * kH * 4);
  const size_t part = p.ksplit > 1 ? (size_t)p.ksplit * p.Mpad * (p.ldh + p.ldc) * 4 : 0;
  p.off_pg = o;
  o = align256(o + part);
  p.off_pu = o;
  o = align256(o + part);
  p.bytes = o;
  return p;
}

size_t batch_ws_bytes(int M, int n_hot, int cap) { return batch_plan(M, n_hot, cap).bytes; }

static void launch_skinny(const BUpArgs& ua, const BDownArgs& da, bool up, hipStream_t st) {
  if (up)
    hipLaunchKernelGGL(k_bup_s<1>, dim3(ua.hot_wg + ua.ldc / 16), dim3(kThreads), 0, st, ua);
  else
    hipLaunchKernelGGL(k_bdown_hot_s<1>, dim3(kH / 16), dim3(kThreads), 0, st, da);
}

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
  float* y = reinterpret_cast<float*>(ws + p.off_y);
  const bool skinny = M <= kSkinnyMax;

  const uint16_t* xa = x;
  if (norm_w) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(kThreads), 0, st, x, norm_w, eps, xn);
    OI2_CHECK_LAUNCH();
    xa = xn;
  }
  const int32_t* dlist = dslots;
  const int32_t* dtotal = total;
  if (has_cold && active->n_chunks == 1) {
    dlist = active->slots;   // already dense: the kernels clamp the count to the capacity
    dtotal = active->counts;
  } else if (has_cold) {
    ActiveList al{active->slots, active->counts, active->n_chunks, active->chunk};
    hipLaunchKernelGGL(k_bcompact, dim3(1), dim3(kThreads), 0, st, al, cap, dslots, total);
    OI2_CHECK_LAUNCH();
  }
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
  ua.hot_wg = skinny ? p.ldh / 16 : p.ldh / kBN;
  if (has_cold) {
    ua.records = cold->records;
    ua.n_records = cold->n_records;
    ua.cold_gbias = cold->gate_bias;
    ua.dslots = dlist;
    ua.total = dtotal;
    ua.cap = cap;
  }
  ua.hc = hc;
  ua.ldc = p.ldc;
  ua.ksplit = skinny ? 1 : p.ksplit;
  ua.pg = reinterpret_cast<float*>(ws + p.off_pg);
  ua.pu = reinterpret_cast<float*>(ws + p.off_pu);
  ua.ldp = p.ldh + p.ldc;
  ua.Mpad = p.Mpad;
  BDownArgs da{};
  da.M = M;
  da.hh = hh;
  da.ldh = p.ldh;
  da.hot_blocks = p.hot_blocks;
  da.hot_splits = p.hot_splits;
  if (n_hot) {
    da.down_q = hot->down_q;
    da.down_stride = hot->down_stride;
    da.down_s = hot->down_scale;
  }
  if (has_cold) {
    da.hc = hc;
    da.ldc = p.ldc;
    da.records = cold->records;
    da.n_records = cold->n_records;
    da.dslots = dlist;
    da.total = dtotal;
    da.cap = cap;
  }
  da.y = y;

  if (p.ldh + p.ldc > 0) {
    if (skinny)
      launch_skinny(ua, da, true, st);
    else
      hipLaunchKernelGGL(k_bup, dim3(p.ldh / kBN + p.ldc / kBN, p.mt, ua.ksplit), dim3(kThreads), 0,
                         st, ua);
    OI2_CHECK_LAUNCH();
    if (ua.ksplit > 1) {
      const int n = M * ua.ldp;
      int g = (n + kThreads - 1) / kThreads;
      hipLaunchKernelGGL(k_bact, dim3(g > 4096 ? 4096 : g), dim3(kThreads), 0, st, ua);
      OI2_CHECK_LAUNCH();
    }
  }
  const int n4 = M * (kH / 4);
  int grid = (n4 + kThreads - 1) / kThreads;
  grid = grid > 2048 ? 2048 : grid;
  // the hot product writes y outright when one workgroup owns each output
  if (!n_hot || (!skinny && p.hot_splits > 1)) {
    hipLaunchKernelGGL(k_bfill, dim3(grid), dim3(kThreads), 0, st, y, n4);
    OI2_CHECK_LAUNCH();
  }
  if (n_hot) {
    if (skinny)
      launch_skinny(ua, da, false, st);
    else
      hipLaunchKernelGGL(k_bdown_hot, dim3((kH / kBN) * p.hot_splits, p.mt), dim3(kThreads), 0, st,
                         da);
    OI2_CHECK_LAUNCH();
  }
  if (has_cold) {
    // item ranges per output tile: ~512 workgroups in all, at least 2 steps each
    const int steps = (cap + kCI - 1) / kCI;
    int splits = (512 / (kH / kCT)) / p.mt;
    splits = std::max(1, std::min(splits, (steps + 1) / 2));
    hipLaunchKernelGGL(k_bdown_cold, dim3(kH / kCT, splits, p.mt), dim3(kThreads), 0, st, da);
    OI2_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(k_bfinal, dim3(grid), dim3(kThreads), 0, st, y, M, add_residual ? x : nullptr,
                     out, y32);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

}  // namespace oi2
