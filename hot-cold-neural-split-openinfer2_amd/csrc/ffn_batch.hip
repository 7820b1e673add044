// Multi-token hot/cold FFN on the matrix cores: batch decode with a shared
// active cold set and prefill chunks, sparse_ffn (engine.py:173-209) for
// x (M, H) with M >= 2.
//
// After the norm and a compaction of the active list:
//   gate/up  H_hot  (M, n_hot) = act(s_g * X G^T + b, s_u * X U^T)   fp8 rows
//            H_cold (M, n_act) = act(sum_g s_g,g (X Q_g^T)_g + b, ...)  INT4 records
//            k_sbup (M <= 16): one workgroup per CU, RMSNorm fused;
//            k_mup (M < 160): 64 tokens x 32 neurons, 32x32x16 tiles, the
//            activation in the epilogue;
//            k_pgemm_up (M >= 160): 128 tokens x 128 neurons
//   down     Y (M, H) fp32
//            hot  H_hot D_hot^T (fp8 rows, row scale): k_bdown_hot_s,
//                 k_pgemm_down_hot
//            cold H_cold D_cold: k_pgemm_down_cold, the records' down
//                 nibbles transposed into a decoded LDS tile
//            both halves from 17 tokens:
//                 k_pgemm_down_both, one workgroup per output tile and K
//                 range of each half
//   k_bfinal out = x + Y (fp16), y32 = Y
// Up to 16 tokens, the cold down stores one partial sum per item range and
// the last kernel (k_bdown_hot_s, or k_bfinal16 without hot rows) adds them
// in range order to the hot product.  With more tokens every down workgroup
// stores its K range's partial sum of its output tile, and k_bfinal adds
// them in range order.  No path uses atomics, so the
// result is the same on every run.  (fp32 atomics into one Y cost the 512-
// token cold down 65 against 44 us, the 64-token one 28 against 18 us.)
// fp8 and INT4 weights convert to fp16 exactly.  The small-batch gate/up
// kernels apply INT4 group scales (one per 128 K) to each block's fp32
// partial sums, exact up to accumulation; the prefill gate/up and every cold
// down multiply nibble and scale in fp16, rounded once (q * s needs up to 14
// significant bits).
//
// MFMA 16x16x32 f16 operand layout (lane l, element i): A[l%16][8(l/16)+i],
// B[8(l/16)+i][l%16], D[4(l/16)+i][l%16].  Only the pairing of A and B
// elements along K matters, so each 128-wide K block is split among the four
// lane groups as 32 contiguous K per group, 8 per MFMA step.
#include <algorithm>

#include "capi_util.h"
#include "decode_util.h"
#include "ffn_kernels.h"

namespace oi2 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

constexpr int kBM = 64;          // token rows per tile
constexpr int kBK = 128;         // K block = INT4 scale group
constexpr int kLdA = kBK + 8;    // LDS row of the A tile, halves (272 B)

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

// 8 INT4 (one dword, K order) times an fp16 scale, in int4x8_h8's order.
// ((d >> 4k) & 0x000F000F) ^ 0x64086408 is the fp16 1024 + (n ^ 8) for the
// nibble pair (k, k + 4); minus 1032 that is the signed nibble, exactly, and
// the product with the scale rounds once.
__device__ __forceinline__ h8 int4x8_h8_scaled(uint32_t d, _Float16 sc) {
  u32x4 m;
#pragma unroll
  for (int k = 0; k < 4; ++k) m[k] = ((d >> (4 * k)) & 0x000F000Fu) ^ 0x64086408u;
  return (__builtin_bit_cast(h8, m) + (_Float16)-1032.0f) * sc;
}

// Raw buffer loads: one descriptor per operand, a 32-bit per-lane offset and a
// uniform (SGPR) offset, instead of a 64-bit address per row.  Reads at or
// past `bytes` return zero.  (The non-temporal hint that speeds up the
// single-token kernels' weight streams made the small-batch kernels slower:
// 8 tokens x 32 layers 1112 -> 1145 us with it on both k_sbup and
// k_bdown_hot_s, so these loads stay plain.)
__device__ __forceinline__ rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint16_t bload2(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}
constexpr uint32_t kNoOffset = 0x80000000u;   // a lane offset past every buffer

__device__ __forceinline__ f32x4 mfma16(h8 a, h8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t dword_of(const u32x4& a, const u32x4& b, int i) {
  return i < 4 ? a[i] : b[i - 4];
}

// ── gate/up and hot down for prefill-sized token counts ─────────────────────
//
// v_mfma_f32_32x32x16_f16 (lane l, element i): A[l%32][8(l/32)+i],
// B[8(l/32)+i][l%32]; output element j is D[8(j/4) + 4(l/32) + j%4][l%32].
// It sustains about 1.45x the 16x16x32 rate on gfx950.  Each 128-wide K block
// is split between the two lane halves as 64 contiguous K, 8 per MFMA step.
//
// Workgroup tile: 32 MS tokens x 4 waves, each wave one 32-column B tile per
// NB (32 weight rows as gate and up, or 32 down rows).  Both operands go
// through two LDS buffers, one barrier per K block; each block's global loads
// are issued a block ahead.  The barrier waits for LDS traffic only
// (lgkmcnt), not for the global loads in flight.
//
// Cold rows: INT4 nibbles times their group scale, rounded once to fp16 (the
// product needs up to 14 significant bits), so every K block accumulates
// straight into the fp32 tile.

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A tile rows m0 .. m0 + 32 MS - 1: thread t loads 16-byte chunk t & 15 of
// rows t / 16 + 16 i; rows >= M lie past the descriptor's range and read as
// zero.  The K block goes in the uniform offset.
template <int MS>
struct ARows {
  rsrc_t r;
  uint32_t voff[2 * MS];
  __device__ __forceinline__ ARows(const uint16_t* A, int ld, int M, int m0) {
    const int t = threadIdx.x;
    r = buf_rsrc(A, (uint32_t)M * ld * 2);
#pragma unroll
    for (int i = 0; i < 2 * MS; ++i) voff[i] = ((uint32_t)(m0 + (t >> 4) + 16 * i) * ld + 8 * (t & 15)) * 2;
  }
  __device__ __forceinline__ void load(int kb, u32x4 (&ra)[2 * MS]) const {
#pragma unroll
    for (int i = 0; i < 2 * MS; ++i) ra[i] = bload16(r, voff[i], kb * kBK * 2);
  }
};

// The loaded chunks into s[32 MS][kLdA].  PAIR stores each group of 8 halves
// as (x0,x4,x1,x5,x2,x6,x3,x7), the order the INT4 decode produces.
template <int NR, bool PAIR>
__device__ __forceinline__ void store_a_rows(const u32x4 (&r)[NR], uint16_t* s) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    u32x4 v = r[i];
    if (PAIR) {
      const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w;
      v.x = (d0 & 0xFFFFu) | (d2 << 16);
      v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
      v.z = (d1 & 0xFFFFu) | (d3 << 16);
      v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
    }
    *reinterpret_cast<u32x4*>(s + ((t >> 4) + 16 * i) * kLdA + 8 * (t & 15)) = v;
  }
}

// A fragment of 32-row subtile ms, K step s (0..7) of the staged block.
__device__ __forceinline__ h8 a_frag32(const uint16_t* s, int ms, int step) {
  const int l = lane_id();
  return *reinterpret_cast<const h8*>(s + (32 * ms + (l & 31)) * kLdA + 64 * (l >> 5) + 8 * step);
}

// Gate/up for 32 MS tokens x 128 weight rows (hot rows first, then items of
// the dense active list).  Both operands go through two LDS buffers: each K
// block's token rows and weight rows are loaded as whole 16-byte chunks
// (eight lanes per 128-byte weight row, so every load instruction reads full
// cache lines) by the staging waves.  Weight rows are padded to 136 bytes (fp8) or 72 bytes (INT4): the
// 32 rows a wave reads at one column then fall on distinct banks.  Wave w
// owns rows 32 w + (l & 31); B tile 0 is the gate row, tile 1 the up row.
// The linear workgroup index is mapped so that the token tiles of one row
// tile run on the same XCD (workgroups go round-robin over the 8 XCDs),
// sharing its L2 for the weights.
constexpr int kLdB8 = 128 + 8;   // bytes per fp8 weight row of a K block in LDS
constexpr int kLdB4 = 64 + 8;    // bytes per INT4 weight row of a K block in LDS

// MS x NB MFMA tiles for the eight K steps of one block, both operands from
// LDS (B tile nb is weight rows 128 nb + 32 w + (l & 31)).  Each step's
// fragments are read into their own registers at the start of the step
// before (its LDS reads are issued ahead of that step's MFMAs, so a read has
// a whole step of MFMAs to land; read just after its previous use it had
// ~six), and converted between the MFMAs (512 tokens: 81 -> 77 us per
// layer for the gate/up).
template <int MS, int NB, bool INT4>
__device__ __forceinline__ void mma_block_lds(const uint16_t* sA, const uint8_t* sB, const uint16_t* sSc,
                                              f32x16 (&acc)[MS][NB]) {
  constexpr int kValuPerMfma = INT4 ? 4 : 1;
  const int w = threadIdx.x >> 6, l = lane_id();
  const int row = 32 * w + (l & 31), h = l >> 5;
  _Float16 sc[2] = {(_Float16)0.0f, (_Float16)0.0f};
  if constexpr (INT4) {
    sc[0] = __builtin_bit_cast(_Float16, sSc[row]);
    sc[1] = __builtin_bit_cast(_Float16, sSc[128 + row]);
  }
  auto b_frag = [&](int st, h8 (&bf)[NB]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (INT4) {
        const uint32_t d = *reinterpret_cast<const uint32_t*>(sB + (128 * nb + row) * kLdB4 + 32 * h + 4 * st);
        bf[nb] = int4x8_h8_scaled(d, sc[nb]);
      } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(sB + (128 * nb + row) * kLdB8 + 64 * h + 8 * st);
        bf[nb] = fp8x8_h8(v[0], v[1]);
      }
    }
  };
  h8 av[2][MS], bf[2][NB];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) av[0][ms] = a_frag32(sA, ms, 0);
  b_frag(0, bf[0]);
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const int cur = st & 1;
    if (st < 7) {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) av[cur ^ 1][ms] = a_frag32(sA, ms, st + 1);
      b_frag(st + 1, bf[cur ^ 1]);
    }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = mfma32(av[cur][ms], bf[cur][nb], acc[ms][nb]);
    if (st < 7) __builtin_amdgcn_sched_group_barrier(0x100, MS + NB, 0);   // the next step's LDS reads
#pragma unroll
    for (int i = 0; i < NB * MS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // one MFMA
      if (st < 7) __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU
    }
  }
}

// gated_act with the activation chosen at compile time (the same operations,
// so the same bits).
template <bool RELU, bool BOTH>
__device__ __forceinline__ float gated_act_t(float g, float u) {
  const float ag = RELU ? fmaxf(g, 0.0f) : silu(g);
  const float au = BOTH ? (RELU ? fmaxf(u, 0.0f) : silu(u)) : u;
  return ag * au;
}

// The gate/up epilogue of one lane's column: for each of the MS x 16
// accumulator elements, h = act(g sg + gb, u su) (zero when !ok), stored as
// fp16 at dst[m * ld + c] through a descriptor that drops rows m >= M.  The
// activation is chosen once, outside the element loop, and no element takes
// a branch, so the elements' exp / divide chains overlap.  (Taken per
// element, the choice and the row test made a prefill tile's epilogue a
// chain of 64 basic blocks: ~14 us of a 98 us tile.)
template <int MS, bool RELU, bool BOTH>
__device__ __forceinline__ void up_epilogue_t(const f32x16 (&acc)[MS][2], float sg, float su, float gb, bool ok,
                                              uint16_t* dst, int M, int ld, int c, int m0) {
  const rsrc_t rd = buf_rsrc(dst, (uint32_t)M * ld * 2);
  const int h = lane_id() >> 5;
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int m = m0 + 32 * ms + 8 * (j >> 2) + 4 * h + (j & 3);
      const float hv = gated_act_t<RELU, BOTH>(fmaf(acc[ms][0][j], sg, gb), acc[ms][1][j] * su);
      __builtin_amdgcn_raw_buffer_store_b16(float_to_half_bits(ok ? hv : 0.f), rd, ((uint32_t)m * ld + c) * 2, 0, 0);
    }
}
template <int MS>
__device__ __forceinline__ void up_epilogue(const BUpArgs& a, const f32x16 (&acc)[MS][2], float sg, float su,
                                            float gb, bool ok, uint16_t* dst, int ld, int c, int m0) {
  if (a.relu) {
    if (a.both) up_epilogue_t<MS, true, true>(acc, sg, su, gb, ok, dst, a.M, ld, c, m0);
    else up_epilogue_t<MS, true, false>(acc, sg, su, gb, ok, dst, a.M, ld, c, m0);
  } else {
    if (a.both) up_epilogue_t<MS, false, true>(acc, sg, su, gb, ok, dst, a.M, ld, c, m0);
    else up_epilogue_t<MS, false, false>(acc, sg, su, gb, ok, dst, a.M, ld, c, m0);
  }
}

// 8 waves: waves 0-3 only multiply (mma_block_lds, then the epilogue of
// their 32 rows), waves 4-7 only stage, each K block two blocks ahead of its
// use: their loads, waits and LDS stores stay out of the multiplying waves'
// instruction streams, and every SIMD holds one wave of each kind (with all
// eight waves doing both, one wave per SIMD, a 512-token tile took 80 us
// against 70).  One barrier per block: the multiplying waves are done with
// buffer kb & 1's previous block, and the staging waves have written block
// kb + 1.
template <int MS, bool HOT>
__device__ __forceinline__ void pgemm_up_tile(const BUpArgs& a, int nt, int m0, int total, int i0,
                                                 uint16_t* sA, uint8_t* sB, uint16_t* sSc) {
  constexpr int kAbuf = 32 * MS * kLdA;   // halves per A buffer
  constexpr int kBbuf = 256 * kLdB8;      // bytes per B buffer (INT4 rows use kLdB4 of it)
  constexpr int NR = HOT ? 8 : 4;         // 16-byte weight chunks staged per thread
  constexpr int kNB = kH / kBK;
  static_assert(kNB % 2 == 0, "the block loop is unrolled by two");
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  auto item_rec = [&](int it) {
    const int slot = it < total ? a.dslots[it] : -1;
    return (slot >= 0 && slot < a.n_records) ? (uint32_t)slot * kRecBytes : kNoOffset;
  };
  if (w >= 4) {
    // staging thread t: token rows (t >> 4) + 16 i, chunk t & 15; hot, chunk
    // t & 7 of tile rows (t >> 3) + 32 i (i < 4 gate, else up); cold, chunk
    // t & 3 of items (t >> 2) + 64 (i & 1), gate for i < 2, up for i >= 2,
    // and the scale of item t & 127 (gate, up by t >> 7).  Rows past M or
    // n_hot and invalid items read as zero.
    const int t = threadIdx.x - 256;
    const rsrc_t rx = buf_rsrc(a.xn, (uint32_t)a.M * kH * 2);
    uint32_t aoff[2 * MS];
#pragma unroll
    for (int i = 0; i < 2 * MS; ++i) aoff[i] = ((uint32_t)(m0 + (t >> 4) + 16 * i) * kH + 8 * (t & 15)) * 2;
    const rsrc_t rw = HOT ? buf_rsrc(a.gate_q, (uint32_t)a.n_hot * kH)
                          : buf_rsrc(a.records, (uint32_t)a.n_records * kRecBytes);
    const rsrc_t ru = buf_rsrc(a.up_q, HOT ? (uint32_t)a.n_hot * kH : 0u);
    uint32_t voff[4], vsc = 0;
    if constexpr (HOT) {
#pragma unroll
      for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)(nt * 128 + (t >> 3) + 32 * i) * kH + 16 * (t & 7);
    } else {
      const uint32_t v0 = item_rec(i0 + (t >> 2)), v1 = item_rec(i0 + (t >> 2) + 64);
      voff[0] = v0 + kOffGate + 16 * (t & 3);
      voff[1] = v1 + kOffGate + 16 * (t & 3);
      voff[2] = v0 + kOffUp + 16 * (t & 3);
      voff[3] = v1 + kOffUp + 16 * (t & 3);
      vsc = item_rec(i0 + (t & 127)) + (t >> 7) * 2 * kGroups;
    }
    u32x4 ra[2][2 * MS], rb[2][NR];
    uint16_t rsc[2] = {0, 0};
    auto load = [&](int kb, int sl) {
#pragma unroll
      for (int i = 0; i < 2 * MS; ++i) ra[sl][i] = bload16(rx, aoff[i], kb * kBK * 2);
      if constexpr (HOT) {
#pragma unroll
        for (int i = 0; i < 8; ++i) rb[sl][i] = bload16(i < 4 ? rw : ru, voff[i & 3], kb * kBK);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) rb[sl][i] = bload16(rw, voff[i], 64 * kb);
        rsc[sl] = bload2(rw, vsc, kOffScales + 2 * kb);
      }
    };
    auto store = [&](int buf, int sl) {
      uint16_t* A = sA + buf * kAbuf;
#pragma unroll
      for (int i = 0; i < 2 * MS; ++i) {
        u32x4 v = ra[sl][i];
        if constexpr (!HOT) {   // (x0,x4,x1,x5,x2,x6,x3,x7): the INT4 decode's pair order
          const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w;
          v.x = (d0 & 0xFFFFu) | (d2 << 16);
          v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
          v.z = (d1 & 0xFFFFu) | (d3 << 16);
          v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x4*>(A + ((t >> 4) + 16 * i) * kLdA + 8 * (t & 15)) = v;
      }
      uint8_t* B = sB + buf * kBbuf;
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        uint8_t* d = HOT ? B + ((t >> 3) + 32 * i) * kLdB8 + 16 * (t & 7)
                         : B + ((t >> 2) + 64 * i) * kLdB4 + 16 * (t & 3);
        reinterpret_cast<u32x2*>(d)[0] = u32x2{rb[sl][i].x, rb[sl][i].y};
        reinterpret_cast<u32x2*>(d)[1] = u32x2{rb[sl][i].z, rb[sl][i].w};
      }
      if constexpr (!HOT) sSc[buf * 256 + t] = rsc[sl];
    };
    // block b sits in register slot and LDS buffer b & 1
    load(0, 0);
    load(1, 1);
    store(0, 0);
    load(2, 0);
    lds_barrier();   // block 0 in buffer 0
#pragma unroll 1
    for (int k0 = 0; k0 < kNB; k0 += 2) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int kb = k0 + u;
        // block kb + 1 into the buffer block kb - 1 left, then its slot
        // loads block kb + 3 (the last passes load the last block again)
        if (kb + 1 < kNB) {
          store(u ^ 1, u ^ 1);
          load(min(kb + 3, kNB - 1), u ^ 1);
        }
        lds_barrier();
      }
    }
    return;
  }
  f32x16 acc[MS][2];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) acc[ms][0] = acc[ms][1] = f32x16{};
  lds_barrier();   // block 0 in buffer 0
#pragma unroll 1
  for (int k0 = 0; k0 < kNB; k0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      mma_block_lds<MS, 2, !HOT>(sA + u * kAbuf, sB + u * kBbuf, sSc + u * 256, acc);
      lds_barrier();
    }
  }
  // epilogue: this lane's column, rows m0 + 32 ms + 8 (j / 4) + 4 (l / 32) + j % 4
  const int col = 32 * w + (l & 31);
  if constexpr (HOT) {
    const int row = nt * 128 + col;
    const bool ok = row < a.n_hot;
    const float sg = ok ? a.gate_s[row] : 0.f, su = ok ? a.up_s[row] : 0.f;
    const float gb = (ok && a.hot_gbias) ? a.hot_gbias[row] : 0.f;
    up_epilogue<MS>(a, acc, sg, su, gb, ok, a.hh, a.ldh, row, m0);
  } else {
    const int item = i0 + col;
    const int slot = item < total ? a.dslots[item] : -1;
    const bool ok = slot >= 0 && slot < a.n_records;
    const float gb = (ok && a.cold_gbias) ? a.cold_gbias[slot] : 0.f;
    up_epilogue<MS>(a, acc, 1.0f, 1.0f, gb, ok, a.hc, a.ldc, item, m0);
  }
}

template <int MS>
__global__ __launch_bounds__(2 * kThreads) void k_pgemm_up(BUpArgs a, int hot_tiles, int n_tiles, int mt) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2 * 32 * MS * kLdA];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2 * 256 * kLdB8];
  __shared__ uint16_t sSc[2 * 256];
  const int b = blockIdx.x;
  const int q = b >> 3;
  const int nt = (q / mt) * 8 + (b & 7), mtile = q % mt;
  if (nt >= n_tiles) return;   // the whole workgroup
  const int m0 = mtile * 32 * MS;
  if (nt < hot_tiles) {
    pgemm_up_tile<MS, true>(a, nt, m0, 0, 0, sA, sB, sSc);
    return;
  }
  const int total = min(*a.total, a.cap);
  const int i0 = (nt - hot_tiles) * 128;
  if (i0 >= total) return;   // the whole workgroup
  pgemm_up_tile<MS, false>(a, nt, m0, total, i0, sA, sB, sSc);
}

// ── gate/up for 17 .. 191 tokens ────────────────────────────────────────────
//
// Workgroup tile: 64 tokens x 32 neurons (hot fp8 rows, or cold items of the
// dense active list), 512 threads.  The whole K range stays in one
// workgroup, so the activation is applied in the epilogue (no partial sums
// leave it).  Wave w takes K step w (16 of every 128-wide block) for both
// 32-token subtiles and both the gate and the up rows: four independent
// 32x32x16 MFMAs per block, each weight fragment decoded once for two of
// them, and two waves per SIMD (two workgroups per CU) to hide each one's
// LDS and decode latency.  (With four waves, each on one subtile and half of
// every block, a tile took ~34 us whatever it held: one wave per SIMD ran a
// chain of LDS reads, decodes and MFMAs with nothing to overlap it.)
// Operands go through two LDS buffers; each block's token rows and weight
// rows are loaded two blocks ahead into registers.  At the end the eight
// waves' sums meet in LDS in a fixed order (w and w + 4, then the four pairs
// in wave order), and each wave applies the activation to an eighth of the
// tile.
// A cold tile's group scales (32 gate + 32 up per item) go to LDS once, up
// front.
// Wide tiles (NW = 2: 64 neurons, eight MFMAs per block and wave) make up
// the difference when a batch of at most 64 tokens has more 32-neuron units
// than the GPU has CUs: every tile then runs in one round, one per CU, where
// narrow tiles alone would put a second tile on some CUs (a CU with two
// takes ~1.5x as long as one with one).
constexpr int kMupN = 32;                            // neurons per subtile
constexpr int kMupThreads = 512;
constexpr int kMupBbuf = 128 * kLdB8;                // bytes per B buffer (2 subtiles x 32 x 2 rows)
constexpr int kMupAbuf = 64 * kLdA * 2;              // bytes per A buffer
constexpr int kMupSc = 2 * kMupAbuf + 2 * kMupBbuf;  // the scales' byte offset
constexpr int kMupRedBuf = 2 * 2 * 16 * 64 * 4;      // one wave's sums of a subtile: [ms][g][j][lane] fp32
constexpr int kMupLds = std::max(kMupSc + 2 * kMupN * 2 * kGroups * 2, 4 * kMupRedBuf);

// n0: the tile's first hot row (HOT) or dense list item (cold).
template <bool HOT, int NW>
__device__ __forceinline__ void mup_tile(const BUpArgs& a, int n0, int m0, int total, uint8_t* smem) {
  constexpr int TW = kMupN * NW;   // neurons of the tile
  uint16_t* sA = reinterpret_cast<uint16_t*>(smem);
  uint8_t* sB = smem + 2 * kMupAbuf;
  uint16_t* sSc = reinterpret_cast<uint16_t*>(smem + kMupSc);
  const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = lane_id(), h = l >> 5, col = l & 31;
  // cold, narrow: waves 0-3 stage the 4 KB weight block, waves 4-7 issue the
  // same load over an empty range (every wave runs the same loads, so the
  // compiler's wait counts stay exact); wide: all eight stage the 8 KB
  const bool bstore = HOT || NW == 2 || w < 4;
  // A staging: chunk t & 15 (8 halves) of token rows m0 + (t >> 4) + 32 i;
  // rows past M read zero
  const rsrc_t rx = buf_rsrc(a.xn, (uint32_t)a.M * kH * 2);
  uint32_t aoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) aoff[i] = ((uint32_t)(m0 + (t >> 4) + 32 * i) * kH + 8 * (t & 15)) * 2;
  // B staging (LDS row 64 s + 32 gu + n: neuron n of subtile s, gate for
  // gu = 0, up for 1): hot, chunk t & 7 of rows 64 s + (t >> 3), s < NW;
  // cold, chunk t & 3 of item t >> 3 (t < 256 when narrow), gate for
  // (t >> 2) & 1 == 0 else up.  Absent rows read zero.
  const rsrc_t rw = HOT ? buf_rsrc(w < 4 ? a.gate_q : a.up_q, (uint32_t)a.n_hot * kH)
                        : buf_rsrc(a.records, (NW == 2 || w < 4) ? (uint32_t)a.n_records * kRecBytes : 0u);
  auto item_rec = [&](int it) {
    const int slot = it < total ? a.dslots[it] : -1;
    return (slot >= 0 && slot < a.n_records) ? (uint32_t)slot * kRecBytes : kNoOffset;
  };
  constexpr int NBL = HOT ? NW : 1;   // B loads per thread and block
  uint32_t boff[NBL];
  if constexpr (HOT) {
#pragma unroll
    for (int sb = 0; sb < NW; ++sb) boff[sb] = (uint32_t)(n0 + 32 * sb + ((t >> 3) & 31)) * kH + 16 * (t & 7);
  } else {
    const int it = NW == 2 ? t >> 3 : (t >> 3) & 31;
    const uint32_t v = item_rec(n0 + it);
    boff[0] = v + (((t >> 2) & 1) ? kOffUp : kOffGate) + 16 * (t & 3);
    // scales: item t >> 3, 16-byte piece t & 7 of its gate (64 B) and up
    // (64 B) scale arrays, stored as sSc[gate, up][group][item] (a block's
    // items side by side: lanes read consecutive halves)
    if (NW == 2 || w < 4) {
      const u32x4 sv = bload16(rw, v + kOffScales + 16 * (t & 7), 0);
      const int g0 = 8 * (t & 3), gu = (t >> 2) & 1;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        sSc[(gu * kGroups + g0 + k) * TW + it] = (uint16_t)(sv[k >> 1] >> (16 * (k & 1)));
    }
  }
  u32x4 ra[2][2], rb[2][NBL];
  auto load = [&](int kb, int sl) {
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[sl][i] = bload16(rx, aoff[i], kb * kBK * 2);
#pragma unroll
    for (int sb = 0; sb < NBL; ++sb) rb[sl][sb] = bload16(rw, boff[sb], HOT ? kb * kBK : 64 * kb);
  };
  auto store = [&](int buf, int sl) {
    uint16_t* A = sA + buf * (kMupAbuf / 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      u32x4 v = ra[sl][i];
      if constexpr (!HOT) {   // (x0,x4,x1,x5,x2,x6,x3,x7): the INT4 decode's pair order
        const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w;
        v.x = (d0 & 0xFFFFu) | (d2 << 16);
        v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
        v.z = (d1 & 0xFFFFu) | (d3 << 16);
        v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
      }
      *reinterpret_cast<u32x4*>(A + ((t >> 4) + 32 * i) * kLdA + 8 * (t & 15)) = v;
    }
    if (bstore) {
#pragma unroll
      for (int sb = 0; sb < NBL; ++sb) {
        uint8_t* d;
        if constexpr (HOT) {
          d = sB + buf * kMupBbuf + (64 * sb + (t >> 3)) * kLdB8 + 16 * (t & 7);
        } else {
          const int it = t >> 3;   // < 32 when narrow
          d = sB + buf * kMupBbuf + (64 * (it >> 5) + 32 * ((t >> 2) & 1) + (it & 31)) * kLdB4 + 16 * (t & 3);
        }
        reinterpret_cast<u32x2*>(d)[0] = u32x2{rb[sl][sb].x, rb[sl][sb].y};
        reinterpret_cast<u32x2*>(d)[1] = u32x2{rb[sl][sb].z, rb[sl][sb].w};
      }
    }
  };
  f32x16 acc[2][2][NW];   // [token subtile][gate, up][neuron subtile]
#pragma unroll
  for (int ms = 0; ms < 2; ++ms)
#pragma unroll
    for (int sb = 0; sb < NW; ++sb) acc[ms][0][sb] = acc[ms][1][sb] = f32x16{};
  // K step w of block kb: rows 64 s + col (gate) and 64 s + 32 + col (up),
  // this lane's 8 K
  auto mma_block = [&](int buf, int kb) {
    const uint16_t* A = sA + buf * (kMupAbuf / 2);
    const uint8_t* B = sB + buf * kMupBbuf;
    h8 bg[NW], bu[NW];
#pragma unroll
    for (int sb = 0; sb < NW; ++sb) {
      if constexpr (HOT) {
        const u32x2 vg = *reinterpret_cast<const u32x2*>(B + (64 * sb + col) * kLdB8 + 64 * h + 8 * w);
        const u32x2 vu = *reinterpret_cast<const u32x2*>(B + (64 * sb + 32 + col) * kLdB8 + 64 * h + 8 * w);
        bg[sb] = fp8x8_h8(vg[0], vg[1]);
        bu[sb] = fp8x8_h8(vu[0], vu[1]);
      } else {
        const _Float16 sg = __builtin_bit_cast(_Float16, sSc[kb * TW + 32 * sb + col]);
        const _Float16 su = __builtin_bit_cast(_Float16, sSc[(kGroups + kb) * TW + 32 * sb + col]);
        const uint32_t dg = *reinterpret_cast<const uint32_t*>(B + (64 * sb + col) * kLdB4 + 32 * h + 4 * w);
        const uint32_t du = *reinterpret_cast<const uint32_t*>(B + (64 * sb + 32 + col) * kLdB4 + 32 * h + 4 * w);
        bg[sb] = int4x8_h8_scaled(dg, sg);
        bu[sb] = int4x8_h8_scaled(du, su);
      }
    }
#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
      const h8 av = a_frag32(A, ms, w);
#pragma unroll
      for (int sb = 0; sb < NW; ++sb) {
        acc[ms][0][sb] = mfma32(av, bg[sb], acc[ms][0][sb]);
        acc[ms][1][sb] = mfma32(av, bu[sb], acc[ms][1][sb]);
      }
    }
  };

  constexpr int kNB = kH / kBK;
  static_assert(kNB % 2 == 0, "the block loop is unrolled by two");
  load(0, 0);
  load(1, 1);
  store(0, 0);
  lds_barrier();
#pragma unroll 1
  for (int k0 = 0; k0 < kNB; k0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kb = k0 + u;
      // slot u held block kb, already in LDS buffer u: refill it with kb + 2
      // (the last two passes load the last block again, unused)
      load(min(kb + 2, kNB - 1), u);
      __builtin_amdgcn_sched_barrier(0);
      mma_block(u, kb);
      __builtin_amdgcn_sched_barrier(0);
      if (kb + 1 < kNB) store(u ^ 1, u ^ 1);
      lds_barrier();
    }
  }

  // the epilogue's operands of this lane's columns, loaded while the sums meet
  float sg[NW], su[NW], gb[NW];
  bool ok[NW];
#pragma unroll
  for (int sb = 0; sb < NW; ++sb) {
    sg[sb] = su[sb] = gb[sb] = 0.f;
    if constexpr (HOT) {
      const int row = n0 + 32 * sb + col;
      ok[sb] = row < a.n_hot;
      if (ok[sb]) {
        sg[sb] = a.gate_s[row];
        su[sb] = a.up_s[row];
        gb[sb] = a.hot_gbias ? a.hot_gbias[row] : 0.f;
      }
    } else {
      const int item = n0 + 32 * sb + col;
      const int slot = item < total ? a.dslots[item] : -1;
      ok[sb] = slot >= 0 && slot < a.n_records;
      gb[sb] = (ok[sb] && a.cold_gbias) ? a.cold_gbias[slot] : 0.f;
    }
  }
  // the eight waves' sums of each neuron subtile meet in LDS (the operand
  // buffers are free now): waves 4-7 store theirs, waves 0-3 add them to
  // their own and store the pair; then wave w adds the four pairs (in wave
  // order) for its four (token subtile, row group) pairs and writes those
  // outputs
  float* red = reinterpret_cast<float*>(smem);
  auto red_at = [&](int buf, int ms, int g, int j) { return red + buf * (kMupRedBuf / 4) + ((ms * 2 + g) * 16 + j) * 64 + l; };
  const int ms = w >> 2;
#pragma unroll
  for (int sb = 0; sb < NW; ++sb) {
    if (sb > 0) __syncthreads();   // the previous subtile's sums are read
    if (w >= 4) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int j = 0; j < 16; ++j) *red_at(w - 4, q, g, j) = acc[q][g][sb][j];
    }
    __syncthreads();
    if (w < 4) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int j = 0; j < 16; ++j) *red_at(w, q, g, j) = acc[q][g][sb][j] + *red_at(w, q, g, j);
    }
    __syncthreads();
    // wave w: token subtile ms = w >> 2, output rows j = 4 (w & 3) .. + 3,
    // i.e. tokens m0 + 32 ms + 8 (w & 3) + 4 h + i, i < 4
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * (w & 3) + i;
      float gs = 0.f, us = 0.f;
#pragma unroll
      for (int bq = 0; bq < 4; ++bq) {
        gs += *red_at(bq, ms, 0, j);
        us += *red_at(bq, ms, 1, j);
      }
      const int m = m0 + 32 * ms + 8 * (j >> 2) + 4 * h + (j & 3);
      if (m >= a.M) continue;
      if constexpr (HOT) {
        const float hv = ok[sb] ? gated_act(fmaf(gs, sg[sb], gb[sb]), us * su[sb], a.relu, a.both) : 0.f;
        a.hh[(size_t)m * a.ldh + n0 + 32 * sb + col] = float_to_half_bits(hv);
      } else {
        const float hv = ok[sb] ? gated_act(gs + gb[sb], us, a.relu, a.both) : 0.f;
        a.hc[(size_t)m * a.ldc + n0 + 32 * sb + col] = float_to_half_bits(hv);
      }
    }
  }
}

// Tiles: the hot rows' 32-neuron units, then the dense list's, each side's
// first `wide_*` tiles two units wide.  Grid: tiles rounded up to 8, x token
// tiles, the token tiles of one weight tile on one XCD (workgroups go
// round-robin over the 8 XCDs), sharing its L2 for the weights.
// (WIDE = false: no wide tile, and the narrow tile's registers allow two
// workgroups per CU.)
struct MupTiles {
  int hot_units, wide_hot, wide_cold, n_tiles;
};
template <bool WIDE>
__global__ __launch_bounds__(kMupThreads) void k_mup(BUpArgs a, MupTiles mtl, int mt) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kMupLds];
  const int b = blockIdx.x;
  const int q = b >> 3;
  const int nt = (q / mt) * 8 + (b & 7), mtile = q % mt;
  if (nt >= mtl.n_tiles) return;   // the whole workgroup
  const int m0 = mtile * 64;
  const int hot_tiles = mtl.hot_units - mtl.wide_hot;
  if (nt < hot_tiles) {
    if (WIDE && nt < mtl.wide_hot)
      mup_tile<true, WIDE ? 2 : 1>(a, 64 * nt, m0, 0, smem);
    else
      mup_tile<true, 1>(a, kMupN * (nt + mtl.wide_hot), m0, 0, smem);
    return;
  }
  const int total = min(*a.total, a.cap);
  const int c = nt - hot_tiles;
  const int i0 = c < mtl.wide_cold ? 64 * c : kMupN * (c + mtl.wide_cold);
  if (i0 >= total) return;   // the whole workgroup
  if (WIDE && c < mtl.wide_cold)
    mup_tile<false, WIDE ? 2 : 1>(a, i0, m0, total, smem);
  else
    mup_tile<false, 1>(a, i0, m0, total, smem);
}

// Hot down for 32 MS tokens x 128 NB outputs (4 waves x 32 NB) over the K
// blocks of one of `splits` ranges, whose partial sum of y it stores.  The
// down rows of each K block are staged through padded LDS like the gate/up
// weights (thread t: chunk t & 7 of rows t / 8 + 32 i); chunks past the row
// stride read as zero (the stride is a multiple of 64, so a chunk never
// straddles it).  Same XCD-aware index mapping.  At 128 tokens a wave's 32
// output rows took 4 A fragments per B fragment from LDS; NB = 2 halves the
// LDS reads per MFMA.  The K blocks are loaded D ahead into D register sets
// (a range of a few blocks at 17-191 tokens is otherwise one load latency
// per block).
// Hot down main loop: acc += the token rows m0 .. of H_hot over K blocks
// [kb0, kb1) times the down rows of output tile nt (unscaled).
template <int MS, int NB, int D>
__device__ __forceinline__ void hot_down_blocks(const BDownArgs& a, int nt, int m0, int kb0, int kb1,
                                                f32x16 (&acc)[MS][NB], uint16_t* sA, uint8_t* sB) {
  constexpr int kAbuf = 32 * MS * kLdA;
  constexpr int kBbuf = 128 * NB * kLdB8;
  const int t = threadIdx.x, w = t >> 6, l = lane_id();
  const ARows<MS> arows(a.hh, a.ldh, a.M, m0);
  const rsrc_t rd = buf_rsrc(a.down_q, (uint32_t)kH * a.down_stride);
  uint32_t voff[4 * NB];
#pragma unroll
  for (int i = 0; i < 4 * NB; ++i)
    voff[i] = (uint32_t)(nt * 128 * NB + (t >> 3) + 32 * i) * a.down_stride + 16 * (t & 7);
  struct Stage {
    u32x4 ra[2 * MS], rb[4 * NB];
    bool in;   // the block's chunk lies inside the row stride
  };
  auto load = [&](int kb, Stage& S) {
    arows.load(kb, S.ra);
    S.in = kb * kBK + 16 * (t & 7) < a.down_stride;
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) S.rb[i] = bload16(rd, voff[i], kb * kBK);
  };
  auto store = [&](int buf, const Stage& S) {
    store_a_rows<2 * MS, false>(S.ra, sA + buf * kAbuf);
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) {
      const u32x4 v = S.in ? S.rb[i] : u32x4{0u, 0u, 0u, 0u};
      uint8_t* d = sB + buf * kBbuf + ((t >> 3) + 32 * i) * kLdB8 + 16 * (t & 7);
      reinterpret_cast<u32x2*>(d)[0] = u32x2{v.x, v.y};
      reinterpret_cast<u32x2*>(d)[1] = u32x2{v.z, v.w};
    }
  };
  // set i holds block kb + i of each D-block round; block b + 1 is staged
  // while block b is multiplied, and set b % D reloads block b + D
  Stage S[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load(min(kb0 + i, kb1 - 1), S[i]);
  store(0, S[0]);
  lds_barrier();
  for (int kb = kb0; kb < kb1; kb += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int bk = kb + i, cur = (bk - kb0) & 1;
      if (bk >= kb1) break;   // workgroup-uniform
      load(min(bk + D, kb1 - 1), S[i]);
      __builtin_amdgcn_sched_barrier(0);
      mma_block_lds<MS, NB, false>(sA + cur * kAbuf, sB + cur * kBbuf, nullptr, acc);
      __builtin_amdgcn_sched_barrier(0);
      if (bk + 1 >= kb1) break;
      store(cur ^ 1, S[(i + 1) % D]);
      lds_barrier();
    }
  }
}

template <int MS, int NB, int D>
__global__ __launch_bounds__(kThreads) void k_pgemm_down_hot(BDownArgs a, int mt, int splits) {
  constexpr int kAbuf = 32 * MS * kLdA;
  constexpr int kBbuf = 128 * NB * kLdB8;
  constexpr int kTiles = kH / (128 * NB);
  __shared__ __attribute__((aligned(16))) uint16_t sA[2 * kAbuf];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2 * kBbuf];
  const int b = blockIdx.x;
  const int q = b >> 3, per = mt * splits;
  const int nt = (q / per) * 8 + (b & 7), rem = q % per;
  if (nt >= kTiles) return;   // the whole workgroup
  const int mtile = rem % mt, split = rem / mt;
  const int kb0 = split * a.hot_blocks / splits, kb1 = (split + 1) * a.hot_blocks / splits;
  if (kb0 >= kb1) return;
  const int m0 = mtile * 32 * MS;
  const int w = threadIdx.x >> 6, l = lane_id();
  f32x16 acc[MS][NB];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = f32x16{};
  hot_down_blocks<MS, NB, D>(a, nt, m0, kb0, kb1, acc, sA, sB);
  // this range's partial sum of y (rows past M dropped by the store's range;
  // no element takes a branch)
  const rsrc_t ry = buf_rsrc(a.y + (size_t)split * a.M * kH, (uint32_t)a.M * kH * 4);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = nt * 128 * NB + 128 * nb + 32 * w + (l & 31);
    const float sd = a.down_s[row];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int m = m0 + 32 * ms + 8 * (j >> 2) + 4 * (l >> 5) + (j & 3);
        __builtin_amdgcn_raw_buffer_store_b32(as_u32(acc[ms][nb][j] * sd), ry, ((uint32_t)m * kH + row) * 4, 0, 0);
      }
  }
}

// Cold down for 128 tokens x 256 outputs (4 waves x 64) over a range of the
// dense active list, 64 items per K block.  The records hold each item's down
// nibbles contiguous along the outputs, while the MFMA wants 8 consecutive
// items per lane, so every block is transposed on the way into LDS: thread
// (ig = t & 7, jg = t >> 3) loads one dword (8 outputs) from each of the
// items 8 ig .. 8 ig + 7, transposes the 8 x 8 nibble block in registers,
// decodes each output's 8 items times their group scales (rounded once to
// fp16, in int4x8_h8's pair order; the H tile is staged in the same order)
// and writes 16-byte rows of the tile T[output][item].  The next block's
// record dwords and H tile are loaded a block ahead; the record offsets of
// the whole range sit in an LDS table, so no load waits for another.
constexpr int kDcItems = 64;                // items per K block
constexpr int kLdC = kDcItems + 8;          // LDS row of T and of the H tile, halves (144 B)
constexpr int kDcMaxItems = 2048;           // items per workgroup (record offset table)

// 8 x 8 nibble transpose: r[k] nibble n -> r[n] nibble k.
__device__ __forceinline__ void nibble_transpose8(uint32_t (&r)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {   // 16-bit halves between rows k and k + 4
    const uint32_t a = r[k], b = r[k + 4];
    r[k] = (a & 0x0000FFFFu) | (b << 16);
    r[k + 4] = (a >> 16) | (b & 0xFFFF0000u);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {   // bytes between rows k and k + 2
    const int k = (i & 1) + 4 * (i >> 1);
    const uint32_t a = r[k], b = r[k + 2];
    r[k] = (a & 0x00FF00FFu) | ((b << 8) & 0xFF00FF00u);
    r[k + 2] = ((a >> 8) & 0x00FF00FFu) | (b & 0xFF00FF00u);
  }
#pragma unroll
  for (int k = 0; k < 8; k += 2) {   // nibbles between rows k and k + 1
    const uint32_t a = r[k], b = r[k + 1];
    r[k] = (a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u);
    r[k + 1] = ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u);
  }
}

// Workgroup = 256 outputs x 32 MS tokens x one range of K blocks (items).
// PART (at most 16 tokens): the range's sum goes to a.part[split] as
// (H, 16) fp32, an empty range storing zeros; otherwise it is added into y.
// Cold down main loop: acc += the token rows m0 .. of H_cold over the dense
// list's K blocks [kb0, kb1) (64 items each) times the items' down columns
// for outputs j0 .. j0 + 255.  Wave w multiplies outputs j0 + 64 w + 32 nb
// (+ lane).
template <int MS>
__device__ __forceinline__ void cold_down_blocks(const BDownArgs& a, int j0, int m0, int total, int kb0, int kb1,
                                                 f32x16 (&acc)[MS][2], uint16_t* sT, uint16_t* sH,
                                                 uint32_t* s_rec, uint16_t* s_sc) {
  constexpr int NB = 2;
  constexpr int kT = 256 * kLdC, kA = 32 * MS * kLdC;   // halves per buffer
  const int t = threadIdx.x, w = t >> 6, l = lane_id();
  const int i_base = kb0 * kDcItems, n_items = (kb1 - kb0) * kDcItems;

  // record offsets of the range (items past the list or with invalid slots
  // point past the records and read as zero)
  for (int i = t; i < n_items; i += kThreads) {
    const int it = i_base + i;
    const int slot = it < total ? a.dslots[it] : -1;
    s_rec[i] = (slot >= 0 && slot < a.n_records) ? (uint32_t)slot * kRecBytes : kNoOffset;
  }
  __syncthreads();

  const rsrc_t rr = buf_rsrc(a.records, (uint32_t)a.n_records * kRecBytes);
  const rsrc_t rh = buf_rsrc(a.hc, (uint32_t)a.M * a.ldc * 2);
  const int ig = t & 7, jg = t >> 3;
  const uint32_t dbyte = kOffDown + (j0 + 8 * jg) / 2;                        // this thread's dword
  // the wave's down scale group: its threads' outputs j0 + 8 jg, jg in
  // [8 w, 8 w + 8), all lie in group (j0 + 64 w) / kGroup
  const uint32_t sbyte = kOffScales + 2 * (2 * kGroups + (j0 + 64 * w) / kGroup);
  // H tile: thread t loads chunk t & 7 (8 items) of token rows t / 8 + 32 r
  uint32_t hoff[MS];
#pragma unroll
  for (int r = 0; r < MS; ++r) hoff[r] = ((uint32_t)(m0 + (t >> 3) + 32 * r) * a.ldc + 8 * (t & 7)) * 2;

  // a K block's loads, held in registers until it is decoded into LDS
  struct Blk {
    uint32_t dq[8];   // this thread's record dword of items 8 ig .. 8 ig + 7
    uint32_t sc;      // lane l: the wave's down scale of item l of the block
    u32x4 hv[MS];     // the H tile
    int kb;
  };
  auto load_block = [&](int kb, Blk& B) {
    B.kb = kb;
    const int ib = (kb - kb0) * kDcItems + 8 * ig;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      B.dq[k] = __builtin_amdgcn_raw_buffer_load_b32(rr, (int)(s_rec[ib + k] + dbyte), 0, 0);
    // one scale per item per wave (the wave's outputs share a group): one
    // 2-byte load per lane instead of eight per thread, handed to the
    // threads that decode the item through the wave's own LDS row
    B.sc = bload2(rr, s_rec[(kb - kb0) * kDcItems + l] + sbyte, 0);
#pragma unroll
    for (int r = 0; r < MS; ++r) B.hv[r] = bload16(rh, hoff[r], kb * kDcItems * 2);
  };
  // decode the loaded block into buffer `buf`
  auto store_block = [&](int buf, const Blk& B) {
    const int hkb = B.kb;
    uint32_t c[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = B.dq[k];
    nibble_transpose8(c);
    // the wave's LDS row: written by lane l, read back 8 items per thread
    // by the same wave (its LDS operations complete in order)
    s_sc[w * kDcItems + l] = (uint16_t)B.sc;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const u32x4 s8 = *reinterpret_cast<const u32x4*>(s_sc + w * kDcItems + 8 * ig);   // items 0..7, 2 a dword
    // the items' scales in pair order (i0, i4, i1, i5, ...)
    const h8 sv = __builtin_bit_cast(h8, u32x4{__builtin_amdgcn_perm(s8.z, s8.x, 0x05040100u),
                                               __builtin_amdgcn_perm(s8.z, s8.x, 0x07060302u),
                                               __builtin_amdgcn_perm(s8.w, s8.y, 0x05040100u),
                                               __builtin_amdgcn_perm(s8.w, s8.y, 0x07060302u)});
    uint16_t* T = sT + buf * kT;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      u32x4 m;
#pragma unroll
      for (int k = 0; k < 4; ++k) m[k] = ((c[n] >> (4 * k)) & 0x000F000Fu) ^ 0x64086408u;
      const h8 v = (__builtin_bit_cast(h8, m) + (_Float16)-1032.0f) * sv;
      *reinterpret_cast<h8*>(T + (8 * jg + n) * kLdC + 8 * ig) = v;
    }
    uint16_t* Hs = sH + buf * kA;
    // H columns past the list's end may hold anything (the gate/up kernels
    // write only the item tiles they own): keep items < total only
    const int keep = total - (hkb * kDcItems + 8 * (t & 7));
    uint32_t km[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      km[d] = (2 * d < keep ? 0x0000FFFFu : 0u) | (2 * d + 1 < keep ? 0xFFFF0000u : 0u);
#pragma unroll
    for (int r = 0; r < MS; ++r) {
      const uint32_t d0 = B.hv[r].x & km[0], d1 = B.hv[r].y & km[1], d2 = B.hv[r].z & km[2], d3 = B.hv[r].w & km[3];
      u32x4 v;
      v.x = (d0 & 0xFFFFu) | (d2 << 16);
      v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
      v.z = (d1 & 0xFFFFu) | (d3 << 16);
      v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
      *reinterpret_cast<u32x4*>(Hs + ((t >> 3) + 32 * r) * kLdC + 8 * (t & 7)) = v;
    }
  };

  // blocks are loaded two ahead: block kb + 2's loads go out while block kb
  // is multiplied and block kb + 1 (loaded an iteration earlier) is decoded
  auto mma_block = [&](int cur) {
    const uint16_t* T = sT + cur * kT;
    const uint16_t* Hs = sH + cur * kA;
#pragma unroll
    for (int st = 0; st < kDcItems / 16; ++st) {
      const int col = 16 * st + 8 * (l >> 5);
      h8 bf[NB], av[MS];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bf[nb] = *reinterpret_cast<const h8*>(T + (64 * w + 32 * nb + (l & 31)) * kLdC + col);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) av[ms] = *reinterpret_cast<const h8*>(Hs + (32 * ms + (l & 31)) * kLdC + col);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = mfma32(av[ms], bf[nb], acc[ms][nb]);
    }
  };
  Blk B0, B1;
  load_block(kb0, B0);
  load_block(min(kb0 + 1, kb1 - 1), B1);
  store_block(0, B0);
  lds_barrier();
  for (int kb = kb0; kb < kb1; kb += 2) {
    // block kb in LDS buffer 0, block kb + 1 in B1
    load_block(min(kb + 2, kb1 - 1), B0);
    __builtin_amdgcn_sched_barrier(0);
    mma_block(0);
    __builtin_amdgcn_sched_barrier(0);
    if (kb + 1 >= kb1) break;   // workgroup-uniform
    store_block(1, B1);
    lds_barrier();
    // block kb + 1 in LDS buffer 1, block kb + 2 in B0
    load_block(min(kb + 3, kb1 - 1), B1);
    __builtin_amdgcn_sched_barrier(0);
    mma_block(1);
    __builtin_amdgcn_sched_barrier(0);
    store_block(0, B0);
    lds_barrier();
  }
}

template <int MS, bool PART>
__global__ __launch_bounds__(kThreads) void k_pgemm_down_cold(BDownArgs a, int mt, int splits) {
  constexpr int NB = 2;
  constexpr int kT = 256 * kLdC, kA = 32 * MS * kLdC;   // halves per buffer
  static_assert(!PART || MS == 1, "partial sums hold 16 tokens");
  __shared__ __attribute__((aligned(16))) uint16_t sT[2 * kT];
  __shared__ __attribute__((aligned(16))) uint16_t sH[2 * kA];
  __shared__ uint32_t s_rec[kDcMaxItems];
  __shared__ __attribute__((aligned(16))) uint16_t s_sc[4 * kDcItems];   // per wave: the block's item scales
  const int b = blockIdx.x;
  const int q = b >> 3, per = mt * splits;
  const int jt = (q / per) * 8 + (b & 7), rem = q % per;
  if (jt >= kH / 256) return;   // the whole workgroup
  const int mtile = rem % mt, split = rem / mt;
  const int total = min(*a.total, a.cap);
  const int n_blk = (total + kDcItems - 1) / kDcItems;
  const int kb0 = split * n_blk / splits, kb1 = (split + 1) * n_blk / splits;
  const int t = threadIdx.x, w = t >> 6, l = lane_id();
  const int m0 = mtile * 32 * MS, j0 = jt * 256;
  // (from 17 tokens) this range's partial sum of y, rows past M dropped
  const rsrc_t ry = buf_rsrc(PART ? nullptr : a.y + (size_t)(a.cold_split0 + split) * a.M * kH,
                             PART ? 0u : (uint32_t)a.M * kH * 4);
  if (kb0 >= kb1) {   // the whole workgroup: an empty range sums to zero
    if (PART) {
      f32x4* dst = reinterpret_cast<f32x4*>(a.part + ((size_t)split * kH + j0 + t) * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      for (int i = t; i < 32 * MS * 64; i += kThreads)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, ry,
                                                ((uint32_t)(m0 + (i >> 6)) * kH + j0 + 4 * (i & 63)) * 4, 0, 0);
    }
    return;
  }
  f32x16 acc[MS][NB];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = f32x16{};
  cold_down_blocks<MS>(a, j0, m0, total, kb0, kb1, acc, sT, sH, s_rec, s_sc);
  if (PART) {
    // rows 0..15 of the 32x32 tile: elements 0..7, four consecutive rows each
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float* dst = a.part + ((size_t)split * kH + j0 + 64 * w + 32 * nb + (l & 31)) * 16 + 4 * (l >> 5);
#pragma unroll
      for (int g = 0; g < 2; ++g)
        *reinterpret_cast<f32x4*>(dst + 8 * g) =
            f32x4{acc[0][nb][4 * g], acc[0][nb][4 * g + 1], acc[0][nb][4 * g + 2], acc[0][nb][4 * g + 3]};
    }
    return;
  }
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * ms + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
        __builtin_amdgcn_raw_buffer_store_b32(as_u32(acc[ms][nb][e]), ry,
                                              ((uint32_t)m * kH + j0 + 64 * w + 32 * nb + (l & 31)) * 4, 0, 0);
      }
}

// The hot and the cold down of one 32 MS-token x 256-output tile in one
// workgroup, over range `split` of the hot K blocks and range `split` of the
// list's K blocks, so each range stores one partial sum (the final add reads
// fewer).  The hot sums take their row scales before the cold sums join
// them.  8 waves: waves 4-7 load each block (the hot range's blocks first,
// then the list's) and stage it into LDS, the hot block as loaded, the cold
// block decoded as in cold_down_blocks; waves 0-3 only multiply.  Blocks are
// loaded two ahead and go through two LDS buffers, one barrier per block;
// a buffer holds either kind.  (With 4 waves doing both, 512 tokens took
// 4219 against 3958 us per 32 layers, 64 tokens 1868 against 1834.)
template <int MS>
__global__ __launch_bounds__(2 * kThreads) void k_pgemm_down_both(BDownArgs a, int mt, int splits) {
  constexpr int NB = 2;
  constexpr int kHotA = 32 * MS * kLdA * 2, kHotB = 256 * kLdB8;   // bytes per buffer
  constexpr int kColdT = 256 * kLdC * 2, kColdH = 32 * MS * kLdC * 2;
  constexpr int kBuf = kHotA + kHotB > kColdT + kColdH ? kHotA + kHotB : kColdT + kColdH;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kBuf];
  __shared__ uint32_t s_rec[kDcMaxItems];
  __shared__ __attribute__((aligned(16))) uint16_t s_sc[4 * kDcItems];
  const int b = blockIdx.x;
  const int q = b >> 3, per = mt * splits;
  const int jt = (q / per) * 8 + (b & 7), rem = q % per;
  if (jt >= kH / 256) return;   // the whole workgroup
  const int mtile = rem % mt, split = rem / mt;
  const int m0 = mtile * 32 * MS, j0 = jt * 256;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int hb0 = split * a.hot_blocks / splits, hb1 = (split + 1) * a.hot_blocks / splits;
  const int total = min(*a.total, a.cap);
  const int n_blk = (total + kDcItems - 1) / kDcItems;
  const int cb0 = split * n_blk / splits, cb1 = (split + 1) * n_blk / splits;
  const int nh = max(hb1 - hb0, 0), nc = max(cb1 - cb0, 0), n = nh + nc;
  if (w >= 4) {
    // staging thread t: token rows (t >> 4) + 16 i of H_hot, chunk t & 15;
    // down rows (t >> 3) + 32 i of the tile, chunk t & 7; the record dword
    // of outputs j0 + 8 (t >> 3) of items 8 (t & 7) .. + 7, and chunk t & 7
    // of H_cold rows (t >> 3) + 32 r
    const int t = threadIdx.x - 256, wp = w - 4;
    for (int i = t; i < nc * kDcItems; i += kThreads) {
      const int it = cb0 * kDcItems + i;
      const int slot = it < total ? a.dslots[it] : -1;
      s_rec[i] = (slot >= 0 && slot < a.n_records) ? (uint32_t)slot * kRecBytes : kNoOffset;
    }
    const rsrc_t rha = buf_rsrc(a.hh, (uint32_t)a.M * a.ldh * 2);
    const rsrc_t rd = buf_rsrc(a.down_q, (uint32_t)kH * a.down_stride);
    const rsrc_t rr = buf_rsrc(a.records, (uint32_t)a.n_records * kRecBytes);
    const rsrc_t rhc = buf_rsrc(a.hc, (uint32_t)a.M * a.ldc * 2);
    uint32_t aoff[2 * MS], doff[8], hoff[MS];
#pragma unroll
    for (int i = 0; i < 2 * MS; ++i) aoff[i] = ((uint32_t)(m0 + (t >> 4) + 16 * i) * a.ldh + 8 * (t & 15)) * 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) doff[i] = (uint32_t)(j0 + (t >> 3) + 32 * i) * a.down_stride + 16 * (t & 7);
#pragma unroll
    for (int r = 0; r < MS; ++r) hoff[r] = ((uint32_t)(m0 + (t >> 3) + 32 * r) * a.ldc + 8 * (t & 7)) * 2;
    const int ig = t & 7;
    const uint32_t dbyte = kOffDown + (j0 + 8 * (t >> 3)) / 2;
    const uint32_t sbyte = kOffScales + 2 * (2 * kGroups + (j0 + 64 * wp) / kGroup);
    // a slot holds one block of either kind: hot, the token rows in R[0, 2 MS)
    // and the down rows in R[2 MS, 2 MS + 8); cold, the record dwords in
    // R[0, 2), the scale in R[2].x and H_cold in R[3, 3 + MS)
    constexpr int kR = 2 * MS + 8;
    u32x4 R[2][kR];
    auto load = [&](int i, int sl) {
      if (i < nh) {   // workgroup-uniform
        const int kb = hb0 + i;
#pragma unroll
        for (int r = 0; r < 2 * MS; ++r) R[sl][r] = bload16(rha, aoff[r], kb * kBK * 2);
#pragma unroll
        for (int r = 0; r < 8; ++r) R[sl][2 * MS + r] = bload16(rd, doff[r], kb * kBK);
      } else {
        const int kb = cb0 + i - nh;
        const int ib = (i - nh) * kDcItems;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          R[sl][k >> 2][k & 3] = __builtin_amdgcn_raw_buffer_load_b32(rr, (int)(s_rec[ib + 8 * ig + k] + dbyte), 0, 0);
        R[sl][2].x = bload2(rr, s_rec[ib + l] + sbyte, 0);
#pragma unroll
        for (int r = 0; r < MS; ++r) R[sl][3 + r] = bload16(rhc, hoff[r], kb * kDcItems * 2);
      }
    };
    auto store = [&](int i, int buf, int sl) {
      uint8_t* base = smem + buf * kBuf;
      if (i < nh) {
        const int kb = hb0 + i;
        const bool in = kb * kBK + 16 * (t & 7) < a.down_stride;   // the chunk lies inside the row stride
        uint16_t* A = reinterpret_cast<uint16_t*>(base);
#pragma unroll
        for (int r = 0; r < 2 * MS; ++r)
          *reinterpret_cast<u32x4*>(A + ((t >> 4) + 16 * r) * kLdA + 8 * (t & 15)) = R[sl][r];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const u32x4 v = in ? R[sl][2 * MS + r] : u32x4{0u, 0u, 0u, 0u};
          uint8_t* d = base + kHotA + ((t >> 3) + 32 * r) * kLdB8 + 16 * (t & 7);
          reinterpret_cast<u32x2*>(d)[0] = u32x2{v.x, v.y};
          reinterpret_cast<u32x2*>(d)[1] = u32x2{v.z, v.w};
        }
      } else {
        const int kb = cb0 + i - nh;
        uint32_t c[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) c[k] = R[sl][k >> 2][k & 3];
        nibble_transpose8(c);
        s_sc[wp * kDcItems + l] = (uint16_t)R[sl][2].x;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const u32x4 s8 = *reinterpret_cast<const u32x4*>(s_sc + wp * kDcItems + 8 * ig);
        const h8 sv = __builtin_bit_cast(h8, u32x4{__builtin_amdgcn_perm(s8.z, s8.x, 0x05040100u),
                                                   __builtin_amdgcn_perm(s8.z, s8.x, 0x07060302u),
                                                   __builtin_amdgcn_perm(s8.w, s8.y, 0x05040100u),
                                                   __builtin_amdgcn_perm(s8.w, s8.y, 0x07060302u)});
        uint16_t* T = reinterpret_cast<uint16_t*>(base);
#pragma unroll
        for (int nn = 0; nn < 8; ++nn) {
          u32x4 m;
#pragma unroll
          for (int k = 0; k < 4; ++k) m[k] = ((c[nn] >> (4 * k)) & 0x000F000Fu) ^ 0x64086408u;
          const h8 v = (__builtin_bit_cast(h8, m) + (_Float16)-1032.0f) * sv;
          *reinterpret_cast<h8*>(T + (8 * (t >> 3) + nn) * kLdC + 8 * ig) = v;
        }
        uint16_t* Hs = reinterpret_cast<uint16_t*>(base + kColdT);
        const int keep = total - (kb * kDcItems + 8 * ig);
        uint32_t km[4];
#pragma unroll
        for (int d = 0; d < 4; ++d)
          km[d] = (2 * d < keep ? 0x0000FFFFu : 0u) | (2 * d + 1 < keep ? 0xFFFF0000u : 0u);
#pragma unroll
        for (int r = 0; r < MS; ++r) {
          const u32x4 hv = R[sl][3 + r];
          const uint32_t d0 = hv.x & km[0], d1 = hv.y & km[1], d2 = hv.z & km[2], d3 = hv.w & km[3];
          u32x4 v;
          v.x = (d0 & 0xFFFFu) | (d2 << 16);
          v.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
          v.z = (d1 & 0xFFFFu) | (d3 << 16);
          v.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
          *reinterpret_cast<u32x4*>(Hs + ((t >> 3) + 32 * r) * kLdC + 8 * ig) = v;
        }
      }
    };
    // block i sits in register slot and LDS buffer i & 1; the record table
    // is complete at the first barrier, before any record load
    if (nh > 0) load(0, 0);
    if (nh > 1) load(1, 1);
    lds_barrier();
    if (n > 0) {   // workgroup-uniform
      if (nh == 0) load(0, 0);
      if (nh <= 1 && n > 1) load(1, 1);
      store(0, 0, 0);
      if (n > 2) load(2, 0);
      lds_barrier();   // block 0 in buffer 0
#pragma unroll 1
      for (int i0 = 0; i0 < n; i0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i = i0 + u;
          if (i >= n) break;
          // block i + 1 into the buffer block i - 1 left, then its slot
          // loads block i + 3
          if (i + 1 < n) {
            store(i + 1, u ^ 1, u ^ 1);
            __builtin_amdgcn_sched_barrier(0);
            if (i + 3 < n) load(i + 3, u ^ 1);
          }
          lds_barrier();
        }
      }
    }
    return;
  }
  f32x16 acc[MS][NB];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = f32x16{};
  float sd_pre[NB];   // the row scales, loaded up front (loaded between the loops they cost spills)
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) sd_pre[nb] = a.down_s[j0 + 128 * nb + 32 * w + (l & 31)];
  auto scale_hot = [&]() {   // the hot sums take their row scales before the cold ones join
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) acc[ms][nb] *= sd_pre[nb];
    }
  };
  auto cold_mma = [&](const uint8_t* base) {
    const uint16_t* T = reinterpret_cast<const uint16_t*>(base);
    const uint16_t* Hs = reinterpret_cast<const uint16_t*>(base + kColdT);
    h8 bf[2][NB], av[2][MS];
    auto frags = [&](int st, h8 (&b)[NB], h8 (&av_)[MS]) {
      const int col = 16 * st + 8 * (l >> 5);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        b[nb] = *reinterpret_cast<const h8*>(T + (128 * nb + 32 * w + (l & 31)) * kLdC + col);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) av_[ms] = *reinterpret_cast<const h8*>(Hs + (32 * ms + (l & 31)) * kLdC + col);
    };
    frags(0, bf[0], av[0]);
#pragma unroll
    for (int st = 0; st < kDcItems / 16; ++st) {
      const int cur = st & 1;
      if (st + 1 < kDcItems / 16) frags(st + 1, bf[cur ^ 1], av[cur ^ 1]);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[ms][nb] = mfma32(av[cur][ms], bf[cur][nb], acc[ms][nb]);
    }
  };
  lds_barrier();   // the record table
  if (n > 0) lds_barrier();   // block 0 in buffer 0
  // block i in buffer i & 1, one barrier after each
#pragma unroll 1
  for (int i = 0; i < nh; ++i) {
    const uint8_t* base = smem + (i & 1) * kBuf;
    mma_block_lds<MS, NB, false>(reinterpret_cast<const uint16_t*>(base), base + kHotA, nullptr, acc);
    lds_barrier();
  }
  if (nh > 0) scale_hot();
#pragma unroll 1
  for (int i = nh; i < n; ++i) {
    cold_mma(smem + (i & 1) * kBuf);
    lds_barrier();
  }
  // this range's partial sum of y (rows past M dropped by the store's range)
  const rsrc_t ry = buf_rsrc(a.y + (size_t)split * a.M * kH, (uint32_t)a.M * kH * 4);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = j0 + 128 * nb + 32 * w + (l & 31);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * ms + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
        __builtin_amdgcn_raw_buffer_store_b32(as_u32(acc[ms][nb][e]), ry, ((uint32_t)m * kH + row) * 4, 0, 0);
      }
  }
}

// ── gate/up for at most 16 tokens, RMSNorm fused ─────────────────────────────

constexpr int kSbGroups = 256;      // workgroups: one per CU
constexpr int kSbThreads = 512;     // 8 waves; wave w takes K [512 w, 512 w + 512)
constexpr int kHotEarly = 4;        // hot chunks each wave loads before the prologue

// Workgroup g takes hot rows [g hr, g hr + hr) (hr = a.hot_per_wg, tiles of
// 16 rows) and items g, g + 256, g + 512, ... of the dense active list
// (tiles of 16), so every CU reads about the same number of weight lines.
// It first normalises the M <= MMAX token rows itself (x_n = fp16((x r) w),
// the rounding of nn.RMSNorm's fp16 output) into LDS: the two halves of the
// workgroup take alternate rows, thread e of a half holds elements
// [16 e, 16 e + 16) of them.  Half of the first hot tile's weight loads are
// in flight by then; the rest, and the first cold tile's record loads, go
// out right after (with all of them first a wave would stall issuing at a
// full memory queue, and the prologue's barriers wait for the slowest wave).
// Hot rows: lane (t, q) = (l & 15, l >> 4) loads 16 bytes of row t at K
// 512 w + 64 c + 16 q, the B operand of two 16x16x32 steps (K + 8 s, s < 2);
// the A operand of the same steps is token t's x_n at the same K.
// Cold items: the lane's 16 bytes are 32 nibbles of item t at K
// 512 w + 128 b + 32 q (four steps, decoded in int4x8_h8's order, the A
// operand permuted to match); the group scale multiplies each 128-K block's
// partial sums.  The 8 waves' sums of a tile meet in LDS and are added in
// wave order.
template <int MMAX>
__global__ __launch_bounds__(kSbThreads) void k_sbup(BUpArgs a, const uint16_t* x, const uint16_t* norm_w,
                                                     float eps) {
  constexpr int kLdX = kH + 8;          // halves per staged row: rows on distinct banks
  constexpr int kRows = MMAX / 2;       // token rows per half of the workgroup
  constexpr int kRed = 7 * 4 * kWave * 4;   // the first hot and cold tiles' wave sums
  constexpr int kScr = MMAX * 256 > kRed ? MMAX * 256 : kRed;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[MMAX * kLdX];
  __shared__ __attribute__((aligned(16))) float s_scr[kScr];   // norm partials, then the wave sums
  const int tid = threadIdx.x, l = lane_id();
  // the wave index as a scalar, so that K offsets go in the buffer
  // instructions' scalar offset operand
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = l & 15, q = l >> 4;
  const int M = a.M;
  const int g = blockIdx.x;
  const int hr = a.hot_per_wg;
  const int n_ht = (hr + 15) / 16;
  const int hot0 = g * hr;
  // Every load below is unconditional (absent data reads zero through a
  // short or empty descriptor), so the compiler issues them back to back and
  // waits for exactly the ones each step uses.  A wave's loads complete in
  // order: the token rows first (the prologue waits on them), then the list
  // (the first cold tile's loads wait on it), then the weights.
  // This thread's token rows (half hf, rows 2 k + hf; rows past M read zero)
  // and norm weights:
  const int hf = tid >> 8, e16 = tid & 255;
  const rsrc_t rx = buf_rsrc(x, (uint32_t)M * kH * 2);
  const rsrc_t rw = buf_rsrc(norm_w, norm_w ? (uint32_t)kH * 2 : 0u);
  u32x4 xin[kRows][2];
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const uint32_t off = ((uint32_t)(2 * k + hf) * kH + 16 * e16) * 2;
    xin[k][0] = bload16(rx, off, 0);
    xin[k][1] = bload16(rx, off, 16);
  }
  u32x4 wn[2];
  wn[0] = bload16(rw, 32 * e16, 0);
  wn[1] = bload16(rw, 32 * e16, 16);
  // lane t's item of tile 0 is g + 256 t
  const bool list = a.ldc > 0;
  const rsrc_t rlt = buf_rsrc(a.total, list ? 4u : 0u);
  const rsrc_t rls = buf_rsrc(a.dslots, list ? (uint32_t)a.cap * 4 : 0u);
  int raw_total = (int)__builtin_amdgcn_raw_buffer_load_b32(rlt, 0, 0, 0);
  int raw_slot = (int)__builtin_amdgcn_raw_buffer_load_b32(rls, 4 * (g + kSbGroups * t), 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  const int kq = 512 * w;
  const rsrc_t rg = buf_rsrc(a.gate_q, (uint32_t)a.n_hot * kH);
  const rsrc_t ru = buf_rsrc(a.up_q, (uint32_t)a.n_hot * kH);
  const rsrc_t rr = buf_rsrc(a.records, (uint32_t)a.n_records * kRecBytes);
  const rsrc_t rgs = buf_rsrc(a.gate_s, (uint32_t)a.n_hot * 4);
  const rsrc_t rus = buf_rsrc(a.up_s, (uint32_t)a.n_hot * 4);
  const rsrc_t rhb = buf_rsrc(a.hot_gbias, a.hot_gbias ? (uint32_t)a.n_hot * 4 : 0u);
  const rsrc_t rcb = buf_rsrc(a.cold_gbias, a.cold_gbias ? (uint32_t)a.n_records * 4 : 0u);
  u32x4 WG[8], WU[8];                   // one hot tile's chunks
  float hsg, hsu, hgb;                  // and its row scales and gate bias (zero past the rows)
  // chunks [c0, c1) of hot tile ti
  auto hot_issue = [&](int ti, int c0, int c1) {
    const int r = 16 * ti + t, col = hot0 + r;
    // rows past this workgroup's share or past n_hot read zero
    const bool in = r < hr && col < a.n_hot;
    const uint32_t voff = in ? (uint32_t)col * kH + 16 * q : kNoOffset;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c < c0 || c >= c1) continue;
      WG[c] = bload16(rg, voff, kq + 64 * c);
      WU[c] = bload16(ru, voff, kq + 64 * c);
    }
    if (c0 > 0) return;
    const uint32_t soff = in ? (uint32_t)col * 4 : kNoOffset;
    hsg = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rgs, soff, 0, 0));
    hsu = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rus, soff, 0, 0));
    hgb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rhb, soff, 0, 0));
  };
  u32x4 CG[4], CU[4], SC[2];            // one cold tile's blocks and group scales
  float cgb;                            // and its items' gate bias
  auto cold_issue = [&](int slot) {
    const bool in = slot >= 0 && slot < a.n_records;
    const uint32_t ro = in ? (uint32_t)slot * kRecBytes : kNoOffset;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      CG[b] = bload16(rr, ro + kOffGate + 16 * q, 256 * w + 64 * b);
      CU[b] = bload16(rr, ro + kOffUp + 16 * q, 256 * w + 64 * b);
    }
    // the 8 group scales around the wave's 4 (16 bytes at 2 mod 16)
    SC[0] = bload16(rr, ro + kOffScales, 16 * (w >> 1));
    SC[1] = bload16(rr, ro + kOffScales + 2 * kGroups, 16 * (w >> 1));
    cgb = __builtin_bit_cast(float,
                             __builtin_amdgcn_raw_buffer_load_b32(rcb, in ? (uint32_t)slot * 4 : kNoOffset, 0, 0));
  };
  // the first hot tile's loads go out unconditionally (a missing tile reads
  // zero): with the same loads on every path the compiler can wait for the
  // token rows alone in the prologue
  hot_issue(0, 0, kHotEarly);
  __builtin_amdgcn_sched_barrier(0);

  // prologue: sum-of-squares partials of this thread's rows, then x_n (rows
  // past M come out zero and are never read)
  if (norm_w) {
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const int m = 2 * k + hf;
      float v[16];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        v[2 * d] = half_bits_to_float((uint16_t)(xin[k][0][d] & 0xFFFFu));
        v[2 * d + 1] = half_bits_to_float((uint16_t)(xin[k][0][d] >> 16));
        v[8 + 2 * d] = half_bits_to_float((uint16_t)(xin[k][1][d] & 0xFFFFu));
        v[8 + 2 * d + 1] = half_bits_to_float((uint16_t)(xin[k][1][d] >> 16));
      }
      s_scr[m * 256 + e16] = ssq16(v);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float wf[16];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      wf[2 * d] = half_bits_to_float((uint16_t)(wn[0][d] & 0xFFFFu));
      wf[2 * d + 1] = half_bits_to_float((uint16_t)(wn[0][d] >> 16));
      wf[8 + 2 * d] = half_bits_to_float((uint16_t)(wn[1][d] & 0xFFFFu));
      wf[8 + 2 * d + 1] = half_bits_to_float((uint16_t)(wn[1][d] >> 16));
    }
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const int m = 2 * k + hf;
      // the canonical factor: lane l sums partials 4 l .. 4 l + 3, then a DPP tree
      const f32x4 pp = reinterpret_cast<const f32x4*>(s_scr + m * 256)[l];
      const float rn = rsqrtf(wave_sum((pp.x + pp.y) + (pp.z + pp.w)) * (1.0f / kH) + eps);
      u32x4 v0 = xin[k][0], v1 = xin[k][1];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float e0 = xn_exact(half_bits_to_float((uint16_t)(v0[d] & 0xFFFFu)), rn, wf[2 * d]);
        const float e1 = xn_exact(half_bits_to_float((uint16_t)(v0[d] >> 16)), rn, wf[2 * d + 1]);
        const float e2 = xn_exact(half_bits_to_float((uint16_t)(v1[d] & 0xFFFFu)), rn, wf[8 + 2 * d]);
        const float e3 = xn_exact(half_bits_to_float((uint16_t)(v1[d] >> 16)), rn, wf[8 + 2 * d + 1]);
        v0[d] = (uint32_t)float_to_half_bits(e0) | ((uint32_t)float_to_half_bits(e1) << 16);
        v1[d] = (uint32_t)float_to_half_bits(e2) | ((uint32_t)float_to_half_bits(e3) << 16);
      }
      u32x4* sx = reinterpret_cast<u32x4*>(s_x + m * kLdX + 16 * e16);
      sx[0] = v0;
      sx[1] = v1;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const int m = 2 * k + hf;
      u32x4* sx = reinterpret_cast<u32x4*>(s_x + m * kLdX + 16 * e16);
      sx[0] = xin[k][0];
      sx[1] = xin[k][1];
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  hot_issue(0, kHotEarly, 8);
  // the list's values are first used here
  asm volatile("" : "+v"(raw_total), "+v"(raw_slot));
  const int total = list ? min(raw_total, a.cap) : 0;
  const int n_items = total > g ? (total - g + kSbGroups - 1) / kSbGroups : 0;   // this workgroup's
  const int n_ct = (n_items + 15) / 16;
  int slot = list && g + kSbGroups * t < total ? raw_slot : -1;
  cold_issue(slot);
  __builtin_amdgcn_sched_barrier(0);

  const bool ta = t < M;                 // this lane's A row is a token
  const uint16_t* xa = s_x + t * kLdX + kq + 16 * q;   // hot: K kq + 64 c + 16 q + 8 s
  const uint16_t* xc = s_x + t * kLdX + kq + 32 * q;   // cold: K kq + 128 b + 32 q + 8 s
  f32x4* s_red = reinterpret_cast<f32x4*>(s_scr);      // [7][4][kWave], later [7][2][kWave]
  // one hot tile (rows t) and one cold tile (items t) of products
  auto hot_mfma = [&](f32x4& accg, f32x4& accu) {
    accg = f32x4{0.f, 0.f, 0.f, 0.f};
    accu = accg;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const h8 A = ta ? *reinterpret_cast<const h8*>(xa + 64 * c + 8 * st) : h8{};
        accg = mfma16(A, fp8x8_h8(WG[c][2 * st], WG[c][2 * st + 1]), accg);
        accu = mfma16(A, fp8x8_h8(WU[c][2 * st], WU[c][2 * st + 1]), accu);
      }
  };
  auto cold_mfma = [&](f32x4& accg, f32x4& accu) {
    accg = f32x4{0.f, 0.f, 0.f, 0.f};
    accu = accg;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 tg = {0.f, 0.f, 0.f, 0.f}, tu = tg;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        h8 A = ta ? *reinterpret_cast<const h8*>(xc + 128 * b + 8 * st) : h8{};
        A = __builtin_shufflevector(A, A, 0, 4, 1, 5, 2, 6, 3, 7);
        tg = mfma16(A, int4x8_h8(CG[b][st]), tg);
        tu = mfma16(A, int4x8_h8(CU[b][st]), tu);
      }
      // group 4 w + b of each vector: half (w & 1) of the 16 loaded bytes
      const int gi = 4 * (w & 1) + b;
      const uint32_t sg2 = SC[0][gi >> 1], su2 = SC[1][gi >> 1];
      const float sg = half_bits_to_float((uint16_t)((gi & 1) ? sg2 >> 16 : sg2 & 0xFFFFu));
      const float su = half_bits_to_float((uint16_t)((gi & 1) ? su2 >> 16 : su2 & 0xFFFFu));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        accg[e] = fmaf(sg, tg[e], accg[e]);
        accu[e] = fmaf(su, tu[e], accu[e]);
      }
    }
  };
  // wave 0's epilogue of one tile: lane column `col` of hh or hc, the value
  // if `valid`, zero if only `write`
  auto store_tile = [&](f32x4 accg, f32x4 accu, bool hot, int col, bool valid, bool write, float sg,
                        float su, float gb) {
    if (!write) return;
    uint16_t* dst = hot ? a.hh : a.hc;
    const int ld = hot ? a.ldh : a.ldc;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * q + e;
      const float h = valid ? gated_act(fmaf(accg[e], sg, gb), accu[e] * su, a.relu, a.both) : 0.f;
      dst[(size_t)m * ld + col] = float_to_half_bits(h);
    }
  };

  // the first hot tile and the first cold tile share one exchange of the 8
  // waves' sums through LDS; wave 0 adds them in wave order
  {
    f32x4 hg, hu, cg, cu;
    hot_mfma(hg, hu);
    cold_mfma(cg, cu);
    __syncthreads();
    if (w > 0) {
      s_red[((w - 1) * 4) * kWave + l] = hg;
      s_red[((w - 1) * 4 + 1) * kWave + l] = hu;
      s_red[((w - 1) * 4 + 2) * kWave + l] = cg;
      s_red[((w - 1) * 4 + 3) * kWave + l] = cu;
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int v = 0; v < 7; ++v) {
        hg += s_red[(v * 4) * kWave + l];
        hu += s_red[(v * 4 + 1) * kWave + l];
        cg += s_red[(v * 4 + 2) * kWave + l];
        cu += s_red[(v * 4 + 3) * kWave + l];
      }
      const int col = hot0 + t;
      store_tile(hg, hu, true, col, t < hr && col < a.n_hot, t < hr && col < a.ldh, hsg, hsu, hgb);
      const int it = g + kSbGroups * t;
      store_tile(cg, cu, false, it, it < total && slot >= 0 && slot < a.n_records, it < total, 1.f, 1.f, cgb);
    }
  }
  // further tiles (more than 16 rows or items per workgroup), one exchange each
  auto finish = [&](f32x4 accg, f32x4 accu, bool hot, int col, bool valid, bool write, float sg, float su,
                    float gb) {
    __syncthreads();
    if (w > 0) {
      s_red[((w - 1) * 2) * kWave + l] = accg;
      s_red[((w - 1) * 2 + 1) * kWave + l] = accu;
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int v = 0; v < 7; ++v) {
        accg += s_red[(v * 2) * kWave + l];
        accu += s_red[(v * 2 + 1) * kWave + l];
      }
      store_tile(accg, accu, hot, col, valid, write, sg, su, gb);
    }
  };
  for (int ti = 1; ti < n_ht; ++ti) {
    hot_issue(ti, 0, 8);
    f32x4 accg, accu;
    hot_mfma(accg, accu);
    const int r = 16 * ti + t, col = hot0 + r;
    finish(accg, accu, true, col, r < hr && col < a.n_hot, r < hr && col < a.ldh, hsg, hsu, hgb);
  }
  for (int ti = 1; ti < n_ct; ++ti) {
    const int it = g + kSbGroups * (16 * ti + t);
    slot = it < total ? a.dslots[it] : -1;
    cold_issue(slot);
    f32x4 accg, accu;
    cold_mfma(accg, accu);
    finish(accg, accu, false, it, it < total && slot >= 0 && slot < a.n_records, it < total, 1.f, 1.f, cgb);
  }
}

// ── down ────────────────────────────────────────────────────────────────────

// Hot half for at most 16 tokens, the last small-batch kernel: workgroup =
// 16 output rows, the 4 waves split the K blocks and meet in LDS.  Each
// wave's activation fragments (L2-resident, written by the gate/up kernel)
// are loaded before its down rows, so no load waits behind another in the
// loop.  The workgroup owns its rows outright: it adds the hot product to y
// (the cold part, or zero) and writes out = fp16(res + y) and y32.
template <int MS>
__global__ __launch_bounds__(kThreads) void k_bdown_hot_s(BDownArgs a) {
  static_assert(MS == 1, "at most 16 tokens");
  constexpr int NBmax = 8;   // ldh <= 4096: at most 32 blocks, 8 per wave
  constexpr int kPre = 16;   // cold ranges whose partial sums are loaded up front
  __shared__ f32x4 s_red[3][MS][kWave];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int h = blockIdx.x * 16 + (l & 15);
  // Every load is issued before any is used, all unconditional (past a range
  // reads zero), so each step waits only for its own: first wave 0's epilogue
  // inputs (output h, tokens 4 (l >> 4) + e: the first kPre cold ranges'
  // partial sums, the row scale, the residual), then every wave's activation
  // fragments and down rows.
  const rsrc_t rp = buf_rsrc(a.part, (uint32_t)a.n_part * kH * 16 * 4);
  const uint32_t pofs = ((uint32_t)h * 16 + 4 * (l >> 4)) * 4;
  u32x4 pv[kPre];
#pragma unroll
  for (int u = 0; u < kPre; ++u)
    pv[u] = bload16(rp, (w == 0 && u < a.n_part) ? pofs + (uint32_t)u * kH * 16 * 4 : kNoOffset, 0);
  const float sd = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 buf_rsrc(a.down_s, kH * 4), 4 * (uint32_t)h, 0, 0));
  const rsrc_t rres = buf_rsrc(a.res, a.res ? (uint32_t)a.M * kH * 2 : 0u);
  uint16_t rb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 4 * (l >> 4) + e;
    rb[e] = bload2(rres, w == 0 && t < a.M ? ((uint32_t)t * kH + h) * 2 : kNoOffset, 0);
  }
  const int nb = a.hot_blocks;
  const int b0 = w * nb / 4, b1 = (w + 1) * nb / 4;
  const int m = l & 15;
  const rsrc_t rh = buf_rsrc(a.hh, (uint32_t)a.M * a.ldh * 2);
  const uint32_t hro = m < a.M ? ((uint32_t)m * a.ldh + 32 * (l >> 4)) * 2 : kNoOffset;
  h8 A[NBmax][4];
#pragma unroll
  for (int b = 0; b < NBmax; ++b)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      A[b][s] = __builtin_bit_cast(
          h8, bload16(rh, b0 + b < b1 ? hro + ((uint32_t)(b0 + b) * kBK + 8 * s) * 2 : kNoOffset, 0));
  const rsrc_t rd = buf_rsrc(a.down_q, (uint32_t)kH * a.down_stride);
  u32x4 D[NBmax][2];
#pragma unroll
  for (int b = 0; b < NBmax; ++b) {
    const int k = (b0 + b) * kBK + 32 * (l >> 4);
    const uint32_t ro = (uint32_t)h * a.down_stride + k;
    const bool in = b0 + b < b1;
    D[b][0] = bload16(rd, (in && k < a.down_stride) ? ro : kNoOffset, 0);
    D[b][1] = bload16(rd, (in && k + 16 < a.down_stride) ? ro + 16 : kNoOffset, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // wave 0: the cold ranges' partial sums in range order (past kPre, loaded now)
  f32x4 yc = {0.f, 0.f, 0.f, 0.f};
  if (w == 0) {
#pragma unroll
    for (int u = 0; u < kPre; ++u)
      yc += f32x4{as_f32(pv[u].x), as_f32(pv[u].y), as_f32(pv[u].z), as_f32(pv[u].w)};
    for (int u = kPre; u < a.n_part; ++u) {
      const u32x4 v = bload16(rp, pofs + (uint32_t)u * kH * 16 * 4, 0);
      yc += f32x4{as_f32(v.x), as_f32(v.y), as_f32(v.z), as_f32(v.w)};
    }
  }
  // blocks past this wave's share hold zeros and add nothing
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < NBmax; ++b)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const h8 bv = fp8x8_h8(dword_of(D[b][0], D[b][1], 2 * s), dword_of(D[b][0], D[b][1], 2 * s + 1));
      acc = mfma16(A[b][s], bv, acc);
    }
  if (w > 0) s_red[w - 1][0][l] = acc;
  lds_barrier();
  if (w != 0) return;
  const f32x4 v = acc + s_red[0][0][l] + s_red[1][0][l] + s_red[2][0][l];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 4 * (l >> 4) + e;
    if (t >= a.M) continue;
    const size_t i = (size_t)t * kH + h;
    const float y = yc[e] + v[e] * sd;
    if (a.y32) a.y32[i] = y;
    if (a.out) a.out[i] = float_to_half_bits(half_bits_to_float(rb[e]) + y);
  }
}

// y = 0 over M rows.
__global__ __launch_bounds__(kThreads) void k_bfill(float* y, int n4) {
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n4; q += gridDim.x * kThreads)
    reinterpret_cast<f32x4*>(y)[q] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// out = res + y (fp16), y32 = y; y the sum in order of the n_ys partial sums
// ys[s] (M, H), the same on every run.
__global__ __launch_bounds__(kThreads) void k_bfinal(const float* ys, int n_ys, int M, const uint16_t* res,
                                                    uint16_t* out, float* y32) {
  const int n4 = M * (kH / 4);
  for (int q = blockIdx.x * kThreads + threadIdx.x; q < n4; q += gridDim.x * kThreads) {
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    {
      // four partial sums in flight per pass, added in range order
      const f32x4* yp = reinterpret_cast<const f32x4*>(ys) + q;
      int sp = 0;
      for (; sp + 4 <= n_ys; sp += 4) {
        f32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = yp[(size_t)(sp + k) * n4];
#pragma unroll
        for (int k = 0; k < 4; ++k) y += v[k];
      }
      for (; sp < n_ys; ++sp) y += yp[(size_t)sp * n4];
    }
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

// k_bfinal for one row per workgroup that also writes the next layer's
// normalised rows: xn = RMSNorm(out) with weight w (k_rmsnorm's arithmetic on
// the fp16 out, so the same bits as a norm launch after the call).  1024
// threads, thread t adding elements 4 t .. 4 t + 3 of row blockIdx.x over
// every partial sum, eight loads in flight: with 256 threads of 16 elements,
// four in flight, 64 rows (64 workgroups) took 7.0 us.  The sum of squares
// is taken as k_rmsnorm takes it (16 consecutive elements per partial, in
// order) from the fp16 outputs staged in LDS.
constexpr int kFnThreads = 1024;
__global__ __launch_bounds__(kFnThreads) void k_bfinal_norm(const float* ys, int n_ys, int M, const uint16_t* res,
                                                            uint16_t* out, float* y32, const uint16_t* w, float eps,
                                                            uint16_t* xn) {
  static_assert(kH == 4 * kFnThreads, "four elements per thread");
  __shared__ __attribute__((aligned(16))) float s_o[kH];
  __shared__ __attribute__((aligned(16))) float s_parts[kThreads];
  const int t = threadIdx.x;
  const size_t e0 = (size_t)blockIdx.x * kH + 4 * t;
  const size_t stride4 = (size_t)M * kH / 4;
  const f32x4* yp = reinterpret_cast<const f32x4*>(ys + e0);
  f32x4 y = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x2 rv = res ? *reinterpret_cast<const u32x2*>(res + e0) : u32x2{0u, 0u};
  const u32x2 wb = *reinterpret_cast<const u32x2*>(w + 4 * t);
  // the partial sums in order, as k_bfinal adds them, eight in flight
  int sp = 0;
  for (; sp + 8 <= n_ys; sp += 8) {
    f32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = yp[(size_t)(sp + k) * stride4];
#pragma unroll
    for (int k = 0; k < 8; ++k) y += v[k];
  }
  for (; sp < n_ys; ++sp) y += yp[(size_t)sp * stride4];
  if (y32) *reinterpret_cast<f32x4*>(y32 + e0) = y;
  float o[4];
  uint16_t ob[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t rb = (uint16_t)(rv[e >> 1] >> (16 * (e & 1)));
    ob[e] = float_to_half_bits(half_bits_to_float(rb) + y[e]);
    o[e] = half_bits_to_float(ob[e]);
  }
  if (out)
    *reinterpret_cast<u32x2*>(out + e0) =
        u32x2{(uint32_t)ob[0] | ((uint32_t)ob[1] << 16), (uint32_t)ob[2] | ((uint32_t)ob[3] << 16)};
  *reinterpret_cast<f32x4*>(s_o + 4 * t) = f32x4{o[0], o[1], o[2], o[3]};
  __syncthreads();
  if (t < kThreads) {
    float v16[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) v16[e] = s_o[16 * t + e];
    s_parts[t] = ssq16(v16);
  }
  __syncthreads();
  const float r = r_from_parts(s_parts, eps);
  uint16_t xb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    xb[e] = float_to_half_bits(xn_exact(o[e], r, half_bits_to_float((uint16_t)(wb[e >> 1] >> (16 * (e & 1))))));
  *reinterpret_cast<u32x2*>(xn + e0) =
      u32x2{(uint32_t)xb[0] | ((uint32_t)xb[1] << 16), (uint32_t)xb[2] | ((uint32_t)xb[3] << 16)};
}

// Up to 16 tokens without hot rows: out = res + y (fp16), y32 = y, y the sum
// in range order of the cold ranges' partial sums part[s] (H, 16).  Thread t takes output column
// t / 4 and rows 4 (t & 3) .. + 3: the four threads of a column read its 64
// bytes of each partial together.
__global__ __launch_bounds__(kThreads) void k_bfinal16(const float* part, int n_part, int M, const uint16_t* res,
                                                      uint16_t* out, float* y32) {
  const int q = blockIdx.x * kThreads + threadIdx.x;
  const int j = q >> 2, m0 = 4 * (q & 3);
  if (j >= kH) return;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  const f32x4* pp = reinterpret_cast<const f32x4*>(part + (size_t)j * 16 + m0);
  int sp = 0;
  for (; sp + 4 <= n_part; sp += 4) {
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = pp[(size_t)(sp + k) * kH * 4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y += v[k];
  }
  for (; sp < n_part; ++sp) y += pp[(size_t)sp * kH * 4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + i;
    if (m >= M) break;
    if (y32) y32[(size_t)m * kH + j] = y[i];
    if (out) {
      const float r = res ? half_bits_to_float(res[(size_t)m * kH + j]) : 0.f;
      out[(size_t)m * kH + j] = float_to_half_bits(r + y[i]);
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
  int M, Mpad, mt, ldh, hot_blocks, cap, ldc, hot_splits;
  bool prefill;
  int pms, pmt;   // prefill tiles: 32-token subtiles per tile, token tiles
  int cold_splits;   // at most 16 tokens: the cold down's item ranges
  int both_splits;   // from 17 tokens with both halves: the joint down's ranges (0: separate downs)
  size_t off_xn, off_hh, off_hc, off_dslots, off_total, off_y, off_part, bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kSkinnyMax = 16;    // token counts up to this use the one-tile split-K kernels
// token counts from this use the 128-token tile kernels (160 tokens: 3072
// against 3099 us per 32 layers on 64-token tiles; 128 tokens: 2888 against 2578)
constexpr int kPrefillMin = 160;

// hot down output tiles: 256 outputs each on the 128-token tiles, else 128
static int hot_down_tiles(int pms) { return pms == 4 ? kH / 256 : kH / 128; }

// Cold down grid: 16 output tiles x token tiles (32 tokens up to 16 tokens,
// else 128) x item ranges, about 256 workgroups; a range holds at most
// kDcMaxItems items.
static int cold_down_splits(int M, int cap) {
  const int mtc = M <= kSkinnyMax ? 1 : M < kPrefillMin ? (M + 63) / 64 : (M + 127) / 128;
  const int n_blk = (cap + kDcItems - 1) / kDcItems;
  const int min_splits = (n_blk + kDcMaxItems / kDcItems - 1) / (kDcMaxItems / kDcItems);
  return std::max(min_splits, std::min(n_blk, std::max(1, 256 / (16 * mtc))));
}

static BatchPlan batch_plan(int M, int n_hot, int cap) {
  BatchPlan p{};
  p.M = M;
  p.Mpad = (M + kBM - 1) / kBM * kBM;
  p.mt = p.Mpad / kBM;
  p.ldh = n_hot > 0 ? (n_hot + kBK - 1) / kBK * kBK : 0;
  p.hot_blocks = p.ldh / kBK;
  p.cap = cap;
  p.ldc = cap > 0 ? (cap + 127) / 128 * 128 : 0;
  p.prefill = M >= kPrefillMin;
  if (M > kSkinnyMax) {
    // 64-token tiles (k_mup and the down kernels at two 32-token subtiles)
    // below the prefill sizes, 128-token tiles from them on (measured from
    // 192 to 448 tokens, 128-token tiles are as fast or faster than 64-token
    // ones even where they leave tokens of the last tile empty: 192 tokens
    // 3011 against 3142 us per 32 layers, 320 tokens 3587 against 4822)
    p.pms = p.prefill ? 4 : 2;
    p.pmt = (M + 32 * p.pms - 1) / (32 * p.pms);
    // hot down: output tiles (128 outputs, 256 on the 128-token tiles) x token
    // tiles x K splits, about 256 workgroups
    p.hot_splits = std::max(1, std::min(p.hot_blocks, 256 / (hot_down_tiles(p.pms) * p.pmt)));
  } else {
    p.hot_splits = p.mt >= 4 ? 1 : 4 / p.mt;
  }
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
  // up to 16 tokens: y (M, H); from 17: one (M, H) partial sum per down range
  // (separate hot and cold downs, or the ranges of the joint one)
  p.both_splits = 0;
  if (M > kSkinnyMax && n_hot > 0 && cap > 0) {
    if (p.pms == 4)
      p.both_splits = std::max(p.hot_splits, cold_down_splits(M, cap));
    else
      p.both_splits = std::max(cold_down_splits(M, cap), std::min(p.hot_blocks, 256 / (16 * p.pmt)));
  }
  const int y_parts = M <= kSkinnyMax ? 1
                                      : std::max(p.both_splits, (n_hot > 0 ? p.hot_splits : 0) +
                                                                    (cap > 0 ? cold_down_splits(M, cap) : 0));
  o = align256(o + (size_t)std::max(1, y_parts) * M * kH * 4);
  p.cold_splits = (M <= kSkinnyMax && cap > 0) ? cold_down_splits(M, cap) : 0;
  p.off_part = o;
  o = align256(o + (size_t)p.cold_splits * kH * 16 * 4);
  p.bytes = o;
  return p;
}

// The current device's CU count (cached per device).
static int device_cus() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cache[dev] = c;
  }
  return cache[dev];
}

// k_mup's tiles: one token tile with more 32-neuron units than CUs makes just
// enough tiles two units wide (list items first) to run them all in one
// round; up to twice the CU count.
static MupTiles mup_tiles(const BatchPlan& p) {
  MupTiles m{};
  m.hot_units = p.ldh / kMupN;
  const int cold_units = p.ldc / kMupN, units = m.hot_units + cold_units;
  const int wide = p.pmt == 1 ? std::min(std::max(0, units - device_cus()), units / 2) : 0;
  m.wide_cold = std::min(wide, cold_units / 2);
  m.wide_hot = std::min(wide - m.wide_cold, m.hot_units / 2);
  m.n_tiles = units - m.wide_hot - m.wide_cold;
  return m;
}

size_t batch_ws_bytes(int M, int n_hot, int cap) { return batch_plan(M, n_hot, cap).bytes; }

static void launch_skinny(const BUpArgs& ua, const BDownArgs& da, bool up, const uint16_t* x,
                          const uint16_t* norm_w, float eps, hipStream_t st) {
  if (up && ua.M <= 8)
    hipLaunchKernelGGL(k_sbup<8>, dim3(kSbGroups), dim3(kSbThreads), 0, st, ua, x, norm_w, eps);
  else if (up)
    hipLaunchKernelGGL(k_sbup<16>, dim3(kSbGroups), dim3(kSbThreads), 0, st, ua, x, norm_w, eps);
  else
    hipLaunchKernelGGL(k_bdown_hot_s<1>, dim3(kH / 16), dim3(kThreads), 0, st, da);
}

int batch_ffn(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const oi2_hot* hot,
              const oi2_cold* cold, const oi2_active* active, int relu, int both, int add_residual,
              uint16_t* out, float* y32, void* workspace, size_t workspace_bytes, hipStream_t st,
              const uint16_t* xn_in, const uint16_t* next_w, float next_eps, uint16_t* xn_next) {
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

  const uint16_t* xa = xn_in ? xn_in : x;
  if (norm_w && !skinny && !xn_in) {   // the skinny gate/up kernel normalises the rows itself
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
  ua.hot_per_wg = (n_hot + kSbGroups - 1) / kSbGroups;
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

  if (skinny) {
    // gate/up, the cold down's partial sums per item range, then the hot
    // down, which adds them to its product and writes the outputs
    const int n4 = M * (kH / 4);
    const int grid = std::min(2048, (n4 + kThreads - 1) / kThreads);
    if (p.ldh + p.ldc > 0) {
      launch_skinny(ua, da, true, xa, xn_in ? nullptr : norm_w, eps, st);
    } else {
      hipLaunchKernelGGL(k_bfill, dim3(grid), dim3(kThreads), 0, st, y, n4);
    }
    OI2_CHECK_LAUNCH();
    float* part = reinterpret_cast<float*>(ws + p.off_part);
    if (has_cold) {
      da.part = part;
      da.n_part = p.cold_splits;
      hipLaunchKernelGGL((k_pgemm_down_cold<1, true>), dim3(16 * p.cold_splits), dim3(kThreads), 0, st, da, 1,
                         p.cold_splits);
      OI2_CHECK_LAUNCH();
    }
    if (n_hot) {
      da.res = add_residual ? x : nullptr;
      da.out = out;
      da.y32 = y32;
      launch_skinny(ua, da, false, x, norm_w, eps, st);
    } else if (has_cold) {   // cold only: the final add of the ranges' partial sums
      hipLaunchKernelGGL(k_bfinal16, dim3(kH * 4 / kThreads), dim3(kThreads), 0, st, part, p.cold_splits, M,
                         add_residual ? x : nullptr, out, y32);
    } else {
      hipLaunchKernelGGL(k_bfinal, dim3(grid), dim3(kThreads), 0, st, y, 1, M, add_residual ? x : nullptr, out, y32);
    }
    OI2_CHECK_LAUNCH();
    if (next_w) {   // the next layer's rows (no final launch of its own here to fold them into)
      hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(kThreads), 0, st, out, next_w, next_eps, xn_next);
      OI2_CHECK_LAUNCH();
    }
    return OI2_OK;
  }
  const int n4 = M * (kH / 4);
  int grid = (n4 + kThreads - 1) / kThreads;
  grid = grid > 2048 ? 2048 : grid;
  // the final add of the n_ys partial sums, with the next layer's rows when asked
  auto final_add = [&](int n_ys) {
    if (next_w)
      hipLaunchKernelGGL(k_bfinal_norm, dim3(M), dim3(kFnThreads), 0, st, y, n_ys, M, add_residual ? x : nullptr,
                         out, y32, next_w, next_eps, xn_next);
    else
      hipLaunchKernelGGL(k_bfinal, dim3(grid), dim3(kThreads), 0, st, y, n_ys, M, add_residual ? x : nullptr, out,
                         y32);
  };
  // each down range stores its own partial sum of y (hot ranges, then cold);
  // k_bfinal adds them in that order
  const int hot_splits = n_hot ? p.hot_splits : 0;
  const int cold_splits = has_cold ? cold_down_splits(M, cap) : 0;
  da.cold_split0 = hot_splits;
  if (p.ldh + p.ldc > 0) {
    if (p.prefill) {
      const int hot_tiles = p.ldh / 128, n_tiles = hot_tiles + p.ldc / 128;
      const dim3 grid((n_tiles + 7) / 8 * 8 * p.pmt);
      hipLaunchKernelGGL(k_pgemm_up<4>, grid, dim3(2 * kThreads), 0, st, ua, hot_tiles, n_tiles, p.pmt);
    } else {
      const MupTiles mtl = mup_tiles(p);
      const dim3 grid((mtl.n_tiles + 7) / 8 * 8 * p.pmt);
      if (mtl.wide_hot + mtl.wide_cold > 0)
        hipLaunchKernelGGL(k_mup<true>, grid, dim3(kMupThreads), 0, st, ua, mtl, p.pmt);
      else
        hipLaunchKernelGGL(k_mup<false>, grid, dim3(kMupThreads), 0, st, ua, mtl, p.pmt);
    }
    OI2_CHECK_LAUNCH();
  }
  if (n_hot && has_cold && p.both_splits > 0) {
    // one launch for both downs (128- or 64-token tiles): one partial sum per range
    const int splits = p.both_splits;
    const dim3 grid(16 * p.pmt * splits);
    if (p.pms == 4)
      hipLaunchKernelGGL((k_pgemm_down_both<4>), grid, dim3(2 * kThreads), 0, st, da, p.pmt, splits);
    else
      hipLaunchKernelGGL((k_pgemm_down_both<2>), grid, dim3(2 * kThreads), 0, st, da, p.pmt, splits);
    OI2_CHECK_LAUNCH();
    final_add(splits);
    OI2_CHECK_LAUNCH();
    return OI2_OK;
  }
  if (n_hot) {
    const dim3 grid(hot_down_tiles(p.pms) * p.pmt * p.hot_splits);
    if (p.pms == 4)
      hipLaunchKernelGGL((k_pgemm_down_hot<4, 2, 1>), grid, dim3(kThreads), 0, st, da, p.pmt, p.hot_splits);
    else
      hipLaunchKernelGGL((k_pgemm_down_hot<2, 1, 4>), grid, dim3(kThreads), 0, st, da, p.pmt, p.hot_splits);
    OI2_CHECK_LAUNCH();
  }
  if (has_cold) {
    if (p.prefill) {
      const int mtc = (M + 127) / 128;
      hipLaunchKernelGGL((k_pgemm_down_cold<4, false>), dim3(16 * mtc * cold_splits), dim3(kThreads), 0, st, da,
                         mtc, cold_splits);
    } else {
      const int mtc = (M + 63) / 64;
      hipLaunchKernelGGL((k_pgemm_down_cold<2, false>), dim3(16 * mtc * cold_splits), dim3(kThreads), 0, st, da,
                         mtc, cold_splits);
    }
    OI2_CHECK_LAUNCH();
  }
  final_add(hot_splits + cold_splits);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

}  // namespace oi2
