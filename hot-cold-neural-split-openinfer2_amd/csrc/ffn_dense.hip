// sparse_ffn (engine.py:173-209) on dense weights, exactly as the reference
// engine calls it: the hot half as the fp16 tensors SparseFFNLayer widens its
// fp8 file to (gate/up (n_hot, H), down (H, n_hot)), the cold half as the fp32
// tensors ColdWeightStore.read_neurons returns (gate/up (n, H), down (H, n)),
// x (rows, H) fp16.  Either half may also come as fp16, bf16 or fp32.
//
//   h     = act(x G^T) * (act)(x U^T)   per half, fp32 (engine.py:163-170)
//   y     = h_hot D_hot^T + h_cold D_cold^T   fp32
//   out   = fp16(y)
//
// Two kernels per half, both HBM-bound GEMVs over the weight matrices:
//   k_dense_up   one wave per neuron row: the wave streams the gate and up
//                rows (lane l: elements 8 l + 512 k, k < 8) and dots them
//                with up to four tokens held in LDS; the activation is applied
//                in registers and h goes to the workspace.
//   k_dense_down one wave per two output rows: the rows of D (stride n, so
//                any alignment) stream through buffer loads whose range ends
//                at the matrix end; h comes through LDS in 2048-neuron chunks.
// Tokens go in passes of up to four, each pass re-reading the weights, so the
// path suits decode batches; prefill-sized batches belong on the fp8/INT4
// matrix-core path.
#include "capi_util.h"
#include "ffn_kernels.h"

namespace oi2 {
namespace {

constexpr int kDTok = 4;              // tokens per pass
constexpr int kDChunk = 2048;         // neurons of h per LDS chunk in the down kernel
constexpr int kDRowsPerWave = 2;      // output rows per wave in the down kernel

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 rload16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// 8 consecutive weights of dtype DT starting at element `e` of a matrix
// (byte offset e * size), as floats.  Past the buffer's range they read 0.
template <int DT>
__device__ __forceinline__ void load8(rsrc_t r, uint32_t e, float w[8]) {
  if constexpr (DT == OI2_DTYPE_F32) {
    const u32x4 a = rload16(r, 4 * e), b = rload16(r, 4 * e + 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      w[k] = as_f32(a[k]);
      w[4 + k] = as_f32(b[k]);
    }
  } else {
    const u32x4 a = rload16(r, 2 * e);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t d = a[k];
      if constexpr (DT == OI2_DTYPE_BF16) {
        w[2 * k] = bf16_bits_to_float((uint16_t)(d & 0xFFFFu));
        w[2 * k + 1] = bf16_bits_to_float((uint16_t)(d >> 16));
      } else {
        w[2 * k] = half_bits_to_float((uint16_t)(d & 0xFFFFu));
        w[2 * k + 1] = half_bits_to_float((uint16_t)(d >> 16));
      }
    }
  }
}

template <int DT>
constexpr uint32_t dsize() { return DT == OI2_DTYPE_F32 ? 4u : 2u; }

// The first `cnt` (< 8) of those weights one element at a time, the rest 0:
// the tail of a row whose length is not a multiple of 8, where a 16-byte
// access could reach past the end of the matrix.
template <int DT>
__device__ __forceinline__ void load_tail(rsrc_t r, uint32_t e, int cnt, float w[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v = 0.0f;
    if (i < cnt) {
      if constexpr (DT == OI2_DTYPE_F32) {
        v = as_f32(__builtin_amdgcn_raw_buffer_load_b32(r, 4 * (e + i), 0, 0));
      } else {
        const uint16_t b = __builtin_amdgcn_raw_buffer_load_b16(r, 2 * (e + i), 0, 0);
        v = DT == OI2_DTYPE_BF16 ? bf16_bits_to_float(b) : half_bits_to_float(b);
      }
    }
    w[i] = v;
  }
}

// h[t][n] = act(g) * (act(u) | u), g = x_t . G[n], u = x_t . U[n].
// Workgroup: 4 waves, one row per wave; tokens [t0, t0 + TB) of the pass.
template <int DT, int TB>
__global__ __launch_bounds__(256) void k_dense_up(const uint16_t* x, int rows, int t0,
                                                  const void* gate, const void* up, int n,
                                                  int relu, int both, float* h) {
  __shared__ u32x4 s_x[TB][kH / 8];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int row = blockIdx.x * 4 + w;
  const bool valid = row < n;
  const uint32_t nbytes = (uint32_t)n * kH * dsize<DT>();
  const rsrc_t rg = make_rsrc(gate, nbytes), ru = make_rsrc(up, nbytes);
  // the row's weights first: a lane past the last row reads zeros
  float gw[8][8], uw[8][8];
  const uint32_t rbase = valid ? (uint32_t)row * kH : (uint32_t)n * kH;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    load8<DT>(rg, rbase + 8 * (lane + 64 * k), gw[k]);
    load8<DT>(ru, rbase + 8 * (lane + 64 * k), uw[k]);
  }
  // the pass's tokens into LDS
  for (int i = threadIdx.x; i < TB * (kH / 8); i += 256) {
    const int t = i / (kH / 8), c = i % (kH / 8);
    s_x[t][c] = (t0 + t < rows) ? reinterpret_cast<const u32x4*>(x + (size_t)(t0 + t) * kH)[c]
                                : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  float pg[TB], pu[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) pg[t] = pu[t] = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const u32x4 xv = s_x[t][lane + 64 * k];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float x0 = half_bits_to_float((uint16_t)(xv[d] & 0xFFFFu));
        const float x1 = half_bits_to_float((uint16_t)(xv[d] >> 16));
        pg[t] = fmaf(gw[k][2 * d], x0, pg[t]);
        pg[t] = fmaf(gw[k][2 * d + 1], x1, pg[t]);
        pu[t] = fmaf(uw[k][2 * d], x0, pu[t]);
        pu[t] = fmaf(uw[k][2 * d + 1], x1, pu[t]);
      }
    }
  }
  wave_sums_to_last(pg);
  wave_sums_to_last(pu);
  if (valid && lane == 63) {
#pragma unroll
    for (int t = 0; t < TB; ++t)
      if (t0 + t < rows) h[(size_t)(t0 + t) * n + row] = gated_act(pg[t], pu[t], relu, both);
  }
}

// y[t][j] (+)= sum_n h[t][n] D[j][n] for the pass's tokens; with out, also
// out[t][j] = fp16(y).  Workgroup: 4 waves x 2 rows.
template <int DT, int TB>
__global__ __launch_bounds__(256) void k_dense_down(const float* h, int rows, int t0, const void* down,
                                                    int n, int accumulate, float* y32, uint16_t* out) {
  __shared__ f32x4 s_h[TB][kDChunk / 4];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int j0 = (blockIdx.x * 4 + w) * kDRowsPerWave;
  const rsrc_t rd = make_rsrc(down, (uint32_t)((size_t)kH * n * dsize<DT>()));
  float acc[kDRowsPerWave][TB];
#pragma unroll
  for (int r = 0; r < kDRowsPerWave; ++r)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[r][t] = 0.0f;
  for (int c0 = 0; c0 < n; c0 += kDChunk) {
    // this chunk's weights: lane l takes elements c0 + 8 (l + 64 k), k < 4
    float dw[kDRowsPerWave][4][8];
#pragma unroll
    for (int r = 0; r < kDRowsPerWave; ++r)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e = c0 + 8 * (lane + 64 * k);
        const uint32_t off = (uint32_t)(j0 + r) * (uint32_t)n + (uint32_t)e;
        if (e + 8 <= n)
          load8<DT>(rd, off, dw[r][k]);
        else   // the row's last elements; nothing past them (the next row's head)
          load_tail<DT>(rd, off, n - e, dw[r][k]);
      }
    __syncthreads();   // the previous chunk's h is no longer read
    for (int i = threadIdx.x; i < TB * (kDChunk / 4); i += 256) {
      const int t = i / (kDChunk / 4), c = i % (kDChunk / 4);
      const int e = c0 + 4 * c;
      f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (t0 + t < rows) {
        const float* hr = h + (size_t)(t0 + t) * n;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (e + q < n) ? hr[e + q] : 0.0f;
      }
      s_h[t][c] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        const f32x4 ha = s_h[t][2 * (lane + 64 * k)], hb = s_h[t][2 * (lane + 64 * k) + 1];
#pragma unroll
        for (int r = 0; r < kDRowsPerWave; ++r) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[r][t] = fmaf(dw[r][k][q], ha[q], acc[r][t]);
            acc[r][t] = fmaf(dw[r][k][4 + q], hb[q], acc[r][t]);
          }
        }
      }
  }
#pragma unroll
  for (int r = 0; r < kDRowsPerWave; ++r) wave_sums_to_last(acc[r]);
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < kDRowsPerWave; ++r)
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (t0 + t >= rows) continue;
        const size_t o = (size_t)(t0 + t) * kH + j0 + r;
        const float v = accumulate ? y32[o] + acc[r][t] : acc[r][t];
        y32[o] = v;
        if (out) out[o] = float_to_half_bits(v);
      }
  }
}

__global__ __launch_bounds__(256) void k_dense_zero(int rows, float* y32, uint16_t* out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < (size_t)rows * kH) {
    y32[i] = 0.0f;
    if (out) out[i] = 0;
  }
}

template <int DT, int TB>
void launch_up(const uint16_t* x, int rows, int t0, const void* g, const void* u, int n, int relu,
               int both, float* h, hipStream_t st) {
  hipLaunchKernelGGL((k_dense_up<DT, TB>), dim3((n + 3) / 4), dim3(256), 0, st, x, rows, t0, g, u, n,
                     relu, both, h);
}

template <int DT, int TB>
void launch_down(const float* h, int rows, int t0, const void* d, int n, int accumulate, float* y32,
                 uint16_t* out, hipStream_t st) {
  hipLaunchKernelGGL((k_dense_down<DT, TB>), dim3(kH / (4 * kDRowsPerWave)), dim3(256), 0, st, h, rows,
                     t0, d, n, accumulate, y32, out);
}

template <int TB>
void launch_half_tb(int dt, const uint16_t* x, int rows, int t0, const void* g, const void* u,
                    const void* d, int n, int relu, int both, float* h, int accumulate, float* y32,
                    uint16_t* out, hipStream_t st) {
  if (dt == OI2_DTYPE_F32) {
    launch_up<OI2_DTYPE_F32, TB>(x, rows, t0, g, u, n, relu, both, h, st);
    launch_down<OI2_DTYPE_F32, TB>(h, rows, t0, d, n, accumulate, y32, out, st);
  } else if (dt == OI2_DTYPE_BF16) {
    launch_up<OI2_DTYPE_BF16, TB>(x, rows, t0, g, u, n, relu, both, h, st);
    launch_down<OI2_DTYPE_BF16, TB>(h, rows, t0, d, n, accumulate, y32, out, st);
  } else {
    launch_up<OI2_DTYPE_F16, TB>(x, rows, t0, g, u, n, relu, both, h, st);
    launch_down<OI2_DTYPE_F16, TB>(h, rows, t0, d, n, accumulate, y32, out, st);
  }
}

// One half over every pass of up to four tokens.
void launch_half(int dt, const uint16_t* x, int rows, const void* g, const void* u, const void* d, int n,
                 int relu, int both, float* h, int accumulate, float* y32, uint16_t* out,
                 hipStream_t st) {
  for (int t0 = 0; t0 < rows; t0 += kDTok) {
    const int tb = rows - t0;
    if (tb >= 4)
      launch_half_tb<4>(dt, x, rows, t0, g, u, d, n, relu, both, h, accumulate, y32, out, st);
    else if (tb == 3)
      launch_half_tb<3>(dt, x, rows, t0, g, u, d, n, relu, both, h, accumulate, y32, out, st);
    else if (tb == 2)
      launch_half_tb<2>(dt, x, rows, t0, g, u, d, n, relu, both, h, accumulate, y32, out, st);
    else
      launch_half_tb<1>(dt, x, rows, t0, g, u, d, n, relu, both, h, accumulate, y32, out, st);
  }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

bool dtype_ok(int dt) { return dt == OI2_DTYPE_F32 || dt == OI2_DTYPE_BF16 || dt == OI2_DTYPE_F16; }

}  // namespace
}  // namespace oi2

using namespace oi2;

extern "C" {

size_t oi2_sparse_ffn_dense_workspace_bytes(int32_t rows, int32_t n_hot, int32_t n_cold) {
  if (rows < 0 || n_hot < 0 || n_cold < 0) return 0;
  return align256((size_t)rows * (size_t)(n_hot > n_cold ? n_hot : n_cold) * sizeof(float)) +
         align256((size_t)rows * kH * sizeof(float));
}

int oi2_sparse_ffn_dense(const uint16_t* x, int32_t rows, int32_t act, int32_t act_on_both,
                         int32_t n_hot, int32_t hot_dtype, const void* gate_hot, const void* up_hot,
                         const void* down_hot, int32_t n_cold, int32_t cold_dtype,
                         const void* gate_cold, const void* up_cold, const void* down_cold,
                         uint16_t* out, float* y32, void* workspace, size_t workspace_bytes,
                         void* stream) {
  clear_error();
  OI2_CHECK_ARG(rows >= 0 && n_hot >= 0 && n_cold >= 0, "negative size");
  OI2_CHECK_ARG(act == OI2_ACT_SILU || act == OI2_ACT_RELU, "act %d is not OI2_ACT_*", act);
  if (rows == 0) return OI2_OK;
  OI2_CHECK_ARG(x && (uintptr_t)x % 16 == 0, "x must be non-null and 16-byte aligned");
  OI2_CHECK_ARG(out || y32, "both outputs are null");
  OI2_CHECK_ARG(!out || (uintptr_t)out % 2 == 0, "out must be 2-byte aligned");
  // the buffer loads address each matrix with 32-bit byte offsets
  const size_t lim = (size_t)1 << 31;
  if (n_hot > 0) {
    OI2_CHECK_ARG(dtype_ok(hot_dtype), "hot_dtype %d is not OI2_DTYPE_F16, _F32 or _BF16", hot_dtype);
    OI2_CHECK_ARG(gate_hot && up_hot && down_hot, "hot weights are null");
    OI2_CHECK_ARG((uintptr_t)gate_hot % 16 == 0 && (uintptr_t)up_hot % 16 == 0,
                  "hot gate/up must be 16-byte aligned");
    OI2_CHECK_ARG((size_t)n_hot * kH * (hot_dtype == OI2_DTYPE_F32 ? 4 : 2) < lim,
                  "hot half too large (%d neurons)", n_hot);
  }
  if (n_cold > 0) {
    OI2_CHECK_ARG(dtype_ok(cold_dtype), "cold_dtype %d is not OI2_DTYPE_F16, _F32 or _BF16",
                  cold_dtype);
    OI2_CHECK_ARG(gate_cold && up_cold && down_cold, "cold weights are null");
    OI2_CHECK_ARG((uintptr_t)gate_cold % 16 == 0 && (uintptr_t)up_cold % 16 == 0,
                  "cold gate/up must be 16-byte aligned");
    OI2_CHECK_ARG((size_t)n_cold * kH * (cold_dtype == OI2_DTYPE_F32 ? 4 : 2) < lim,
                  "cold half too large (%d neurons)", n_cold);
  }
  const size_t need = oi2_sparse_ffn_dense_workspace_bytes(rows, n_hot, n_cold);
  OI2_CHECK_ARG(workspace && workspace_bytes >= need, "workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  float* h = reinterpret_cast<float*>(ws);
  float* y = y32 ? y32
                 : reinterpret_cast<float*>(ws + align256((size_t)rows *
                                                          (size_t)(n_hot > n_cold ? n_hot : n_cold) * 4));
  const int relu = act == OI2_ACT_RELU, both = act_on_both ? 1 : 0;
  if (n_hot == 0 && n_cold == 0) {   // engine.py:207-208: zeros
    const size_t m = (size_t)rows * kH;
    hipLaunchKernelGGL(k_dense_zero, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, rows, y, out);
    OI2_CHECK_LAUNCH();
    return OI2_OK;
  }
  if (n_hot > 0) {
    launch_half(hot_dtype, x, rows, gate_hot, up_hot, down_hot, n_hot, relu, both, h, 0, y,
                n_cold > 0 ? nullptr : out, st);
    OI2_CHECK_LAUNCH();
  }
  if (n_cold > 0) {
    launch_half(cold_dtype, x, rows, gate_cold, up_cold, down_cold, n_cold, relu, both, h,
                n_hot > 0 ? 1 : 0, y, out, st);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

}  // extern "C"
