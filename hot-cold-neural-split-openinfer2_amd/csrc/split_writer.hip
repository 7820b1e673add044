// Device split writer: the cold half of split_dense's per-layer loop
// (splitter.py:229-256) with quantize_int4 (splitter.py:81-108), producing the
// byte image of one section of cold_weights.bin in device memory.
//
// quantize_int4 per 128-element group g of a vector:
//   s = max(max|g|, 1e-8) / 7                        (fp32, correctly rounded)
//   q = clamp(round_half_even(g / s), -8, 7)         (fp32 divide, then rint)
//   nibbles: element 2k low, 2k + 1 high; scale stored as fp16 (RNE)
// Section: 16-byte header <HHIq (layer, expert, n_cold, 0), n_cold records
// of 6400 bytes, zero padding to a 4096-byte multiple.  Record: u16 nid, gate,
// up and down nibbles (2048 B each), gate/up/down scales (32 fp16 each), zero
// padding from byte 6338.
#include "capi_util.h"
#include "ffn_kernels.h"

namespace oi2 {

namespace {

constexpr int kPage = 4096;
constexpr int kHeader = 16;
constexpr int kRawRecord = kOffScales + 3 * kGroups * 2;   // 6338

struct QuantArgs {
  const float* src[3];        // gate, up, down
  int64_t row_stride[3];      // elements between consecutive source rows
  int64_t elem_stride[3];     // elements between consecutive vector elements
  const uint16_t* nids;
  const int32_t* rows;        // source row of record k
  int n;
  uint8_t* records;           // record k at records + 6400 k
};

// One workgroup per (record k = blockIdx.x, vector m = blockIdx.y): thread t
// quantises elements 16 t .. 16 t + 15, i.e. one eighth of group t / 8.
__global__ __launch_bounds__(kThreads) void k_quantize_records(QuantArgs a) {
  const int k = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int64_t es = a.elem_stride[m];
  const float* v = a.src[m] + (int64_t)a.rows[k] * a.row_stride[m] + (int64_t)(16 * t) * es;
  float x[16];
  if (es == 1 && (reinterpret_cast<uintptr_t>(v) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 q = reinterpret_cast<const f32x4*>(v)[i];
      x[4 * i] = q.x;
      x[4 * i + 1] = q.y;
      x[4 * i + 2] = q.z;
      x[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = v[i * es];
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
  // the 8 threads of a group are consecutive lanes
  amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
  amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
  amax = fmaxf(amax, __shfl_xor(amax, 4, kWave));
  const float s = __fdiv_rn(fmaxf(amax, 1e-8f), 7.0f);

  uint8_t* rec = a.records + (size_t)k * kRecBytes;
  uint16_t* out = reinterpret_cast<uint16_t*>(rec + kOffGate + m * (kH / 2) + 8 * t);   // 2-byte aligned
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t half = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float r = __builtin_rintf(__fdiv_rn(x[4 * p + j], s));
      const int q = (int)fminf(fmaxf(r, -8.0f), 7.0f);
      half |= (uint32_t)(q & 0xF) << (4 * j);
    }
    out[p] = (uint16_t)half;
  }
  if ((t & 7) == 0)
    reinterpret_cast<uint16_t*>(rec + kOffScales + m * kGroups * 2)[t >> 3] = float_to_half_bits(s);
  if (m == 0) {
    if (t == 0) reinterpret_cast<uint16_t*>(rec)[0] = a.nids[k];
    if (t < (kRecBytes - kRawRecord) / 2) reinterpret_cast<uint16_t*>(rec + kRawRecord)[t] = 0;
  }
}

// Header and trailing zero padding of a section with n records.
__global__ __launch_bounds__(kThreads) void k_section_frame(uint8_t* section, int layer, int expert, int n,
                                                            size_t body, size_t total) {
  const int t = threadIdx.x;
  if (t == 0) {
    uint32_t* h = reinterpret_cast<uint32_t*>(section);
    h[0] = (uint32_t)(layer & 0xFFFF) | ((uint32_t)(expert & 0xFFFF) << 16);
    h[1] = (uint32_t)n;
    h[2] = 0;
    h[3] = 0;
  }
  for (size_t i = body + t; i < total; i += kThreads) section[i] = 0;
}

size_t section_bytes(int64_t n) {
  const size_t body = kHeader + (size_t)n * kRecBytes;
  return (body + kPage - 1) / kPage * kPage;
}

}  // namespace

}  // namespace oi2

using namespace oi2;

extern "C" size_t oi2_section_bytes(int32_t n_cold) { return n_cold < 0 ? 0 : section_bytes(n_cold); }

extern "C" int oi2_quantize_section(int32_t layer, int32_t expert, int32_t n, const uint16_t* nids,
                                    const int32_t* rows, const float* gate, const float* up,
                                    const float* down, const int64_t* row_stride,
                                    const int64_t* elem_stride, uint8_t* section,
                                    size_t section_bytes_, void* stream) {
  OI2_CHECK_ARG(n >= 0, "n must be non-negative, got %d", n);
  OI2_CHECK_ARG(layer >= 0 && layer <= 0xFFFF && expert >= 0 && expert <= 0xFFFF,
                "layer and expert must fit the header's u16 fields");
  OI2_CHECK_ARG(section && (uintptr_t)section % 16 == 0, "section must be 16-byte aligned device memory");
  const size_t need = section_bytes(n);
  OI2_CHECK_ARG(section_bytes_ >= need, "section buffer of %zu bytes is smaller than the %zu required",
                section_bytes_, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n > 0) {
    OI2_CHECK_ARG(nids && rows && gate && up && down && row_stride && elem_stride,
                  "nids, rows, gate, up, down and the strides are required");
    QuantArgs a{};
    a.src[0] = gate;
    a.src[1] = up;
    a.src[2] = down;
    for (int m = 0; m < 3; ++m) {
      OI2_CHECK_ARG(row_stride[m] >= 0 && elem_stride[m] >= 1, "strides must be non-negative (element: >= 1)");
      a.row_stride[m] = row_stride[m];
      a.elem_stride[m] = elem_stride[m];
    }
    a.nids = nids;
    a.rows = rows;
    a.n = n;
    a.records = section + kHeader;
    hipLaunchKernelGGL(k_quantize_records, dim3(n, 3), dim3(kThreads), 0, st, a);
    OI2_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(k_section_frame, dim3(1), dim3(kThreads), 0, st, section, layer, expert, n,
                     (size_t)kHeader + (size_t)n * kRecBytes, need);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}
