// oi2_ffn_forward_noalloc: the single-token decode FFN of oi2_ffn_forward
// (the same k_prep / k_ffn_up / k_ffn_down launches, token by token) for
// callers that cannot allocate device memory: code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc.  Its scratch (h_hot, the
// cold partial rows, x * w, the norm partials) is one file-scope device
// array, `scratch`, of kNoAllocBytes: room for n_hot up to 4096 and
// kNoAllocColdWG cold partial rows, which covers any list with an expected
// active count up to kNoAllocMaxExpected records.  Each GPU holds
// its own copy until the process ends.
//
// In host code `scratch` names a host-side stand-in, not the device array:
// the device address is looked up once per device with hipGetSymbolAddress
// (with that device current) and only that address is ever handed to a
// kernel.  Every call on a GPU shares that GPU's array and leaves its
// contents behind; the kernels write every scratch word before reading it,
// so nothing needs clearing between calls.  Calls that overlap on one GPU
// (concurrent streams, or threads) race on the array.
#include <mutex>

#include "capi_util.h"
#include "ffn_kernels.h"

namespace oi2 {

constexpr int kNoAllocColdWG = 256;
constexpr int kNoAllocMaxExpected = 1024;
constexpr size_t kNoAllocBytes = ffn_ws_bytes(kH, kNoAllocColdWG);   // 4,220,160 bytes
static_assert(cold_rows_bound(kNoAllocMaxExpected) <= kNoAllocColdWG,
              "the scratch holds the partial rows of every list the limit admits");
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The calling thread's current device's copy of `scratch`, looked up on the
// first call on that device.
int scratch_for_current_device(void** out) {
  int dev = -1;
  OI2_CHECK_HIP(hipGetDevice(&dev));
  OI2_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d beyond the %d this library tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    OI2_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    OI2_CHECK_ARG(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return OI2_OK;
}

}  // namespace
}  // namespace oi2

using namespace oi2;

extern "C" {

size_t oi2_ffn_noalloc_scratch_bytes(void) { return kNoAllocBytes; }

int32_t oi2_ffn_noalloc_max_expected(void) { return kNoAllocMaxExpected; }

int oi2_ffn_forward_noalloc(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                            const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active,
                            int32_t act, int32_t act_on_both, int32_t add_residual, uint16_t* out,
                            float* y32, void* stream) {
  clear_error();
  FfnCall c;
  int rc = ffn_validate(x, batch, norm_w, hot, cold, active, act, &c);
  if (rc || batch == 0) return rc;
  const int expected = active && active->expected > 0 && active->expected < c.cap ? active->expected : c.cap;
  OI2_CHECK_ARG(!c.has_cold || expected <= kNoAllocMaxExpected,
                "expected active count %d is beyond the %d records the static scratch of this "
                "entry point covers (set oi2_active.expected)",
                expected, kNoAllocMaxExpected);
  void* base = nullptr;
  rc = scratch_for_current_device(&base);
  if (rc) return rc;
  return ffn_decode_tokens(x, batch, norm_w, eps, hot, cold, active, act, act_on_both, add_residual,
                           out, y32, c, ffn_ws(base, c.n_hot, kNoAllocColdWG), (hipStream_t)stream);
}

}  // extern "C"
