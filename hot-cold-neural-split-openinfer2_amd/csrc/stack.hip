// FFN-only decode stack: DesdemonaEngine.forward's layer loop (engine.py:421-438)
// restricted to the FFN sublayers, batch 1, entirely on device.
//
// Per token: layer 0's active set is predicted from the input (engine.py:422),
// then for each layer L two launches:
//   ffn_up(L)   hot + cold gate/up of layer L, and the down projection of
//               layer L+1's predictor on RMSNorm_{L+1}(x_L) (the lookahead,
//               engine.py:432-436)
//   ffn_down(L) x_{L+1} = x_L + FFN_L, and layer L+1's logits, threshold and
//               compacted active set
// so there is no host synchronisation inside a token.  The launch sequence
// is captured once into a hipGraph per (x_in, x_out, stream) and replayed.
#include <algorithm>
#include <string>
#include <vector>

#include "capi_util.h"
#include "ffn_kernels.h"

namespace oi2 {

struct StackLayer {
  oi2_layer l;
  bool has_pred;
  int32_t* all_slots = nullptr;   // device: every record slot, for layers without a predictor
  int32_t* all_count = nullptr;   // device: one int
  int n_all = 0;
};

}  // namespace oi2

struct oi2_stack {
  std::vector<oi2::StackLayer> layers;
  int n_layers = 0, inter = 0, n_chunks = 0, relu = 0, both = 0, max_hot = 0, max_rank = 0;
  float eps = 0.0f, thr = 0.0f;
  uint16_t* xbuf = nullptr;      // (n_layers, H): output of each layer
  uint16_t* xw = nullptr;        // (H) fp16 x * w of the layer about to run
  float* ssq = nullptr;          // 256 sum-of-squares partials of that x
  float* h_hot = nullptr;
  float* cold_part = nullptr;    // (kMaxColdWG, H) partial rows of the current layer
  int cold_cap = 0;
  double* z = nullptr;
  int32_t* sel_counts = nullptr; // (n_layers, n_chunks)
  int32_t* sel_slots = nullptr;  // (n_layers, n_chunks * 256)
  int32_t* sel_ids = nullptr;
  int cold_wg = 1;
  int cold_wpc = 1;
  bool use_graph = true;
  // staging: each layer's active records are copied one layer ahead, on a
  // side stream, from their source (device or pinned host memory) into one
  // of two HBM buffers, and the FFN reads them there
  bool staged = false;
  int copy_wg = 0;                           // workgroups of the staging copy kernel
  hipStream_t side = nullptr;
  hipStream_t own = nullptr;                 // runs a staged token asked for on the NULL stream
  uint8_t* stage[2] = {nullptr, nullptr};
  std::vector<const uint8_t*> src;           // per layer: device-visible address of the records
  uint32_t* stage_sync = nullptr;            // sel / ready counters and the error word
  oi2::StageLayer* stage_tab = nullptr;      // per layer: what the copy kernel stages
  uint32_t stage_spin = 1u << 20;            // poll bound of the staged waits
  hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_null_in = nullptr, ev_null_out = nullptr;
  struct GraphEntry {
    hipGraphExec_t exec;
    const void* in;
    void* out;
    hipStream_t stream;
  };
  std::vector<GraphEntry> graphs;   // small cache keyed by (x_in, x_out, stream)
  // persistent token kernel: its own active lists (kTokChunks chunks of
  // tok_chunk ids per layer), signal area and cold activations
  bool tok_ok = false;       // this configuration supports it
  bool tok = false;          // decodes use it (when not staged)
  std::string tok_why;
  int tok_npw = 0, tok_chunk = 0;
  oi2::TokLayer* tok_layers = nullptr;
  uint32_t* tok_sync = nullptr;
  uint32_t tok_spin = 1u << 20;       // poll bound of the kernel's device-wide waits
  uint16_t* tok_xw = nullptr;    // one slice per layer of everything the launch writes
  float* tok_ssq = nullptr;
  float* tok_h = nullptr;
  double* tok_z = nullptr;
  float* tok_cpart = nullptr;
  int32_t* tok_sel_counts = nullptr;
  int32_t* tok_sel_slots = nullptr;
  int32_t* tok_sel_ids = nullptr;
  std::vector<int32_t*> tok_static;   // all-record lists of layers without a predictor
};

namespace oi2 {


// Launch arguments of layer L's two kernels.  x_in is the token entering the
// stack and x_out the buffer that receives the last layer's output.
static ActiveList layer_list(const oi2_stack* s, int L) {
  const StackLayer& SL = s->layers[L];
  if (SL.has_pred)
    return ActiveList{s->sel_slots + (size_t)L * s->n_chunks * kSelChunk,
                      s->sel_counts + (size_t)L * s->n_chunks, s->n_chunks, kSelChunk};
  return ActiveList{SL.all_slots, SL.all_count, 1, SL.n_all};
}

static void layer_args(const oi2_stack* s, int L, const uint16_t* x_in, uint16_t* x_out,
                       UpArgs& ua, DownArgs& da) {
  const int n = s->n_layers;
  const size_t sel_stride = (size_t)s->n_chunks * kSelChunk;
  const StackLayer& SL = s->layers[L];
  const oi2_layer& l = SL.l;
  // staged: the next layer's predictor runs in its own launches, ahead of
  // this layer's FFN, so its selection can start the next copy early
  const bool pred_next = (L + 1 < n) && s->layers[L + 1].has_pred && !s->staged;
  const uint16_t* xl = (L == 0) ? x_in : s->xbuf + (size_t)(L - 1) * kH;

  ua = UpArgs{};
  ua.tok = TokenIn{xl, s->xw, s->ssq, s->eps, 1};
  ua.relu = s->relu;
  ua.both = s->both;
  ua.n_hot = l.hot.n_hot;
  ua.gate_q = l.hot.gate_q;
  ua.up_q = l.hot.up_q;
  ua.gate_s = l.hot.gate_scale;
  ua.up_s = l.hot.up_scale;
  ua.hot_gbias = l.hot.gate_bias;
  ua.h_hot = s->h_hot;
  const bool has_cold = l.cold.n_records > 0;
  if (has_cold) {
    ua.cold_gbias = l.cold.gate_bias;
    ua.act = layer_list(s, L);
    if (s->staged) {
      ua.records = s->stage[L & 1];
      ua.n_records = s->cold_cap;
      ua.act.slots = nullptr;
      ua.stage_ready = s->stage_sync + stage_ready_word(L);
      ua.stage_target = (uint32_t)s->copy_wg;   // one arrival per copy workgroup
      ua.stage_err = s->stage_sync + stage_err_word(n);
      ua.stage_spin = s->stage_spin;
      ua.stage_src = s->src[L];
      ua.stage_src_n = l.cold.n_records;
      ua.stage_slots = layer_list(s, L).slots;
    } else {
      ua.records = s->src[L];
      ua.n_records = l.cold.n_records;
    }
    ua.cold_part = s->cold_part;
    const ColdSplit cs = SL.has_pred ? ColdSplit{s->cold_wpc, s->cold_wg} : cold_split(1, SL.n_all);
    ua.cold_wpc = cs.wpc;
    ua.wg_cold = cs.wg;
  }
  ua.wg_hot = (l.hot.n_hot + 7) / 8;
  if (pred_next) {
    const oi2_layer& ln = s->layers[L + 1].l;
    ua.pd_w = ln.pred.down_w;
    ua.pd_rank = ln.pred.rank;
    ua.pd_bf16 = ln.pred.dtype == OI2_DTYPE_BF16;
    ua.pd_norm_w = ln.norm_w;
    ua.pd_z = s->z;
    ua.wg_pred = (ln.pred.rank + 3) / 4;
  }

  da = DownArgs{};
  da.res = xl;
  da.h_hot = s->h_hot;
  da.n_hot = l.hot.n_hot;
  da.down_stride = l.hot.down_stride;
  da.down_q = l.hot.down_q;
  da.down_s = l.hot.down_scale;
  if (has_cold) {
    da.cold_part = s->cold_part;
    da.cold_wg = ua.wg_cold;
  }
  da.out = s->xbuf + (size_t)L * kH;
  da.out2 = (L == n - 1) ? x_out : nullptr;
  if (L + 1 < n) {
    da.next_norm_w = s->layers[L + 1].l.norm_w;
    da.xw_out = s->xw;
    da.ssq_out = s->ssq;
  }
  if (pred_next) {
    const oi2_layer& ln = s->layers[L + 1].l;
    da.pu_w = ln.pred.up_w;
    da.pu_b = ln.pred.up_b;
    da.pu_rank = ln.pred.rank;
    da.pu_bf16 = ln.pred.dtype == OI2_DTYPE_BF16;
    da.inter = ln.pred.inter;
    da.pd_z = s->z;
    da.thr = s->thr;
    da.lut = ln.lut;
    da.sel_slots = s->sel_slots + (size_t)(L + 1) * sel_stride;
    da.sel_ids = s->sel_ids + (size_t)(L + 1) * sel_stride;
    da.sel_counts = s->sel_counts + (size_t)(L + 1) * s->n_chunks;
    da.wg_pred = s->n_chunks;
  }
  da.wg_down = kDownWG;
}

static int launch_up(const UpArgs& ua, hipStream_t st) {
  const int grid = ua.wg_cold + ua.wg_pred + ua.wg_hot;
  if (grid > 0) {
    hipLaunchKernelGGL(k_ffn_up, dim3(grid), dim3(kThreads), 0, st, ua);
    OI2_CHECK_LAUNCH();
  }
  return OI2_OK;
}

static int launch_down(const DownArgs& da, hipStream_t st) {
  hipLaunchKernelGGL(k_ffn_down, dim3(da.wg_pred + da.wg_down), dim3(kThreads), 0, st, da);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

// Layer P's predictor on x (its RMSNorm from the shared sum-of-squares
// partials of x): logits, threshold and the compacted active set sel[P].
static int launch_predictor(oi2_stack* s, int P, const uint16_t* x, hipStream_t st) {
  const oi2_layer& lp = s->layers[P].l;
  const size_t sel_stride = (size_t)s->n_chunks * kSelChunk;
  UpArgs ua{};
  ua.tok = TokenIn{x, s->xw, s->ssq, s->eps, 1};
  ua.pd_w = lp.pred.down_w;
  ua.pd_rank = lp.pred.rank;
  ua.pd_bf16 = lp.pred.dtype == OI2_DTYPE_BF16;
  ua.pd_norm_w = lp.norm_w;
  ua.pd_z = s->z;
  ua.wg_pred = (lp.pred.rank + 3) / 4;
  hipLaunchKernelGGL(k_pred_up, dim3(ua.wg_pred), dim3(kThreads), 0, st, ua);
  OI2_CHECK_LAUNCH();
  DownArgs da{};
  da.pu_w = lp.pred.up_w;
  da.pu_b = lp.pred.up_b;
  da.pu_rank = lp.pred.rank;
  da.pu_bf16 = lp.pred.dtype == OI2_DTYPE_BF16;
  da.inter = lp.pred.inter;
  da.pd_z = s->z;
  da.thr = s->thr;
  da.lut = lp.lut;
  da.sel_slots = s->sel_slots + (size_t)P * sel_stride;
  da.sel_ids = s->sel_ids + (size_t)P * sel_stride;
  da.sel_counts = s->sel_counts + (size_t)P * s->n_chunks;
  da.sel_flag = s->staged ? s->stage_sync + stage_sel_word(P) : nullptr;
  da.wg_pred = s->n_chunks;
  hipLaunchKernelGGL(k_pred_down, dim3(da.wg_pred), dim3(kThreads), 0, st, da);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

// Staged decode: layer P's list is complete (its predictor's selection
// workgroups signal that themselves; a layer without one is signalled here,
// at the point of the main stream where its predictor would run).
static int launch_selection(oi2_stack* s, int P, const uint16_t* x, hipStream_t st) {
  if (s->layers[P].has_pred) return launch_predictor(s, P, x, st);
  hipLaunchKernelGGL(k_stage_signal, dim3(1), dim3(64), 0, st, s->stage_sync + stage_sel_word(P));
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

static StageArgs stage_args(const oi2_stack* s, int L) {
  StageArgs g{};
  g.src = s->src[L];
  g.n_records = s->layers[L].l.cold.n_records;
  g.act = layer_list(s, L);
  g.cap = s->cold_cap;
  g.dst = s->stage[L & 1];
  return g;
}

static int launch_gather(const oi2_stack* s, int L, hipStream_t st) {
  if (s->layers[L].l.cold.n_records == 0) return OI2_OK;
  const StageArgs g = stage_args(s, L);
  hipLaunchKernelGGL(k_stage_gather, dim3(s->copy_wg), dim3(kThreads), 0, st, g);
  OI2_CHECK_LAUNCH();
  return OI2_OK;
}

static inline const uint16_t* layer_input(const oi2_stack* s, int L, const uint16_t* x_in) {
  return L == 0 ? x_in : s->xbuf + (size_t)(L - 1) * kH;
}

// Staged token.  Main stream: clear the signal counters, then
// selection(L+1) on x_L ahead of FFN(L) for every layer; FFN(L)'s cold
// workgroups wait on the device until layer L's records are staged.  Side
// stream: one k_stage_copy for the whole token, which copies each layer's
// records as soon as its selection is signalled.  The two streams meet once
// at the start of the token and once at its end; everything in between is
// ordered by device-side signals with bounded waits.
static int stack_launch_staged_on(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st);

static int stack_launch_staged(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st) {
  if (st != nullptr) return stack_launch_staged_on(s, x_in, x_out, st);
  // On the NULL stream the token runs on the stack's own stream, ordered
  // after the NULL stream's earlier work and before its later work: the
  // NULL stream's implicit synchronisation with other streams must not come
  // between the two streams that signal each other.
  OI2_CHECK_HIP(hipEventRecord(s->ev_null_in, nullptr));
  OI2_CHECK_HIP(hipStreamWaitEvent(s->own, s->ev_null_in, 0));
  int rc = stack_launch_staged_on(s, x_in, x_out, s->own);
  if (rc) return rc;
  OI2_CHECK_HIP(hipEventRecord(s->ev_null_out, s->own));
  OI2_CHECK_HIP(hipStreamWaitEvent(nullptr, s->ev_null_out, 0));
  return OI2_OK;
}

static int stack_launch_staged_on(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st) {
  const int n = s->n_layers;
  // the counters start at zero every token; the error word is kept until
  // oi2_stack_status reports it
  hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(kThreads), 0, st, s->stage_sync,
                     stage_err_word(n), 0u);
  OI2_CHECK_LAUNCH();
  hipLaunchKernelGGL(k_prep, dim3(1), dim3(kThreads), 0, st, x_in, s->layers[0].l.norm_w, s->xw,
                     s->ssq);
  OI2_CHECK_LAUNCH();
  OI2_CHECK_HIP(hipEventRecord(s->ev_fork, st));
  OI2_CHECK_HIP(hipStreamWaitEvent(s->side, s->ev_fork, 0));
  StageCopyArgs ca{};
  ca.layers = s->stage_tab;
  ca.n_layers = n;
  ca.cap = s->cold_cap;
  ca.sync = s->stage_sync;
  ca.spin = s->stage_spin;
  hipLaunchKernelGGL(k_stage_copy, dim3(s->copy_wg), dim3(kThreads), 0, s->side, ca);
  OI2_CHECK_LAUNCH();
  int rc = launch_selection(s, 0, x_in, st);
  if (rc) return rc;
  for (int L = 0; L < n; ++L) {
    if (L + 1 < n && (rc = launch_selection(s, L + 1, layer_input(s, L, x_in), st))) return rc;
    UpArgs ua;
    DownArgs da;
    layer_args(s, L, x_in, x_out, ua, da);
    if ((rc = launch_up(ua, st)) || (rc = launch_down(da, st))) return rc;
  }
  OI2_CHECK_HIP(hipEventRecord(s->ev_join, s->side));
  OI2_CHECK_HIP(hipStreamWaitEvent(st, s->ev_join, 0));
  return OI2_OK;
}

static inline bool use_tok(const oi2_stack* s) { return s->tok && s->tok_ok && !s->staged; }

static TokArgs tok_args(const oi2_stack* s, const uint16_t* x_in, uint16_t* x_out) {
  TokArgs a{};
  a.layers = s->tok_layers;
  a.n_layers = s->n_layers;
  a.x_in = x_in;
  a.x_out = x_out;
  a.xbuf = s->xbuf;
  a.xw = s->tok_xw;
  a.ssq = s->tok_ssq;
  a.h = s->tok_h;
  a.z = s->tok_z;
  a.cpart = s->tok_cpart;
  a.sync = s->tok_sync;
  a.spin = s->tok_spin;
  a.eps = s->eps;
  a.thr = s->thr;
  a.relu = s->relu;
  a.both = s->both;
  return a;
}

// The token as one persistent launch (it computes layer 0's x * w and
// sum-of-squares partials itself, and its signal words need no clearing).
static int stack_launch_tok(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st) {
  return tok_launch(tok_args(s, x_in, x_out), s->tok_npw, st);
}

// The two-launch-per-layer sequence (or the staged one).
static int stack_launch_layers(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st) {
  if (s->staged) return stack_launch_staged(s, x_in, x_out, st);
  hipLaunchKernelGGL(k_prep, dim3(1), dim3(kThreads), 0, st, x_in, s->layers[0].l.norm_w, s->xw,
                     s->ssq);
  OI2_CHECK_LAUNCH();
  // layer 0's active set from the token itself
  if (s->layers[0].has_pred) {
    int rc = launch_predictor(s, 0, x_in, st);
    if (rc) return rc;
  }
  for (int L = 0; L < s->n_layers; ++L) {
    UpArgs ua;
    DownArgs da;
    layer_args(s, L, x_in, x_out, ua, da);
    int rc = launch_up(ua, st);
    if (rc == OI2_OK) rc = launch_down(da, st);
    if (rc) return rc;
  }
  return OI2_OK;
}

static int stack_launch(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, hipStream_t st) {
  return use_tok(s) ? stack_launch_tok(s, x_in, x_out, st) : stack_launch_layers(s, x_in, x_out, st);
}

// Device-visible address of a record array: device memory as is, pinned host
// memory through its mapping.  Anything else (pageable memory) is rejected,
// since a kernel reading it would fault.
static int device_view(const uint8_t* p, const uint8_t** out) {
  hipPointerAttribute_t at{};
  if (hipPointerGetAttributes(&at, p) != hipSuccess ||
      (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeHost)) {
    (void)hipGetLastError();
    return OI2_EINVAL;
  }
  if (at.type == hipMemoryTypeHost) {
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, (void*)p, 0) != hipSuccess || !dp) {
      (void)hipGetLastError();
      return OI2_EINVAL;
    }
    p = (const uint8_t*)dp;
  }
  *out = p;
  return OI2_OK;
}

static void staging_free(oi2_stack* s) {
  if (s->own) (void)hipStreamDestroy(s->own);
  s->own = nullptr;
  for (auto* e : {&s->ev_fork, &s->ev_join, &s->ev_null_in, &s->ev_null_out}) {
    if (*e) (void)hipEventDestroy(*e);
    *e = nullptr;
  }
  for (auto& b : s->stage) {
    if (b) (void)hipFree(b);
    b = nullptr;
  }
  if (s->stage_sync) (void)hipFree(s->stage_sync);
  if (s->stage_tab) (void)hipFree(s->stage_tab);
  s->stage_sync = nullptr;
  s->stage_tab = nullptr;
  if (s->side) (void)hipStreamDestroy(s->side);
  s->side = nullptr;
  s->staged = false;
}

static void stack_free(oi2_stack* s) {
  staging_free(s);
  for (auto& L : s->layers) {
    if (L.all_slots) (void)hipFree(L.all_slots);
    if (L.all_count) (void)hipFree(L.all_count);
  }
  for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.exec);
  s->graphs.clear();
  for (int32_t* p : s->tok_static)
    if (p) (void)hipFree(p);
  s->tok_static.clear();
  for (void* p : {(void*)s->tok_layers, (void*)s->tok_sync, (void*)s->tok_xw, (void*)s->tok_ssq,
                  (void*)s->tok_h, (void*)s->tok_z, (void*)s->tok_sel_counts,
                  (void*)s->tok_sel_slots, (void*)s->tok_sel_ids, (void*)s->tok_cpart})
    if (p) (void)hipFree(p);
  for (void* p : {(void*)s->xbuf, (void*)s->xw, (void*)s->ssq, (void*)s->h_hot, (void*)s->cold_part,
                  (void*)s->z, (void*)s->sel_counts,
                  (void*)s->sel_slots, (void*)s->sel_ids})
    if (p) (void)hipFree(p);
}

// Decide whether the persistent token kernel can run this stack and, if so,
// allocate its buffers and build the device-resident layer table.  An
// unsupported configuration is not an error (tok_why says why); an
// allocation failure is.
static int tok_setup(oi2_stack* s) {
  s->tok_ok = false;
  s->tok = false;
  char why[160] = {0};
  const int n = s->n_layers;
  const int chunk = (s->inter + kTokChunks - 1) / kTokChunks;
  int max_hot = 0, max_rank = 0;
  for (int L = 0; L < n && !why[0]; ++L) {
    const StackLayer& SL = s->layers[L];
    const oi2_layer& l = SL.l;
    max_hot = std::max(max_hot, l.hot.n_hot);
    if (l.hot.n_hot > kTokMaxHot) snprintf(why, sizeof why, "layer %d: n_hot %d > %d", L, l.hot.n_hot, kTokMaxHot);
    if (SL.has_pred) {
      max_rank = std::max(max_rank, l.pred.rank);
      if (l.pred.dtype != OI2_DTYPE_BF16 || l.pred.rank > kTokMaxRank)
        snprintf(why, sizeof why, "layer %d: the predictor is not bf16 of rank <= %d", L, kTokMaxRank);
    }
    if (l.cold.n_records > 0) {
      hipPointerAttribute_t at{};
      if (hipPointerGetAttributes(&at, l.cold.records) != hipSuccess || at.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        snprintf(why, sizeof why, "layer %d: cold records are not in device memory", L);
      }
    }
  }
  const int npw = max_hot <= 2 * kTokWorkers * kTokGroups ? 2 : 3;   // hot neurons per worker wave
  if (!why[0] && chunk > kTokMaxChunk)
    snprintf(why, sizeof why, "inter %d > %d", s->inter, kTokChunks * kTokMaxChunk);
  int resident = 0;
  if (!why[0] && tok_resident(npw, &resident) != OI2_OK) return OI2_EHIP;
  if (!why[0] && resident < kTokGroups)
    snprintf(why, sizeof why, "the device holds %d of the %d workgroups at once", resident, kTokGroups);
  if (why[0]) {
    s->tok_why = why;
    return OI2_OK;
  }
  hipError_t e = hipSuccess;
  auto alloc = [&](void** p, size_t bytes) {
    if (e == hipSuccess) e = hipMalloc(p, bytes);
  };
  const size_t sel = (size_t)n * kTokChunks * chunk;
  alloc((void**)&s->tok_layers, (size_t)n * sizeof(TokLayer));
  alloc((void**)&s->tok_sync, (size_t)kTokSyncWords * 4);
  alloc((void**)&s->tok_xw, (size_t)n * kH * 2);
  alloc((void**)&s->tok_ssq, (size_t)n * kTokGroups * 4);
  alloc((void**)&s->tok_h, (size_t)n * kTokMaxHot * 4);
  alloc((void**)&s->tok_z, (size_t)n * 4 * kTokMaxRank * sizeof(double));
  alloc((void**)&s->tok_cpart, (size_t)n * kTokGroups * kH * 4);
  alloc((void**)&s->tok_sel_counts, (size_t)n * kTokChunks * 4);
  alloc((void**)&s->tok_sel_slots, sel * 4);
  alloc((void**)&s->tok_sel_ids, sel * 4);
  if (e == hipSuccess) e = hipMemset(s->tok_sel_counts, 0, (size_t)n * kTokChunks * 4);
  // h slices past n_hot are never written and must read as zero
  if (e == hipSuccess) e = hipMemset(s->tok_h, 0, (size_t)n * kTokMaxHot * 4);
  // the signal words start at zero once; launches count on from there
  if (e == hipSuccess) e = hipMemset(s->tok_sync, 0, (size_t)kTokSyncWords * 4);
  std::vector<TokLayer> tab(n);
  for (int L = 0; L < n && e == hipSuccess; ++L) {
    const StackLayer& SL = s->layers[L];
    const oi2_layer& l = SL.l;
    TokLayer& T = tab[L];
    T = TokLayer{};
    T.n_hot = l.hot.n_hot;
    T.down_stride = l.hot.down_stride;
    T.gate_q = l.hot.gate_q;
    T.up_q = l.hot.up_q;
    T.gate_s = l.hot.gate_scale;
    T.up_s = l.hot.up_scale;
    T.hot_gbias = l.hot.gate_bias;
    T.down_q = l.hot.down_q;
    T.down_s = l.hot.down_scale;
    T.norm_w = l.norm_w;
    T.n_records = l.cold.n_records;
    T.records = l.cold.records;
    T.cold_gbias = l.cold.gate_bias;
    int32_t* own_slots = s->tok_sel_slots + (size_t)L * kTokChunks * chunk;
    int32_t* own_ids = s->tok_sel_ids + (size_t)L * kTokChunks * chunk;
    int32_t* own_counts = s->tok_sel_counts + (size_t)L * kTokChunks;
    if (SL.has_pred) {
      T.rank = l.pred.rank;
      T.inter = l.pred.inter;
      T.pd_w = static_cast<const uint16_t*>(l.pred.down_w);
      T.pu_w = static_cast<const uint16_t*>(l.pred.up_w);
      T.pu_b = static_cast<const uint16_t*>(l.pred.up_b);
      T.lut = l.lut;
      T.sel_slots = own_slots;
      T.sel_ids = own_ids;
      T.sel_counts = own_counts;
      T.sel_chunk = chunk;
    }
    if (l.cold.n_records > 0) {
      if (SL.has_pred) {
        T.act_slots = own_slots;
        T.act_counts = own_counts;
        T.act_chunk = chunk;
      } else {
        // every cold record, ascending neuron id (engine.py:282-283), cut into
        // kTokChunks chunks
        std::vector<int32_t> lut(s->inter);
        e = hipMemcpy(lut.data(), l.lut, (size_t)s->inter * 4, hipMemcpyDeviceToHost);
        std::vector<int32_t> all;
        for (int i = 0; i < s->inter; ++i)
          if (lut[i] >= 0 && lut[i] < l.cold.n_records) all.push_back(lut[i]);
        const int ca = std::max<int>(1, ((int)all.size() + kTokChunks - 1) / kTokChunks);
        std::vector<int32_t> host((size_t)kTokChunks * ca + kTokChunks, -1);
        for (int c = 0; c < kTokChunks; ++c) {
          const int b = c * ca, m = std::max(0, std::min(ca, (int)all.size() - b));
          for (int k = 0; k < m; ++k) host[(size_t)c * ca + k] = all[b + k];
          host[(size_t)kTokChunks * ca + c] = m;
        }
        int32_t* buf = nullptr;
        alloc((void**)&buf, host.size() * 4);
        if (buf) s->tok_static.push_back(buf);
        if (e == hipSuccess) e = hipMemcpy(buf, host.data(), host.size() * 4, hipMemcpyHostToDevice);
        T.act_slots = buf;
        T.act_counts = buf + (size_t)kTokChunks * ca;
        T.act_chunk = ca;
      }
    }
  }
  if (e == hipSuccess) e = hipMemcpy(s->tok_layers, tab.data(), (size_t)n * sizeof(TokLayer), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    set_error("token kernel allocation failed: %s", hipGetErrorString(e));
    return OI2_ENOMEM;
  }
  s->tok_npw = npw;
  s->tok_chunk = chunk;
  s->tok_ok = true;
  s->tok = true;
  return OI2_OK;
}

static void drop_graphs(oi2_stack* s) {
  for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.exec);
  s->graphs.clear();
}

}  // namespace oi2

using namespace oi2;

extern "C" {

int oi2_stack_create(const oi2_layer* layers, int32_t n_layers, int32_t inter, float eps,
                     int32_t act, int32_t act_on_both, float threshold_logit, oi2_stack** out) {
  clear_error();
  OI2_CHECK_ARG(out, "out is null");
  *out = nullptr;
  OI2_CHECK_ARG(layers && n_layers > 0, "need at least one layer");
  OI2_CHECK_ARG(inter > 0 && inter <= 65536, "inter %d out of range", inter);
  OI2_CHECK_ARG(act == OI2_ACT_SILU || act == OI2_ACT_RELU, "act %d", act);
  oi2_stack* s = new oi2_stack();
  s->n_layers = n_layers;
  s->inter = inter;
  s->n_chunks = (inter + kSelChunk - 1) / kSelChunk;
  s->eps = eps;
  s->relu = act == OI2_ACT_RELU;
  s->both = act_on_both != 0;
  s->thr = threshold_logit;
  int max_records = 0;
  for (int L = 0; L < n_layers; ++L) {
    StackLayer SL;
    SL.l = layers[L];
    SL.has_pred = layers[L].pred.down_w != nullptr;
    const oi2_hot& h = SL.l.hot;
    if (h.n_hot > 0 &&
        (h.down_stride < h.n_hot || h.down_stride % 16 || h.down_stride > 4096 || !h.gate_q ||
         !h.up_q || !h.down_q || !h.gate_scale || !h.up_scale || !h.down_scale)) {
      set_error("layer %d: invalid hot weights", L);
      stack_free(s);
      delete s;
      return OI2_EINVAL;
    }
    if (!SL.l.norm_w || (SL.l.cold.n_records > 0 && (!SL.l.cold.records || !SL.l.lut))) {
      set_error("layer %d: norm weight, cold records and lut are required", L);
      stack_free(s);
      delete s;
      return OI2_EINVAL;
    }
    // records: device memory, or pinned host memory read over PCIe
    const uint8_t* src = nullptr;
    if (SL.l.cold.n_records > 0 &&
        ((uintptr_t)SL.l.cold.records % 16 || device_view(SL.l.cold.records, &src) != OI2_OK)) {
      set_error("layer %d: records must be 16-byte aligned device or pinned host memory", L);
      stack_free(s);
      delete s;
      return OI2_EINVAL;
    }
    s->src.push_back(src);
    if (SL.has_pred) {
      const oi2_predictor& p = SL.l.pred;
      if (!p.up_w || !p.up_b || p.inter != inter || p.rank <= 0 || p.rank > 256 || p.rank % 8 ||
          (p.dtype != OI2_DTYPE_F32 && p.dtype != OI2_DTYPE_BF16)) {
        set_error("layer %d: invalid predictor", L);
        stack_free(s);
        delete s;
        return OI2_EINVAL;
      }
      s->max_rank = std::max(s->max_rank, p.rank);
    }
    s->max_hot = std::max(s->max_hot, h.n_hot);
    max_records = std::max(max_records, SL.l.cold.n_records);
    s->layers.push_back(SL);
  }
  s->cold_cap = std::max(s->n_chunks * kSelChunk, max_records);
  {
    const ColdSplit cs = cold_split(s->n_chunks, s->cold_cap);
    s->cold_wpc = cs.wpc;
    s->cold_wg = cs.wg;
  }
  const size_t sel = (size_t)n_layers * s->n_chunks * kSelChunk;
  hipError_t e = hipSuccess;
  auto alloc = [&](void** p, size_t bytes) {
    if (e == hipSuccess) e = hipMalloc(p, bytes);
  };
  alloc((void**)&s->xbuf, (size_t)n_layers * kH * 2);
  alloc((void**)&s->xw, (size_t)kH * 2);
  alloc((void**)&s->ssq, (size_t)kDownWG * 4);
  alloc((void**)&s->h_hot, (size_t)(s->max_hot + 64) * 4);
  alloc((void**)&s->cold_part, (size_t)kMaxColdWG * kH * 4);
  alloc((void**)&s->z, (size_t)(s->max_rank + 64) * sizeof(double));
  alloc((void**)&s->sel_counts, (size_t)n_layers * s->n_chunks * 4);
  alloc((void**)&s->sel_slots, sel * 4);
  alloc((void**)&s->sel_ids, sel * 4);
  // layers without a predictor fetch every cold record (engine.py:282-283):
  // ascending neuron id order, i.e. the lut's non-negative entries in order
  for (auto& SL : s->layers) {
    if (e != hipSuccess || SL.has_pred || SL.l.cold.n_records == 0) continue;
    std::vector<int32_t> lut(inter);
    e = hipMemcpy(lut.data(), SL.l.lut, (size_t)inter * 4, hipMemcpyDeviceToHost);
    std::vector<int32_t> all;
    for (int i = 0; i < inter; ++i)
      if (lut[i] >= 0 && lut[i] < SL.l.cold.n_records) all.push_back(lut[i]);
    SL.n_all = std::max<int>(1, (int)all.size());
    alloc((void**)&SL.all_slots, (size_t)SL.n_all * 4);
    alloc((void**)&SL.all_count, 4);
    const int cnt = (int)all.size();
    if (e == hipSuccess && cnt) e = hipMemcpy(SL.all_slots, all.data(), (size_t)cnt * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(SL.all_count, &cnt, 4, hipMemcpyHostToDevice);
  }
  if (e == hipSuccess) e = hipMemset(s->sel_counts, 0, (size_t)n_layers * s->n_chunks * 4);
  if (e != hipSuccess) {
    set_error("stack allocation failed: %s", hipGetErrorString(e));
    stack_free(s);
    delete s;
    return OI2_ENOMEM;
  }
  const int rc = tok_setup(s);
  if (rc != OI2_OK) {
    stack_free(s);
    delete s;
    return rc;
  }
  *out = s;
  return OI2_OK;
}

int oi2_stack_decode(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out, "null argument");
  OI2_CHECK_ARG(((uintptr_t)x_in | (uintptr_t)x_out) % 16 == 0, "x must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  // a staged token is launched directly: its two streams wait on each other
  // on the device, so both must be running at once, which direct launches on
  // two streams guarantee and a graph's branches need not
  if (!s->use_graph || st == nullptr || s->staged) return stack_launch(s, x_in, x_out, st);
  for (auto& g : s->graphs)
    if (g.in == x_in && g.out == x_out && g.stream == st) {
      OI2_CHECK_HIP(hipGraphLaunch(g.exec, st));
      return OI2_OK;
    }
  if (s->graphs.size() >= 8) {
    OI2_CHECK_HIP(hipGraphExecDestroy(s->graphs.front().exec));
    s->graphs.erase(s->graphs.begin());
  }
  hipGraph_t g = nullptr;
  OI2_CHECK_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  int rc = stack_launch(s, x_in, x_out, st);
  hipError_t ec = hipStreamEndCapture(st, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  OI2_CHECK_HIP(ec);
  hipGraphExec_t exec = nullptr;
  hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  OI2_CHECK_HIP(ei);
  s->graphs.push_back({exec, x_in, x_out, st});
  OI2_CHECK_HIP(hipGraphLaunch(exec, st));
  return OI2_OK;
}

int oi2_stack_predict(oi2_stack* s, int32_t layer, const uint16_t* x, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x, "null argument");
  OI2_CHECK_ARG((uintptr_t)x % 16 == 0, "x must be 16-byte aligned");
  OI2_CHECK_ARG(layer >= 0 && layer < s->n_layers, "layer %d of %d", layer, s->n_layers);
  OI2_CHECK_ARG(!s->staged, "per-layer calls do not stage; turn staging off");
  if (!s->layers[layer].has_pred) return OI2_OK;   // the layer takes every cold record
  hipStream_t st = (hipStream_t)stream;
  // the predictor normalises x from its sum-of-squares partials
  hipLaunchKernelGGL(k_prep, dim3(1), dim3(kThreads), 0, st, x, s->layers[layer].l.norm_w, s->xw, s->ssq);
  OI2_CHECK_LAUNCH();
  return launch_predictor(s, layer, x, st);
}

int oi2_stack_layer(oi2_stack* s, int32_t layer, const uint16_t* x_in, uint16_t* x_out, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out, "null argument");
  OI2_CHECK_ARG(((uintptr_t)x_in | (uintptr_t)x_out) % 16 == 0, "x must be 16-byte aligned");
  OI2_CHECK_ARG(x_in + kH <= x_out || x_out + kH <= x_in, "x_in and x_out overlap");
  OI2_CHECK_ARG(layer >= 0 && layer < s->n_layers, "layer %d of %d", layer, s->n_layers);
  OI2_CHECK_ARG(!s->staged, "per-layer calls do not stage; turn staging off");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_prep, dim3(1), dim3(kThreads), 0, st, x_in, s->layers[layer].l.norm_w, s->xw, s->ssq);
  OI2_CHECK_LAUNCH();
  UpArgs ua;
  DownArgs da;
  layer_args(s, layer, x_in, x_out, ua, da);
  // the caller's input and output; the next layer's input is not this
  // output (attention comes between), so no norm partials are passed on
  ua.tok = TokenIn{x_in, s->xw, s->ssq, s->eps, 1};
  da.res = x_in;
  da.out = x_out;
  da.out2 = nullptr;
  da.next_norm_w = nullptr;
  da.xw_out = nullptr;
  da.ssq_out = nullptr;
  int rc = launch_up(ua, st);
  if (rc == OI2_OK) rc = launch_down(da, st);
  return rc;
}

int oi2_stack_set_expected_active(oi2_stack* s, int32_t expected) {
  clear_error();
  OI2_CHECK_ARG(s && expected >= 0, "bad argument");
  const ColdSplit cs = cold_split(s->n_chunks, expected > 0 ? expected : s->cold_cap);
  s->cold_wpc = cs.wpc;
  s->cold_wg = cs.wg;
  for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.exec);
  s->graphs.clear();
  return OI2_OK;
}

int oi2_stack_set_graph(oi2_stack* s, int32_t enable) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  s->use_graph = enable != 0;
  return OI2_OK;
}

int oi2_stack_set_staging(oi2_stack* s, int32_t copy_workgroups) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  OI2_CHECK_ARG(copy_workgroups >= 0 && copy_workgroups <= 1024, "copy_workgroups %d out of range",
                copy_workgroups);
  for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.exec);
  s->graphs.clear();
  OI2_CHECK_HIP(hipDeviceSynchronize());
  staging_free(s);
  if (!copy_workgroups) return OI2_OK;
  for (int L = 0; L < s->n_layers; ++L)
    if (s->layers[L].l.cold.n_records > 0 && s->layers[L].l.cold.gate_bias) {
      set_error("layer %d: staging does not support a cold gate bias", L);
      return OI2_EUNSUPPORTED;
    }
  const int n = s->n_layers;
  hipError_t e = hipStreamCreateWithFlags(&s->side, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->own, hipStreamNonBlocking);
  for (int b = 0; b < 2 && e == hipSuccess; ++b)
    e = hipMalloc((void**)&s->stage[b], (size_t)s->cold_cap * kRecBytes);
  if (e == hipSuccess) e = hipMalloc((void**)&s->stage_sync, (size_t)stage_sync_words(n) * 4);
  if (e == hipSuccess) e = hipMemset(s->stage_sync, 0, (size_t)stage_sync_words(n) * 4);
  if (e == hipSuccess) e = hipMalloc((void**)&s->stage_tab, (size_t)n * sizeof(StageLayer));
  for (auto* ev : {&s->ev_fork, &s->ev_join, &s->ev_null_in, &s->ev_null_out})
    if (e == hipSuccess) e = hipEventCreateWithFlags(ev, hipEventDisableTiming);
  if (e == hipSuccess) {
    // what the copy kernel stages per layer: the same lists the FFN reads
    std::vector<StageLayer> tab(n);
    for (int L = 0; L < n; ++L) {
      tab[L] = StageLayer{};
      if (s->layers[L].l.cold.n_records == 0) continue;
      tab[L].src = s->src[L];
      tab[L].n_records = s->layers[L].l.cold.n_records;
      tab[L].act = layer_list(s, L);
      tab[L].dst = s->stage[L & 1];
      tab[L].sel_target = s->layers[L].has_pred ? (uint32_t)s->n_chunks : 1u;
    }
    e = hipMemcpy(s->stage_tab, tab.data(), (size_t)n * sizeof(StageLayer), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    set_error("staging set-up failed: %s", hipGetErrorString(e));
    staging_free(s);
    return OI2_ENOMEM;
  }
  s->staged = true;
  s->copy_wg = copy_workgroups;
  return OI2_OK;
}

int oi2_stack_profile_staging(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                              float* gather_us, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out && gather_us, "null argument");
  OI2_CHECK_ARG(s->staged, "staging is not enabled on this stack");
  OI2_CHECK_ARG(reps > 0 && reps <= 1024, "reps %d out of range", reps);
  hipStream_t st = (hipStream_t)stream;
  hipEvent_t ev[2] = {nullptr, nullptr};
  int rc = OI2_OK;
  for (auto& e : ev)
    if (rc == OI2_OK && hipEventCreate(&e) != hipSuccess) {
      set_error("hipEventCreate failed");
      rc = OI2_EHIP;
    }
  // one token fixes the active sets; then every layer's copy back to back on
  // the launch stream; then the token again, so the buffers hold its state
  if (rc == OI2_OK) rc = stack_launch(s, x_in, x_out, st);
  if (rc == OI2_OK && hipStreamSynchronize(st) != hipSuccess) rc = OI2_EHIP;
  if (rc == OI2_OK && hipEventRecord(ev[0], st) != hipSuccess) rc = OI2_EHIP;
  for (int r = 0; rc == OI2_OK && r < reps; ++r)
    for (int L = 0; rc == OI2_OK && L < s->n_layers; ++L) rc = launch_gather(s, L, st);
  if (rc == OI2_OK && hipEventRecord(ev[1], st) != hipSuccess) rc = OI2_EHIP;
  if (rc == OI2_OK) rc = stack_launch(s, x_in, x_out, st);
  if (rc == OI2_OK && hipStreamSynchronize(st) != hipSuccess) rc = OI2_EHIP;
  float t = 0.0f;
  if (rc == OI2_OK && hipEventElapsedTime(&t, ev[0], ev[1]) != hipSuccess) rc = OI2_EHIP;
  if (rc == OI2_EHIP && !oi2_last_error()[0]) set_error("HIP call failed while profiling");
  if (rc == OI2_OK) *gather_us = (float)(t * 1e3 / ((double)reps * s->n_layers));
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int oi2_stack_profile(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                      float* up_us, float* down_us, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out && up_us && down_us, "null argument");
  OI2_CHECK_ARG(reps > 0 && reps <= 1024, "reps %d out of range", reps);
  OI2_CHECK_ARG(!s->staged, "kernel profiling needs staging disabled");
  hipStream_t st = (hipStream_t)stream;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  int rc = OI2_OK;
  for (auto& e : ev)
    if (rc == OI2_OK && hipEventCreate(&e) != hipSuccess) {
      set_error("hipEventCreate failed");
      rc = OI2_EHIP;
    }
  // one real token (two-launch sequence) fixes every layer's active set; then
  // every layer's ffn_up back to back, reps times, then every layer's ffn_down
  // the same way
  if (rc == OI2_OK) rc = stack_launch_layers(s, x_in, x_out, st);
  std::vector<UpArgs> ua(s->n_layers);
  std::vector<DownArgs> da(s->n_layers);
  for (int L = 0; L < s->n_layers; ++L) layer_args(s, L, x_in, x_out, ua[L], da[L]);
  if (rc == OI2_OK && hipEventRecord(ev[0], st) != hipSuccess) rc = OI2_EHIP;
  for (int r = 0; rc == OI2_OK && r < reps; ++r)
    for (int L = 0; rc == OI2_OK && L < s->n_layers; ++L) rc = launch_up(ua[L], st);
  if (rc == OI2_OK && hipEventRecord(ev[1], st) != hipSuccess) rc = OI2_EHIP;
  for (int r = 0; rc == OI2_OK && r < reps; ++r)
    for (int L = 0; rc == OI2_OK && L < s->n_layers; ++L) rc = launch_down(da[L], st);
  if (rc == OI2_OK && hipEventRecord(ev[2], st) != hipSuccess) rc = OI2_EHIP;
  // the timing launches overwrite the selections: run the token again so the
  // stack's state (and x_out) is that of x_in
  if (rc == OI2_OK) rc = stack_launch(s, x_in, x_out, st);
  if (rc == OI2_OK && hipStreamSynchronize(st) != hipSuccess) {
    set_error("hipStreamSynchronize failed");
    rc = OI2_EHIP;
  }
  float t_up = 0.0f, t_down = 0.0f;
  if (rc == OI2_OK && (hipEventElapsedTime(&t_up, ev[0], ev[1]) != hipSuccess ||
                       hipEventElapsedTime(&t_down, ev[1], ev[2]) != hipSuccess)) {
    set_error("hipEventElapsedTime failed");
    rc = OI2_EHIP;
  }
  if (rc == OI2_OK) {
    const double n = (double)reps * s->n_layers;
    *up_us = (float)(t_up * 1e3 / n);
    *down_us = (float)(t_down * 1e3 / n);
  }
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int oi2_stack_trace(oi2_stack* s, uint16_t* xs, int32_t* counts, int32_t* slots, int32_t* ids,
                    void* stream) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  hipStream_t st = (hipStream_t)stream;
  const bool tk = use_tok(s);
  const int nc = tk ? kTokChunks : s->n_chunks;
  const size_t sel = (size_t)s->n_layers * nc * (tk ? s->tok_chunk : kSelChunk);
  if (xs) OI2_CHECK_HIP(hipMemcpyAsync(xs, s->xbuf, (size_t)s->n_layers * kH * 2, hipMemcpyDeviceToDevice, st));
  if (counts)
    OI2_CHECK_HIP(hipMemcpyAsync(counts, tk ? s->tok_sel_counts : s->sel_counts, (size_t)s->n_layers * nc * 4,
                                 hipMemcpyDeviceToDevice, st));
  if (slots)
    OI2_CHECK_HIP(hipMemcpyAsync(slots, tk ? s->tok_sel_slots : s->sel_slots, sel * 4, hipMemcpyDeviceToDevice, st));
  if (ids) OI2_CHECK_HIP(hipMemcpyAsync(ids, tk ? s->tok_sel_ids : s->sel_ids, sel * 4, hipMemcpyDeviceToDevice, st));
  return OI2_OK;
}

int oi2_stack_selection_layout(const oi2_stack* s, int32_t* n_chunks, int32_t* chunk) {
  clear_error();
  OI2_CHECK_ARG(s && n_chunks && chunk, "null argument");
  const bool tk = use_tok(s);
  *n_chunks = tk ? kTokChunks : s->n_chunks;
  *chunk = tk ? s->tok_chunk : kSelChunk;
  return OI2_OK;
}

int oi2_stack_set_token_kernel(oi2_stack* s, int32_t enable) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  if (enable && !s->tok_ok) {
    set_error("the persistent token kernel does not support this stack: %s", s->tok_why.c_str());
    return OI2_EUNSUPPORTED;
  }
  drop_graphs(s);
  s->tok = enable != 0;
  return OI2_OK;
}

int32_t oi2_stack_token_kernel(const oi2_stack* s) { return (s && use_tok(s)) ? 1 : 0; }

int oi2_stack_set_wait_bound(oi2_stack* s, int32_t polls) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  OI2_CHECK_ARG(polls >= 1 && polls <= (1 << 24), "wait bound %d out of range 1 .. %d", polls, 1 << 24);
  s->tok_spin = (uint32_t)polls;
  s->stage_spin = (uint32_t)polls;
  drop_graphs(s);   // the bound is a kernel argument
  return OI2_OK;
}

int oi2_stack_status(oi2_stack* s, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s, "null stack");
  OI2_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
  if (s->staged) {
    // the staged path's device-side waits keep their own error word, set
    // until reported here
    uint32_t err = 0;
    uint32_t* ew = s->stage_sync + stage_err_word(s->n_layers);
    OI2_CHECK_HIP(hipStreamSynchronize(s->side));
    OI2_CHECK_HIP(hipStreamSynchronize(s->own));
    OI2_CHECK_HIP(hipMemcpy(&err, ew, 4, hipMemcpyDeviceToHost));
    if (err != 0) {
      OI2_CHECK_HIP(hipMemset(ew, 0, 4));
      set_error("staged decode: a device-side wait for records ran past its bound in a token "
                "decoded since the previous status check");
      return OI2_EHIP;
    }
    return OI2_OK;
  }
  if (!use_tok(s)) return OI2_OK;
  // the error word is nonzero once any launch since the signal words were
  // last cleared had a wait run past its bound (it holds that launch's epoch
  // base + 1); it stays set until reported here, so an overrun in any token
  // since the previous status call is reported, not only in the last one
  uint32_t err = 0;
  OI2_CHECK_HIP(hipMemcpy(&err, s->tok_sync + kTokSyncErr, 4, hipMemcpyDeviceToHost));
  if (err != 0) {
    // a wait that gave up lets its group run ahead of an epoch, so the
    // counters may no longer line up with the epochs: start them over
    OI2_CHECK_HIP(hipMemset(s->tok_sync, 0, (size_t)kTokSyncWords * 4));
    set_error("persistent token kernel: a device-wide wait ran past its bound in a token "
              "decoded since the previous status check");
    return OI2_EHIP;
  }
  return OI2_OK;
}

int oi2_stack_profile_token(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                            float* token_us, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out && token_us, "null argument");
  OI2_CHECK_ARG(reps > 0 && reps <= 4096, "reps %d out of range", reps);
  OI2_CHECK_ARG(use_tok(s), "the persistent token kernel is not in use on this stack");
  hipStream_t st = (hipStream_t)stream;
  std::vector<hipEvent_t> ev(2 * (size_t)reps, nullptr);
  int rc = OI2_OK;
  for (auto& e : ev)
    if (rc == OI2_OK && hipEventCreate(&e) != hipSuccess) {
      set_error("hipEventCreate failed");
      rc = OI2_EHIP;
    }
  if (rc == OI2_OK) rc = stack_launch_tok(s, x_in, x_out, st);
  const TokArgs a = tok_args(s, x_in, x_out);
  for (int r = 0; rc == OI2_OK && r < reps; ++r) {
    if (hipEventRecord(ev[2 * r], st) != hipSuccess) rc = OI2_EHIP;
    if (rc == OI2_OK) rc = tok_launch(a, s->tok_npw, st);
    if (rc == OI2_OK && hipEventRecord(ev[2 * r + 1], st) != hipSuccess) rc = OI2_EHIP;
  }
  if (rc == OI2_OK && hipStreamSynchronize(st) != hipSuccess) rc = OI2_EHIP;
  double total = 0.0;
  for (int r = 0; rc == OI2_OK && r < reps; ++r) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]) != hipSuccess) rc = OI2_EHIP;
    total += ms;
  }
  if (rc == OI2_EHIP && !oi2_last_error()[0]) set_error("HIP call failed while profiling");
  if (rc == OI2_OK) *token_us = (float)(total * 1e3 / reps);
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int oi2_stack_trace_token(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, uint64_t* trace,
                          size_t trace_bytes, void* stream) {
  clear_error();
  OI2_CHECK_ARG(s && x_in && x_out && trace, "null argument");
  OI2_CHECK_ARG(use_tok(s), "the persistent token kernel is not in use on this stack");
  const size_t need = (size_t)std::min(s->n_layers, kTokTraceLayers) * kTokGroups * kTokTracePoints * 8;
  OI2_CHECK_ARG(trace_bytes >= need, "trace buffer of %zu bytes is smaller than the %zu required",
                trace_bytes, need);
  TokArgs a = tok_args(s, x_in, x_out);
  a.trace = trace;
  return tok_launch(a, s->tok_npw, (hipStream_t)stream);
}

int oi2_stack_destroy(oi2_stack* s) {
  clear_error();
  if (!s) return OI2_OK;
  stack_free(s);
  delete s;
  return OI2_OK;
}

}  // extern "C"
