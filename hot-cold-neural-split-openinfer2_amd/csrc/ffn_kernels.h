// Argument blocks and kernel declarations shared by the decode-path sources.
#pragma once
#include "oi2.h"
#include "oi2_device.h"

namespace oi2 {

constexpr int kThreads = 256;
constexpr int kRowsPerDownWG = 16;
constexpr int kDownWG = kH / kRowsPerDownWG;   // 256 output tiles
constexpr int kSelChunk = 256;
constexpr int kMaxChunks = 256;
// Cold work of the single-token kernels: about kColdItemsPerWave active items
// per wave, at most kMaxColdWaves waves plus one per chunk, four waves per
// workgroup, each workgroup one fp32 partial row of y.
constexpr int kColdItemsPerWave = 2;
constexpr int kMaxColdWaves = 1024;
constexpr int kMaxColdWG = (kMaxColdWaves + kMaxChunks + 3) / 4;   // 320

// Active items in chunks: chunk c holds counts[c] items at slots[c * chunk ..].
// slots == nullptr: item at position p uses record p.
struct ActiveList {
  const int32_t* slots;
  const int32_t* counts;
  int n_chunks;
  int chunk;
};

// Normalised-token inputs every FFN workgroup shares: xw = fp16(x * w) (the
// norm weight applied, not yet scaled) and 256 partial sums of x^2 from which
// each wave derives r = rsqrt(mean(x^2) + eps); x_n = r * xw.
struct TokenIn {
  const uint16_t* x;        // (H) fp16 token (the predictor normalises it exactly)
  const uint16_t* xw;       // (H) fp16 x * norm weight, or x when use_norm == 0
  const float* ssq;         // 256 partial sums of x^2
  float eps;
  int use_norm;
  // non-null: the norm weight, and the kernel forms xw and the partials from
  // x itself (k_prep's arithmetic) instead of reading xw and ssq
  const uint16_t* norm_w;
};

struct UpArgs {
  TokenIn tok;
  int relu, both;
  // hot gate/up
  int n_hot;
  const uint8_t* gate_q;
  const uint8_t* up_q;
  const float* gate_s;
  const float* up_s;
  const float* hot_gbias;
  float* h_hot;             // (n_hot)
  // cold gate/up: one wave per active record
  const uint8_t* records;
  int n_records;
  const float* cold_gbias;
  ActiveList act;
  float* cold_part;         // (wg_cold, H) partial down sums, one row per workgroup
  int cold_wpc;             // cold waves per chunk of the list
  // predictor down projection (lookahead layer): z = D q, q = cast(fp16(x r w'))
  const void* pd_w;
  int pd_rank;
  int pd_bf16;
  const uint16_t* pd_norm_w;  // null: q = cast(x)
  const float* pd_q;          // precomputed query (H), or null
  double* pd_z;
  int wg_cold, wg_pred, wg_hot;
  // staged records: the cold workgroups wait until *stage_ready reaches
  // stage_target before reading them (null: no wait).  A wait that gives up
  // (or finds the error word set) reads the layer's records from where the
  // copy takes them, stage_src (n records), through the chunked slot list
  // stage_slots, so the output is the same either way.
  const uint32_t* stage_ready;
  uint32_t stage_target;
  uint32_t* stage_err;
  uint32_t stage_spin;
  const uint8_t* stage_src;
  int stage_src_n;
  const int32_t* stage_slots;
};

struct DownArgs {
  const uint16_t* res;      // residual (H) fp16 or null
  // hot down
  const float* h_hot;
  int n_hot;
  int down_stride;
  const uint8_t* down_q;
  const float* down_s;
  // cold down: partial rows from ffn_up's cold workgroups
  const float* cold_part;
  int cold_wg;              // ffn_up's cold workgroup count
  // outputs
  uint16_t* out;
  uint16_t* out2;
  float* y32;
  const uint16_t* next_norm_w;  // norm weight of the next layer, or null
  uint16_t* xw_out;             // fp16(out * next_norm_w)
  float* ssq_out;               // 256 partial sums of out^2
  // predictor up projection + selection
  const void* pu_w;
  const void* pu_b;
  int pu_rank;
  int pu_bf16;
  int inter;
  const double* pd_z;
  float thr;
  const int32_t* lut;
  int32_t* sel_slots;
  int32_t* sel_ids;
  int32_t* sel_counts;
  float* logits_out;
  float* probs_out;
  uint8_t* mask_out;
  uint32_t* sel_flag;       // each selection workgroup adds 1 once its chunk is written (or null)
  int wg_pred, wg_down;
};

// Staging of one layer's active cold records (see k_stage_gather).
struct StageArgs {
  const uint8_t* src;       // record 0 of the layer's records, 16-byte aligned
  int n_records;
  ActiveList act;
  int cap;                  // items beyond this are ignored
  uint8_t* dst;             // staging records, list position p at dst + 6400 p
};

__global__ void k_stage_gather(StageArgs a);

// Staged decode with device-side signals (one token at a time).  The sync
// area holds, one 128-byte line each: sel[L] (workgroups of layer L's
// selection kernel that have written their chunk of the active list, or 1
// from k_stage_signal for a layer without a predictor), ready[L] (copy
// workgroups done with layer L's records) and an error word set when a wait
// runs past its bound.  The counters are cleared by k_fill_u32 at the start of
// every token.
constexpr int kStageLine = 32;    // words per counter
__host__ __device__ constexpr int stage_sel_word(int L) { return kStageLine * (2 * L); }
__host__ __device__ constexpr int stage_ready_word(int L) { return kStageLine * (2 * L + 1); }
__host__ __device__ constexpr int stage_err_word(int n_layers) { return kStageLine * (2 * n_layers); }
__host__ __device__ constexpr int stage_sync_words(int n_layers) { return kStageLine * (2 * n_layers + 1); }

struct StageLayer {
  const uint8_t* src;       // the layer's records (device or pinned host memory)
  int n_records;            // 0: nothing to stage
  ActiveList act;
  uint8_t* dst;             // staging buffer: list position p at dst + 6400 p
  uint32_t sel_target;      // sel[L] value meaning the list is complete
};

struct StageCopyArgs {
  const StageLayer* layers; // (n_layers) device table
  int n_layers;
  int cap;
  uint32_t* sync;
  uint32_t spin;            // poll bound of each wait
};

__global__ void k_stage_copy(StageCopyArgs a);
__global__ void k_stage_signal(uint32_t* word);
__global__ void k_fill_u32(uint32_t* p, int n, uint32_t v);

// Multi-token FFN on the matrix cores (ffn_batch.hip).
struct BUpArgs {
  const uint16_t* xn;       // (M, H) fp16 normalised tokens
  int M;
  int relu, both;
  int n_hot;
  const uint8_t* gate_q;
  const uint8_t* up_q;
  const float* gate_s;
  const float* up_s;
  const float* hot_gbias;
  uint16_t* hh;             // (Mpad, ldh) fp16 hot activations, zero past n_hot
  int ldh;
  const uint8_t* records;
  int n_records;
  const float* cold_gbias;
  const int32_t* dslots;    // dense active list
  const int32_t* total;
  int cap;
  uint16_t* hc;             // (Mpad, ldc) fp16 cold activations
  int ldc;
  int Mpad;
  int hot_per_wg;           // k_sbup: hot rows per workgroup (n_hot over 256 workgroups)
};

struct BDownArgs {
  int M;
  const uint16_t* hh;
  int ldh;
  const uint8_t* down_q;
  int down_stride;
  const float* down_s;
  int hot_blocks;           // 128-wide K blocks of the hot product
  int hot_splits;
  const uint16_t* hc;
  int ldc;
  const uint8_t* records;
  int n_records;
  const int32_t* dslots;
  const int32_t* total;
  int cap;
  // from 17 tokens: (splits, M, H) fp32, one partial sum of y per down range
  // (the hot ranges, then the cold ranges from cold_split0), which k_bfinal
  // adds in that order
  float* y;
  int cold_split0;
  // at most 16 tokens: the cold down's partial sums, n_part item ranges of
  // (H, 16) fp32; k_bdown_hot_s, the last of the small-batch kernels, adds
  // them in range order to the hot product -> out = fp16(res + y) (res may
  // be null), and y32 = y when asked
  float* part;
  int n_part;
  const uint16_t* res;
  uint16_t* out;
  float* y32;
};

__global__ void k_bup(BUpArgs a);
__global__ void k_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, uint16_t* out);

size_t batch_ws_bytes(int M, int n_hot, int cap);
// Scratch carve-up of the single-token decode FFN (k_prep / k_ffn_up /
// k_ffn_down): h_hot, cold partial rows (one per cold workgroup), the cold
// item total, x * w and the norm's sum-of-squares partials.
struct FfnWs {
  float* h_hot;
  float* cold_part;
  uint16_t* xw;
  float* ssq;
};

__host__ __device__ constexpr size_t ffn_align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Bytes of that scratch for n_hot hot neurons and cold_wg cold workgroups.
__host__ __device__ constexpr size_t ffn_ws_bytes(int n_hot, int cold_wg) {
  return ffn_align256((size_t)(n_hot > 0 ? n_hot : 0) * 4 + 64) +
         ffn_align256((size_t)cold_wg * kH * 4) + ffn_align256(kH * 2) +
         ffn_align256(kDownWG * 4);
}

FfnWs ffn_ws(void* base, int n_hot, int cold_wg);

// A validated oi2_ffn_forward request.
struct FfnCall {
  int n_hot = 0;
  bool has_cold = false;
  int cap = 0;       // capacity of the active list
  int wg_cold = 0;   // cold workgroups of the launch (from the expected count)
  int cold_wpc = 0;  // cold waves per chunk
};

int ffn_validate(const uint16_t* x, int batch, const uint16_t* norm_w, const oi2_hot* hot,
                 const oi2_cold* cold, const oi2_active* active, int act, FfnCall* c);
int ffn_decode_tokens(const uint16_t* x, int batch, const uint16_t* norm_w, float eps,
                      const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active, int act,
                      int act_on_both, int add_residual, uint16_t* out, float* y32,
                      const FfnCall& c, const FfnWs& ws, hipStream_t st);
// The cold split of a list of n_chunks chunks with about `expected` items:
// wpc waves per chunk, wg workgroups (never more than cold_rows_bound of any
// expected count at least as large, nor than kMaxColdWG).
struct ColdSplit {
  int wpc;
  int wg;
};
ColdSplit cold_split(int n_chunks, int expected);
// Partial rows (cold workgroups) that any list of up to kMaxChunks chunks
// with at most `capacity` expected items can need.
constexpr int cold_rows_bound(int capacity) {
  const int waves = (capacity + kColdItemsPerWave - 1) / kColdItemsPerWave;
  const int wv = waves < 1 ? 1 : (waves > kMaxColdWaves ? kMaxColdWaves : waves);
  return (wv + kMaxChunks - 1 + 3) / 4;
}

// With xn_in the rows are taken as already normalised (no norm launch);
// with next_w the call also writes xn_next = RMSNorm(out) with that weight.
int batch_ffn(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const oi2_hot* hot,
              const oi2_cold* cold, const oi2_active* active, int relu, int both, int add_residual,
              uint16_t* out, float* y32, void* workspace, size_t workspace_bytes, hipStream_t st,
              const uint16_t* xn_in = nullptr, const uint16_t* next_w = nullptr, float next_eps = 0.f,
              uint16_t* xn_next = nullptr);

// Exclusive prefix of the (clamped) chunk counts into s_prefix[0..n_chunks];
// all threads of a 256-thread workgroup call it (it contains barriers).
__device__ __forceinline__ void chunk_prefix(const ActiveList& al, int* s_prefix) {
  const int t = threadIdx.x;
  int c = 0;
  if (t < al.n_chunks) {
    c = al.counts[t];
    c = c < 0 ? 0 : (c > al.chunk ? al.chunk : c);
  }
  s_prefix[t + 1] = c;
  if (t == 0) s_prefix[0] = 0;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {
    int v = (t >= off) ? s_prefix[t + 1 - off] : 0;
    __syncthreads();
    s_prefix[t + 1] += v;
    __syncthreads();
  }
}
// ── persistent token kernel (token.hip) ─────────────────────────────────────

constexpr int kTokGroups = 256;            // workgroups (one per CU), one output tile each
constexpr int kTokThreads = 512;           // a control wave and 7 worker waves
constexpr int kTokWorkers = kTokThreads / 64 - 1;
constexpr int kTokChunks = 256;            // active-list chunks: one per group
constexpr int kTokMaxChunk = 64;           // ids per chunk (one lane each)
constexpr int kTokMaxRank = 64;
constexpr int kTokMaxHot = 4096;           // h staged in LDS; also the per-layer h slice
constexpr int kTokSyncWords = 2048 + 192;
constexpr int kTokSyncErr = 2048 + 128;       // epoch base + 1 of a launch whose wait ran past its bound
constexpr int kTokSyncGoD = 64 * 8;           // XCD 0's flag of the D phase

// One layer as the token kernel reads it (a device-resident table).
struct TokLayer {
  // hot half
  int n_hot, down_stride;
  const uint8_t* gate_q;
  const uint8_t* up_q;
  const float* gate_s;
  const float* up_s;
  const float* hot_gbias;
  const uint8_t* down_q;
  const float* down_s;
  // cold half and the active list it reads (kTokChunks chunks of act_chunk)
  int n_records, act_chunk;
  const uint8_t* records;
  const float* cold_gbias;
  const int32_t* act_slots;
  const int32_t* act_counts;
  const uint16_t* norm_w;
  // this layer's predictor (run one layer ahead); pd_w null: none
  int rank, inter;
  const uint16_t* pd_w;     // (rank, H) bf16
  const uint16_t* pu_w;     // (inter, rank) bf16
  const uint16_t* pu_b;     // (inter) bf16
  const int32_t* lut;
  int32_t* sel_slots;       // where its list is written: chunk c at c * sel_chunk
  int32_t* sel_ids;
  int32_t* sel_counts;
  int sel_chunk;
};

struct TokArgs {
  const TokLayer* layers;
  int n_layers;
  const uint16_t* x_in;
  uint16_t* x_out;
  // Everything below is written at most once per launch and read only after
  // the signal that completes it, so it is read with cached loads: one slice
  // per layer.
  uint16_t* xbuf;           // (n_layers, H) layer outputs
  uint16_t* xw;             // (n_layers, H) x_L * norm weight of layer L
  float* ssq;               // (n_layers, 256) sum-of-squares partials of x_L
  float* h;                 // (n_layers, kTokMaxHot) hot activations, zero past n_hot
  double* z;                // (n_layers, 4 * kTokMaxRank) predictor down projection of layer L:
                            // quarter q of row r at 4 r + q
  float* cpart;             // (n_layers, kTokGroups, H) cold down partial of each chunk with items
  uint32_t* sync;           // kTokSyncWords, zero at allocation
  uint32_t spin;            // poll bound of every device-wide wait
  uint64_t* trace;          // null, or (min(n_layers, kTokTraceLayers), kTokGroups, kTokTracePoints)
                            // s_memrealtime stamps of each group's control wave
  float eps, thr;
  int relu, both;
};

// The control wave's trace points per layer: 0 the U phase starts (the
// previous D signal seen), 1 B1, 2 B2, 3 the U arrival issued, 4 the U signal
// seen, 5 D1a, 6 D1b, 7 the D arrival issued.
constexpr int kTokTracePoints = 8;
constexpr int kTokTraceLayers = 64;

int tok_launch(const TokArgs& a, int npw, hipStream_t st);
int tok_resident(int npw, int* resident);

__global__ void k_prep(const uint16_t* x, const uint16_t* w, uint16_t* xw, float* ssq);
__global__ void k_ffn_up(UpArgs a);
__global__ void k_ffn_down(DownArgs a);
__global__ void k_pred_up(UpArgs a);
__global__ void k_pred_down(DownArgs a);
__global__ void k_compact_dense(const int32_t* slots, const int32_t* ids, const int32_t* counts,
                                int n_chunks, int32_t* dslots, int32_t* dids, int32_t* total);

}  // namespace oi2
