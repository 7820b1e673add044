/*
 * oi2.h - C ABI of the MI355X (gfx950) hot/cold sparse-FFN decode library.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream passed
 * as void* (hipStream_t; NULL = the default stream), enqueues its work
 * asynchronously on that stream and returns an int status: OI2_OK (0) or an
 * error code, with a message available from oi2_last_error() on the calling
 * thread.  Nothing throws across the ABI.  Entry points that need scratch
 * memory take a caller-provided workspace (size from the matching *_bytes
 * query) and allocate nothing; the stack handle allocates once, at creation
 * (and when staging is switched on).
 *
 * Layouts (H = 4096, the hidden size the cold-record format is sized for):
 *   activations   fp16, row-major (batch, H)
 *   hot weights   fp8 e4m3fn (OCP) with fp32 per-row scales:
 *                 gate/up (n_hot, H), down (H, down_stride) row-major, columns
 *                 n_hot..down_stride-1 zero
 *   cold records  the split format's 6400-byte records (splitter.py:23-39),
 *                 consecutive, record 0 at a 16-byte aligned address
 *   predictor     fp32 or bf16: down (rank, H), up (inter, rank), bias (inter)
 *
 * Citations are file:line in the reference (OpenInfer2) checkout.
 */
#ifndef OI2_H
#define OI2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OI2_ABI_VERSION 2

enum {
  OI2_OK = 0,
  OI2_EINVAL = 1,       /* bad argument (shape, pointer, size) */
  OI2_EHIP = 2,         /* a HIP runtime call failed */
  OI2_ENOMEM = 3,       /* workspace too small / allocation failed at creation */
  OI2_EUNSUPPORTED = 4, /* valid request outside what this build implements */
  OI2_EIO = 5           /* reading the cold-record file failed */
};

enum { OI2_ACT_SILU = 0, OI2_ACT_RELU = 1 };          /* engine.py:165 */
enum { OI2_DTYPE_F32 = 0, OI2_DTYPE_BF16 = 1, OI2_DTYPE_F16 = 2 };

/* Hot FP8 half of one layer: the tensors SparseFFNLayer loads from
 * hot_weights/layer_XXX_expert_000.pt (engine.py:252-264, written at
 * splitter.py:221-226), kept at fp8 with per-row scales (1.0 reproduces the
 * reference's unscaled cast). */
typedef struct oi2_hot {
  int32_t n_hot;
  int32_t down_stride;        /* bytes per down row; >= n_hot, multiple of 16 */
  const uint8_t* gate_q;      /* (n_hot, H) */
  const uint8_t* up_q;        /* (n_hot, H) */
  const uint8_t* down_q;      /* (H, down_stride) */
  const float* gate_scale;    /* (n_hot) */
  const float* up_scale;      /* (n_hot) */
  const float* down_scale;    /* (H) */
  const float* gate_bias;     /* (n_hot) gate pre-activation shift, or NULL */
} oi2_hot;

/* One layer's cold section: the records that ColdWeightStore.read_neurons
 * decodes (splitter.py:354-403), in device memory (or, for a decode stack,
 * pinned host memory, read over PCIe). */
typedef struct oi2_cold {
  const uint8_t* records;     /* record slot 0 */
  int32_t n_records;
  const float* gate_bias;     /* per record slot, or NULL */
} oi2_cold;

/* The active cold set: record slots grouped in n_chunks chunks of capacity
 * `chunk`; counts[c] valid entries start at slots[c * chunk].  A plain list of
 * n slots is one chunk with counts -> {n}.  counts live in device memory, so a
 * predictor's output feeds the FFN without a host round trip. */
typedef struct oi2_active {
  const int32_t* slots;
  const int32_t* counts;
  int32_t n_chunks;           /* 1..256 */
  int32_t chunk;
  int32_t expected;           /* expected active count sizing the launch
                                 (0: the capacity n_chunks * chunk); any
                                 count up to the capacity is handled */
} oi2_active;

/* NeuronPredictor weights (predictor.py:55-75): sigmoid(up(down(x))). */
typedef struct oi2_predictor {
  int32_t inter;              /* intermediate size I (<= 65536) */
  int32_t rank;               /* low-rank width (multiple of 4, <= 256) */
  int32_t dtype;              /* OI2_DTYPE_F32 or OI2_DTYPE_BF16 */
  const void* down_w;         /* (rank, H), no bias (predictor.py:67) */
  const void* up_w;           /* (inter, rank) (predictor.py:68) */
  const void* up_b;           /* (inter) */
} oi2_predictor;

/* ---- library ---------------------------------------------------------- */
const char* oi2_last_error(void);
int oi2_abi_version(void);
/* NEURON_RECORD_BYTES, splitter.py:75-76 */
int oi2_record_bytes(void);

/* ---- cold records ------------------------------------------------------- */
/* Replaces the per-neuron dequant loop of ColdWeightStore.read_neurons
 * (splitter.py:369-403) and dequantize_int4 (splitter.py:111-124): decodes
 * records[slots[k]] for k < n into gate (n, H), up (n, H) and down_t (H, n),
 * fp32, bit-exact.  Slot lookup / absent-id skipping is the caller's. */
int oi2_dequant_records(const uint8_t* records, int32_t n_records, const int32_t* slots,
                        int32_t n, float* gate, float* up, float* down_t, void* stream);

/* ---- norm --------------------------------------------------------------- */
/* nn.RMSNorm as SparseFFNLayer.input_layernorm (engine.py:247-249, :289,
 * :295): out = x * rsqrt(mean(x^2) + eps) * w over rows of H fp16 values. */
int oi2_rmsnorm(const uint16_t* x, const uint16_t* w, int32_t rows, float eps,
                uint16_t* out, void* stream);

/* ---- FFN ---------------------------------------------------------------- */
/* Workspace bytes for oi2_ffn_forward at this batch / hot size and an active
 * list of capacity cold_capacity (n_chunks * chunk). */
size_t oi2_ffn_workspace_bytes(int32_t batch, int32_t n_hot, int32_t cold_capacity);

/* sparse_ffn (engine.py:173-209) and SparseFFNLayer.forward
 * (engine.py:292-312) for `batch` tokens sharing one active cold set:
 *   x_n  = norm_w ? RMSNorm(x) : x
 *   y    = hot(x_n) + cold(x_n)        fp32, hot = fp8 GEMV, cold = fused
 *                                      INT4 gather/dequant/act/down
 *   out  = (add_residual ? x : 0) + y  fp16 (may be NULL)
 *   y32  = y                           fp32 (may be NULL)
 * hot may be NULL or n_hot 0; cold/active may be NULL or empty (then that
 * half contributes nothing, engine.py:194-209).  act: OI2_ACT_*. */
int oi2_ffn_forward(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                    const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active,
                    int32_t act, int32_t act_on_both, int32_t add_residual, uint16_t* out,
                    float* y32, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference (its layers each run their own
 * input_layernorm, engine.py:295).  oi2_ffn_forward for one layer of a chain
 * of layers run back to back (engine.py:424-438) at batch >= 2, with the
 * RMSNorm moved across the layer boundary, for callers that run several
 * layers on one batch (batched decode, prefill chunks):
 *   xn_in       (may be NULL) RMSNorm(x) as the previous call of the chain
 *               wrote it: the call takes it as x_n and launches no norm
 *               (x is still the residual; norm_w is then not read)
 *   next_norm_w (may be NULL) the next layer's norm weight: the call also
 *               writes xn_next = RMSNorm(out) with it and next_eps, (batch, H)
 *               fp16; needs out.  From 17 tokens the final add of the call
 *               writes it, so the next call has one launch fewer.
 * The outputs are the same bits as oi2_ffn_forward calls with their own
 * norms.  Pointers 16-byte aligned; the workspace as oi2_ffn_forward's. */
int oi2_ffn_forward_chain(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                          const uint16_t* xn_in, const oi2_hot* hot, const oi2_cold* cold,
                          const oi2_active* active, int32_t act, int32_t act_on_both, int32_t add_residual,
                          uint16_t* out, float* y32, const uint16_t* next_norm_w, float next_eps,
                          uint16_t* xn_next, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for oi2_sparse_ffn_dense. */
size_t oi2_sparse_ffn_dense_workspace_bytes(int32_t rows, int32_t n_hot, int32_t n_cold);

/* sparse_ffn (engine.py:173-209) on the dense tensors the reference passes
 * it: the hot half as SparseFFNLayer's widened fp16 tensors
 * (engine.py:255-261) and the cold half as ColdWeightStore.read_neurons's
 * fp32 tensors (splitter.py:397-403), gate/up (n, H) row-major and down
 * (H, n) row-major (any n: rows of down need no alignment), each half of one
 * dtype (OI2_DTYPE_F16, _F32 or _BF16); x (rows, H) fp16.
 *   y   = down_h act(gate_h x, up_h x) + down_c act(gate_c x, up_c x)
 *         fp32 accumulation, the halves summed in fp32
 *   y32 = y (may be NULL), out = fp16(y) (may be NULL; not both)
 * n_hot or n_cold 0 drops that half; both 0 gives zeros (engine.py:207-208).
 * gate/up must be 16-byte aligned, each matrix under 2 GiB. */
int oi2_sparse_ffn_dense(const uint16_t* x, int32_t rows, int32_t act, int32_t act_on_both,
                         int32_t n_hot, int32_t hot_dtype, const void* gate_hot, const void* up_hot,
                         const void* down_hot, int32_t n_cold, int32_t cold_dtype,
                         const void* gate_cold, const void* up_cold, const void* down_cold,
                         uint16_t* out, float* y32, void* workspace, size_t workspace_bytes,
                         void* stream);

/* No counterpart in the reference.  oi2_ffn_forward without a workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc): the same single-token
 * decode kernels, the tokens of a batch run one after another (batch >= 2 is
 * not routed to the matrix-core path), their scratch in a static device
 * array of oi2_ffn_noalloc_scratch_bytes() bytes per GPU, held until the
 * process ends.  Limits: n_hot <= 4096 and an expected active count
 * (oi2_active.expected, or the list capacity when 0) of at most
 * oi2_ffn_noalloc_max_expected() records (more items than expected are still
 * processed); larger requests fail with OI2_EINVAL.  Allocates nothing.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race. */
int oi2_ffn_forward_noalloc(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                            const oi2_hot* hot, const oi2_cold* cold, const oi2_active* active,
                            int32_t act, int32_t act_on_both, int32_t add_residual, uint16_t* out,
                            float* y32, void* stream);
/* Bytes of that static scratch array, and its largest expected active count. */
size_t oi2_ffn_noalloc_scratch_bytes(void);
int32_t oi2_ffn_noalloc_max_expected(void);

/* ---- predictor ---------------------------------------------------------- */
size_t oi2_predict_workspace_bytes(const oi2_predictor* p);

/* PredictorRegistry.predict (predictor.py:435-456) with NeuronPredictor's
 * forward / predict_mask (predictor.py:70-79) for `rows` query rows h of
 * dtype h_dtype (OI2_DTYPE_F16, _F32 or _BF16), each cast straight to the
 * predictor dtype as predictor.py:455 does (fp16 and bf16 widen exactly to
 * an fp32 predictor; fp32 rounds to nearest-even for a bf16 one): logits
 * (rows, inter) fp32, probs = sigmoid(logits) fp32 and/or mask (rows, inter)
 * bytes = sigmoid(logit) >= threshold, evaluated as logit >= threshold_logit
 * (log(p / (1 - p)); the float32 sigmoid's saturation point 16.6355 for
 * p == 1).  Any output may be NULL. */
int oi2_predict(const void* h, int32_t h_dtype, int32_t rows, const oi2_predictor* p,
                float threshold_logit, float* logits, float* probs, uint8_t* mask,
                void* workspace, size_t workspace_bytes, void* stream);

/* SparseFFNLayer._cold_ids_for (engine.py:274-283) on device: query =
 * mean over the `batch` rows of RMSNorm(x) (norm_w may be NULL for an already
 * normalised x), predicted-active ids in ascending order, minus ids whose
 * lut entry is < 0 (hot or absent from the section, which read_neurons skips,
 * splitter.py:371-372).  Output is chunked (chunk = 256): counts[c] (device
 * ints, n_chunks = ceil(inter / 256)), slots[c*256 + k] = lut[id] and
 * ids[c*256 + k] = id.  If total is non-NULL it receives the dense count and
 * slots/ids are additionally compacted in place into dense ascending order
 * (dense_slots / dense_ids, length >= inter). */
int oi2_predict_select(const uint16_t* x, int32_t batch, const uint16_t* norm_w, float eps,
                       const oi2_predictor* p, float threshold_logit, const int32_t* lut,
                       int32_t* slots, int32_t* ids, int32_t* counts, int32_t* dense_slots,
                       int32_t* dense_ids, int32_t* total, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---- whole decode step ------------------------------------------------- */
/* One layer of the FFN-only decode stack: the per-layer state that
 * DesdemonaEngine passes to SparseFFNLayer (engine.py:391-398). */
typedef struct oi2_layer {
  oi2_hot hot;
  oi2_cold cold;
  const int32_t* lut;         /* (inter) id -> record slot, -1 for hot / absent */
  const uint16_t* norm_w;     /* (H) fp16 post_attention_layernorm weight */
  oi2_predictor pred;         /* pred.down_w == NULL: no predictor, fetch all */
} oi2_layer;

typedef struct oi2_stack oi2_stack;

/* DesdemonaEngine.forward's layer loop restricted to the FFN sublayers
 * (engine.py:421-438), batch 1: layer 0's cold set is predicted from the
 * input, layer L+1's from layer L's input (the one-sublayer lookahead), and
 * x_{L+1} = x_L + FFN_L(RMSNorm_L(x_L)).  `layers` is copied; the pointed-to
 * device memory must outlive the stack.  Allocates its workspaces here. */
int oi2_stack_create(const oi2_layer* layers, int32_t n_layers, int32_t inter, float eps,
                     int32_t act, int32_t act_on_both, float threshold_logit,
                     oi2_stack** out);
/* One token through all layers: x_out (H) fp16 from x_in (H) fp16. */
int oi2_stack_decode(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, void* stream);
/* The same layers one at a time, for a caller that runs other sublayers
 * (attention) between them, as DesdemonaEngine.forward does
 * (engine.py:421-438), batch 1:
 *   oi2_stack_predict(s, L, x): layer L's cold set predicted from x (the
 *     engine predicts layer 0's from the embedded token, engine.py:422);
 *   oi2_stack_layer(s, L, x_in, x_out): x_out = x_in + FFN_L(RMSNorm_L(x_in))
 *     over the set held for layer L (SparseFFNLayer.forward,
 *     engine.py:292-312), and layer L+1's set predicted from x_in, the
 *     engine's lookahead from layer L's post-attention state
 *     (engine.py:431-436), inside the same two kernels.
 * Both are launched directly on `stream` (a caller may capture them); not
 * with staging.  x_in and x_out must not overlap. */
int oi2_stack_predict(oi2_stack* s, int32_t layer, const uint16_t* x, void* stream);
int oi2_stack_layer(oi2_stack* s, int32_t layer, const uint16_t* x_in, uint16_t* x_out, void* stream);
/* Size the cold gather launch for about `expected` active cold records per
 * layer (any count up to the capacity is still processed; this only sets how
 * many workgroups the pass uses).  0 restores the capacity. */
int oi2_stack_set_expected_active(oi2_stack* s, int32_t expected);
/* Replay the launch sequence through a captured hipGraph (default 1) or launch
 * it directly (0).  Graphs are never used on the NULL stream. */
int oi2_stack_set_graph(oi2_stack* s, int32_t enable);
/* Cold-record staging, the device counterpart of the prefetch pipeline
 * (SparseFFNLayer.submit_cold_fetch / _fetch_cold, engine.py:266-272,
 * 285-290, submitted one layer ahead at engine.py:432-436).  Enabled, each
 * token runs layer L+1's selection (predictor, or a signal for a layer
 * without one) on x_L ahead of layer L's FFN.  One copy kernel on a side
 * stream spans the token: as soon as a layer's list is signalled complete on
 * the device it copies that layer's active records from the layer's record
 * pointer into one of two HBM staging buffers and signals them ready; the
 * FFN's cold workgroups wait on the device for that signal.  The record
 * pointers may then be pinned host memory (hipHostMalloc, or a pinned torch
 * tensor): the copy reads it over PCIe.  Device memory also works (pageable
 * memory is rejected at creation).  copy_workgroups: workgroups of the copy
 * kernel (256 threads, one record per wave at a time, each holding its CU's
 * whole LDS so no FFN workgroup shares the CU), 0 disables staging.  Staged
 * tokens are launched directly, never through a graph.  Every device-side
 * wait is bounded (oi2_stack_set_wait_bound); oi2_stack_status reports one
 * that ran past its bound.  Synchronises the device; drops captured graphs. */
int oi2_stack_set_staging(oi2_stack* s, int32_t copy_workgroups);
/* With staging enabled: decode x_in once (fixing the active sets), time
 * every layer's record copy back to back `reps` times between two hipEvents
 * on `stream`, decode x_in again, and write the mean microseconds per
 * layer copy. */
int oi2_stack_profile_staging(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                              float* gather_us, void* stream);
/* Average kernel durations on the decode path.  Decodes x_in once (fixing
 * every layer's active set), then launches every layer's ffn_up kernel back
 * to back `reps` times between two hipEvents on `stream`, then every layer's
 * ffn_down the same way, then decodes x_in again so the stack's state and
 * x_out are those of x_in.  Waits for the stream and writes the mean
 * microseconds per ffn_up launch and per ffn_down launch. */
int oi2_stack_profile(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                      float* up_us, float* down_us, void* stream);
/* Each layer's output (n_layers, H) fp16 and the active sets of the last
 * decode: counts (n_layers, n_chunks) and slots/ids (n_layers, n_chunks*chunk)
 * in the layout oi2_stack_selection_layout reports, copied to device buffers
 * supplied by the caller (any may be NULL).  Chunk c holds counts[c] ids,
 * ascending; the chunks in order give _cold_ids_for's list (engine.py:274-283). */
int oi2_stack_trace(oi2_stack* s, uint16_t* xs, int32_t* counts, int32_t* slots, int32_t* ids,
                    void* stream);
/* The chunking of the active sets oi2_stack_trace returns: n_chunks chunks of
 * at most `chunk` ids per layer (n_chunks * chunk >= inter). */
int oi2_stack_selection_layout(const oi2_stack* s, int32_t* n_chunks, int32_t* chunk);
/* The whole token as one persistent kernel (default on where supported):
 * every layer's FFN and the lookahead predictor run in a single launch of
 * 256 co-resident workgroups (one per CU) that hand the phases over through
 * device-wide counters, each loading its next layer's weights before it waits
 * (the same layer loop, engine.py:421-438, with no launch boundary between
 * layers).
 * Needs HBM-resident records, bf16 predictors of rank <= 64, n_hot <= 4096
 * and inter <= 16384, and no staging; returns OI2_EUNSUPPORTED otherwise.
 * 0 selects the two-launch-per-layer sequence.  Drops captured graphs. */
int oi2_stack_set_token_kernel(oi2_stack* s, int32_t enable);
/* 1 when decodes run as the persistent token kernel, else 0. */
int32_t oi2_stack_token_kernel(const oi2_stack* s);
/* Waits for `stream`; OI2_EHIP if a device-wide wait of any persistent-kernel
 * token, or a staged token's wait for its records, decoded since the
 * previous call ran past its bound (the tokens decoded since then are to be
 * taken as invalid; the signal words are reset so the next token is clean),
 * else OI2_OK. */
int oi2_stack_status(oi2_stack* s, void* stream);
/* No counterpart in the reference: the bound, in polls, of every device-wide
 * wait of the persistent kernel and of the staged path (default 1 << 20;
 * 1 .. 1 << 24).  A wait past it gives up, so the token is invalid and
 * oi2_stack_status reports it; the kernels still run to their end.  For
 * tests of that failure path.  Drops captured graphs. */
int oi2_stack_set_wait_bound(oi2_stack* s, int32_t polls);
/* Mean microseconds of the persistent token kernel alone: decodes x_in once,
 * then `reps` more launches timed between hipEvents on `stream`; leaves the
 * state of decoding x_in. */
int oi2_stack_profile_token(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, int32_t reps,
                            float* token_us, void* stream);
/* No counterpart in the reference (the reference's profiler times whole
 * layers from the host): decodes x_in once on the persistent token kernel
 * with its control waves stamping s_memrealtime (a 100 MHz counter) at eight
 * points of every layer, and writes the stamps to `trace` (device memory),
 * laid out (min(n_layers, 64), 256 groups, 8 points) as uint64: 0 the U phase
 * starts, 1 its inputs are in LDS (B1), 2 the U products are in LDS (B2),
 * 3 the U arrival is issued, 4 the U signal is seen, 5 the D inputs are in
 * LDS (D1a), 6 the next list is in LDS (D1b), 7 the D arrival is issued.
 * Leaves the state of decoding x_in; the stamps stay in LDS until the end. */
int oi2_stack_trace_token(oi2_stack* s, const uint16_t* x_in, uint16_t* x_out, uint64_t* trace,
                          size_t trace_bytes, void* stream);
int oi2_stack_destroy(oi2_stack* s);

/* ---- cold records read from the split file ------------------------------ */
typedef struct oi2_file_store oi2_file_store;

/* ColdWeightStore.__init__ (splitter.py:317-330) without a device copy: opens
 * cold_weights.bin for reading.  index is cold_index.npy's data, n_sections
 * pairs (section byte offset, n_cold) as uint64 (splitter.py:188, 256; the
 * (layer, expert) grid flattened, section = layer * n_experts + expert).
 * direct_io = 0 maps the file (splitter.py:322-323) and copies records out
 * of the mapping; 1 opens it with O_DIRECT and reads whole 4 KB pages into
 * aligned bounce buffers, bypassing the page cache (OI2_EUNSUPPORTED where
 * the file system refuses O_DIRECT).  threads: reader threads (1 .. 64),
 * each taking a contiguous run of a request's records in file order. */
int oi2_file_store_open(const char* path, const uint64_t* index, int32_t n_sections, int32_t direct_io,
                        int32_t threads, oi2_file_store** out);
/* The byte side of ColdWeightStore.read_neurons (splitter.py:354-403):
 * records slots[0..n) of `section` (record k at section offset + 16 + 6400 k)
 * copied whole, in request order (duplicates kept), into host memory
 * dst (n x 6400 bytes; pinned memory lets one hipMemcpyAsync move the
 * batch to the device).  Slot lookup from neuron ids is the caller's (an
 * absent id has no slot and is skipped before the call, as read_neurons
 * skips it).  Synchronous: returns once every record is in place; OI2_EIO
 * if a read fails.  One call at a time per handle. */
int oi2_file_store_read(oi2_file_store* fs, int32_t section, const int32_t* slots, int32_t n,
                        uint8_t* dst);
/* The cold fetch of SparseFFNLayer._fetch_cold (engine.py:266-272:
 * read_neurons, then .to(device)) for a caller's worker thread: reads the
 * records as oi2_file_store_read into host_buf (pinned, n x 6400 bytes), then
 * enqueues one hipMemcpyAsync of them to dst (device, n x 6400 bytes) on
 * `stream` and returns; host_buf must stay untouched until that copy has
 * run (an event recorded on `stream` after the call marks it). */
int oi2_file_store_stage(oi2_file_store* fs, int32_t section, const int32_t* slots, int32_t n,
                         uint8_t* host_buf, uint8_t* dst, void* stream);
/* O_DIRECT reads only: records whose page ranges lie within `bytes` of each
 * other are read with one pread (the gap read and dropped); 0 merges only
 * touching ranges.  Default 16384; at most 524288.  No reference
 * counterpart: a tuning knob of the direct-I/O reads (splitter.py:322-323
 * reads through a mapping). */
int oi2_file_store_set_read_gap(oi2_file_store* fs, int64_t bytes);
/* ColdWeightStore.close (splitter.py:405-407). */
int oi2_file_store_close(oi2_file_store* fs);

/* ---- grouped-query attention (decode) ----------------------------------- */
/* One layer's attention weights as GroupedQueryAttention holds them
 * (engine.py:66-88): q_proj, k_proj, v_proj, o_proj kept at fp8 e4m3fn,
 * the reference's storage (splitter.py:175-177), unscaled; row-major
 * (out_features, in_features).  head_dim = H / n_q must be 128. */
typedef struct oi2_attn {
  int32_t n_q;                /* query heads: H / 128 */
  int32_t n_kv;               /* kv heads; n_q / n_kv in {1, 2, 4, 8} */
  const uint8_t* wq;          /* (n_q * 128, H) */
  const uint8_t* wk;          /* (n_kv * 128, H) */
  const uint8_t* wv;          /* (n_kv * 128, H) */
  const uint8_t* wo;          /* (H, n_q * 128) */
  const uint16_t* norm_w;     /* (H) fp16 input_layernorm (ones for nn.RMSNorm's default) */
} oi2_attn;

/* Workspace of oi2_attn_forward for batch x seq query rows attending to
 * positions [0, past + seq): q, the attention output, and the sequence
 * split's partial sums only when past + seq exceeds 1024 positions (the
 * splits the launch picks for that span); 0 for invalid sizes. */
size_t oi2_attn_workspace_bytes(int32_t batch, int32_t seq, int32_t n_q, int32_t n_kv, int32_t past);
/* GroupedQueryAttention.forward (engine.py:90-125) for x (batch, seq, H)
 * fp16: x_n = RMSNorm(x); q, k, v = x_n W^T; RoPE on q and k with cos / sin
 * (seq, 64) fp32, the call's positions as the engine slices them
 * (engine.py:414-416; rounded to fp16 as engine.py:153-154 does); k and v
 * written into k_cache / v_cache (batch, n_kv, cache_cap, 128) fp16 at
 * positions past .. past + seq - 1 (the reference's torch.cat,
 * engine.py:105-109, done in place: positions below past are the cache);
 * attention of each query over positions [0, past + seq), causal when
 * `causal` (the reference: causal exactly when it has no cache,
 * engine.py:121); out (batch * seq, H) fp16 = o_proj(attn), the tensor the
 * reference returns.  x_out, if not NULL, receives fp16(x + out), the
 * engine's residual add (engine.py:427).  Three kernels on `stream`. */
int oi2_attn_forward(const uint16_t* x, int32_t batch, int32_t seq, const oi2_attn* w, float eps,
                     const float* cos, const float* sin, uint16_t* k_cache, uint16_t* v_cache,
                     int32_t cache_cap, int32_t past, int32_t causal, uint16_t* out, uint16_t* x_out,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---- split writer ------------------------------------------------------- */
/* Bytes of one cold_weights.bin section with n_cold records: the 16-byte
 * <HHIq header, n_cold x 6400, zero padding to a 4096 multiple
 * (splitter.py:229-254).  0 for a negative count. */
size_t oi2_section_bytes(int32_t n_cold);
/* The cold half of split_dense's per-layer loop on the device
 * (splitter.py:229-256, quantize_int4 splitter.py:81-108): quantise n
 * neurons to INT4 records and frame them as one section, byte-identical to
 * the reference writer's.  Record k stores nids[k]; its gate, up and down
 * vectors are read as
 *   src[m][rows[k] * row_stride[m] + e * elem_stride[m]],  e = 0 .. 4095,
 * for m = 0 (gate), 1 (up), 2 (down), fp32 device memory.  With the model's
 * gate/up (I, H), down (H, I), rows = nids, row_stride = {H, H, 1} and
 * elem_stride = {1, 1, I} this is gate[nid], up[nid] and down[:, nid].
 * nids and rows are device arrays of n; row_stride and elem_stride are host
 * arrays of 3.  section: 16-byte aligned device memory of at least
 * oi2_section_bytes(n) bytes (header, records and padding all written). */
int oi2_quantize_section(int32_t layer, int32_t expert, int32_t n, const uint16_t* nids,
                         const int32_t* rows, const float* gate, const float* up, const float* down,
                         const int64_t* row_stride, const int64_t* elem_stride, uint8_t* section,
                         size_t section_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* OI2_H */
