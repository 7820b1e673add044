// Argument blocks and kernel declarations shared by the decode-path sources.
#pragma once
#include "oi2_device.h"

namespace oi2 {

constexpr int kThreads = 256;
constexpr int kRowsPerDownWG = 16;
constexpr int kSelChunk = 256;
constexpr int kMaxChunks = 256;
constexpr int kMaxColdWG = 256;
constexpr int kRecordsPerColdWG = 8;   // target records per cold workgroup (2 per wave)
constexpr int kLdsRed = kH + kH / 32;

struct ActiveList {
  const int32_t* slots;
  const int32_t* counts;
  int n_chunks;
  int chunk;
};

struct UpArgs {
  const uint16_t* x;        // (H) fp16 token
  const uint16_t* norm_w;   // (H) fp16 or null: x is already normalised
  float eps;
  int relu, both;
  // hot
  int n_hot;
  const uint8_t* gate_q;
  const uint8_t* up_q;
  const float* gate_s;
  const float* up_s;
  const float* hot_gbias;
  float* h_hot;
  // cold
  const uint8_t* records;
  int n_records;
  const float* cold_gbias;
  ActiveList act;
  float* partials;          // (wg_cold, H)
  int* n_part_out;          // cold workgroup 0 publishes how many partial rows it used
  // predictor down projection of the lookahead layer
  const void* pd_w;
  int pd_rank;
  int pd_bf16;
  const uint16_t* pd_norm_w;  // norm applied to x for the query, or null
  const float* pd_q;          // precomputed query (H), or null
  float* pd_z;                // (rank)
  int wg_cold, wg_pred, wg_hot;
};

struct DownArgs {
  const uint16_t* res;      // residual (H) fp16 or null
  const float* h_hot;
  int n_hot;
  int down_stride;
  const uint8_t* down_q;
  const float* down_s;
  const float* partials;
  int n_partials;           // used when n_part_in is null
  const int* n_part_in;     // partial rows written by ffn_up's cold workgroups
  uint16_t* out;
  uint16_t* out2;
  float* y32;
  // predictor up projection + selection
  const void* pu_w;
  const void* pu_b;
  int pu_rank;
  int pu_bf16;
  int inter;
  const float* pd_z;
  float thr;
  const int32_t* lut;
  int32_t* sel_slots;
  int32_t* sel_ids;
  int32_t* sel_counts;
  float* logits_out;
  float* probs_out;
  uint8_t* mask_out;
  int wg_pred, wg_down;
};

__global__ void k_ffn_up(UpArgs a);
__global__ void k_ffn_down(DownArgs a);
__global__ void k_pred_up(UpArgs a);
__global__ void k_pred_down(DownArgs a);
__global__ void k_compact_dense(const int32_t* slots, const int32_t* ids, const int32_t* counts,
                                int n_chunks, int32_t* dslots, int32_t* dids, int32_t* total);

}  // namespace oi2
