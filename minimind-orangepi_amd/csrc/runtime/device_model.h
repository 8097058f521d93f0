// device_model.h -- device copy of the model weights (internal to the runtime).
#pragma once

#include "config.h"
#include "device.h"
#include "../kernels/kernels.h"

#include <cstddef>
#include <vector>

namespace minimind::model {

struct LayerDev {
  const float* input_norm = nullptr;
  const float* post_norm = nullptr;
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  const __half* qkv = nullptr;      // [(Hq + 2 Hkv) d][H]  rows q | k | v
  const __half* o = nullptr;        // [H][Hq d]
  const __half* gate_up = nullptr;  // [2F][H]  rows gate_0, up_0, gate_1, up_1, ...
  const __half* down = nullptr;     // [H][F]
};

struct DeviceModel {
  MiniMindConfig cfg;
  Arena arena;
  const __half* embed = nullptr;    // [V][H]
  const __half* lm_head = nullptr;  // [V][H] (aliases embed when identical)
  const float* final_norm = nullptr;
  std::vector<LayerDev> layers;
  const float* inv_freq = nullptr;  // [d/2] RoPE frequencies, formula of decoder_layer.cpp:114
  mmr::GemvPlan plan_qkv, plan_o, plan_gu, plan_down, plan_lm;
  bool gemm_prefill = false;  // every projection's K suits the prefill GEMM
  // Shapes below the GEMV / attention kernels' (the reference's toy model):
  // every step is one launch of the one-workgroup kernel (tiny.hip).
  bool tiny = false;
  std::size_t weight_bytes = 0;
};

// Floats of the prefill split-K partial buffer for chunks of up to
// `chunk_rows` rows: the largest splits x rows x N over the four projections
// (QKV, O, gate_up, down) and every row count 1..chunk_rows.  Fewer rows can
// take more K splits (the GEMM tiling aims at a block count), so the product
// is not largest at chunk_rows.  Host arithmetic only.
int64_t prefill_partial_floats(const MiniMindConfig& cfg, int64_t chunk_rows);

// Attention splits of a single-sequence decode step over n_keys keys with
// `tile`-key tiles (the step graph's bucket).  Never decreases as n_keys
// grows: the KV backing reserved before a graph is captured covers every
// context its split count serves.  Host arithmetic only.
int decode_attention_splits(int64_t n_keys, int tile);

}  // namespace minimind::model
