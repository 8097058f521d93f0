// decoder_layer.h -- one dense decoder layer's decode step on the device.
//
// Counterpart of the reference's run_dense_decoder_layer_device
// (decoder_layer.h:50-80, decoder_layer.cpp:617-659) and its LayerKvCache
// (decoder_layer.h:40-48): the same op order (norm -> fused QKV -> q/k norm +
// RoPE -> KV append -> attention -> O + residual -> norm -> gate_up + SwiGLU
// -> down + residual) as the four GEMVs and one attention launch the
// whole-model step uses, over a caller-owned hidden vector, a caller-owned
// KV cache and a position held in device memory.  Nothing here allocates or
// synchronises, so a call can be recorded into a hipGraph.
#pragma once

#include "config.h"
#include "device.h"
#include "device_model.h"
#include "weights.h"
#include "../kernels/kernels.h"

#include <cstddef>
#include <cstdint>
#include <memory>

namespace minimind::model {

// Launch shapes of the layer's four projections; the whole-model step uses
// the same ones.
struct LayerPlans {
  mmr::GemvPlan qkv, o, gate_up, down;
};
LayerPlans plan_layer(const MiniMindConfig& c);

// RoPE frequencies of the reference formula (decoder_layer.cpp:114):
// inv_freq[i] = 1 / powf(theta, 2i / d).
std::vector<float> rope_inv_freq(const MiniMindConfig& c);

// Device copy of one layer (the reference's AscendLayerWeights,
// ascend_weights.h:15-33): fp16 matrices in the runtime's fused layout (qkv
// rows [q; k; v], gate/up rows interleaved), fp32 gains, and the config's
// RoPE frequencies.  upload() owns its memory; view() shares a loaded
// model's layer and keeps that model's weights alive.
struct DeviceLayerWeights {
  MiniMindConfig cfg;
  LayerDev w;
  LayerPlans plans;
  const float* inv_freq = nullptr;
  std::shared_ptr<const void> owner;

  static std::shared_ptr<DeviceLayerWeights> upload(const MiniMindConfig& c, const DenseLayerWeights& host);
  static std::shared_ptr<DeviceLayerWeights> view(const std::shared_ptr<const DeviceModel>& model, int64_t layer);
};

// Validates one layer's host weights against the config (sizes of every
// member), as the LanguageModel constructor does for each layer.
void check_layer_weights(const MiniMindConfig& c, const DenseLayerWeights& w);
// Uploads one layer in the fused fp16 layout into `ar` (planned with
// plan_layer_bytes); returns the device view and adds its bytes to *bytes.
std::size_t plan_layer_bytes(const MiniMindConfig& c);
LayerDev upload_layer(Arena& ar, const MiniMindConfig& c, const DenseLayerWeights& w);

// One call's buffers: the reference's hidden / out DeviceTensors, its
// LayerKvCache and the per-call scratch.
struct DecoderLayerIo {
  const float* hidden = nullptr;      // [H] fp32
  float* out = nullptr;               // [H] fp32, may alias hidden
  const int32_t* position = nullptr;  // device int32: RoPE position and cache row of the new token
  mmr::KvSegs seg;                    // the layer's cache segments (KvStore::layer)
  int rows = 0;                       // backed cache rows
  int capacity = 0;                   // usable positions, all backed (a position >= capacity sets *err)
  mmr::KvDtype kv = mmr::kKvF32;
  int splits = 1;                     // attention context splits
  float* workspace = nullptr;         // decoder_layer_workspace_floats(cfg, splits) floats
  int32_t* err = nullptr;             // device int32, set to 1 on an out-of-range position
};

std::size_t decoder_layer_workspace_floats(const MiniMindConfig& c, int splits);
void enqueue_decoder_layer(const DeviceLayerWeights& w, const DecoderLayerIo& io, hipStream_t stream);

}  // namespace minimind::model
