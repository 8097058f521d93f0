// weights.h -- host-side weights, the MMRTW001 runtime format, and the seeded
// synthetic-weight generator used by tests and benchmarks.
#pragma once

#include "config.h"

#include <cstdint>
#include <string>
#include <vector>

namespace minimind::model {

// Same members as the reference's dense layer (decoder_layer.h:19-35, dense
// subset): fp32 row-major matrices [out][in].
struct DenseLayerWeights {
  std::vector<float> input_norm;
  std::vector<float> post_attention_norm;
  std::vector<float> q_norm;
  std::vector<float> k_norm;
  std::vector<float> q_proj;
  std::vector<float> k_proj;
  std::vector<float> v_proj;
  std::vector<float> o_proj;
  std::vector<float> gate_proj;
  std::vector<float> up_proj;
  std::vector<float> down_proj;
};

// language_model.h:15-21 of the reference.
struct DenseModelWeights {
  std::vector<float> embed_tokens;
  std::vector<DenseLayerWeights> layers;
  std::vector<float> final_norm;
  std::vector<float> lm_head;
};

// MMRTW001 (runtime_loader.cpp:121-167 of the reference): magic "MMRTW001",
// then per tensor u64 name length, name, u64 element count, fp32 LE payload, in
// the fixed order embed, norm, lm_head, then per layer input_layernorm,
// post_attention_layernorm, q_norm, k_norm, q, k, v, o, gate, up, down.
DenseModelWeights read_weights(const MiniMindConfig& config, const std::string& path);
void write_weights(const MiniMindConfig& config, const DenseModelWeights& weights, const std::string& path);
void write_config(const MiniMindConfig& config, const std::string& path);

// Seeded synthetic weights.  SplitMix64(seed) drives Box-Muller normals:
// element i of the drawn stream uses the pair p = i / 2 built from draws
// 2p+1 and 2p+2 (u = (draw >> 11) * 2^-53, r = sqrt(-2 ln(1 - u1)),
// cos(2 pi u2) for even i, sin for odd i); value = float(std * z), rounded to
// the nearest fp16 (ties to even) when round_fp16.  Matrices are drawn in
// MMRTW001 order; RMSNorm gains are 1.0 and draw nothing; with
// tie_word_embeddings lm_head copies the embedding.
DenseModelWeights synthesize_weights(const MiniMindConfig& config, uint64_t seed, double std, bool round_fp16);
// Streams the same weights to <dir>/weights.bin and writes the config file.
void write_synthetic_model(const std::string& dir, const MiniMindConfig& config, uint64_t seed, double std,
                           bool round_fp16);
// `count` token ids floor(u * vocab) from SplitMix64(seed) draws 1..count.
std::vector<int32_t> synthesize_prompt(uint64_t seed, int64_t count, int64_t vocab);
// Fills out[0..count) with stream elements [first, first + count).
void synthesize_normals(uint64_t seed, uint64_t first, uint64_t count, double std, bool round_fp16, float* out);

// IEEE binary16 round-to-nearest-even conversions.
uint16_t float_to_half(float value);
float half_to_float(uint16_t value);

}  // namespace minimind::model
