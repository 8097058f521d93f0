// language_model.h -- device-resident MiniMind dense model on gfx950.
//
// Mirrors the reference C++ API (language_model.h:22-49, runtime_loader.h:9-10)
// so callers switch by relinking: LanguageModel(config, weights), make_state,
// forward_token, forward_next_token, prefill_next_token, generate_stream,
// generate, argmax_token, load_runtime_language_model,
// has_runtime_language_model.
//
// Differences a caller can observe (all deliberate):
//  * there is no CPU path: every step runs the HIP kernels; shapes the kernels
//    do not support raise std::invalid_argument at construction instead of
//    falling back silently;
//  * weights live on the GPU as fp16 (round to nearest even at upload), norm
//    gains and activations stay fp32;
//  * the KV cache has a capacity chosen in make_state; exceeding it raises
//    std::length_error.  Device memory backs it in 64-token pages grouped in
//    doubling segments, added as the context reaches them (512 positions up
//    front), never moved or reallocated;
//  * one decode step is one hipGraph replay; the next token, the position and
//    the token sequence stay in device memory between steps.
#pragma once

#include "config.h"
#include "weights.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace minimind::model {

enum class KvCacheDtype : int { kFloat16 = 0, kFloat32 = 1 };

struct DeviceModel;
struct DeviceState;

// Per-sequence decode state (reference DecoderState, language_model.h:22-25).
// Owns the device KV cache, the token sequence and the captured step graphs.
struct DecoderState {
  DecoderState();
  ~DecoderState();
  DecoderState(DecoderState&&) noexcept;
  DecoderState& operator=(DecoderState&&) noexcept;
  DecoderState(const DecoderState&) = delete;
  DecoderState& operator=(const DecoderState&) = delete;

  int64_t position = 0;  // tokens already in the cache (host mirror)
  int64_t capacity() const;
  // KV positions backed by device memory so far (the cache grows in
  // doubling segments as the context reaches them) and the bytes they hold.
  int64_t kv_backed() const;
  std::size_t kv_device_bytes() const;
  KvCacheDtype kv_dtype() const;
  void* stream() const;  // hipStream_t all work of this state runs on
  std::unique_ptr<DeviceState> device;
};

struct BatchDeviceState;

// A batch of independent sequences decoded in lockstep, each at its own
// position, with a paged KV cache (64-token pages mapped through a per-sequence
// page table).  The reference has no batched state (its DecoderState holds one
// sequence, language_model.h:22-25); this serves BASELINE configs[4].
struct BatchState {
  BatchState();
  ~BatchState();
  BatchState(BatchState&&) noexcept;
  BatchState& operator=(BatchState&&) noexcept;
  BatchState(const BatchState&) = delete;
  BatchState& operator=(const BatchState&) = delete;

  int64_t steps = 0;  // batched steps run since the prompts were set (host mirror)
  int64_t batch() const;
  int64_t capacity() const;  // positions per sequence
  void* stream() const;
  std::unique_ptr<BatchDeviceState> device;
};

class LanguageModel {
 public:
  LanguageModel(MiniMindConfig config, DenseModelWeights weights);
  ~LanguageModel();
  LanguageModel(LanguageModel&&) noexcept;
  LanguageModel& operator=(LanguageModel&&) noexcept;

  const MiniMindConfig& config() const noexcept { return config_; }

  // capacity 0 = max_position_embeddings.
  DecoderState make_state() const;
  DecoderState make_state(int64_t capacity, KvCacheDtype kv = KvCacheDtype::kFloat32) const;

  std::vector<float> forward_token(int32_t token, DecoderState& state) const;
  int32_t forward_next_token(int32_t token, DecoderState& state) const;
  int32_t prefill_next_token(const std::vector<int32_t>& prompt_tokens, DecoderState& state) const;
  void generate_stream(const std::vector<int32_t>& prompt_tokens, int64_t max_new_tokens,
                       const std::function<void(int32_t)>& on_token) const;
  std::vector<int32_t> generate(const std::vector<int32_t>& prompt_tokens, int64_t max_new_tokens) const;

  // ---- device-resident fast path (no host round trip per token) ----
  // Enqueue `n` greedy steps; step i consumes seq[position] (the token the
  // previous step produced) and appends its prediction.  `first_token`
  // (if >= 0) is written to seq[position] first.  Returns immediately.
  void enqueue_decode(DecoderState& state, int64_t n, int32_t first_token = -1) const;
  // Upload prompt tokens and run them through the model (chunked batched
  // prefill kernels, or one decode step per token where the GEMM shapes are
  // unsupported); the prompt's last row predicts the first generated token.
  void enqueue_prefill(DecoderState& state, const std::vector<int32_t>& prompt_tokens) const;
  // Wait for the state's stream and raise if a kernel flagged an error.
  void synchronize(DecoderState& state) const;
  // seq[first, first + count) of the state (prompt and generated ids).
  std::vector<int32_t> read_sequence(DecoderState& state, int64_t first, int64_t count) const;
  // Logits of the last executed step.
  std::vector<float> read_logits(DecoderState& state) const;
  // Enqueue `count` launches of one step kernel (0 qkv, 1 attention, 2 o,
  // 3 gate_up, 4 down, 5 lm_head, 6 argmax finalize without bookkeeping),
  // cycling over layers from `layer`.  Used to time single kernels;
  // overwrites scratch buffers.
  void enqueue_kernel(DecoderState& state, int kernel, int64_t layer, int64_t count) const;
  // Average time per launch (us) of `count` back-to-back launches of one step
  // kernel, from HIP events on the state's stream.  With graphs enabled the
  // launches are captured into one hipGraph (a dependent chain, as in the
  // step) and replayed once after a warm replay, so host launch overhead never
  // paces them; otherwise they are launched eagerly after 32 warm launches.
  double time_kernel(DecoderState& state, int kernel, int64_t layer, int64_t count) const;
  // Reset position to 0 (the cache contents are overwritten as it refills).
  void reset_state(DecoderState& state) const;
  // Back KV positions [0, positions) now (at most the capacity), so decoding
  // up to there allocates nothing; otherwise segments are added as the
  // context reaches them.
  void reserve_kv(DecoderState& state, int64_t positions) const;

  // ---- batched decode (independent sequences in lockstep) ----
  BatchState make_batch_state(int64_t batch, int64_t capacity, KvCacheDtype kv = KvCacheDtype::kFloat16) const;
  // Upload one prompt per sequence (lengths may differ) into a fresh batch and
  // run max-length batched steps: sequence b consumes its prompt, then its own
  // predictions, so each sequence decodes exactly as it would alone.
  void enqueue_batch_prefill(BatchState& state, const std::vector<std::vector<int32_t>>& prompts) const;
  // `n` more batched steps: every sequence appends one greedy token per step.
  void enqueue_batch_decode(BatchState& state, int64_t n) const;
  void synchronize(BatchState& state) const;
  std::vector<int32_t> read_batch_sequence(BatchState& state, int64_t index, int64_t first, int64_t count) const;
  // Logits of sequence `index` at the last executed step.
  std::vector<float> read_batch_logits(BatchState& state, int64_t index) const;

  const DeviceModel& device_model() const { return *device_; }
  std::shared_ptr<const DeviceModel> shared_device_model() const { return device_; }
  std::size_t device_weight_bytes() const;

 private:
  void launch_step(DecoderState& state) const;
  void launch_batch_step(BatchState& state) const;

  MiniMindConfig config_;
  std::shared_ptr<DeviceModel> device_;
};

int32_t argmax_token(const std::vector<float>& logits);
LanguageModel load_runtime_language_model(const std::string& model_dir);
// The reference's built-in toy model (language_model.cpp:415-470): one layer,
// hidden 4, 2 query / 1 KV heads of head_dim 2, FFN 8, vocab 8, 16
// positions, identity projections and fixed embedding / lm_head tables.  The
// CLI tools fall back to it when no model directory is given.  Its shapes run
// on the small-model step kernel.
std::pair<MiniMindConfig, DenseModelWeights> toy_model_weights();
LanguageModel make_toy_language_model();
bool has_runtime_language_model(const std::string& model_dir);

}  // namespace minimind::model
