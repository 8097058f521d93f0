// kernels.h -- host-side launch interface of the gfx950 kernels.
//
// Every launcher takes plain device pointers and an explicit stream, performs
// no allocation and no synchronisation, and is therefore safe to record into a
// hipGraph.  Shape checks live in the callers (C-ABI layer and LanguageModel).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mmr {

// ---------------------------------------------------------------- GEMV ----
// y = W x with W fp16 row-major [rows][k] (weights streamed from HBM once),
// x/y fp32, fp32 accumulation.
enum GemvPrologue : int {
  kProPlain = 0,       // x used as given
  kProRmsNorm = 1,     // x := x * (scale * norm_w)      decoder_layer.cpp:32-42
  kProRmsNormFinal = 2,// x := (x * scale) * norm_w      language_model.cpp:24-38
  kProEmbedRmsNorm = 3 // x := embed[seq[*pos]] (fp16 -> fp32), then kProRmsNorm;
                       //      block 0 also stores the raw row to h_out
};

enum GemvEpilogue : int {
  kEpiStore = 0,     // y[r] = dot
  kEpiResidual = 1,  // y[r] = residual[r] + dot
  kEpiSwiGlu = 2,    // rows interleaved (gate_0, up_0, gate_1, up_1, ...):
                     //   y[i] = silu(gate_i) * up_i      decoder_layer.cpp:175-182
  kEpiArgmax = 3     // y[r] = dot (optional), token = first argmax over r
};

struct GemvArgs {
  const __half* w = nullptr;
  int rows = 0;
  int k = 0;
  const float* x = nullptr;
  const float* norm_w = nullptr;
  float eps = 0.0f;
  // kProEmbedRmsNorm
  const __half* embed = nullptr;
  const int32_t* seq = nullptr;
  const int32_t* pos = nullptr;
  int vocab = 0;
  float* h_out = nullptr;
  // outputs
  float* y = nullptr;
  const float* residual = nullptr;
  // kEpiArgmax
  unsigned long long* best = nullptr;  // packed (value, ~index) key, zero before first use
  unsigned int* counter = nullptr;      // zero before first use
  int32_t* token_out = nullptr;
  // optional decode-step bookkeeping with kEpiArgmax: the step at position
  // p = *step_pos writes its prediction to step_seq[p + 1] when
  // p + 1 >= *step_prompt_len, then advances *step_pos.
  int32_t* step_seq = nullptr;
  int32_t* step_pos = nullptr;
  const int32_t* step_prompt_len = nullptr;
  int seq_len = 0;
};

struct GemvPlan {
  int lanes_per_row = 32;  // 16, 32 or 64
  int rows_per_group = 1;  // 1, 2 or 4 (even for kEpiSwiGlu)
  int chunks_per_lane = 3; // 16-byte chunks of a row per lane
  int blocks = 0;
};

// Picks a launch shape; lanes_per_row / rows_per_group of 0 mean "auto".
// Returns false when k is not a multiple of 8 or exceeds the supported range.
bool gemv_plan(int rows, int k, GemvEpilogue epi, int lanes_per_row, int rows_per_group, GemvPlan* plan);
hipError_t launch_gemv(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, const GemvPlan& plan,
                       hipStream_t stream);
constexpr int kGemvBlock = 256;

// ----------------------------------------------------------- attention ----
// GQA decode attention for one query token over a resident KV cache laid out
// [kv_head][capacity][head_dim], split along the context into `splits` ranges
// per KV head and merged with a log-sum-exp combine by the last block.
enum AttnMode : int {
  kAttnFused = 0,     // q/k RMSNorm + RoPE from the raw projection, append k/v at
                      // index *pos, attend over *pos + 1 keys
  kAttnFromCache = 1  // q given (already normalised/rotated), attend over `tokens` keys
};

enum KvDtype : int { kKvF16 = 0, kKvF32 = 1 };

struct AttnArgs {
  const float* qkv = nullptr;  // fused: [Hq*D + 2*Hkv*D]
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* rope_cos = nullptr;  // [max_pos][D/2]
  const float* rope_sin = nullptr;
  const int32_t* pos = nullptr;     // fused: index of the new token
  const float* q = nullptr;         // from-cache: [Hq*D]
  int tokens = 0;                   // from-cache: cached keys
  void* kcache = nullptr;
  void* vcache = nullptr;
  int capacity = 0;
  int max_pos = 0;
  int hq = 0, hkv = 0, d = 0;
  int splits = 1;
  float* part = nullptr;            // [Hkv][splits][R][D+2]
  unsigned int* counters = nullptr; // [Hkv], zero on first use, re-armed by the kernel
  float* out = nullptr;             // [Hq*D]
  int32_t* err = nullptr;           // set to 1 when *pos is out of range
};

constexpr int kAttnMaxGroup = 8;  // Hq / Hkv supported
size_t attention_partial_floats(int hq, int hkv, int d, int splits);
int attention_tile_tokens(int d);
bool attention_supported(int hq, int hkv, int d);
hipError_t launch_attention(const AttnArgs& a, AttnMode mode, KvDtype kv, hipStream_t stream);

// qkv post-process as a standalone op (reference K2): per-head q/k RMSNorm +
// RoPE at `position`, q -> query_out, k/v appended at cache index `index`.
struct QkvPostArgs {
  const float* qkv = nullptr;
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int position = 0;
  int index = 0;
  void* kcache = nullptr;
  void* vcache = nullptr;
  int capacity = 0;
  int hq = 0, hkv = 0, d = 0;
  float* query_out = nullptr;
};
hipError_t launch_qkv_postprocess(const QkvPostArgs& a, KvDtype kv, hipStream_t stream);

// ------------------------------------------------------------- support ----
hipError_t launch_rms_norm_rows(const float* in, const float* w, float eps, int rows, int cols, float* out,
                                hipStream_t stream);
hipError_t launch_add(const float* a, const float* b, int64_t n, float* out, hipStream_t stream);
hipError_t launch_swiglu_rows(const float* gate_up, int rows, int cols, float* out, hipStream_t stream);
hipError_t launch_embedding_gather(const __half* table, const int32_t* ids, int tokens, int vocab, int hidden,
                                   float* out, int32_t* err, hipStream_t stream);

}  // namespace mmr
