// capi.cpp -- extern "C" boundary of libmmr.so (declared in include/mmr.h).
//
// Thin: argument checks, exception -> status translation, then a kernel
// launcher (op-level) or the LanguageModel (model-level).
#include "../../include/mmr.h"

#include "kernels/kernels.h"
#include "host_ops.h"
#include "runtime/decoder_layer.h"
#include "runtime/device.h"
#include "runtime/device_model.h"
#include "runtime/kv_store.h"
#include "runtime/prefill_layer.h"
#include "runtime/language_model.h"

#include <algorithm>
#include <cstdint>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

using namespace minimind::model;

struct mmr_model {
  std::unique_ptr<LanguageModel> lm;
};
struct mmr_state {
  DecoderState st;
};
struct mmr_batch_state {
  BatchState st;
};
struct mmr_rope_table {
  DeviceBuffer inv_freq;  // [d/2]: 1 / powf(theta, 2i / d); cos/sin(pos * inv_freq) on the device
  int64_t max_positions = 0;
  int64_t head_dim = 0;
  const float* data() const { return static_cast<const float*>(inv_freq.data()); }
};
struct mmr_kv_cache {
  minimind::model::KvStore store;  // one layer
  int dtype = MMR_KV_F32;
  int64_t prefilled = 0;  // rows a prefill-layer call filled; 0 = empty (reset clears it)
  int64_t kv_heads() const { return store.kv_heads(); }
  int64_t head_dim() const { return store.head_dim(); }
  int64_t capacity() const { return store.capacity(); }
  int64_t usable() const { return std::min(store.capacity(), store.backed()); }  // backed positions
  mmr::KvDtype kv() const { return dtype == MMR_KV_F16 ? mmr::kKvF16 : mmr::kKvF32; }
};
struct mmr_layer_weights {
  std::shared_ptr<DeviceLayerWeights> w;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return MMR_OK;
  } catch (const std::invalid_argument& e) {
    return fail(MMR_ERR_INVALID_ARGUMENT, e.what());
  } catch (const std::out_of_range& e) {
    return fail(MMR_ERR_OUT_OF_RANGE, e.what());
  } catch (const std::length_error& e) {
    return fail(MMR_ERR_LENGTH, e.what());
  } catch (const std::exception& e) {
    return fail(MMR_ERR_RUNTIME, e.what());
  } catch (...) {
    return fail(MMR_ERR_RUNTIME, "unknown error");
  }
}

void require(bool ok, const char* msg) {
  if (!ok) throw std::invalid_argument(msg);
}

hipStream_t as_stream(mmr_stream_t s) { return static_cast<hipStream_t>(s); }

void hip(hipError_t st, const char* what) { check_hip(st, what); }

MiniMindConfig to_cpp(const mmr_config& c) {
  MiniMindConfig m = default_minimind_config();
  m.hidden_size = c.hidden_size;
  m.num_hidden_layers = c.num_hidden_layers;
  m.vocab_size = c.vocab_size;
  m.num_attention_heads = c.num_attention_heads;
  m.num_key_value_heads = c.num_key_value_heads;
  m.head_dim = c.head_dim;
  m.intermediate_size = c.intermediate_size;
  m.max_position_embeddings = c.max_position_embeddings;
  m.bos_token_id = c.bos_token_id;
  m.eos_token_id = c.eos_token_id;
  m.use_moe = c.use_moe != 0;
  m.tie_word_embeddings = c.tie_word_embeddings != 0;
  m.rms_norm_eps = c.rms_norm_eps;
  m.rope_theta = c.rope_theta;
  m.moe_intermediate_size = c.intermediate_size;
  return m;
}

mmr_config to_c(const MiniMindConfig& m) {
  mmr_config c;
  c.hidden_size = m.hidden_size;
  c.num_hidden_layers = m.num_hidden_layers;
  c.vocab_size = m.vocab_size;
  c.num_attention_heads = m.num_attention_heads;
  c.num_key_value_heads = m.num_key_value_heads;
  c.head_dim = m.head_dim;
  c.intermediate_size = m.intermediate_size;
  c.max_position_embeddings = m.max_position_embeddings;
  c.bos_token_id = m.bos_token_id;
  c.eos_token_id = m.eos_token_id;
  c.use_moe = m.use_moe ? 1 : 0;
  c.tie_word_embeddings = m.tie_word_embeddings ? 1 : 0;
  c.rms_norm_eps = m.rms_norm_eps;
  c.rope_theta = m.rope_theta;
  return c;
}

void check_matvec_shape(int64_t rows, int64_t cols) {
  require(rows > 0 && cols > 0, "rows and cols must be positive");
  require(cols % 8 == 0 && cols <= 4096, "cols must be a multiple of 8 and <= 4096");
  require(rows < (int64_t{1} << 30), "rows too large");
}

// Argmax workspace: per-block partial values, then per-block indices.
size_t argmax_ws_bytes(const mmr::GemvPlan& p) { return static_cast<size_t>(p.blocks) * 8; }

int auto_splits(int64_t tokens, int64_t head_dim) {
  const int tile = mmr::attention_tile_tokens(static_cast<int>(head_dim));
  const int64_t tiles = (tokens + tile - 1) / tile;
  return static_cast<int>(tiles < 1 ? 1 : (tiles > 512 ? 512 : tiles));
}

// Attention workspace: the split partials, o [Hkv][splits][R][d] then (m, l)
// [Hkv][splits][R][2], fp32.
size_t attention_ws_bytes(int64_t hq, int64_t hkv, int64_t d, int splits) {
  return mmr::attention_partial_floats(static_cast<int>(hq), static_cast<int>(hkv), static_cast<int>(d), splits) * 4;
}

void check_attention_shape(int64_t hq, int64_t hkv, int64_t d) {
  require(mmr::attention_supported(static_cast<int>(hq), static_cast<int>(hkv), static_cast<int>(d)),
          "unsupported heads/head_dim: need Hq % Hkv == 0, Hq/Hkv <= 8, head_dim in {16,32,64,96,128}");
  require(hkv <= 64, "kv_heads must be <= 64");
}

// Rows [0, tokens) must be backed: op-level calls never allocate.
void require_backed(const mmr_kv_cache* c, int64_t tokens) {
  if (tokens > c->usable())
    throw std::length_error("KV cache rows [0, " + std::to_string(tokens) + ") are not backed (" +
                            std::to_string(c->usable()) + " are): call mmr_kv_cache_reserve first");
}

}  // namespace

extern "C" {

const char* mmr_last_error(void) { return g_last_error.c_str(); }
int mmr_version(void) { return 1; }

int mmr_device_count(int* count) {
  return guarded([&] {
    require(count, "null count");
    *count = 0;
    const hipError_t st = hipGetDeviceCount(count);
    if (st != hipSuccess) *count = 0;
  });
}

int mmr_malloc(void** ptr, size_t bytes) {
  return guarded([&] {
    require(ptr, "null ptr");
    hip(hipMalloc(ptr, bytes), "hipMalloc");
  });
}
int mmr_free(void* ptr) {
  return guarded([&] { hip(hipFree(ptr), "hipFree"); });
}
int mmr_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return guarded([&] { hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D"); });
}
int mmr_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return guarded([&] { hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H"); });
}
int mmr_memcpy_d2d_async(void* dst, const void* src, size_t bytes, mmr_stream_t stream) {
  return guarded([&] {
    hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "hipMemcpyAsync D2D");
  });
}
int mmr_memset(void* dst, int value, size_t bytes) {
  return guarded([&] { hip(hipMemset(dst, value, bytes), "hipMemset"); });
}
int mmr_stream_create(mmr_stream_t* stream) {
  return guarded([&] {
    require(stream, "null stream");
    hipStream_t s = nullptr;
    hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
  });
}
int mmr_stream_destroy(mmr_stream_t stream) {
  return guarded([&] { hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy"); });
}
int mmr_stream_synchronize(mmr_stream_t stream) {
  return guarded([&] { hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); });
}
int mmr_device_synchronize(void) {
  return guarded([&] { hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}
int mmr_event_create(void** event) {
  return guarded([&] {
    require(event, "null event");
    hipEvent_t e = nullptr;
    hip(hipEventCreate(&e), "hipEventCreate");
    *event = e;
  });
}
int mmr_event_destroy(void* event) {
  return guarded([&] { hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy"); });
}
int mmr_event_record(void* event, mmr_stream_t stream) {
  return guarded([&] { hip(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "hipEventRecord"); });
}
int mmr_event_elapsed_ms(void* start, void* stop, float* ms) {
  return guarded([&] {
    require(ms, "null ms");
    hip(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize");
    hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
        "hipEventElapsedTime");
  });
}
int mmr_graph_capture_begin(mmr_stream_t stream) {
  return guarded([&] {
    require(stream, "graph capture needs a created stream");
    hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  });
}
int mmr_graph_capture_end(mmr_stream_t stream, void** graph) {
  return guarded([&] {
    require(stream && graph, "null argument");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    hip(hipStreamEndCapture(as_stream(stream), &g), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t st = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip(st, "hipGraphInstantiate");
    *graph = exec;
  });
}
int mmr_graph_launch(void* graph, mmr_stream_t stream) {
  return guarded([&] {
    require(graph, "null graph");
    hip(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), as_stream(stream)), "hipGraphLaunch");
  });
}
int mmr_graph_destroy(void* graph) {
  return guarded([&] {
    if (graph) hip(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)), "hipGraphExecDestroy");
  });
}
int mmr_launch_floor_us(int kernels, int blocks, int load_store, int reps, float* us_per_kernel) {
  return guarded([&] {
    require(us_per_kernel, "null us_per_kernel");
    require(kernels > 0 && kernels <= 4096 && blocks > 0 && blocks <= 65536 && reps > 0, "probe size out of range");
    hip(mmr::measure_launch_floor(kernels, blocks, load_store != 0, reps, us_per_kernel), "launch floor probe");
  });
}
int mmr_gemm_k_splits(int64_t m, int64_t n, int64_t k, int* splits) {
  return guarded([&] {
    require(splits, "null splits");
    require(m > 0 && n > 0 && k > 0 && m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX, "shape out of range");
    *splits = mmr::gemm_k_splits(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
  });
}
int mmr_splitk_block_tile(int block, int row_blocks, int chunks, int* row_block, int* chunk) {
  return guarded([&] {
    require(row_block && chunk, "null argument");
    require(row_blocks > 0 && chunks > 0 && block >= 0 && static_cast<int64_t>(row_blocks) * chunks <= INT32_MAX &&
                block < row_blocks * chunks,
            "block out of range");
    const mmr::SplitKTile t = mmr::splitk_block_tile(block, row_blocks, chunks);
    *row_block = t.row_block;
    *chunk = t.chunk;
  });
}
int mmr_decode_attention_splits(int64_t n_keys, int64_t head_dim, int* splits) {
  return guarded([&] {
    require(splits, "null splits");
    require(n_keys > 0 && n_keys <= INT32_MAX, "n_keys out of range");
    require(head_dim > 0 && head_dim <= 128 && mmr::attention_supported(1, 1, static_cast<int>(head_dim)),
            "unsupported head_dim");
    *splits = minimind::model::decode_attention_splits(
        n_keys, mmr::attention_tile_tokens(static_cast<int>(head_dim)));
  });
}
int mmr_prefill_partial_floats(const mmr_config* config, int64_t chunk_rows, int64_t* floats) {
  return guarded([&] {
    require(config && floats, "null argument");
    require(chunk_rows >= 0, "chunk_rows must be non-negative");
    *floats = minimind::model::prefill_partial_floats(to_cpp(*config), chunk_rows);
  });
}
int mmr_f32_to_f16(const float* src, uint16_t* dst, size_t n) {
  return guarded([&] {
    require(src && dst, "null buffer");
    for (size_t i = 0; i < n; ++i) dst[i] = float_to_half(src[i]);
  });
}
int mmr_f16_to_f32(const uint16_t* src, float* dst, size_t n) {
  return guarded([&] {
    require(src && dst, "null buffer");
    for (size_t i = 0; i < n; ++i) dst[i] = half_to_float(src[i]);
  });
}

// ------------------------------------------------------------------ ops --

int mmr_matvec_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* residual, float* y,
                   mmr_stream_t stream) {
  return mmr_matvec_f16_ex(w, rows, cols, x, nullptr, 0.0f, MMR_PRO_PLAIN,
                           residual ? MMR_EPI_RESIDUAL : MMR_EPI_STORE, residual, y, 0, 0, stream);
}

namespace {

// The GEMV entry points with x in fp32 (x) or fp16 (xh); exactly one is set.
void enqueue_matvec(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const uint16_t* xh,
                    const float* norm_w, float eps, int prologue, int epilogue, const float* residual, float* y,
                    int lanes_per_row, int rows_per_group, mmr_stream_t stream) {
    check_matvec_shape(rows, cols);
    require(w && (x || xh) && y, "null buffer");
    require(prologue >= MMR_PRO_PLAIN && prologue <= MMR_PRO_RMSNORM_FINAL, "unknown prologue");
    require(epilogue >= MMR_EPI_STORE && epilogue <= MMR_EPI_SWIGLU, "unknown epilogue");
    require(prologue == MMR_PRO_PLAIN || norm_w, "RMSNorm prologue needs norm_w");
    require(epilogue != MMR_EPI_RESIDUAL || residual, "residual epilogue needs residual");
    require(prologue != MMR_PRO_RMSNORM_FINAL, "the final-norm prologue is fused with argmax only");
    mmr::GemvPlan plan;
    require(mmr::gemv_plan(static_cast<int>(rows), static_cast<int>(cols), static_cast<mmr::GemvEpilogue>(epilogue),
                           lanes_per_row, rows_per_group, &plan),
            "unsupported launch shape (lanes_per_row 16/32/64, rows_per_group 1/2/4, even for SwiGLU)");
    mmr::GemvArgs a;
    a.w = reinterpret_cast<const __half*>(w);
    a.rows = static_cast<int>(rows);
    a.k = static_cast<int>(cols);
    a.x = x;
    a.x_half = reinterpret_cast<const __half*>(xh);
    a.norm_w = norm_w;
    a.eps = eps;
    a.y = y;
    a.residual = residual;
    hip(mmr::launch_gemv(a, static_cast<mmr::GemvPrologue>(prologue), static_cast<mmr::GemvEpilogue>(epilogue), plan,
                         as_stream(stream)),
        "matvec launch");
}

void enqueue_matvec_argmax(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const uint16_t* xh,
                           const float* norm_w, float eps, float* logits, int32_t* token_out, void* workspace,
                           size_t workspace_bytes, mmr_stream_t stream) {
  check_matvec_shape(rows, cols);
  require(w && (x || xh) && token_out && workspace, "null buffer");
  mmr::GemvPlan plan;
  require(mmr::gemv_plan(static_cast<int>(rows), static_cast<int>(cols), mmr::kEpiArgmax, 0, 0, &plan),
          "unsupported shape");
  require(workspace_bytes >= argmax_ws_bytes(plan), "workspace too small");
  char* ws = static_cast<char*>(workspace);
  mmr::GemvArgs a;
  a.w = reinterpret_cast<const __half*>(w);
  a.rows = static_cast<int>(rows);
  a.k = static_cast<int>(cols);
  a.x = x;
  a.x_half = reinterpret_cast<const __half*>(xh);
  a.norm_w = norm_w;
  a.eps = eps;
  a.y = logits;
  a.part_val = reinterpret_cast<float*>(ws);
  a.part_idx = reinterpret_cast<int*>(ws + static_cast<size_t>(plan.blocks) * 4);
  hip(mmr::launch_gemv(a, norm_w ? mmr::kProRmsNormFinal : mmr::kProPlain, mmr::kEpiArgmax, plan, as_stream(stream)),
      "matvec argmax launch");
  mmr::ArgmaxFinalizeArgs f;
  f.part_val = a.part_val;
  f.part_idx = a.part_idx;
  f.parts = plan.blocks;
  f.token_out = token_out;
  hip(mmr::launch_argmax_finalize(f, as_stream(stream)), "argmax finalize launch");
}

}  // namespace

int mmr_matvec_f16_ex(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* norm_w, float eps,
                      int prologue, int epilogue, const float* residual, float* y, int lanes_per_row,
                      int rows_per_group, mmr_stream_t stream) {
  return guarded([&] {
    require(x, "null buffer");
    enqueue_matvec(w, rows, cols, x, nullptr, norm_w, eps, prologue, epilogue, residual, y, lanes_per_row,
                   rows_per_group, stream);
  });
}

int mmr_matvec_f16x(const uint16_t* w, int64_t rows, int64_t cols, const uint16_t* x, const float* residual, float* y,
                    mmr_stream_t stream) {
  return guarded([&] {
    require(x, "null buffer");
    enqueue_matvec(w, rows, cols, nullptr, x, nullptr, 0.0f, MMR_PRO_PLAIN, residual ? MMR_EPI_RESIDUAL : MMR_EPI_STORE,
                   residual, y, 0, 0, stream);
  });
}

size_t mmr_matvec_argmax_workspace_size(int64_t rows, int64_t cols) {
  mmr::GemvPlan plan;
  if (rows <= 0 || rows >= (int64_t{1} << 30) ||
      !mmr::gemv_plan(static_cast<int>(rows), static_cast<int>(cols), mmr::kEpiArgmax, 0, 0, &plan))
    return 0;
  return argmax_ws_bytes(plan);
}

int mmr_matvec_argmax_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* norm_w, float eps,
                          float* logits, int32_t* token_out, void* workspace, size_t workspace_bytes,
                          mmr_stream_t stream) {
  return guarded([&] {
    require(x, "null buffer");
    enqueue_matvec_argmax(w, rows, cols, x, nullptr, norm_w, eps, logits, token_out, workspace, workspace_bytes,
                          stream);
  });
}

int mmr_matvec_argmax_f16x(const uint16_t* w, int64_t rows, int64_t cols, const uint16_t* x, float* logits,
                           int32_t* token_out, void* workspace, size_t workspace_bytes, mmr_stream_t stream) {
  return guarded([&] {
    require(x, "null buffer");
    enqueue_matvec_argmax(w, rows, cols, nullptr, x, nullptr, 0.0f, logits, token_out, workspace, workspace_bytes,
                          stream);
  });
}

int mmr_rope_table_create(int64_t max_positions, int64_t head_dim, float theta, mmr_rope_table** out) {
  return guarded([&] {
    require(out, "null out");
    require(max_positions > 0 && max_positions <= (int64_t{1} << 24), "max_positions out of range");
    require(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 128, "head_dim must be even and <= 128");
    require(theta > 0.0f, "theta must be positive");
    auto t = std::make_unique<mmr_rope_table>();
    const int64_t half = head_dim / 2;
    std::vector<float> inv(static_cast<size_t>(half));
    for (int64_t i = 0; i < half; ++i)
      inv[static_cast<size_t>(i)] =
          1.0F / std::pow(theta, static_cast<float>(i * 2) / static_cast<float>(head_dim));
    t->inv_freq.reset(inv.size() * sizeof(float));
    hip(hipMemcpy(t->inv_freq.data(), inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
    t->max_positions = max_positions;
    t->head_dim = head_dim;
    *out = t.release();
  });
}

int mmr_rope_table_destroy(mmr_rope_table* table) {
  return guarded([&] { delete table; });
}

int mmr_kv_cache_create(int64_t kv_heads, int64_t head_dim, int64_t capacity, int kv_dtype, mmr_kv_cache** out) {
  return guarded([&] {
    require(out, "null out");
    require(kv_heads > 0 && head_dim > 0 && capacity > 0, "dimensions must be positive");
    require(kv_dtype == MMR_KV_F16 || kv_dtype == MMR_KV_F32, "unknown kv dtype");
    require(head_dim <= 128, "head_dim must be <= 128");
    auto c = std::make_unique<mmr_kv_cache>();
    c->dtype = kv_dtype;
    c->store = minimind::model::KvStore(1, kv_heads, head_dim, c->kv(), capacity);
    c->store.reserve(std::min<int64_t>(capacity, mmr::kv_segment_tokens(0)));
    *out = c.release();
  });
}

int mmr_kv_cache_destroy(mmr_kv_cache* cache) {
  return guarded([&] { delete cache; });
}

int mmr_kv_cache_reserve(mmr_kv_cache* cache, int64_t tokens) {
  return guarded([&] {
    require(cache, "null argument");
    require(tokens >= 0, "tokens must be non-negative");
    cache->store.reserve(tokens);
  });
}

int mmr_kv_cache_reset(mmr_kv_cache* cache) {
  return guarded([&] {
    require(cache, "null argument");
    cache->store.release_tail();
    cache->prefilled = 0;
  });
}

int mmr_kv_cache_info(const mmr_kv_cache* cache, int64_t* kv_heads, int64_t* head_dim, int64_t* capacity,
                      int* kv_dtype) {
  return guarded([&] {
    require(cache, "null argument");
    if (kv_heads) *kv_heads = cache->kv_heads();
    if (head_dim) *head_dim = cache->head_dim();
    if (capacity) *capacity = cache->capacity();
    if (kv_dtype) *kv_dtype = cache->dtype;
  });
}

int mmr_kv_cache_backed(const mmr_kv_cache* cache, int64_t* tokens, uint64_t* device_bytes) {
  return guarded([&] {
    require(cache, "null argument");
    if (tokens) *tokens = cache->usable();
    if (device_bytes) *device_bytes = cache->store.device_bytes();
  });
}

int mmr_kv_cache_segment(const mmr_kv_cache* cache, int index, void** keys, void** values, int64_t* first_token,
                         int64_t* tokens) {
  return guarded([&] {
    require(cache && keys && values && first_token && tokens, "null argument");
    require(index >= 0 && index < mmr::kKvSegments, "segment index out of range");
    const mmr::KvSeg& sg = cache->store.layer(0).s[index];
    *keys = sg.k;
    *values = sg.v;
    *first_token = mmr::kv_segment_first(index);
    *tokens = sg.k ? std::max<int64_t>(0, std::min<int64_t>(mmr::kv_segment_tokens(index),
                                                            cache->usable() - *first_token))
                   : 0;
  });
}

int mmr_kv_cache_write(mmr_kv_cache* cache, int64_t first, int64_t count, const void* keys, const void* values) {
  return guarded([&] {
    require(cache && keys && values, "null argument");
    require(first >= 0 && count >= 0 && first + count <= cache->capacity(), "rows outside the cache capacity");
    cache->store.write_rows(0, first, count, keys, values);
  });
}

int mmr_kv_cache_read(const mmr_kv_cache* cache, int64_t first, int64_t count, void* keys, void* values) {
  return guarded([&] {
    require(cache && keys && values, "null argument");
    require(first >= 0 && count >= 0 && first + count <= cache->usable(), "rows outside the backed cache");
    cache->store.read_rows(0, first, count, keys, values);
  });
}

int mmr_decode_qkv_postprocess(const float* qkv, const float* q_norm, const float* k_norm, mmr_kv_cache* cache,
                               int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t position,
                               const mmr_rope_table* rope, float eps, float* query, mmr_stream_t stream) {
  return guarded([&] {
    require(qkv && q_norm && k_norm && cache && rope && query, "null argument");
    check_attention_shape(q_heads, kv_heads, head_dim);
    require(cache->kv_heads() == kv_heads && cache->head_dim() == head_dim, "cache shape mismatch");
    require(rope->head_dim == head_dim, "rope table head_dim mismatch");
    require(tokens >= 1 && tokens <= cache->capacity(), "tokens must be in [1, capacity]");
    require_backed(cache, tokens);
    require(position >= 0 && position < rope->max_positions, "position outside the rope table");
    mmr::QkvPostArgs a;
    a.qkv = qkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.inv_freq = rope->data();
    a.position = static_cast<int>(position);
    a.index = static_cast<int>(tokens - 1);
    a.seg = cache->store.layer(0);
    a.hq = static_cast<int>(q_heads);
    a.hkv = static_cast<int>(kv_heads);
    a.d = static_cast<int>(head_dim);
    a.query_out = query;
    hip(mmr::launch_qkv_postprocess(a, cache->kv(), as_stream(stream)), "qkv postprocess launch");
  });
}

size_t mmr_attention_workspace_size(int64_t q_heads, int64_t kv_heads, int64_t head_dim, int splits) {
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || head_dim <= 0) return 0;
  if (splits <= 0) splits = 512;
  return attention_ws_bytes(q_heads, kv_heads, head_dim, splits);
}

namespace {

// mmr_attention_from_cache with the split partials in `part` (checked by the
// callers to hold attention_ws_bytes for `splits`).
void enqueue_attention_from_cache(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                                  int64_t kv_heads, int64_t head_dim, float* out, float* part, int splits,
                                  mmr_stream_t stream) {
  mmr::AttnArgs a;
  a.q = query;
  a.tokens = static_cast<int>(tokens);
  a.seg = cache->store.layer(0);
  a.capacity = static_cast<int>(cache->usable());
  a.rows = static_cast<int>(cache->store.backed());
  a.hq = static_cast<int>(q_heads);
  a.hkv = static_cast<int>(kv_heads);
  a.d = static_cast<int>(head_dim);
  a.splits = splits;
  a.part = part;
  hip(mmr::launch_attention(a, mmr::kAttnFromCache, cache->kv(), as_stream(stream)), "attention launch");
  hip(mmr::launch_attention_combine(a.part, a.hq, a.hkv, a.d, splits, out, as_stream(stream)),
      "attention combine launch");
}

void check_attention_from_cache(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, const float* out, int* splits) {
  require(query && cache && out, "null argument");
  check_attention_shape(q_heads, kv_heads, head_dim);
  require(cache->kv_heads() == kv_heads && cache->head_dim() == head_dim, "cache shape mismatch");
  require(tokens >= 1 && tokens <= cache->capacity(), "tokens must be in [1, capacity]");
  require_backed(cache, tokens);
  if (*splits <= 0) *splits = auto_splits(tokens, head_dim);
  require(*splits <= 4096, "splits too large");
}

}  // namespace

int mmr_attention_from_cache(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, float* out, void* workspace, size_t workspace_bytes,
                             int splits, mmr_stream_t stream) {
  return guarded([&] {
    check_attention_from_cache(query, cache, tokens, q_heads, kv_heads, head_dim, out, &splits);
    require(workspace != nullptr, "null argument");
    require(workspace_bytes >= attention_ws_bytes(q_heads, kv_heads, head_dim, splits), "workspace too small");
    enqueue_attention_from_cache(query, cache, tokens, q_heads, kv_heads, head_dim, out,
                                 static_cast<float*>(workspace), splits, stream);
  });
}

// ---- mmr_attention_from_cache_noalloc: the split partials in a static
// device array instead of a caller workspace.  One copy per GPU, held until
// the process ends.  In host code `scratch` names a host-side stand-in, never
// the device copy: every use goes through the address hipGetSymbolAddress
// returns for the current device, looked up once per device on its first
// call (under g_scratch_mutex) and kept in g_scratch_ptr.
static __device__ __align__(256) float scratch[MMR_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxScratchDevices] = {};

float* device_scratch() {
  int dev = -1;
  hip(hipGetDevice(&dev), "hipGetDevice");
  require(dev >= 0 && dev < kMaxScratchDevices, "device index beyond the static scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    require(p != nullptr, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

int mmr_attention_from_cache_noalloc(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                                     int64_t kv_heads, int64_t head_dim, float* out, int splits,
                                     mmr_stream_t stream) {
  return guarded([&] {
    check_attention_from_cache(query, cache, tokens, q_heads, kv_heads, head_dim, out, &splits);
    const size_t need = attention_ws_bytes(q_heads, kv_heads, head_dim, splits);
    if (need > MMR_NOALLOC_SCRATCH_BYTES)
      throw std::invalid_argument("split partials need " + std::to_string(need) + " bytes, beyond the " +
                                  std::to_string(MMR_NOALLOC_SCRATCH_BYTES) +
                                  "-byte static scratch: use fewer splits or mmr_attention_from_cache");
    enqueue_attention_from_cache(query, cache, tokens, q_heads, kv_heads, head_dim, out, device_scratch(), splits,
                                 stream);
  });
}

int mmr_decode_attention_fused(const float* qkv, const float* q_norm, const float* k_norm, float eps,
                               const mmr_rope_table* rope, const int32_t* position, mmr_kv_cache* cache,
                               int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out, void* workspace,
                               size_t workspace_bytes, int splits, int32_t* error, mmr_stream_t stream) {
  return guarded([&] {
    require(qkv && q_norm && k_norm && rope && position && cache && out && workspace && error, "null argument");
    check_attention_shape(q_heads, kv_heads, head_dim);
    require(cache->kv_heads() == kv_heads && cache->head_dim() == head_dim, "cache shape mismatch");
    require(rope->head_dim == head_dim, "rope table head_dim mismatch");
    // The device position is unknown here: size the splits for the backed rows.
    if (splits <= 0) splits = auto_splits(cache->usable(), head_dim);
    require(splits <= 4096, "splits too large");
    require(workspace_bytes >= attention_ws_bytes(q_heads, kv_heads, head_dim, splits), "workspace too small");
    mmr::AttnArgs a;
    a.qkv = qkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.inv_freq = rope->data();
    a.pos = position;
    a.seg = cache->store.layer(0);
    a.capacity = static_cast<int>(std::min(cache->usable(), rope->max_positions));
    a.rows = static_cast<int>(cache->store.backed());
    a.hq = static_cast<int>(q_heads);
    a.hkv = static_cast<int>(kv_heads);
    a.d = static_cast<int>(head_dim);
    a.splits = splits;
    a.part = static_cast<float*>(workspace);
    a.err = error;
    hip(mmr::launch_attention(a, mmr::kAttnFused, cache->kv(), as_stream(stream)), "fused attention launch");
    hip(mmr::launch_attention_combine(a.part, a.hq, a.hkv, a.d, splits, out, as_stream(stream)),
        "attention combine launch");
  });
}

int mmr_matmul_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, int64_t batch,
                   const float* residual, float* y, mmr_stream_t stream) {
  return guarded([&] {
    require(w && x && y, "null buffer");
    require(rows > 0 && cols > 0 && batch > 0, "rows, cols and batch must be positive");
    require(rows <= (1 << 24) && cols <= (1 << 24) && batch <= (1 << 24), "matrix too large");
    require(cols % 8 == 0, "cols must be a multiple of 8");
    mmr::GemmArgs g;
    g.a = x;
    g.lda = static_cast<int>(cols);
    g.w = reinterpret_cast<const __half*>(w);
    g.residual = residual;
    g.c = y;
    g.ldc = static_cast<int>(rows);
    g.m = static_cast<int>(batch);
    g.n = static_cast<int>(rows);
    g.k = static_cast<int>(cols);
    hip(mmr::launch_gemm(g, as_stream(stream)), "gemm launch");
  });
}

int mmr_prefill_qkv_rows(const float* qkv, const float* q_norm, const float* k_norm, float eps,
                         const mmr_rope_table* rope, mmr_kv_cache* cache, int64_t start_position, int64_t seq_len,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* query, mmr_stream_t stream) {
  return guarded([&] {
    require(qkv && q_norm && k_norm && rope && cache && query, "null argument");
    check_attention_shape(q_heads, kv_heads, head_dim);
    require(cache->kv_heads() == kv_heads && cache->head_dim() == head_dim, "cache shape mismatch");
    require(rope->head_dim == head_dim, "rope table head_dim mismatch");
    require(seq_len >= 1 && start_position >= 0, "seq_len must be positive and start_position non-negative");
    require(start_position + seq_len <= cache->capacity(), "prompt exceeds the cache capacity");
    require_backed(cache, start_position + seq_len);
    require(start_position + seq_len <= rope->max_positions, "positions outside the rope table");
    mmr::QkvRowsArgs a;
    a.qkv = qkv;
    a.qkv_stride = static_cast<int>((q_heads + 2 * kv_heads) * head_dim);
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.inv_freq = rope->data();
    a.start = static_cast<int>(start_position);
    a.row0 = static_cast<int>(start_position);
    a.tokens = static_cast<int>(seq_len);
    a.seg = cache->store.layer(0);
    a.hq = static_cast<int>(q_heads);
    a.hkv = static_cast<int>(kv_heads);
    a.d = static_cast<int>(head_dim);
    a.query = query;
    a.query_stride = static_cast<int>(q_heads * head_dim);
    hip(mmr::launch_qkv_rows(a, cache->kv(), as_stream(stream)), "qkv rows launch");
  });
}

int mmr_cube_matvec_available(void) { return cube_matvec_available() ? 1 : 0; }
int mmr_cube_matmul_available(void) { return cube_matmul_available() ? 1 : 0; }
int mmr_custom_ops_available(void) { return custom_ops_available() ? 1 : 0; }

int mmr_cube_matvec(const float* matrix, int64_t rows, int64_t cols, const float* input, float* out) {
  return guarded([&] { host_matmul(matrix, rows, cols, input, 1, out); });
}

int mmr_cube_matmul(const float* matrix, int64_t rows, int64_t cols, const float* input, int64_t batch, float* out) {
  return guarded([&] { host_matmul(matrix, rows, cols, input, batch, out); });
}

int mmr_cube_matvec_argmax(const float* matrix, int64_t rows, int64_t cols, const float* input, int32_t* token) {
  return guarded([&] {
    require(token, "null argument");
    *token = host_matvec_argmax(matrix, rows, cols, input);
  });
}

int mmr_custom_attention(const float* query, const float* keys, const float* values, int64_t tokens, int64_t q_heads,
                         int64_t kv_heads, int64_t head_dim, float* out) {
  return guarded([&] { host_attention(query, keys, values, tokens, q_heads, kv_heads, head_dim, out); });
}

int mmr_custom_prefill_attention(const float* query, const float* keys, const float* values, mmr_kv_cache** cache,
                                 int64_t seq_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out) {
  return guarded(
      [&] { host_prefill_attention(query, keys, values, cache, seq_len, q_heads, kv_heads, head_dim, out); });
}

int mmr_custom_attention_cached(const float* query, const float* key, const float* value, mmr_kv_cache** cache,
                                int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out) {
  return guarded([&] { host_attention_cached(query, key, value, cache, tokens, q_heads, kv_heads, head_dim, out); });
}

int mmr_layer_weights_create(const mmr_config* config, const float* input_norm, const float* post_attention_norm,
                             const float* q_norm, const float* k_norm, const float* q_proj, const float* k_proj,
                             const float* v_proj, const float* o_proj, const float* gate_proj, const float* up_proj,
                             const float* down_proj, mmr_layer_weights** out) {
  return guarded([&] {
    require(config && out, "null argument");
    require(input_norm && post_attention_norm && q_norm && k_norm && q_proj && k_proj && v_proj && o_proj &&
                gate_proj && up_proj && down_proj,
            "null weight array");
    const MiniMindConfig c = to_cpp(*config);
    // The config sets how many floats are read from each array: validate it first.
    const auto errors = validate_config(c);
    if (!errors.empty()) throw std::invalid_argument("invalid MiniMind config: " + errors.front());
    const auto dev_errors = validate_device_config(c);
    if (!dev_errors.empty()) throw std::invalid_argument("unsupported by the gfx950 runtime: " + dev_errors.front());
    const int64_t H = c.hidden_size, D = c.head_dim, F = c.intermediate_size;
    const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
    const auto vec = [](const float* p, int64_t n) { return std::vector<float>(p, p + n); };
    DenseLayerWeights L;
    L.input_norm = vec(input_norm, H);
    L.post_attention_norm = vec(post_attention_norm, H);
    L.q_norm = vec(q_norm, D);
    L.k_norm = vec(k_norm, D);
    L.q_proj = vec(q_proj, qs * H);
    L.k_proj = vec(k_proj, kvs * H);
    L.v_proj = vec(v_proj, kvs * H);
    L.o_proj = vec(o_proj, H * qs);
    L.gate_proj = vec(gate_proj, F * H);
    L.up_proj = vec(up_proj, F * H);
    L.down_proj = vec(down_proj, H * F);
    auto h = std::make_unique<mmr_layer_weights>();
    h->w = DeviceLayerWeights::upload(c, L);
    *out = h.release();
  });
}

int mmr_model_layer_weights(const mmr_model* model, int64_t layer, mmr_layer_weights** out) {
  return guarded([&] {
    require(model && out, "null argument");
    auto h = std::make_unique<mmr_layer_weights>();
    h->w = DeviceLayerWeights::view(model->lm->shared_device_model(), layer);
    *out = h.release();
  });
}

int mmr_layer_weights_destroy(mmr_layer_weights* weights) {
  delete weights;
  return MMR_OK;
}

size_t mmr_decoder_layer_workspace_size(const mmr_config* config, int splits) {
  if (!config || splits < 1 || splits > 4096) return 0;
  return decoder_layer_workspace_floats(to_cpp(*config), splits) * 4;
}

int mmr_decoder_layer_forward(const mmr_layer_weights* weights, mmr_kv_cache* cache, const float* hidden,
                              const int32_t* position, float* out, void* workspace, size_t workspace_bytes,
                              int splits, int32_t* error, mmr_stream_t stream) {
  return guarded([&] {
    require(weights && weights->w && cache && hidden && position && out && workspace && error, "null argument");
    const MiniMindConfig& c = weights->w->cfg;
    require(cache->kv_heads() == c.num_key_value_heads && cache->head_dim() == c.head_dim,
            "cache shape does not match the layer (kv_heads, head_dim)");
    // The device position is unknown here: size the splits for the backed
    // rows, which follow the context when the cache is grown as it fills.
    if (splits <= 0) splits = auto_splits(cache->usable(), c.head_dim);
    require(splits <= 4096, "splits too large");
    require(workspace_bytes >= decoder_layer_workspace_floats(c, splits) * 4, "workspace too small");
    DecoderLayerIo io;
    io.hidden = hidden;
    io.out = out;
    io.position = position;
    io.seg = cache->store.layer(0);
    io.rows = static_cast<int>(cache->store.backed());
    io.capacity = static_cast<int>(std::min(cache->usable(), c.max_position_embeddings));
    io.kv = cache->kv();
    io.splits = splits;
    io.workspace = static_cast<float*>(workspace);
    io.err = error;
    enqueue_decoder_layer(*weights->w, io, as_stream(stream));
  });
}

size_t mmr_prefill_layer_workspace_size(const mmr_config* config, int64_t seq_len) {
  if (!config || seq_len < 1 || seq_len > (int64_t{1} << 20)) return 0;
  return prefill_scratch_bytes(to_cpp(*config), seq_len);
}

int mmr_prefill_layer_forward(const mmr_layer_weights* weights, mmr_kv_cache* cache, const float* hidden_seq,
                              int64_t start_position, int64_t seq_len, float* out, void* workspace,
                              size_t workspace_bytes, mmr_stream_t stream) {
  return guarded([&] {
    require(weights && weights->w && cache && hidden_seq && out && workspace, "null argument");
    const MiniMindConfig& c = weights->w->cfg;
    require(cache->kv_heads() == c.num_key_value_heads && cache->head_dim() == c.head_dim,
            "cache shape does not match the layer (kv_heads, head_dim)");
    // decoder_layer.cpp:416-418 / :669-671
    require(cache->prefilled == 0, "prefill layer requires an empty KV cache");
    require(seq_len >= 1 && seq_len <= (int64_t{1} << 20) && start_position >= 0,
            "seq_len must be in [1, 2^20] and start_position non-negative");
    require(start_position + seq_len <= c.max_position_embeddings, "positions exceed max_position_embeddings");
    require(seq_len <= cache->capacity(), "prompt exceeds the cache capacity");
    require_backed(cache, seq_len);
    const int H = static_cast<int>(c.hidden_size), F = static_cast<int>(c.intermediate_size);
    const int qs = static_cast<int>(c.num_attention_heads * c.head_dim);
    const int qkv = static_cast<int>((c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim);
    require(mmr::gemm_supported(1, qkv, H) && mmr::gemm_supported(1, H, qs) && mmr::gemm_supported(1, 2 * F, H) &&
                mmr::gemm_supported(1, H, F),
            "the prefill GEMMs need hidden_size, q_size and intermediate_size to be multiples of 8");
    require(workspace_bytes >= prefill_scratch_bytes(c, seq_len), "workspace too small");
    hipStream_t st = as_stream(stream);
    const size_t bytes = static_cast<size_t>(seq_len * H) * sizeof(float);
    if (out != hidden_seq) hip(hipMemcpyAsync(out, hidden_seq, bytes, hipMemcpyDeviceToDevice, st), "copy hidden_seq");
    const PrefillScratch scratch = carve_prefill_scratch(c, seq_len, workspace);
    const LayerDev& w = weights->w->w;
    const int rows = static_cast<int>(seq_len);
    enqueue_prefill_input_norm(c, scratch, rows, out, w.input_norm, st);
    // Keys and values go to cache rows 0 .. seq_len - 1 and rotate to
    // positions start_position + i (device_prefill_attention copies them to
    // the front of the cache, ascend_custom_ops.cpp:796-803).
    PrefillKv kv;
    kv.seg = cache->store.layer(0);
    kv.dtype = cache->kv();
    kv.rope_start = static_cast<int>(start_position);
    kv.row0 = 0;
    // The norm after the last residual feeds no later layer here: it lands
    // in the scratch unused.
    enqueue_prefill_layer(c, w, weights->w->inv_freq, scratch, kv, rows, out, w.input_norm, false, st);
    cache->prefilled = seq_len;  // cache.tokens = seq_len (decoder_layer.cpp:524, :733)
  });
}

int mmr_prefill_attention(const float* query, const mmr_kv_cache* cache, int64_t start_position, int64_t seq_len,
                          int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out, mmr_stream_t stream) {
  return guarded([&] {
    require(query && cache && out, "null argument");
    check_attention_shape(q_heads, kv_heads, head_dim);
    require(cache->kv_heads() == kv_heads && cache->head_dim() == head_dim, "cache shape mismatch");
    require(seq_len >= 1 && start_position >= 0, "seq_len must be positive and start_position non-negative");
    require(start_position + seq_len <= cache->capacity(), "prompt exceeds the cache capacity");
    require_backed(cache, start_position + seq_len);
    mmr::PrefillAttnArgs a;
    a.query = query;
    a.query_stride = static_cast<int>(q_heads * head_dim);
    a.seg = cache->store.layer(0);
    a.start = static_cast<int>(start_position);
    a.tokens = static_cast<int>(seq_len);
    a.hq = static_cast<int>(q_heads);
    a.hkv = static_cast<int>(kv_heads);
    a.d = static_cast<int>(head_dim);
    a.out = out;
    a.out_stride = static_cast<int>(q_heads * head_dim);
    hip(mmr::launch_prefill_attention(a, cache->kv(), as_stream(stream)), "prefill attention launch");
  });
}

int mmr_rms_norm_rows(const float* in, const float* w, float eps, int64_t rows, int64_t cols, float* out,
                      mmr_stream_t stream) {
  return guarded([&] {
    require(in && w && out, "null buffer");
    require(rows >= 0 && cols > 0 && rows < (int64_t{1} << 31), "invalid shape");
    hip(mmr::launch_rms_norm_rows(in, w, eps, static_cast<int>(rows), static_cast<int>(cols), out, as_stream(stream)),
        "rms_norm_rows launch");
  });
}

int mmr_add(const float* a, const float* b, int64_t n, float* out, mmr_stream_t stream) {
  return guarded([&] {
    require(a && b && out, "null buffer");
    hip(mmr::launch_add(a, b, n, out, as_stream(stream)), "add launch");
  });
}

int mmr_swiglu_rows(const float* gate_up, int64_t rows, int64_t cols, float* out, mmr_stream_t stream) {
  return guarded([&] {
    require(gate_up && out, "null buffer");
    require(rows >= 0 && cols > 0, "invalid shape");
    hip(mmr::launch_swiglu_rows(gate_up, static_cast<int>(rows), static_cast<int>(cols), out, as_stream(stream)),
        "swiglu_rows launch");
  });
}

int mmr_embedding_gather(const uint16_t* table, const int32_t* ids, int64_t tokens, int64_t vocab, int64_t hidden,
                         float* out, int32_t* error, mmr_stream_t stream) {
  return guarded([&] {
    require(table && ids && out, "null buffer");
    require(tokens >= 0 && tokens < 65536 && vocab > 0 && hidden > 0, "invalid shape");
    hip(mmr::launch_embedding_gather(reinterpret_cast<const __half*>(table), ids, static_cast<int>(tokens),
                                     static_cast<int>(vocab), static_cast<int>(hidden), out, error, as_stream(stream)),
        "embedding_gather launch");
  });
}

// ---------------------------------------------------------------- model --

int mmr_default_config(mmr_config* out) {
  return guarded([&] {
    require(out, "null out");
    *out = to_c(default_minimind_config());
  });
}

int mmr_load_config(const char* path, mmr_config* out) {
  return guarded([&] {
    require(path && out, "null argument");
    *out = to_c(config_from_file(path));
  });
}

int mmr_has_runtime_model(const char* model_dir, int* out) {
  return guarded([&] {
    require(model_dir && out, "null argument");
    *out = has_runtime_language_model(model_dir) ? 1 : 0;
  });
}

int mmr_model_load(const char* model_dir, mmr_model** out) {
  return guarded([&] {
    require(model_dir && out, "null argument");
    auto m = std::make_unique<mmr_model>();
    m->lm = std::make_unique<LanguageModel>(load_runtime_language_model(model_dir));
    *out = m.release();
  });
}

int mmr_model_create_synthetic(const mmr_config* config, uint64_t seed, double std, int round_fp16,
                               mmr_model** out) {
  return guarded([&] {
    require(config && out, "null argument");
    const MiniMindConfig c = to_cpp(*config);
    const auto errors = validate_config(c);
    if (!errors.empty()) throw std::invalid_argument("invalid MiniMind config: " + errors.front());
    auto m = std::make_unique<mmr_model>();
    m->lm = std::make_unique<LanguageModel>(c, synthesize_weights(c, seed, std, round_fp16 != 0));
    *out = m.release();
  });
}

int mmr_model_free(mmr_model* model) {
  return guarded([&] { delete model; });
}

int mmr_model_config(const mmr_model* model, mmr_config* out) {
  return guarded([&] {
    require(model && out, "null argument");
    *out = to_c(model->lm->config());
  });
}

int mmr_model_weight_bytes(const mmr_model* model, uint64_t* bytes) {
  return guarded([&] {
    require(model && bytes, "null argument");
    *bytes = model->lm->device_weight_bytes();
  });
}

int mmr_write_synthetic_model(const char* model_dir, const mmr_config* config, uint64_t seed, double std,
                              int round_fp16) {
  return guarded([&] {
    require(model_dir && config, "null argument");
    const MiniMindConfig c = to_cpp(*config);
    const auto errors = validate_config(c);
    if (!errors.empty()) throw std::invalid_argument("invalid MiniMind config: " + errors.front());
    write_synthetic_model(model_dir, c, seed, std, round_fp16 != 0);
  });
}

int mmr_model_create_toy(mmr_model** out) {
  return guarded([&] {
    require(out, "null out");
    auto m = std::make_unique<mmr_model>();
    m->lm = std::make_unique<LanguageModel>(make_toy_language_model());
    *out = m.release();
  });
}

int mmr_write_toy_model(const char* model_dir) {
  return guarded([&] {
    require(model_dir, "null argument");
    const auto cw = toy_model_weights();
    std::filesystem::create_directories(model_dir);
    write_config(cw.first, std::string(model_dir) + "/minimind_runtime_config.txt");
    write_weights(cw.first, cw.second, std::string(model_dir) + "/weights.bin");
  });
}

int mmr_synthesize_normals(uint64_t seed, uint64_t first, uint64_t count, double std, int round_fp16, float* out) {
  return guarded([&] {
    require(out || count == 0, "null out");
    synthesize_normals(seed, first, count, std, round_fp16 != 0, out);
  });
}

int mmr_synthesize_prompt(uint64_t seed, int64_t count, int64_t vocab, int32_t* out) {
  return guarded([&] {
    require((out || count == 0) && count >= 0 && vocab > 0, "invalid argument");
    const auto ids = synthesize_prompt(seed, count, vocab);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
  });
}

int mmr_state_create(const mmr_model* model, int64_t capacity, int kv_dtype, mmr_state** out) {
  return guarded([&] {
    require(model && out, "null argument");
    require(kv_dtype == MMR_KV_F16 || kv_dtype == MMR_KV_F32, "unknown kv dtype");
    auto s = std::make_unique<mmr_state>();
    s->st = model->lm->make_state(capacity, kv_dtype == MMR_KV_F16 ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32);
    *out = s.release();
  });
}

int mmr_state_free(mmr_state* state) {
  return guarded([&] { delete state; });
}

int mmr_state_position(const mmr_state* state, int64_t* position) {
  return guarded([&] {
    require(state && position, "null argument");
    *position = state->st.position;
  });
}

int mmr_state_reserve(const mmr_model* model, mmr_state* state, int64_t positions) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->reserve_kv(state->st, positions);
  });
}

int mmr_state_kv_backed(const mmr_state* state, int64_t* tokens, uint64_t* device_bytes) {
  return guarded([&] {
    require(state, "null argument");
    if (tokens) *tokens = state->st.kv_backed();
    if (device_bytes) *device_bytes = state->st.kv_device_bytes();
  });
}

int mmr_state_stream(const mmr_state* state, mmr_stream_t* stream) {
  return guarded([&] {
    require(state && stream, "null argument");
    *stream = state->st.stream();
  });
}

int mmr_state_reset(const mmr_model* model, mmr_state* state) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->reset_state(state->st);
  });
}

int mmr_forward_token(const mmr_model* model, mmr_state* state, int32_t token, float* logits) {
  return guarded([&] {
    require(model && state && logits, "null argument");
    const auto v = model->lm->forward_token(token, state->st);
    std::memcpy(logits, v.data(), v.size() * sizeof(float));
  });
}

int mmr_forward_next_token(const mmr_model* model, mmr_state* state, int32_t token, int32_t* next) {
  return guarded([&] {
    require(model && state && next, "null argument");
    *next = model->lm->forward_next_token(token, state->st);
  });
}

int mmr_prefill_next_token(const mmr_model* model, mmr_state* state, const int32_t* prompt, int64_t n,
                           int32_t* next) {
  return guarded([&] {
    require(model && state && next && (prompt || n == 0) && n >= 0, "null argument");
    *next = model->lm->prefill_next_token(std::vector<int32_t>(prompt, prompt + n), state->st);
  });
}

int mmr_generate(const mmr_model* model, const int32_t* prompt, int64_t n, int64_t max_new_tokens, int32_t* out,
                 int64_t* out_count) {
  return guarded([&] {
    require(model && out_count && (prompt || n == 0) && n >= 0, "null argument");
    require(out || max_new_tokens <= 0, "null out");
    const auto ids = model->lm->generate(std::vector<int32_t>(prompt, prompt + n), max_new_tokens);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
    *out_count = static_cast<int64_t>(ids.size());
  });
}

int mmr_enqueue_prefill(const mmr_model* model, mmr_state* state, const int32_t* prompt, int64_t n) {
  return guarded([&] {
    require(model && state && (prompt || n == 0) && n >= 0, "null argument");
    model->lm->enqueue_prefill(state->st, std::vector<int32_t>(prompt, prompt + n));
  });
}

int mmr_enqueue_decode(const mmr_model* model, mmr_state* state, int64_t steps, int32_t first_token) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->enqueue_decode(state->st, steps, first_token);
  });
}

int mmr_state_synchronize(const mmr_model* model, mmr_state* state) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->synchronize(state->st);
  });
}

int mmr_read_sequence(const mmr_model* model, mmr_state* state, int64_t first, int64_t count, int32_t* out) {
  return guarded([&] {
    require(model && state && (out || count == 0), "null argument");
    const auto ids = model->lm->read_sequence(state->st, first, count);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
  });
}

int mmr_batch_state_create(const mmr_model* model, int64_t batch, int64_t capacity, int kv_dtype,
                           mmr_batch_state** out) {
  return guarded([&] {
    require(model && out, "null argument");
    require(kv_dtype == MMR_KV_F16 || kv_dtype == MMR_KV_F32, "unknown kv dtype");
    auto s = std::make_unique<mmr_batch_state>();
    s->st = model->lm->make_batch_state(batch, capacity,
                                        kv_dtype == MMR_KV_F16 ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32);
    *out = s.release();
  });
}

int mmr_batch_state_free(mmr_batch_state* state) {
  return guarded([&] { delete state; });
}

int mmr_batch_state_info(const mmr_batch_state* state, int64_t* batch, int64_t* capacity, int64_t* steps) {
  return guarded([&] {
    require(state, "null argument");
    if (batch) *batch = state->st.batch();
    if (capacity) *capacity = state->st.capacity();
    if (steps) *steps = state->st.steps;
  });
}

int mmr_batch_state_stream(const mmr_batch_state* state, mmr_stream_t* stream) {
  return guarded([&] {
    require(state && stream, "null argument");
    *stream = state->st.stream();
  });
}

int mmr_batch_prefill(const mmr_model* model, mmr_batch_state* state, const int32_t* tokens, const int64_t* lengths,
                      int64_t batch) {
  return guarded([&] {
    require(model && state && tokens && lengths, "null argument");
    std::vector<std::vector<int32_t>> prompts(static_cast<size_t>(std::max<int64_t>(batch, 0)));
    int64_t off = 0;
    for (int64_t b = 0; b < batch; ++b) {
      require(lengths[b] >= 0, "negative prompt length");
      prompts[b].assign(tokens + off, tokens + off + lengths[b]);
      off += lengths[b];
    }
    model->lm->enqueue_batch_prefill(state->st, prompts);
  });
}

int mmr_batch_decode(const mmr_model* model, mmr_batch_state* state, int64_t steps) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->enqueue_batch_decode(state->st, steps);
  });
}

int mmr_batch_synchronize(const mmr_model* model, mmr_batch_state* state) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->synchronize(state->st);
  });
}

int mmr_batch_read_sequence(const mmr_model* model, mmr_batch_state* state, int64_t index, int64_t first,
                            int64_t count, int32_t* out) {
  return guarded([&] {
    require(model && state && (out || count == 0), "null argument");
    const auto ids = model->lm->read_batch_sequence(state->st, index, first, count);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
  });
}

int mmr_batch_read_logits(const mmr_model* model, mmr_batch_state* state, int64_t index, float* logits) {
  return guarded([&] {
    require(model && state && logits, "null argument");
    const auto v = model->lm->read_batch_logits(state->st, index);
    std::memcpy(logits, v.data(), v.size() * sizeof(float));
  });
}

int mmr_read_logits(const mmr_model* model, mmr_state* state, float* logits) {
  return guarded([&] {
    require(model && state && logits, "null argument");
    const auto v = model->lm->read_logits(state->st);
    std::memcpy(logits, v.data(), v.size() * sizeof(float));
  });
}

int mmr_launch_step_kernel(const mmr_model* model, mmr_state* state, int kernel, int64_t layer, int64_t count) {
  return guarded([&] {
    require(model && state, "null argument");
    model->lm->enqueue_kernel(state->st, kernel, layer, count);
  });
}

int mmr_time_step_kernel(const mmr_model* model, mmr_state* state, int kernel, int64_t layer, int64_t count,
                         double* avg_us) {
  return guarded([&] {
    require(model && state && avg_us, "null argument");
    *avg_us = model->lm->time_kernel(state->st, kernel, layer, count);
  });
}

}  // extern "C"
