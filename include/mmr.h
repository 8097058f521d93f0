/*
 * mmr.h -- C ABI of the MiniMind gfx950 decode runtime (libmmr.so).
 *
 * Plain pointers and sizes only: device buffers are `void*`/typed pointers
 * obtained from mmr_malloc (or any HIP allocation), streams are hipStream_t
 * passed as `mmr_stream_t`.  Every function returns an MMR_* status; on
 * failure mmr_last_error() (thread-local) holds the message.  Op-level entry
 * points never allocate, never synchronise and may be recorded into a
 * hipGraph; model-level entry points mirror the reference C++ API.
 *
 * Each declaration names the reference interface it replaces
 * (paths under lvyufeng/minimind-orangepi, file:line).
 */
#ifndef MMR_H
#define MMR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MMR_OK 0
#define MMR_ERR_INVALID_ARGUMENT 1 /* reference: std::invalid_argument */
#define MMR_ERR_OUT_OF_RANGE 2     /* reference: std::out_of_range (token id) */
#define MMR_ERR_RUNTIME 3          /* reference: std::runtime_error (backend, IO) */
#define MMR_ERR_LENGTH 4           /* KV cache capacity exhausted */

#define MMR_KV_F16 0
#define MMR_KV_F32 1

typedef void* mmr_stream_t;
typedef struct mmr_model mmr_model;
typedef struct mmr_state mmr_state;
typedef struct mmr_batch_state mmr_batch_state;
typedef struct mmr_rope_table mmr_rope_table;
typedef struct mmr_kv_cache mmr_kv_cache;
typedef struct mmr_layer_weights mmr_layer_weights;

/* Fields of MiniMindConfig (src/csrc/models/minimind/config.h:21-45) used by
 * the dense path. */
typedef struct mmr_config {
  int64_t hidden_size;
  int64_t num_hidden_layers;
  int64_t vocab_size;
  int64_t num_attention_heads;
  int64_t num_key_value_heads;
  int64_t head_dim;
  int64_t intermediate_size;
  int64_t max_position_embeddings;
  int32_t bos_token_id;
  int32_t eos_token_id;
  int32_t use_moe;
  int32_t tie_word_embeddings;
  float rms_norm_eps;
  float rope_theta;
} mmr_config;

const char* mmr_last_error(void);
int mmr_version(void);

/* ---- device plumbing: DeviceBuffer / upload_* / runtime()
 *      (src/csrc/models/minimind/ascend_matmul.h:18-101) ------------------- */
int mmr_device_count(int* count);
int mmr_malloc(void** ptr, size_t bytes);
int mmr_free(void* ptr);
int mmr_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mmr_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mmr_memset(void* dst, int value, size_t bytes);
/* Device-to-device copy enqueued on `stream` (HIP's blit kernel). */
int mmr_memcpy_d2d_async(void* dst, const void* src, size_t bytes, mmr_stream_t stream);
int mmr_stream_create(mmr_stream_t* stream);
int mmr_stream_destroy(mmr_stream_t stream);
int mmr_stream_synchronize(mmr_stream_t stream);
int mmr_device_synchronize(void);
int mmr_event_create(void** event);
int mmr_event_destroy(void* event);
int mmr_event_record(void* event, mmr_stream_t stream);
int mmr_event_elapsed_ms(void* start, void* stop, float* ms);
/* Stream capture into a replayable hipGraph (no counterpart in the reference,
 * whose device path launches every op from the host): everything enqueued on
 * `stream` between begin and end (which must not allocate or synchronize)
 * becomes one executable graph, replayed by mmr_graph_launch on any stream. */
int mmr_graph_capture_begin(mmr_stream_t stream);
int mmr_graph_capture_end(mmr_stream_t stream, void** graph);
int mmr_graph_launch(void* graph, mmr_stream_t stream);
int mmr_graph_destroy(void* graph);
/* Measurement aid with no counterpart in the reference: the per-kernel time of
 * a hipGraph chain of `kernels` trivial launches of `blocks` x 256 threads
 * (load_store 0: empty kernels; 1: each loads one float its predecessor
 * wrote and stores one), replayed `reps` times.  Synchronous. */
int mmr_launch_floor_us(int kernels, int blocks, int load_store, int reps, float* us_per_kernel);
/* Test aids with no counterpart in the reference (host arithmetic, no
 * device needed): the K-split count the prefill / batched GEMM takes for an
 * m x n x k product, and the floats of the prefill split-K partial buffer a
 * state with prefill chunks of up to chunk_rows rows allocates (the largest
 * splits x rows x n over the four projections and every row count
 * 1..chunk_rows). */
int mmr_gemm_k_splits(int64_t m, int64_t n, int64_t k, int* splits);
int mmr_prefill_partial_floats(const mmr_config* config, int64_t chunk_rows, int64_t* floats);
/* Test aid, no reference counterpart: the (W row block, K chunk) that block
 * `block` of a batched split-K GEMM launch with grid (row_blocks, chunks)
 * computes (the blocks of one K chunk are placed on one XCD where chunks is a
 * multiple of 8). */
int mmr_splitk_block_tile(int block, int row_blocks, int chunks, int* row_block, int* chunk);
/* Test aid, no reference counterpart (host arithmetic, no device needed): the
 * attention split count a single-sequence decode step takes over n_keys keys
 * (its replayed graph's bucket) for heads of head_dim dimensions. */
int mmr_decode_attention_splits(int64_t n_keys, int64_t head_dim, int* splits);
/* float_to_half / half_to_float (ascend_matmul.h:14-15), but IEEE
 * round-to-nearest-even instead of the reference's ties-away rounding. */
int mmr_f32_to_f16(const float* src, uint16_t* dst, size_t n);
int mmr_f16_to_f32(const uint16_t* src, float* dst, size_t n);

/* ---- projection matvec: device_matmul batch 1 (ascend_matmul.h:102,
 *      ascend_matmul.cpp:385-410) and device_matmul_add (ascend_matmul.h:103-107).
 * y[r] = sum_c W[r*cols + c] * x[c] (+ residual[r] when residual != NULL).
 * W fp16 row-major [rows][cols] (the reference stores W^T; row-major keeps each
 * output row one contiguous HBM stream), x/y/residual fp32 on the device.
 * cols % 8 == 0, cols <= 4096.  residual may alias y. */
int mmr_matvec_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* residual, float* y,
                   mmr_stream_t stream);

#define MMR_PRO_PLAIN 0
#define MMR_PRO_RMSNORM 1       /* x := x * (scale * norm_w), decoder_layer.cpp:32-42 */
#define MMR_PRO_RMSNORM_FINAL 2 /* x := (x * scale) * norm_w, language_model.cpp:24-38 */
#define MMR_EPI_STORE 0
#define MMR_EPI_RESIDUAL 1
#define MMR_EPI_SWIGLU 2 /* rows interleaved gate_0, up_0, ...: y[i] = silu(g_i) * u_i, decoder_layer.cpp:175-182 */
/* Fused variant used by the decode step: RMSNorm prologue (K1 folded in) and
 * residual / SwiGLU epilogue (K5 / K4 folded in).  lanes_per_row (16/32/64)
 * and rows_per_group (1/2/4) select the launch shape; 0 = automatic. */
int mmr_matvec_f16_ex(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* norm_w, float eps,
                      int prologue, int epilogue, const float* residual, float* y, int lanes_per_row,
                      int rows_per_group, mmr_stream_t stream);
/* BASELINE configs[1]'s input format: x fp16 [cols] on the device (widened
 * exactly to fp32 in the kernel), otherwise as mmr_matvec_f16. */
int mmr_matvec_f16x(const uint16_t* w, int64_t rows, int64_t cols, const uint16_t* x, const float* residual, float* y,
                    mmr_stream_t stream);

/* ---- lm_head matvec + argmax: device_matmul_argmax (ascend_matmul.h:108-109,
 *      ascend_matmul.cpp:467-502) / cube_matvec_argmax (ascend_matmul.h:127-130).
 * token_out (device int32) receives the first index of the maximum logit
 * (std::max_element, language_model.cpp:408-413); logits (device fp32,
 * nullable) receives all logits.  norm_w != NULL fuses the final RMSNorm
 * (language_model.cpp:325).  The workspace (device, see _workspace_size)
 * holds per-block partials reduced by a second, one-block launch. */
size_t mmr_matvec_argmax_workspace_size(int64_t rows, int64_t cols);
int mmr_matvec_argmax_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, const float* norm_w, float eps,
                          float* logits, int32_t* token_out, void* workspace, size_t workspace_bytes,
                          mmr_stream_t stream);
/* The same with x fp16 [cols] (configs[1]'s lm_head + argmax shape), no norm. */
int mmr_matvec_argmax_f16x(const uint16_t* w, int64_t rows, int64_t cols, const uint16_t* x, float* logits,
                           int32_t* token_out, void* workspace, size_t workspace_bytes, mmr_stream_t stream);

/* ---- RoPE table: cached_rope_table (ascend_custom_ops.cpp:93-123).  Holds
 * the fp32 frequencies inv_freq[i] = 1 / powf(theta, 2i / d) of the CPU
 * formula (decoder_layer.cpp:114); kernels evaluate cos/sin(float(pos) *
 * inv_freq[i]) in fp32 (the reference uploads an fp16 table). */
int mmr_rope_table_create(int64_t max_positions, int64_t head_dim, float theta, mmr_rope_table** out);
int mmr_rope_table_destroy(mmr_rope_table* table);

/* ---- resident KV cache of one layer: CustomAttentionCache /
 * ensure_attention_cache (ascend_custom_ops.cpp:59-65,126-139), which
 * reallocates and drops its rows when a longer context arrives.  Here the
 * cache holds 64-token pages [kv_head][64][head_dim] (fp16 or fp32) in
 * segments that double: segment 0 = positions [0, 512), segment s >= 1 =
 * [512 << (s - 1), 512 << s).  `capacity` bounds the positions; only the
 * rows reserved so far are backed by device memory, and growing adds
 * segments without moving a row.
 *   create:  backs segment 0 (min(capacity, 512) positions);
 *   reserve: backs positions [0, tokens) (allocates, synchronous; not for
 *            stream capture; tokens > capacity -> MMR_ERR_LENGTH);
 *   reset:   frees every segment past the first and marks the cache empty
 *            for mmr_prefill_layer_forward (synchronises the device; do not
 *            replay graphs recorded with the freed segments);
 *   write / read: host rows [first, first + count), keys and values each
 *            [kv_head][count][head_dim] in the cache dtype (fp16 bits or
 *            fp32); write reserves what it writes, read needs backed rows.
 * Op-level calls never allocate: a call touching unbacked rows fails with
 * MMR_ERR_LENGTH; calls with a device-side position flag positions past the
 * backed rows through *error.  Kernels recorded into a graph keep the
 * segments backed when they were recorded. */
int mmr_kv_cache_create(int64_t kv_heads, int64_t head_dim, int64_t capacity, int kv_dtype, mmr_kv_cache** out);
int mmr_kv_cache_destroy(mmr_kv_cache* cache);
int mmr_kv_cache_reserve(mmr_kv_cache* cache, int64_t tokens);
int mmr_kv_cache_reset(mmr_kv_cache* cache);
/* Shape of a cache (any output pointer may be NULL). */
int mmr_kv_cache_info(const mmr_kv_cache* cache, int64_t* kv_heads, int64_t* head_dim, int64_t* capacity,
                      int* kv_dtype);
/* Backed positions (from 0) and the device bytes held (either may be NULL). */
int mmr_kv_cache_backed(const mmr_kv_cache* cache, int64_t* tokens, uint64_t* device_bytes);
/* Device pointers of segment `index` (NULL while unbacked): keys and values
 * [pages][kv_head][64][head_dim] for positions first_token ..
 * first_token + tokens - 1 (tokens = its backed, usable positions). */
int mmr_kv_cache_segment(const mmr_kv_cache* cache, int index, void** keys, void** values, int64_t* first_token,
                         int64_t* tokens);
int mmr_kv_cache_write(mmr_kv_cache* cache, int64_t first, int64_t count, const void* keys, const void* values);
int mmr_kv_cache_read(const mmr_kv_cache* cache, int64_t first, int64_t count, void* keys, void* values);

/* ---- QKV post-process + KV append: device_decode_qkv_postprocess
 * (ascend_custom_ops.h:132-143, ascend_custom_ops.cpp:825-884).
 * qkv fp32 [Hq*d | Hkv*d | Hkv*d]; per-head RMSNorm with eps (honoured; the
 * AscendC kernel hardcodes 1e-5) then RoPE at `position`; q -> query
 * [Hq*d]; k, v appended at cache index tokens - 1. */
int mmr_decode_qkv_postprocess(const float* qkv, const float* q_norm, const float* k_norm, mmr_kv_cache* cache,
                               int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t position,
                               const mmr_rope_table* rope, float eps, float* query, mmr_stream_t stream);

/* ---- decode attention: device_attention_from_cache (ascend_custom_ops.h:145-151,
 * ascend_custom_ops.cpp:886-916).  Attends `query` [Hq*d] over the first
 * `tokens` cached keys: softmax(q.k / sqrt(d)) v per head, GQA mapping
 * kv = h / (Hq/Hkv) (decoder_layer.cpp:184-234).  Split along the context in
 * `splits` tile sets (0 = automatic), merged by a log-sum-exp combine (a
 * second launch on the same stream).  The workspace holds the split partials. */
size_t mmr_attention_workspace_size(int64_t q_heads, int64_t kv_heads, int64_t head_dim, int splits);
int mmr_attention_from_cache(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, float* out, void* workspace, size_t workspace_bytes,
                             int splits, mmr_stream_t stream);

/* No counterpart in the reference: mmr_attention_from_cache without a
 * workspace argument, for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split partials live in a static device array of the
 * library, MMR_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends;
 * a call whose partials (mmr_attention_workspace_size) exceed it fails with
 * MMR_ERR_INVALID_ARGUMENT.  Allocates nothing; the first call on each GPU
 * looks up that GPU's copy of the array (make it outside stream capture).
 * Every call on one GPU shares the array and leaves its contents behind:
 * calls that overlap on one GPU (several streams or threads) race, so the
 * caller serialises them. */
#define MMR_NOALLOC_SCRATCH_BYTES (2u << 20)
int mmr_attention_from_cache_noalloc(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads,
                                     int64_t kv_heads, int64_t head_dim, float* out, int splits,
                                     mmr_stream_t stream);

/* ---- fused post-process + append + attend (the decode-step form of
 * device_decode_attention, ascend_custom_ops.h:153-161): position read from
 * device memory (*position), k/v appended at that index, attention over
 * *position + 1 keys.  *error (device int32) is set to 1 when the position is
 * out of range. */
int mmr_decode_attention_fused(const float* qkv, const float* q_norm, const float* k_norm, float eps,
                               const mmr_rope_table* rope, const int32_t* position, mmr_kv_cache* cache,
                               int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out, void* workspace,
                               size_t workspace_bytes, int splits, int32_t* error, mmr_stream_t stream);

/* ---- host-vector twins and availability probes: cube_matvec,
 * cube_matmul, cube_matvec_argmax, cube_*_available (ascend_matmul.h:116-133,
 * ascend_matmul.cpp:513-693) and custom_ops_available, custom_attention,
 * custom_prefill_attention, custom_attention_cached (ascend_custom_ops.h:13,
 * 33-55, ascend_custom_ops.cpp:333-530).  Every pointer is host memory; each
 * call uploads, runs the device op, waits and copies back (so these
 * allocate and synchronise, as the reference's do).  Matrices are fp32
 * [rows][cols] rounded to fp16 on upload; inputs and outputs stay fp32 (the
 * reference rounds them to fp16).  Caches the twins create are fp32; a
 * caller's fp16 cache keeps its dtype (also when grown) and receives the rows
 * rounded to fp16 (RNE).  keys/values are in the
 * reference layout [token][kv_head][head_dim]; key/value of the cached form
 * are one token's [kv_head][head_dim], written at row tokens - 1.  The cache
 * argument may be *cache == NULL (a new fp32 cache of at least 2048 tokens
 * is created), a cache of another shape (replaced), or a cache too short
 * (grown, rows kept; the reference starts an empty one).  The probes return
 * 1 when a gfx950 device is visible, else 0. */
int mmr_cube_matvec_available(void);
int mmr_cube_matmul_available(void);
int mmr_custom_ops_available(void);
int mmr_cube_matvec(const float* matrix, int64_t rows, int64_t cols, const float* input, float* out);
int mmr_cube_matmul(const float* matrix, int64_t rows, int64_t cols, const float* input, int64_t batch, float* out);
int mmr_cube_matvec_argmax(const float* matrix, int64_t rows, int64_t cols, const float* input, int32_t* token);
int mmr_custom_attention(const float* query, const float* keys, const float* values, int64_t tokens, int64_t q_heads,
                         int64_t kv_heads, int64_t head_dim, float* out);
int mmr_custom_prefill_attention(const float* query, const float* keys, const float* values, mmr_kv_cache** cache,
                                 int64_t seq_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out);
int mmr_custom_attention_cached(const float* query, const float* key, const float* value, mmr_kv_cache** cache,
                                int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out);

/* ---- one decoder layer: run_dense_decoder_layer_device (decoder_layer.h:50-80,
 * decoder_layer.cpp:617-659) and run_dense_decoder_layer (decoder_layer.cpp:312-407)
 * over a LayerKvCache (decoder_layer.h:40-48).
 * Layer weights: the reference's DenseLayerWeights members (decoder_layer.h:19-35),
 * fp32 host arrays, uploaded as fp16 in the runtime's fused layout
 * (mmr_layer_weights_create), or a view of a loaded model's layer that keeps
 * the model's weights alive (mmr_model_layer_weights).
 * mmr_decoder_layer_forward: out = layer(hidden) for the token at device
 * position *position, which is also the cache row its k/v are appended at;
 * attention runs over *position + 1 keys (the reference's cache.tokens after
 * its increment).  hidden/out [hidden_size] fp32 on the device (out may
 * alias hidden); the cache must match the layer (kv_heads, head_dim); splits
 * 0 = automatic from the cache's backed positions (which follow the context
 * when the caller reserves as it goes).  No allocation, no
 * synchronisation: the call may be recorded into a hipGraph and replayed
 * with the position advanced in device memory.  *error (device int32) is
 * set to 1 when *position is outside the backed rows or
 * max_position_embeddings. */
int mmr_layer_weights_create(const mmr_config* config, const float* input_norm, const float* post_attention_norm,
                             const float* q_norm, const float* k_norm, const float* q_proj, const float* k_proj,
                             const float* v_proj, const float* o_proj, const float* gate_proj, const float* up_proj,
                             const float* down_proj, mmr_layer_weights** out);
int mmr_model_layer_weights(const mmr_model* model, int64_t layer, mmr_layer_weights** out);
int mmr_layer_weights_destroy(mmr_layer_weights* weights);
size_t mmr_decoder_layer_workspace_size(const mmr_config* config, int splits);
int mmr_decoder_layer_forward(const mmr_layer_weights* weights, mmr_kv_cache* cache, const float* hidden,
                              const int32_t* position, float* out, void* workspace, size_t workspace_bytes,
                              int splits, int32_t* error, mmr_stream_t stream);

/* ---- one decoder layer over a prompt: run_dense_prefill_layer_device
 * (decoder_layer.h:74-80, decoder_layer.cpp:661-734) and
 * run_dense_prefill_layer (decoder_layer.cpp:409-527).
 * out = layer(hidden_seq) for seq_len rows [seq_len][hidden_size] fp32 on the
 * device (out may alias hidden_seq), on the fp16 matrix cores with fp32
 * accumulation.  Row i's query and key rotate to position start_position + i;
 * the keys and values go to cache rows 0 .. seq_len - 1 and row i attends
 * rows 0 .. i.  The cache must be empty (no prefill-layer call since it was
 * created or reset; else MMR_ERR_INVALID_ARGUMENT, as the reference throws)
 * and backed for seq_len rows; afterwards it counts as holding seq_len rows.
 * The workspace (mmr_prefill_layer_workspace_size bytes) holds every
 * intermediate: no allocation, no synchronisation, graph-capturable. */
size_t mmr_prefill_layer_workspace_size(const mmr_config* config, int64_t seq_len);
int mmr_prefill_layer_forward(const mmr_layer_weights* weights, mmr_kv_cache* cache, const float* hidden_seq,
                              int64_t start_position, int64_t seq_len, float* out, void* workspace,
                              size_t workspace_bytes, mmr_stream_t stream);

/* ---- prefill (run_dense_prefill_layer_device, decoder_layer.cpp:661-734) ----
 * Batched projection: device_matmul / device_matmul_add with batch = seq_len
 * (ascend_matmul.h:102-107) and cube_matmul (ascend_matmul.h:122-126).
 * y[b][r] = sum_c W[r*cols + c] * x[b][c] (+ residual[b][r]); W fp16
 * row-major [rows][cols], x [batch][cols], y/residual [batch][rows] fp32;
 * fp16 matrix cores on x split into hi + lo fp16 planes (W is exact in
 * fp16), fp32 accumulation.  cols % 8 == 0; residual may alias y. */
int mmr_matmul_f16(const uint16_t* w, int64_t rows, int64_t cols, const float* x, int64_t batch,
                   const float* residual, float* y, mmr_stream_t stream);
/* Rows of the fused qkv projection for positions start_position ..
 * start_position + seq_len - 1: device_qkv_split_rows + q/k
 * device_rms_norm_rows + device_rope_rows (ascend_custom_ops.h:80-107) and
 * the KV-cache write of device_prefill_attention (ascend_custom_ops.h:122-130).
 * qkv [seq_len][(Hq + 2 Hkv) d]; query [seq_len][Hq d]. */
int mmr_prefill_qkv_rows(const float* qkv, const float* q_norm, const float* k_norm, float eps,
                         const mmr_rope_table* rope, mmr_kv_cache* cache, int64_t start_position, int64_t seq_len,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* query, mmr_stream_t stream);
/* Causal attention of device_prefill_attention (ascend_custom_ops.h:122-130):
 * query rows at positions start_position + i attend cache keys 0 ..
 * start_position + i.  out [seq_len][Hq d]. */
int mmr_prefill_attention(const float* query, const mmr_kv_cache* cache, int64_t start_position, int64_t seq_len,
                          int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out, mmr_stream_t stream);

/* ---- support ops (ascend_custom_ops.h:70-79,109-120) ----------------------- */
int mmr_rms_norm_rows(const float* in, const float* w, float eps, int64_t rows, int64_t cols, float* out,
                      mmr_stream_t stream);
int mmr_add(const float* a, const float* b, int64_t n, float* out, mmr_stream_t stream);
int mmr_swiglu_rows(const float* gate_up, int64_t rows, int64_t cols, float* out, mmr_stream_t stream);
int mmr_embedding_gather(const uint16_t* table, const int32_t* ids, int64_t tokens, int64_t vocab, int64_t hidden,
                         float* out, int32_t* error, mmr_stream_t stream);

/* ---- model API: LanguageModel / DecoderState (language_model.h:22-49),
 *      load_runtime_language_model / has_runtime_language_model
 *      (runtime_loader.h:9-10) ---------------------------------------------- */
int mmr_default_config(mmr_config* out);
int mmr_load_config(const char* path, mmr_config* out);
int mmr_has_runtime_model(const char* model_dir, int* out);
int mmr_model_load(const char* model_dir, mmr_model** out);
int mmr_model_create_synthetic(const mmr_config* config, uint64_t seed, double std, int round_fp16,
                               mmr_model** out);
int mmr_model_free(mmr_model* model);
int mmr_model_config(const mmr_model* model, mmr_config* out);
int mmr_model_weight_bytes(const mmr_model* model, uint64_t* bytes);

/* Writes minimind_runtime_config.txt + weights.bin (MMRTW001,
 * runtime_loader.cpp:121-167) with seeded synthetic weights. */
int mmr_write_synthetic_model(const char* model_dir, const mmr_config* config, uint64_t seed, double std,
                              int round_fp16);
/* make_toy_language_model (language_model.cpp:415-470): the reference's
 * built-in toy model (hidden 4, head_dim 2, vocab 8, 16 positions), run on
 * the small-model step kernel; mmr_write_toy_model writes the same model as a
 * runtime directory (config + MMRTW001 weights). */
int mmr_model_create_toy(mmr_model** out);
int mmr_write_toy_model(const char* model_dir);
int mmr_synthesize_normals(uint64_t seed, uint64_t first, uint64_t count, double std, int round_fp16, float* out);
int mmr_synthesize_prompt(uint64_t seed, int64_t count, int64_t vocab, int32_t* out);

/* capacity 0 = max_position_embeddings */
int mmr_state_create(const mmr_model* model, int64_t capacity, int kv_dtype, mmr_state** out);
int mmr_state_free(mmr_state* state);
int mmr_state_position(const mmr_state* state, int64_t* position);
/* KV positions the state has backed with device memory so far (its cache
 * grows in doubling segments of 64-token pages as the context reaches them,
 * 512 positions at creation) and the device bytes they hold; either may be
 * NULL. */
int mmr_state_kv_backed(const mmr_state* state, int64_t* tokens, uint64_t* device_bytes);
/* Back KV positions [0, positions) now (at most the capacity), so decoding up
 * to there allocates nothing (allocates; synchronous). */
int mmr_state_reserve(const mmr_model* model, mmr_state* state, int64_t positions);
int mmr_state_stream(const mmr_state* state, mmr_stream_t* stream);
int mmr_state_reset(const mmr_model* model, mmr_state* state);

/* language_model.cpp:297-308 / :310-333 / :335-366 / :368-406 */
int mmr_forward_token(const mmr_model* model, mmr_state* state, int32_t token, float* logits);
int mmr_forward_next_token(const mmr_model* model, mmr_state* state, int32_t token, int32_t* next);
int mmr_prefill_next_token(const mmr_model* model, mmr_state* state, const int32_t* prompt, int64_t n,
                           int32_t* next);
int mmr_generate(const mmr_model* model, const int32_t* prompt, int64_t n, int64_t max_new_tokens, int32_t* out,
                 int64_t* out_count);

/* Device-resident loop (no host round trip per token). */
int mmr_enqueue_prefill(const mmr_model* model, mmr_state* state, const int32_t* prompt, int64_t n);
int mmr_enqueue_decode(const mmr_model* model, mmr_state* state, int64_t steps, int32_t first_token);
int mmr_state_synchronize(const mmr_model* model, mmr_state* state);
int mmr_read_sequence(const mmr_model* model, mmr_state* state, int64_t first, int64_t count, int32_t* out);
int mmr_read_logits(const mmr_model* model, mmr_state* state, float* logits);

/* ---- batched decode.  No counterpart in the reference,
 * whose DecoderState holds one sequence (language_model.h:22-25): `batch`
 * independent sequences advance one greedy token per step in lockstep, each
 * at its own position, with a paged KV cache (64-token pages through a
 * per-sequence page table) and the projections as batch-row GEMMs.  Each
 * sequence decodes exactly as mmr_forward_next_token would decode it alone;
 * there is no EOS stop (callers cut sequences at EOS). */
int mmr_batch_state_create(const mmr_model* model, int64_t batch, int64_t capacity, int kv_dtype,
                           mmr_batch_state** out);
int mmr_batch_state_free(mmr_batch_state* state);
/* batch, capacity (positions per sequence), steps run since the prompts; any may be NULL */
int mmr_batch_state_info(const mmr_batch_state* state, int64_t* batch, int64_t* capacity, int64_t* steps);
int mmr_batch_state_stream(const mmr_batch_state* state, mmr_stream_t* stream);
/* tokens: the prompts concatenated; lengths[batch].  Fresh state only; runs
 * max(lengths) steps (shorter prompts start generating earlier). */
int mmr_batch_prefill(const mmr_model* model, mmr_batch_state* state, const int32_t* tokens, const int64_t* lengths,
                      int64_t batch);
int mmr_batch_decode(const mmr_model* model, mmr_batch_state* state, int64_t steps);
int mmr_batch_synchronize(const mmr_model* model, mmr_batch_state* state);
int mmr_batch_read_sequence(const mmr_model* model, mmr_batch_state* state, int64_t index, int64_t first,
                            int64_t count, int32_t* out);
int mmr_batch_read_logits(const mmr_model* model, mmr_batch_state* state, int64_t index, float* logits);

/* Enqueue `count` launches of one kernel of the decode step on the state's
 * stream, cycling over layers from `layer` (kernel: 0 qkv, 1 attention,
 * 2 o, 3 gate_up, 4 down, 5 lm_head, 6 argmax finalize without step
 * bookkeeping).  For timing
 * with events recorded on the state's stream; overwrites scratch buffers. */
int mmr_launch_step_kernel(const mmr_model* model, mmr_state* state, int kernel, int64_t layer, int64_t count);
/* Average time per launch in us of `count` back-to-back launches of one step
 * kernel (numbering as above), from HIP events on the state's stream: the
 * launches are captured into one hipGraph and replayed (eager launches after
 * 32 warm ones when the state runs without graphs, MMR_NO_GRAPH).
 * Synchronous; overwrites scratch buffers. */
int mmr_time_step_kernel(const mmr_model* model, mmr_state* state, int kernel, int64_t layer, int64_t count,
                         double* avg_us);

#ifdef __cplusplus
}
#endif
#endif /* MMR_H */
