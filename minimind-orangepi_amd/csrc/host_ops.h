// host_ops.h -- the reference's host-vector operator twins and availability
// probes (ascend_matmul.h:116-133, ascend_custom_ops.h:13,39-55): each call
// takes host vectors, uploads them, runs the gfx950 op through the device-op
// C ABI, waits, and returns host vectors.  For callers that hold plain
// std::vector data; the decode path itself never uses them.
//
// Differences from the reference, deliberate:
//  * activations and the attention caches stay fp32 (the reference rounds
//    queries, keys and values to fp16 on upload); matrices are rounded to fp16
//    (round to nearest even) as every device projection here is;
//  * a CustomAttentionCache that is too small grows and keeps its rows (the
//    reference replaces it with an empty one, ascend_custom_ops.cpp:409-413,
//    :479-483).
#pragma once

#include "../../include/mmr.h"

#include <cstdint>
#include <memory>
#include <vector>

namespace minimind::model {

// A HIP device of the architecture the library was built for is visible.
bool cube_matvec_available();
bool cube_matmul_available();
bool custom_ops_available();

// y = W x (ascend_matmul.cpp:573-629), W host fp32 [rows][cols] row-major.
std::vector<float> cube_matvec(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                               const std::vector<float>& input);
// Y = X W^T for `batch` rows of X (ascend_matmul.cpp:513-571).
std::vector<float> cube_matmul(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                               const std::vector<float>& input, int64_t batch);
// First index of the maximum of W x (ascend_matmul.cpp:631-693).
int32_t cube_matvec_argmax(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                           const std::vector<float>& input);

// Device KV cache owned by a host-side caller (ascend_custom_ops.cpp:59-65):
// layout [kv_head][rows][head_dim], fp32, capacity at least 2048 tokens.
struct CustomAttentionCache {
  CustomAttentionCache(int64_t kv_heads, int64_t head_dim, int64_t capacity);
  ~CustomAttentionCache();
  CustomAttentionCache(const CustomAttentionCache&) = delete;
  CustomAttentionCache& operator=(const CustomAttentionCache&) = delete;
  mmr_kv_cache* handle = nullptr;
  int64_t kv_heads = 0, head_dim = 0, capacity = 0;
};

// Attention of one query over `tokens` keys/values given as host vectors in
// the reference layout [token][kv_head][d] (ascend_custom_ops.cpp:333-387).
std::vector<float> custom_attention(const std::vector<float>& query, const std::vector<float>& keys,
                                    const std::vector<float>& values, int64_t tokens, int64_t q_heads,
                                    int64_t kv_heads, int64_t head_dim);
// Causal attention of seq_len queries over the first seq_len keys, which are
// written into the cache first (ascend_custom_ops.cpp:389-457).
std::vector<float> custom_prefill_attention(const std::vector<float>& query, const std::vector<float>& keys,
                                            const std::vector<float>& values,
                                            std::shared_ptr<CustomAttentionCache>& cache, int64_t seq_len,
                                            int64_t q_heads, int64_t kv_heads, int64_t head_dim);
// Appends one token's key/value ([kv_head][d]) at row tokens - 1 and attends
// the query over the first `tokens` rows (ascend_custom_ops.cpp:459-530).
std::vector<float> custom_attention_cached(const std::vector<float>& query, const std::vector<float>& key,
                                           const std::vector<float>& value,
                                           std::shared_ptr<CustomAttentionCache>& cache, int64_t tokens,
                                           int64_t q_heads, int64_t kv_heads, int64_t head_dim);

// Pointer forms behind the C ABI (mmr_cube_*, mmr_custom_*): the same
// operations on host arrays, the cache passed as an mmr_kv_cache handle that
// the call may create (when *cache is null), replace (other shape) or grow.
void host_matmul(const float* matrix, int64_t rows, int64_t cols, const float* input, int64_t batch, float* out);
int32_t host_matvec_argmax(const float* matrix, int64_t rows, int64_t cols, const float* input);
void host_attention(const float* query, const float* keys, const float* values, int64_t tokens, int64_t q_heads,
                    int64_t kv_heads, int64_t head_dim, float* out);
void host_prefill_attention(const float* query, const float* keys, const float* values, mmr_kv_cache** cache,
                            int64_t seq_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out);
void host_attention_cached(const float* query, const float* key, const float* value, mmr_kv_cache** cache,
                           int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out);

}  // namespace minimind::model
