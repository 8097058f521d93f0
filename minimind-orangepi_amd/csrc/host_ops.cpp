// host_ops.cpp -- host-vector operator twins over the device-op C ABI.
#include "host_ops.h"

#include "runtime/device.h"
#include "runtime/weights.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace minimind::model {

namespace {

// C status -> the reference's exception classes.
void ok(int status) {
  if (status == MMR_OK) return;
  const std::string msg = mmr_last_error();
  switch (status) {
    case MMR_ERR_INVALID_ARGUMENT:
      throw std::invalid_argument(msg);
    case MMR_ERR_OUT_OF_RANGE:
      throw std::out_of_range(msg);
    case MMR_ERR_LENGTH:
      throw std::length_error(msg);
    default:
      throw std::runtime_error(msg);
  }
}

// Capacity a new cache gets: the reference's ensure_attention_cache floor.
constexpr int64_t kMinCacheTokens = 2048;

void require(bool cond, const char* msg) {
  if (!cond) throw std::invalid_argument(msg);
}

void check_heads(int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  require(q_heads > 0 && kv_heads > 0 && head_dim > 0 && q_heads % kv_heads == 0, "invalid attention shape");
}

std::vector<uint16_t> to_half(const float* v, std::size_t n) {
  std::vector<uint16_t> out(n);
  for (std::size_t i = 0; i < n; ++i) out[i] = float_to_half(v[i]);
  return out;
}

// Keys/values of tokens [first, first + count) from the reference layout
// [token][kv_head][d] (fp32) into the cache, as [kv_head][count][d] rows of
// the cache's element type: an fp16 cache gets the rows rounded to fp16
// (RNE), the rounding the decode kernels apply when they append.
void write_rows(mmr_kv_cache* cache, const float* keys, const float* values, int64_t first, int64_t count,
                int64_t kv_heads, int64_t head_dim) {
  int dtype = MMR_KV_F32;
  ok(mmr_kv_cache_info(cache, nullptr, nullptr, nullptr, &dtype));
  const std::size_t n = static_cast<std::size_t>(count * kv_heads * head_dim);
  std::vector<float> kf(n), vf(n);
  for (int64_t t = 0; t < count; ++t)
    for (int64_t h = 0; h < kv_heads; ++h)
      for (int64_t d = 0; d < head_dim; ++d) {
        const std::size_t src = static_cast<std::size_t>((t * kv_heads + h) * head_dim + d);
        const std::size_t dst = static_cast<std::size_t>((h * count + t) * head_dim + d);
        kf[dst] = keys[src];
        vf[dst] = values[src];
      }
  if (dtype == MMR_KV_F16) {
    const auto kh = to_half(kf.data(), n), vh = to_half(vf.data(), n);
    ok(mmr_kv_cache_write(cache, first, count, kh.data(), vh.data()));
  } else {
    ok(mmr_kv_cache_write(cache, first, count, kf.data(), vf.data()));
  }
}

// A cache of this shape holding at least `needed` tokens: created when
// absent, replaced when its shape differs, and when its capacity is short,
// replaced by one of twice the capacity holding the same rows and dtype.
void ensure_cache(mmr_kv_cache** cache, int64_t kv_heads, int64_t head_dim, int64_t needed) {
  int64_t kvh = 0, d = 0, cap = 0;
  int dtype = MMR_KV_F32;
  if (*cache != nullptr) ok(mmr_kv_cache_info(*cache, &kvh, &d, &cap, &dtype));
  if (*cache != nullptr && kvh == kv_heads && d == head_dim && cap >= needed) return;
  const bool keep = *cache != nullptr && kvh == kv_heads && d == head_dim;
  mmr_kv_cache* fresh = nullptr;
  ok(mmr_kv_cache_create(kv_heads, head_dim, std::max(needed, keep ? 2 * cap : kMinCacheTokens),
                         keep ? dtype : MMR_KV_F32, &fresh));
  std::unique_ptr<mmr_kv_cache, int (*)(mmr_kv_cache*)> guard(fresh, mmr_kv_cache_destroy);
  if (keep) {  // rows [0, backed) move over through the host, in the cache layout and dtype
    int64_t backed = 0;
    ok(mmr_kv_cache_backed(*cache, &backed, nullptr));
    const std::size_t bytes = static_cast<std::size_t>(backed * kv_heads * head_dim) * (dtype == MMR_KV_F16 ? 2 : 4);
    std::vector<char> k(bytes), v(bytes);
    ok(mmr_kv_cache_read(*cache, 0, backed, k.data(), v.data()));
    ok(mmr_kv_cache_write(fresh, 0, backed, k.data(), v.data()));
  }
  if (*cache != nullptr) ok(mmr_kv_cache_destroy(*cache));
  *cache = guard.release();
}

// out = attention of `query` [q_heads][d] over the first `tokens` cache rows.
void attend(const float* query, const mmr_kv_cache* cache, int64_t tokens, int64_t q_heads, int64_t kv_heads,
            int64_t head_dim, float* out) {
  const std::size_t qn = static_cast<std::size_t>(q_heads * head_dim);
  DeviceBuffer q(qn * 4), o(qn * 4);
  DeviceBuffer ws(mmr_attention_workspace_size(q_heads, kv_heads, head_dim, 0));
  check_hip(hipMemcpy(q.data(), query, qn * 4, hipMemcpyHostToDevice), "hipMemcpy query");
  ok(mmr_attention_from_cache(static_cast<const float*>(q.data()), cache, tokens, q_heads, kv_heads, head_dim,
                              static_cast<float*>(o.data()), ws.data(), ws.bytes(), 0, nullptr));
  check_hip(hipMemcpy(out, o.data(), qn * 4, hipMemcpyDeviceToHost), "hipMemcpy attention out");
}

}  // namespace

bool custom_ops_available() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
    (void)hipGetLastError();
    return false;
  }
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}
bool cube_matvec_available() { return custom_ops_available(); }
bool cube_matmul_available() { return custom_ops_available(); }

void host_matmul(const float* matrix, int64_t rows, int64_t cols, const float* input, int64_t batch, float* out) {
  require(matrix && input && out, "null argument");
  require(rows > 0 && cols > 0 && batch > 0, "rows, cols and batch must be positive");
  const auto w = to_half(matrix, static_cast<std::size_t>(rows * cols));
  DeviceBuffer dw(w.size() * 2), dx(static_cast<std::size_t>(batch * cols) * 4),
      dy(static_cast<std::size_t>(batch * rows) * 4);
  check_hip(hipMemcpy(dw.data(), w.data(), w.size() * 2, hipMemcpyHostToDevice), "hipMemcpy matrix");
  check_hip(hipMemcpy(dx.data(), input, dx.bytes(), hipMemcpyHostToDevice), "hipMemcpy input");
  const auto* wp = static_cast<const uint16_t*>(dw.data());
  const auto* xp = static_cast<const float*>(dx.data());
  auto* yp = static_cast<float*>(dy.data());
  ok(batch == 1 ? mmr_matvec_f16(wp, rows, cols, xp, nullptr, yp, nullptr)
                : mmr_matmul_f16(wp, rows, cols, xp, batch, nullptr, yp, nullptr));
  check_hip(hipMemcpy(out, dy.data(), dy.bytes(), hipMemcpyDeviceToHost), "hipMemcpy output");
}

int32_t host_matvec_argmax(const float* matrix, int64_t rows, int64_t cols, const float* input) {
  require(matrix && input, "null argument");
  require(rows > 0 && cols > 0, "rows and cols must be positive");
  const auto w = to_half(matrix, static_cast<std::size_t>(rows * cols));
  DeviceBuffer dw(w.size() * 2), dx(static_cast<std::size_t>(cols) * 4), tok(4);
  const std::size_t wsb = mmr_matvec_argmax_workspace_size(rows, cols);
  require(wsb > 0, "unsupported matvec shape: cols must be a multiple of 8 and <= 4096");
  DeviceBuffer ws(wsb);
  check_hip(hipMemcpy(dw.data(), w.data(), w.size() * 2, hipMemcpyHostToDevice), "hipMemcpy matrix");
  check_hip(hipMemcpy(dx.data(), input, dx.bytes(), hipMemcpyHostToDevice), "hipMemcpy input");
  ok(mmr_matvec_argmax_f16(static_cast<const uint16_t*>(dw.data()), rows, cols, static_cast<const float*>(dx.data()),
                           nullptr, 0.0f, nullptr, static_cast<int32_t*>(tok.data()), ws.data(), wsb, nullptr));
  int32_t token = 0;
  check_hip(hipMemcpy(&token, tok.data(), 4, hipMemcpyDeviceToHost), "hipMemcpy token");
  return token;
}

void host_attention(const float* query, const float* keys, const float* values, int64_t tokens, int64_t q_heads,
                    int64_t kv_heads, int64_t head_dim, float* out) {
  require(query && keys && values && out, "null argument");
  check_heads(q_heads, kv_heads, head_dim);
  require(tokens > 0, "tokens must be positive");
  mmr_kv_cache* cache = nullptr;
  ok(mmr_kv_cache_create(kv_heads, head_dim, tokens, MMR_KV_F32, &cache));
  std::unique_ptr<mmr_kv_cache, int (*)(mmr_kv_cache*)> guard(cache, mmr_kv_cache_destroy);
  write_rows(cache, keys, values, 0, tokens, kv_heads, head_dim);
  attend(query, cache, tokens, q_heads, kv_heads, head_dim, out);
}

void host_prefill_attention(const float* query, const float* keys, const float* values, mmr_kv_cache** cache,
                            int64_t seq_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out) {
  require(query && keys && values && cache && out, "null argument");
  check_heads(q_heads, kv_heads, head_dim);
  require(seq_len > 0, "seq_len must be positive");
  ensure_cache(cache, kv_heads, head_dim, seq_len);
  write_rows(*cache, keys, values, 0, seq_len, kv_heads, head_dim);
  const std::size_t n = static_cast<std::size_t>(seq_len * q_heads * head_dim);
  DeviceBuffer q(n * 4), o(n * 4);
  check_hip(hipMemcpy(q.data(), query, n * 4, hipMemcpyHostToDevice), "hipMemcpy query");
  ok(mmr_prefill_attention(static_cast<const float*>(q.data()), *cache, 0, seq_len, q_heads, kv_heads, head_dim,
                           static_cast<float*>(o.data()), nullptr));
  check_hip(hipMemcpy(out, o.data(), n * 4, hipMemcpyDeviceToHost), "hipMemcpy prefill out");
}

void host_attention_cached(const float* query, const float* key, const float* value, mmr_kv_cache** cache,
                           int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out) {
  require(query && key && value && cache && out, "null argument");
  check_heads(q_heads, kv_heads, head_dim);
  require(tokens > 0, "tokens must be positive");
  ensure_cache(cache, kv_heads, head_dim, tokens);
  write_rows(*cache, key, value, tokens - 1, 1, kv_heads, head_dim);
  attend(query, *cache, tokens, q_heads, kv_heads, head_dim, out);
}

std::vector<float> cube_matvec(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                               const std::vector<float>& input) {
  return cube_matmul(matrix, rows, cols, input, 1);
}

std::vector<float> cube_matmul(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                               const std::vector<float>& input, int64_t batch) {
  require(static_cast<int64_t>(matrix.size()) == rows * cols, "matrix size does not match rows * cols");
  require(static_cast<int64_t>(input.size()) == batch * cols, "input size does not match batch * cols");
  std::vector<float> out(static_cast<std::size_t>(std::max<int64_t>(batch * rows, 0)));
  host_matmul(matrix.data(), rows, cols, input.data(), batch, out.data());
  return out;
}

int32_t cube_matvec_argmax(const std::vector<float>& matrix, int64_t rows, int64_t cols,
                           const std::vector<float>& input) {
  require(static_cast<int64_t>(matrix.size()) == rows * cols, "matrix size does not match rows * cols");
  require(static_cast<int64_t>(input.size()) == cols, "input size does not match cols");
  return host_matvec_argmax(matrix.data(), rows, cols, input.data());
}

CustomAttentionCache::CustomAttentionCache(int64_t kvh, int64_t d, int64_t cap)
    : kv_heads(kvh), head_dim(d), capacity(std::max(cap, kMinCacheTokens)) {
  ok(mmr_kv_cache_create(kv_heads, head_dim, capacity, MMR_KV_F32, &handle));
}

CustomAttentionCache::~CustomAttentionCache() {
  if (handle) (void)mmr_kv_cache_destroy(handle);
}

namespace {

// The C++ cache object around a handle the pointer forms may have replaced.
void refresh(std::shared_ptr<CustomAttentionCache>& cache) {
  int dtype = 0;
  ok(mmr_kv_cache_info(cache->handle, &cache->kv_heads, &cache->head_dim, &cache->capacity, &dtype));
}

std::shared_ptr<CustomAttentionCache>& usable(std::shared_ptr<CustomAttentionCache>& cache, int64_t kv_heads,
                                              int64_t head_dim, int64_t needed) {
  if (!cache || cache->kv_heads != kv_heads || cache->head_dim != head_dim)
    cache = std::make_shared<CustomAttentionCache>(kv_heads, head_dim, needed);
  return cache;
}

}  // namespace

std::vector<float> custom_attention(const std::vector<float>& query, const std::vector<float>& keys,
                                    const std::vector<float>& values, int64_t tokens, int64_t q_heads,
                                    int64_t kv_heads, int64_t head_dim) {
  check_heads(q_heads, kv_heads, head_dim);
  require(static_cast<int64_t>(query.size()) == q_heads * head_dim &&
              static_cast<int64_t>(keys.size()) == tokens * kv_heads * head_dim &&
              static_cast<int64_t>(values.size()) == tokens * kv_heads * head_dim,
          "custom_attention shape mismatch");
  std::vector<float> out(query.size());
  host_attention(query.data(), keys.data(), values.data(), tokens, q_heads, kv_heads, head_dim, out.data());
  return out;
}

std::vector<float> custom_prefill_attention(const std::vector<float>& query, const std::vector<float>& keys,
                                            const std::vector<float>& values,
                                            std::shared_ptr<CustomAttentionCache>& cache, int64_t seq_len,
                                            int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  check_heads(q_heads, kv_heads, head_dim);
  require(static_cast<int64_t>(query.size()) == seq_len * q_heads * head_dim &&
              static_cast<int64_t>(keys.size()) == seq_len * kv_heads * head_dim &&
              static_cast<int64_t>(values.size()) == seq_len * kv_heads * head_dim,
          "custom_prefill_attention shape mismatch");
  std::vector<float> out(query.size());
  auto& c = usable(cache, kv_heads, head_dim, seq_len);
  host_prefill_attention(query.data(), keys.data(), values.data(), &c->handle, seq_len, q_heads, kv_heads, head_dim,
                         out.data());
  refresh(c);
  return out;
}

std::vector<float> custom_attention_cached(const std::vector<float>& query, const std::vector<float>& key,
                                           const std::vector<float>& value,
                                           std::shared_ptr<CustomAttentionCache>& cache, int64_t tokens,
                                           int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  check_heads(q_heads, kv_heads, head_dim);
  require(static_cast<int64_t>(query.size()) == q_heads * head_dim &&
              static_cast<int64_t>(key.size()) == kv_heads * head_dim &&
              static_cast<int64_t>(value.size()) == kv_heads * head_dim,
          "custom_attention_cached shape mismatch");
  std::vector<float> out(query.size());
  auto& c = usable(cache, kv_heads, head_dim, tokens);
  host_attention_cached(query.data(), key.data(), value.data(), &c->handle, tokens, q_heads, kv_heads, head_dim,
                        out.data());
  refresh(c);
  return out;
}

}  // namespace minimind::model
