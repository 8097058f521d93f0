#include "kv_store.h"

#include <algorithm>
#include <stdexcept>

namespace minimind::model {

namespace {
// Tokens the segment table can address: segments 0 .. kKvSegments - 1.
constexpr int64_t kMaxTokens =
    int64_t{mmr::kv_segment_first(mmr::kKvSegments - 1)} + mmr::kv_segment_tokens(mmr::kKvSegments - 1);
}  // namespace

KvStore::KvStore(int64_t layers, int64_t kv_heads, int64_t head_dim, mmr::KvDtype dtype, int64_t capacity)
    : layers_(layers), kv_heads_(kv_heads), head_dim_(head_dim), capacity_(capacity), dtype_(dtype) {
  if (layers <= 0 || kv_heads <= 0 || head_dim <= 0) throw std::invalid_argument("invalid KV cache shape");
  if (capacity <= 0) throw std::invalid_argument("KV cache capacity must be positive");
  if (capacity > kMaxTokens) throw std::invalid_argument("KV cache capacity exceeds 1,048,576 positions");
  tables_.resize(static_cast<std::size_t>(layers));
}

int64_t KvStore::segment_pages(int s) const {
  const int64_t first = mmr::kv_segment_first(s);
  const int64_t tokens = std::min<int64_t>(mmr::kv_segment_tokens(s), capacity_ - first);
  return (tokens + mmr::kKvPage - 1) / mmr::kKvPage;
}

void KvStore::reserve(int64_t tokens) {
  if (tokens > capacity_) throw std::length_error("KV cache capacity exhausted");
  while (backed_ < tokens) {
    const int s = segments();
    const int64_t pages = segment_pages(s);
    const std::size_t per = static_cast<std::size_t>(pages * kv_heads_ * mmr::kKvPage * head_dim_) * element_bytes();
    DeviceBuffer buf(per * 2 * static_cast<std::size_t>(layers_));
    // Zeroed before first use (synchronous: a new segment is never written by
    // the stream's queued work, which only reaches backed rows).
    check_hip(hipMemset(buf.data(), 0, buf.bytes()), "hipMemset KV segment");
    char* base = static_cast<char*>(buf.data());
    for (int64_t l = 0; l < layers_; ++l) {
      tables_[static_cast<std::size_t>(l)].s[s].k = base + static_cast<std::size_t>(2 * l) * per;
      tables_[static_cast<std::size_t>(l)].s[s].v = base + static_cast<std::size_t>(2 * l + 1) * per;
    }
    segments_.push_back(std::move(buf));
    backed_ = mmr::kv_segment_first(s) + pages * mmr::kKvPage;
  }
}

void KvStore::release_tail() {
  if (segments_.size() <= 1) return;
  check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
  segments_.resize(1);
  for (auto& t : tables_)
    for (int s = 1; s < mmr::kKvSegments; ++s) t.s[s] = mmr::KvSeg{};
  backed_ = segment_pages(0) * mmr::kKvPage;
}

std::size_t KvStore::device_bytes() const noexcept {
  std::size_t total = 0;
  for (const auto& b : segments_) total += b.bytes();
  return total;
}

void KvStore::copy_rows(int64_t layer, int64_t first, int64_t count, void* host_k, void* host_v,
                        bool to_device) const {
  if (layer < 0 || layer >= layers_) throw std::out_of_range("KV cache layer out of range");
  if (first < 0 || count < 0 || first + count > std::min(capacity_, backed_))
    throw std::out_of_range("KV cache rows out of range");
  const mmr::KvSegs& table = tables_[static_cast<std::size_t>(layer)];
  const std::size_t elem = element_bytes();
  const std::size_t row = static_cast<std::size_t>(head_dim_) * elem;
  // One page's run of rows for every head at once: heads are kKvPage rows
  // apart on the device and `count` rows apart on the host.
  for (int64_t t = first; t < first + count;) {
    const int64_t t1 = std::min(first + count, (t / mmr::kKvPage + 1) * mmr::kKvPage);
    const int s = mmr::kv_segment(static_cast<int>(t));
    const int64_t off = mmr::kv_segment_offset(s, static_cast<int>(t), 0, static_cast<int>(kv_heads_),
                                               static_cast<int>(head_dim_));
    const std::size_t dpitch = mmr::kKvPage * row, hpitch = static_cast<std::size_t>(count) * row;
    const std::size_t width = static_cast<std::size_t>(t1 - t) * row, hoff = static_cast<std::size_t>(t - first) * row;
    char* dk = static_cast<char*>(table.s[s].k) + static_cast<std::size_t>(off) * elem;
    char* dv = static_cast<char*>(table.s[s].v) + static_cast<std::size_t>(off) * elem;
    char* hk = static_cast<char*>(host_k) + hoff;
    char* hv = static_cast<char*>(host_v) + hoff;
    const auto h = static_cast<std::size_t>(kv_heads_);
    if (to_device) {
      check_hip(hipMemcpy2D(dk, dpitch, hk, hpitch, width, h, hipMemcpyHostToDevice), "hipMemcpy2D keys");
      check_hip(hipMemcpy2D(dv, dpitch, hv, hpitch, width, h, hipMemcpyHostToDevice), "hipMemcpy2D values");
    } else {
      check_hip(hipMemcpy2D(hk, hpitch, dk, dpitch, width, h, hipMemcpyDeviceToHost), "hipMemcpy2D keys");
      check_hip(hipMemcpy2D(hv, hpitch, dv, dpitch, width, h, hipMemcpyDeviceToHost), "hipMemcpy2D values");
    }
    t = t1;
  }
}

void KvStore::write_rows(int64_t layer, int64_t first, int64_t count, const void* keys, const void* values) {
  if (first < 0 || count < 0) throw std::out_of_range("KV cache rows out of range");
  reserve(first + count);
  copy_rows(layer, first, count, const_cast<void*>(keys), const_cast<void*>(values), true);
}

void KvStore::read_rows(int64_t layer, int64_t first, int64_t count, void* keys, void* values) const {
  copy_rows(layer, first, count, keys, values, false);
}

}  // namespace minimind::model
