// kv_store.h -- one sequence's KV cache, grown page by page in doubling segments.
//
// Counterpart of the reference's resident attention cache (CustomAttentionCache
// and ensure_attention_cache, ascend_custom_ops.cpp:59-65,126-139, which
// reallocates and drops its rows when a longer context arrives) and of the
// CPU LayerKvCache vectors (decoder_layer.h:40-48).  Here the cache holds
// `layers` layers' keys and values in the segment layout of kernels.h:
// 64-token pages [Hkv][64][d], segment 0 = tokens [0, 512), segment s >= 1 =
// [512 << (s - 1), 512 << s).  Only what reserve() asked for is backed; a
// longer context adds segments and never moves a row.  One allocation per
// segment holds every layer's K and V pages of that segment.  Segments are
// freed only by release_tail() and the destructor, so kernels recorded with an
// earlier segment table stay valid while the store lives.
#pragma once

#include "device.h"
#include "../kernels/kernels.h"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace minimind::model {

class KvStore {
 public:
  KvStore() = default;
  // `capacity` positions at most; nothing is backed until reserve().
  KvStore(int64_t layers, int64_t kv_heads, int64_t head_dim, mmr::KvDtype dtype, int64_t capacity);

  // Back tokens [0, tokens) (whole segments, never past capacity); tokens
  // above capacity raise std::length_error.  Allocates; not for stream capture.
  void reserve(int64_t tokens);
  // Free every segment past the first (the store returns to its first
  // segment's footprint); the caller must not replay launches recorded with
  // the freed segments.  Synchronises the device first.
  void release_tail();

  int64_t capacity() const noexcept { return capacity_; }
  int64_t backed() const noexcept { return backed_; }  // tokens [0, backed) are backed (a multiple of 64 or capacity)
  int64_t layers() const noexcept { return layers_; }
  int64_t kv_heads() const noexcept { return kv_heads_; }
  int64_t head_dim() const noexcept { return head_dim_; }
  mmr::KvDtype dtype() const noexcept { return dtype_; }
  std::size_t element_bytes() const noexcept { return dtype_ == mmr::kKvF16 ? 2 : 4; }
  std::size_t device_bytes() const noexcept;
  int segments() const noexcept { return static_cast<int>(segments_.size()); }
  // Segment table of one layer (unbacked segments null), as kernels take it.
  const mmr::KvSegs& layer(int64_t l) const { return tables_.at(static_cast<std::size_t>(l)); }

  // Host copies of rows [first, first + count) of one layer, keys and values
  // each [kv_head][count][head_dim] in the cache dtype.  write_rows reserves
  // what it writes.  Synchronous.
  void write_rows(int64_t layer, int64_t first, int64_t count, const void* keys, const void* values);
  void read_rows(int64_t layer, int64_t first, int64_t count, void* keys, void* values) const;

 private:
  int64_t segment_pages(int s) const;  // pages of segment s (the last one cut at capacity)
  void copy_rows(int64_t layer, int64_t first, int64_t count, void* host_k, void* host_v, bool to_device) const;

  int64_t layers_ = 0, kv_heads_ = 0, head_dim_ = 0, capacity_ = 0, backed_ = 0;
  mmr::KvDtype dtype_ = mmr::kKvF32;
  std::vector<DeviceBuffer> segments_;
  std::vector<mmr::KvSegs> tables_;  // per layer
};

}  // namespace minimind::model
