// attention_common.h -- layout helpers shared by the attention kernels and the
// O-projection GEMV, whose prologue merges the attention split partials.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace mmr {

template <int D>
constexpr int attn_tile_tokens() {
  return D <= 96 ? 64 : 32;
}

// Split partial of query head h (h-th head of KV group g) from split s:
// [m, l, o[0..d)] at this float offset; layout [Hkv][splits][R][d + 2].
__host__ __device__ inline int64_t attn_partial_offset(int g, int s, int h, int splits, int R, int d) {
  return ((static_cast<int64_t>(g) * splits + s) * R + h) * (d + 2);
}

// 16-byte load unit of a KV element type.
template <typename KV>
struct ChunkOf {
  using type = uint4;
};

}  // namespace mmr
