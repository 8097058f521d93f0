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

// Split partials of query head h (the h-th head of KV group g) from split s,
// two regions one after the other in one fp32 buffer:
//   o  [Hkv][splits][R][d]  unnormalised sum of exp(score - m) * v (rows are
//                           16-byte aligned, so the combine reads float4s);
//   ml [Hkv][splits][R][2]  (m, l): running max and sum of exp(score - m).
// Total hkv * splits * R * (d + 2) floats.
__host__ __device__ inline int64_t attn_o_offset(int g, int s, int h, int splits, int R, int d) {
  return ((static_cast<int64_t>(g) * splits + s) * R + h) * d;
}
__host__ __device__ inline int64_t attn_ml_offset(int g, int s, int h, int splits, int R, int d, int hkv) {
  return static_cast<int64_t>(hkv) * splits * R * d + ((static_cast<int64_t>(g) * splits + s) * R + h) * 2;
}

// 16-byte load unit of a KV element type.
template <typename KV>
struct ChunkOf {
  using type = uint4;
};

}  // namespace mmr
