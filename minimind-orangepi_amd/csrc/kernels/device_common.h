// device_common.h -- small device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace mmr {

constexpr int kWave = 64;  // CDNA wavefront width

// Eight fp16 values packed in 16 bytes -> eight fp32 values (exact).
__device__ __forceinline__ void half8_to_float8(const uint4& u, float* f) {
  const __half2* h = reinterpret_cast<const __half2*>(&u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float2 v = __half22float2(h[i]);
    f[2 * i] = v.x;
    f[2 * i + 1] = v.y;
  }
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = kWidth / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWidth);
  return v;
}

template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = kWidth / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWidth));
  return v;
}

// (value, index) pair ordering used by every argmax in the runtime: larger
// value wins, equal values resolve to the lower index (the first maximum, as
// std::max_element does).
__device__ __forceinline__ bool argmax_better(float v, int i, float best_v, int best_i) {
  return v > best_v || (v == best_v && i < best_i);
}

template <typename T>
__device__ __forceinline__ float to_float(T v);
template <>
__device__ __forceinline__ float to_float<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float to_float<__half>(__half v) {
  return __half2float(v);
}

template <typename T>
__device__ __forceinline__ T from_float(float v);
template <>
__device__ __forceinline__ float from_float<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ __half from_float<__half>(float v) {
  return __float2half_rn(v);
}

}  // namespace mmr
