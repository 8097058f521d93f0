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

// Cross-block handoff without cache maintenance.  On gfx950 a device-scope
// fence (__threadfence) writes back and invalidates the whole L2 of the XCD,
// which evicts the weights the other blocks are streaming.  Values handed to
// the last block are therefore written with agent-scope atomic stores (sc1:
// write-through to the coherence point) and read back with agent-scope atomic
// loads, and the ticket only has to wait for those stores to complete.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Last-block-done ticket.  Every block calls it once after writing its
// partial results with store_coherent / device atomics; it returns true in
// exactly one block (the last to arrive), which may then read every other
// block's partials with load_coherent.  The last block re-arms the counter so
// the next launch (or a graph replay) starts from zero without a memset.
__device__ __forceinline__ bool last_block_ticket(unsigned int* counter, unsigned int expected) {
  __shared__ bool is_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial writes have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == expected - 1u);
    if (is_last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return is_last;
}

// Order-preserving 64-bit key for a first-index argmax through atomicMax:
// high word = float mapped to an unsigned total order (-0 folded into +0),
// low word = ~index so that equal values prefer the lower index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  const unsigned int u = __float_as_uint(v + 0.0f);
  const unsigned int ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(ord) << 32) | static_cast<unsigned int>(0xffffffffu - static_cast<unsigned int>(idx));
}
__device__ __forceinline__ int argmax_key_index(unsigned long long key) {
  return static_cast<int>(0xffffffffu - static_cast<unsigned int>(key & 0xffffffffull));
}

}  // namespace mmr
