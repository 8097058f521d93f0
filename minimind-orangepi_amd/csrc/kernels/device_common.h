// device_common.h -- small device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

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

// a / b for 0 <= a < 2^20 and 1 <= b < 2^20, by a reciprocal multiply.  The
// exact (a + 0.5) / b lies at least 0.5 / b from every integer.  v_rcp_f32 is
// accurate to 1 ulp and the product adds half an ulp, a relative error below
// 2^-22, i.e. an absolute error below (a + 0.5) / b * 2^-22 < 0.5 / b while
// a + 0.5 < 2^21, so the truncation is exact.  (A runtime integer division is
// a long instruction sequence; this is three instructions.)  The GEMV combine
// prologue gives it element indices below 1024 and head indices below 16,
// l2_warm chunk indices below 2^16 (rows x 16-byte chunks of one block).
__device__ __forceinline__ int small_quotient(int a, int b) {
  return static_cast<int>((static_cast<float>(a) + 0.5f) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
}

// Cross-lane reductions without an LDS round trip.  Inside a 16-lane row the
// partners come from DPP permutations (GFX9 encodings): quad_perm [1,0,3,2]
// and [2,3,0,1] pair lanes within a quad, row_half_mirror (lane i <-> 7 - i of
// each half-row) pairs the two quads of a half-row once each quad is uniform,
// and row_mirror (i <-> 15 - i) pairs the two half-rows.  Rows are then
// combined with v_readlane from lanes 0, 16, 32 and 48.  Each step combines
// two disjoint, already uniform halves, so every lane of a group ends with the
// same bits.  Every lane of the wave must be active (wave-uniform control
// flow), as for any cross-lane operation.
namespace dpp {
constexpr int kQuadXor1 = 0xB1;
constexpr int kQuadXor2 = 0x4E;
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
}  // namespace dpp

template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  const int b = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(b, b, kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float read_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Reduction over aligned groups of kWidth lanes (a power of two <= 64); the
// result is in every lane of the group.
template <int kWidth, typename Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  static_assert(kWidth >= 1 && kWidth <= 64 && (kWidth & (kWidth - 1)) == 0, "width must be a power of two <= 64");
  if constexpr (kWidth >= 2) v = op(v, dpp_move<dpp::kQuadXor1>(v));
  if constexpr (kWidth >= 4) v = op(v, dpp_move<dpp::kQuadXor2>(v));
  if constexpr (kWidth >= 8) v = op(v, dpp_move<dpp::kRowHalfMirror>(v));
  if constexpr (kWidth >= 16) v = op(v, dpp_move<dpp::kRowMirror>(v));
  if constexpr (kWidth == 32) {
    const float lo = op(read_lane(v, 0), read_lane(v, 16));
    const float hi = op(read_lane(v, 32), read_lane(v, 48));
    v = (__lane_id() < 32) ? lo : hi;
  } else if constexpr (kWidth == 64) {
    v = op(op(read_lane(v, 0), read_lane(v, 16)), op(read_lane(v, 32), read_lane(v, 48)));
  }
  return v;
}

template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
  return group_reduce<kWidth>(v, OpSum{});
}

template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
  return group_reduce<kWidth>(v, OpMax{});
}

// (value, index) pair ordering used by every argmax in the runtime: larger
// value wins, equal values resolve to the lower index (the first maximum, as
// std::max_element does).
__device__ __forceinline__ bool argmax_better(float v, int i, float best_v, int best_i) {
  return v > best_v || (v == best_v && i < best_i);
}

template <int kCtrl>
__device__ __forceinline__ int dpp_move_int(int v) {
  return __builtin_amdgcn_update_dpp(v, v, kCtrl, 0xF, 0xF, false);
}

// (max, lowest index) over the 64 lanes of a wave with the DPP steps of
// group_reduce, then the four rows' results in row order (v_readlane); every
// lane ends with the result.  The pair order is associative and commutative,
// so the steps cannot change it.  No LDS traffic: nothing waits on lgkmcnt.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  auto take = [&](float ov, int oi) {
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  };
  take(dpp_move<dpp::kQuadXor1>(v), dpp_move_int<dpp::kQuadXor1>(i));
  take(dpp_move<dpp::kQuadXor2>(v), dpp_move_int<dpp::kQuadXor2>(i));
  take(dpp_move<dpp::kRowHalfMirror>(v), dpp_move_int<dpp::kRowHalfMirror>(i));
  take(dpp_move<dpp::kRowMirror>(v), dpp_move_int<dpp::kRowMirror>(i));
  float bv = read_lane(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int row = 16; row < kWave; row += 16) {
    const float rv = read_lane(v, row);
    const int ri = __builtin_amdgcn_readlane(i, row);
    if (argmax_better(rv, ri, bv, bi)) {
      bv = rv;
      bi = ri;
    }
  }
  v = bv;
  i = bi;
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

// silu(g) = g / (1 + e^-g) with e^-g as 2^(-g log2 e) on v_exp_f32 and the
// quotient as a product with v_rcp_f32 (each within an ulp or two): the
// batched down GEMM, the prefill gate_up epilogue and the decode gate_up
// GEMV apply it, where expf and an IEEE divide cost some 30 instructions.
__device__ __forceinline__ float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

using lds_byte = __attribute__((address_space(3))) char;

// One wave-wide direct load: lane l's `bytes` (16 or 4) at sbase + voff land
// in LDS at m0 + l * bytes.  sbase is a scalar (wave-uniform) address and
// voff this lane's 32-bit byte offset (the scalar-base form of the global
// load), m0 the wave's LDS destination.  M0 is an input operand ("{m0}"): the
// compiler writes it before the statement and knows what it holds after, so
// no value of the compiler's own is lost in it.  A write of M0 needs one wait
// state before an LDS-direct load reads it (s_nop).  The instruction is issued
// from inline assembly so that the compiler, which does not see the LDS write,
// inserts no wait for it: the kernel waits with explicit vmcnt.
template <int kBytes>
__device__ __forceinline__ void dma_load(const void* sbase, uint32_t voff, uint32_t m0) {
  if constexpr (kBytes == 16) {
    asm volatile("s_nop 1\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
  } else {
    static_assert(kBytes == 4, "16- or 4-byte loads");
    asm volatile("s_nop 1\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
  }
}

// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_byte*)p));
}

// Warming block j of set.blocks (the first warming block's id is a multiple
// of kXcds, so j % kXcds is the XCD it runs on): loads what the reading
// blocks of every region on the same XCD will read (the XCD's warming blocks
// take every (set.blocks / kXcds)-th of those blocks), with direct-to-LDS
// loads that hold no registers, into the 1 KB per wave at lds (the block's
// scratch, overwritten), and waits for them.
template <int kThreads>
__device__ void l2_warm(const L2WarmSet& set, int j, void* lds) {
  const int xcd = j % kXcds, slot = j / kXcds, slots = set.blocks / kXcds;
  if (slots <= 0) return;  // the launchers pass a positive multiple of kXcds; the loops below need a stride
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_address(lds) + (threadIdx.x / kWave) * (kWave * 16));
#pragma unroll
  for (int r = 0; r < kL2WarmRegions; ++r) {
    const L2Warm& g = set.region[r];
    if (g.base == nullptr) continue;
    const int units = g.units_x * g.units_y;
    const uint32_t seg_chunks = g.seg_bytes / 16;
    for (int u = xcd + kXcds * slot; u < units; u += kXcds * slots) {
      const int ux = u % g.units_x, uy = u / g.units_x;
      const uint32_t lo = static_cast<uint32_t>(ux) * g.rows * g.row_bytes + static_cast<uint32_t>(uy) * g.seg_bytes;
      if (g.seg_bytes == g.row_bytes) {  // whole rows: one contiguous run
        const uint32_t hi = min(lo + static_cast<uint32_t>(g.rows) * g.row_bytes, g.bytes);
        for (uint32_t off = lo + threadIdx.x * 16; off < hi; off += kThreads * 16) dma_load<16>(g.base, off, m0);
      } else {  // one segment of each of the block's rows
        const uint32_t chunks = static_cast<uint32_t>(g.rows) * seg_chunks;
        for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) {
          const uint32_t row = static_cast<uint32_t>(small_quotient(static_cast<int>(c), static_cast<int>(seg_chunks)));
          const uint32_t off = lo + row * g.row_bytes + (c - row * seg_chunks) * 16;
          if (off < g.bytes) dma_load<16>(g.base, off, m0);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
}

}  // namespace mmr
