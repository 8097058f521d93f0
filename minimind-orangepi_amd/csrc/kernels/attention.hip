// attention.hip -- GQA decode attention over a resident KV cache (gfx950).
//
// Replaces, on the decode path:
//  * the QKV post-process + resident KV append (reference K2,
//    mini_mind_decode_qkv_postprocess via device_decode_qkv_postprocess,
//    ascend_custom_ops.cpp:825-884; CPU semantics decoder_layer.cpp:342-359),
//  * the decode attention (reference K3 via device_attention_from_cache,
//    ascend_custom_ops.cpp:886-916; CPU semantics decoder_layer.cpp:184-234).
//
// Layout: per layer the cache holds K and V as [kv_head][capacity][head_dim]
// (fp16 or fp32), so one KV head's context is one contiguous stream.
//
// Grid (splits, kv_heads), 256 threads.  A block owns one KV head and a range
// of 64-token tiles (32 for d = 128) and serves all Hq/Hkv query heads of the
// group from that single read of K/V:
//   1. prologue: per-head q RMSNorm + RoPE (fp32 cos/sin table) into LDS; the
//      block whose range holds the new token also normalises/rotates its k,
//      rounds k and v to the cache dtype and appends them to the cache;
//   2. per tile: K/V staged through LDS with 16-byte coalesced loads, one lane
//      per token computes q.k / sqrt(d), online softmax per head (one wave per
//      head), P.V with one lane per dimension pair;
//   3. the last block of each KV head (ticket counter) merges the per-split
//      (max, sum, o) partials with a log-sum-exp combine in fixed split order,
//      so results are deterministic.
#include "device_common.h"
#include "kernels.h"

namespace mmr {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;

template <int D>
constexpr int tile_tokens() {
  return D <= 96 ? 64 : 32;
}

template <typename KV>
__device__ __forceinline__ void load_chunk(const KV* src, float* dst);
template <>
__device__ __forceinline__ void load_chunk<__half>(const __half* src, float* dst) {
  half8_to_float8(*reinterpret_cast<const uint4*>(src), dst);
}
template <>
__device__ __forceinline__ void load_chunk<float>(const float* src, float* dst) {
  const float4 v = *reinterpret_cast<const float4*>(src);
  dst[0] = v.x;
  dst[1] = v.y;
  dst[2] = v.z;
  dst[3] = v.w;
}

// Per-head RMSNorm of `src` (decoder_layer.cpp:32-42, x * (scale * w)) into
// dst, executed by one wave; d <= 128 so a lane owns dims lane and lane + 64.
template <int D>
__device__ __forceinline__ void wave_rms_norm(const float* src, const float* w, float eps, float* dst, int lane) {
  const float x0 = lane < D ? src[lane] : 0.0f;
  const float x1 = lane + kWave < D ? src[lane + kWave] : 0.0f;
  const float ss = group_sum<kWave>(x0 * x0 + x1 * x1);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
  if (lane < D) dst[lane] = x0 * (scale * w[lane]);
  if (lane + kWave < D) dst[lane + kWave] = x1 * (scale * w[lane + kWave]);
}

// Rotate-half RoPE in place on one head held in LDS (decoder_layer.cpp:139-152).
template <int D>
__device__ __forceinline__ void wave_rope(float* x, const float* cos_row, const float* sin_row, int lane) {
  constexpr int kHalf = D / 2;
  for (int i = lane; i < kHalf; i += kWave) {
    const float first = x[i];
    const float second = x[i + kHalf];
    const float c = cos_row[i];
    const float s = sin_row[i];
    x[i] = first * c - second * s;
    x[i + kHalf] = second * c + first * s;
  }
}

template <typename KV, int D, int MODE>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnArgs a) {
  constexpr int TT = tile_tokens<D>();
  constexpr int LD = D + 4;  // padded row: conflict-free 16-byte LDS reads
  constexpr int CH = 16 / static_cast<int>(sizeof(KV));
  constexpr int kHalf = D / 2;
  __shared__ __align__(16) float q_s[kAttnMaxGroup][D];
  __shared__ __align__(16) float k_s[TT][LD];
  __shared__ __align__(16) float v_s[TT][LD];
  __shared__ float p_s[kAttnMaxGroup][TT];
  __shared__ float knew_s[D];
  __shared__ float vnew_s[D];

  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int R = a.hq / a.hkv;
  const int S = a.splits;

  int n_keys = 0;
  int p = -1;
  if constexpr (MODE == kAttnFused) {
    p = *a.pos;
    if (p < 0 || p >= a.capacity || p >= a.max_pos) {
      if (threadIdx.x == 0 && split == 0 && g == 0) *a.err = 1;
    } else {
      n_keys = p + 1;
    }
  } else {
    n_keys = a.tokens < a.capacity ? a.tokens : a.capacity;
  }
  const int n_tiles = (n_keys + TT - 1) / TT;
  const int tps = n_tiles > 0 ? (n_tiles + S - 1) / S : 1;
  const int active = n_tiles > 0 ? (n_tiles + tps - 1) / tps : 0;
  const int tile_begin = split * tps;
  const int tile_end = min(n_tiles, tile_begin + tps);

  if (tile_begin < tile_end) {
    const bool owns_new = (MODE == kAttnFused) && p >= tile_begin * TT && p < tile_end * TT;
    const float* cos_row = nullptr;
    const float* sin_row = nullptr;
    if constexpr (MODE == kAttnFused) {
      cos_row = a.rope_cos + static_cast<int64_t>(p) * kHalf;
      sin_row = a.rope_sin + static_cast<int64_t>(p) * kHalf;
    }

    // ---- prologue: queries (and the new key/value) ----
    for (int h = wave; h < R; h += kAttnWaves) {
      const int qh = g * R + h;
      if constexpr (MODE == kAttnFused) {
        wave_rms_norm<D>(a.qkv + qh * D, a.q_norm, a.eps, q_s[h], lane);
      } else {
        if (lane < D) q_s[h][lane] = a.q[qh * D + lane];
        if (lane + kWave < D) q_s[h][lane + kWave] = a.q[qh * D + lane + kWave];
      }
    }
    if (owns_new && wave == kAttnWaves - 1) {
      const float* kraw = a.qkv + a.hq * D + g * D;
      const float* vraw = a.qkv + a.hq * D + a.hkv * D + g * D;
      wave_rms_norm<D>(kraw, a.k_norm, a.eps, knew_s, lane);
      if (lane < D) vnew_s[lane] = vraw[lane];
      if (lane + kWave < D) vnew_s[lane + kWave] = vraw[lane + kWave];
    }
    __syncthreads();
    if constexpr (MODE == kAttnFused) {
      for (int h = wave; h < R; h += kAttnWaves) wave_rope<D>(q_s[h], cos_row, sin_row, lane);
      if (owns_new && wave == kAttnWaves - 1) wave_rope<D>(knew_s, cos_row, sin_row, lane);
      __syncthreads();
      if (owns_new && wave == kAttnWaves - 1) {
        // Round to the cache dtype once; this step and later steps then see
        // the same key/value.
        KV* kdst = reinterpret_cast<KV*>(a.kcache) + (static_cast<int64_t>(g) * a.capacity + p) * D;
        KV* vdst = reinterpret_cast<KV*>(a.vcache) + (static_cast<int64_t>(g) * a.capacity + p) * D;
        for (int i = lane; i < D; i += kWave) {
          const KV kq = from_float<KV>(knew_s[i]);
          const KV vq = from_float<KV>(vnew_s[i]);
          kdst[i] = kq;
          vdst[i] = vq;
          knew_s[i] = to_float<KV>(kq);
          vnew_s[i] = to_float<KV>(vq);
        }
      }
      __syncthreads();
    }

    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    const float sqrt_d = sqrtf(static_cast<float>(D));

    const KV* kbase = reinterpret_cast<const KV*>(a.kcache) + static_cast<int64_t>(g) * a.capacity * D;
    const KV* vbase = reinterpret_cast<const KV*>(a.vcache) + static_cast<int64_t>(g) * a.capacity * D;

    for (int tile = tile_begin; tile < tile_end; ++tile) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      // ---- stage K/V tile through LDS ----
      const int nchunks = rows * D / CH;
      for (int c = threadIdx.x; c < nchunks; c += kAttnThreads) {
        const int r = (c * CH) / D;
        const int col = (c * CH) % D;
        if (MODE == kAttnFused && t0 + r == p) continue;
        const int64_t off = static_cast<int64_t>(t0 + r) * D + col;
        load_chunk<KV>(kbase + off, &k_s[r][col]);
        load_chunk<KV>(vbase + off, &v_s[r][col]);
      }
      if (MODE == kAttnFused && p >= t0 && p < t0 + rows) {
        const int r = p - t0;
        for (int i = threadIdx.x; i < D; i += kAttnThreads) {
          k_s[r][i] = knew_s[i];
          v_s[r][i] = vnew_s[i];
        }
      }
      __syncthreads();

      // ---- scores and online softmax: one wave per query head ----
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int h = wave + j * kAttnWaves;
        if (h >= R) break;
        float s = -INFINITY;
        if (lane < rows) {
          float dot = 0.0f;
#pragma unroll
          for (int dd = 0; dd < D; dd += 4) {
            const float4 kv4 = *reinterpret_cast<const float4*>(&k_s[lane][dd]);
            const float4 q4 = *reinterpret_cast<const float4*>(&q_s[h][dd]);
            dot = fmaf(q4.x, kv4.x, dot);
            dot = fmaf(q4.y, kv4.y, dot);
            dot = fmaf(q4.z, kv4.z, dot);
            dot = fmaf(q4.w, kv4.w, dot);
          }
          s = dot / sqrt_d;  // decoder_layer.cpp:213 divides by sqrt(d)
        }
        const float m_tile = group_max<kWave>(s);
        const float m_new = fmaxf(m_run[j], m_tile);
        const float alpha = expf(m_run[j] - m_new);
        const float pv = lane < rows ? expf(s - m_new) : 0.0f;
        l_run[j] = l_run[j] * alpha + group_sum<kWave>(pv);
        if (lane < TT) p_s[h][lane] = pv;
        acc[j][0] *= alpha;
        acc[j][1] *= alpha;
        m_run[j] = m_new;
      }
      __syncthreads();

      // ---- P.V ----
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int h = wave + j * kAttnWaves;
        if (h >= R) break;
        float a0 = acc[j][0];
        float a1 = acc[j][1];
        for (int t = 0; t < rows; ++t) {
          const float pt = p_s[h][t];
          if (lane < D) a0 = fmaf(pt, v_s[t][lane], a0);
          if (lane + kWave < D) a1 = fmaf(pt, v_s[t][lane + kWave], a1);
        }
        acc[j][0] = a0;
        acc[j][1] = a1;
      }
      __syncthreads();
    }

    // ---- per-split partial (m, l, o[D]) ----
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = wave + j * kAttnWaves;
      if (h >= R) break;
      float* dst = a.part + ((static_cast<int64_t>(g) * S + split) * R + h) * (D + 2);
      if (lane == 0) {
        store_coherent(&dst[0], m_run[j]);
        store_coherent(&dst[1], l_run[j]);
      }
      if (lane < D) store_coherent(&dst[2 + lane], acc[j][0]);
      if (lane + kWave < D) store_coherent(&dst[2 + lane + kWave], acc[j][1]);
    }
  }

  // ---- last block of this KV head: log-sum-exp combine ----
  if (last_block_ticket(&a.counters[g], static_cast<unsigned int>(S))) {
    for (int h = wave; h < R; h += kAttnWaves) {
      const float* base = a.part + (static_cast<int64_t>(g) * S * R + h) * (D + 2);
      const int64_t stride = static_cast<int64_t>(R) * (D + 2);
      float M = -INFINITY;
      for (int s = 0; s < active; ++s) M = fmaxf(M, load_coherent(&base[s * stride]));
      float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
      for (int s = 0; s < active; ++s) {
        const float* part = base + s * stride;
        const float w = expf(load_coherent(&part[0]) - M);
        L = fmaf(load_coherent(&part[1]), w, L);
        if (lane < D) o0 = fmaf(load_coherent(&part[2 + lane]), w, o0);
        if (lane + kWave < D) o1 = fmaf(load_coherent(&part[2 + lane + kWave]), w, o1);
      }
      const float inv = active > 0 ? 1.0f / L : 0.0f;
      float* out = a.out + (g * R + h) * D;
      if (lane < D) out[lane] = o0 * inv;
      if (lane + kWave < D) out[lane + kWave] = o1 * inv;
    }
  }
}

// Standalone post-process (reference K2): one wave per head.
template <typename KV, int D>
__global__ __launch_bounds__(kWave) void qkv_postprocess_kernel(QkvPostArgs a) {
  __shared__ float x_s[D];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const bool is_q = b < a.hq;
  const int head = is_q ? b : b - a.hq;
  const float* src = a.qkv + (is_q ? head * D : a.hq * D + head * D);
  wave_rms_norm<D>(src, is_q ? a.q_norm : a.k_norm, a.eps, x_s, lane);
  __syncthreads();
  wave_rope<D>(x_s, a.rope_cos + static_cast<int64_t>(a.position) * (D / 2),
               a.rope_sin + static_cast<int64_t>(a.position) * (D / 2), lane);
  __syncthreads();
  if (is_q) {
    for (int i = lane; i < D; i += kWave) a.query_out[head * D + i] = x_s[i];
  } else {
    const float* vsrc = a.qkv + a.hq * D + a.hkv * D + head * D;
    KV* kdst = reinterpret_cast<KV*>(a.kcache) + (static_cast<int64_t>(head) * a.capacity + a.index) * D;
    KV* vdst = reinterpret_cast<KV*>(a.vcache) + (static_cast<int64_t>(head) * a.capacity + a.index) * D;
    for (int i = lane; i < D; i += kWave) {
      kdst[i] = from_float<KV>(x_s[i]);
      vdst[i] = from_float<KV>(vsrc[i]);
    }
  }
}

template <typename KV, int D>
hipError_t launch_attn_d(const AttnArgs& a, AttnMode mode, hipStream_t s) {
  const dim3 grid(a.splits, a.hkv), block(kAttnThreads);
  if (mode == kAttnFused) {
    attention_kernel<KV, D, kAttnFused><<<grid, block, 0, s>>>(a);
  } else {
    attention_kernel<KV, D, kAttnFromCache><<<grid, block, 0, s>>>(a);
  }
  return hipGetLastError();
}

template <typename KV>
hipError_t launch_attn_kv(const AttnArgs& a, AttnMode mode, hipStream_t s) {
  switch (a.d) {
    case 16: return launch_attn_d<KV, 16>(a, mode, s);
    case 32: return launch_attn_d<KV, 32>(a, mode, s);
    case 64: return launch_attn_d<KV, 64>(a, mode, s);
    case 96: return launch_attn_d<KV, 96>(a, mode, s);
    case 128: return launch_attn_d<KV, 128>(a, mode, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename KV>
hipError_t launch_post_kv(const QkvPostArgs& a, hipStream_t s) {
  const dim3 grid(a.hq + a.hkv), block(kWave);
  switch (a.d) {
    case 16: qkv_postprocess_kernel<KV, 16><<<grid, block, 0, s>>>(a); break;
    case 32: qkv_postprocess_kernel<KV, 32><<<grid, block, 0, s>>>(a); break;
    case 64: qkv_postprocess_kernel<KV, 64><<<grid, block, 0, s>>>(a); break;
    case 96: qkv_postprocess_kernel<KV, 96><<<grid, block, 0, s>>>(a); break;
    case 128: qkv_postprocess_kernel<KV, 128><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool attention_supported(int hq, int hkv, int d) {
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0 || hq / hkv > kAttnMaxGroup) return false;
  return d == 16 || d == 32 || d == 64 || d == 96 || d == 128;
}

int attention_tile_tokens(int d) { return d <= 96 ? 64 : 32; }

size_t attention_partial_floats(int hq, int hkv, int d, int splits) {
  return static_cast<size_t>(hkv) * splits * (hq / hkv) * (d + 2);
}

hipError_t launch_attention(const AttnArgs& a, AttnMode mode, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d) || a.splits <= 0) return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_attn_kv<__half>(a, mode, stream) : launch_attn_kv<float>(a, mode, stream);
}

hipError_t launch_qkv_postprocess(const QkvPostArgs& a, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d)) return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_post_kv<__half>(a, stream) : launch_post_kv<float>(a, stream);
}

}  // namespace mmr
