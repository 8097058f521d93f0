// tiny.hip -- a whole decode step in one workgroup, for models below the
// shapes of the GEMV and attention kernels (hidden not a multiple of 8,
// head_dim outside {16, 32, 64, 96, 128}).  The reference's built-in toy
// model (language_model.cpp:415-470: hidden 4, head_dim 2, vocab 8) is the
// case this serves: its CLI and tests fall back to it when no model directory
// is given (minimind_generate.cpp:84-86, bench_decode.cpp:124-126).
//
// One launch = one step, with the step bookkeeping of the large-model path:
// the token at seq[*pos] goes in, every layer runs in the reference's op
// order (decoder_layer.cpp:312-407), the final norm, lm_head and first-index
// argmax follow (language_model.cpp:310-333, :408-413), the prediction lands
// in seq[*pos + 1] (past the prompt) and *pos advances.  Phases are separated
// by workgroup barriers; activations live in LDS, weights (fp16) and the KV
// cache in global memory.  Speed is not the point at these sizes.
#include "device_common.h"
#include "kernels.h"

#include <climits>

namespace mmr {
namespace {

constexpr int kTinyThreads = 256;
constexpr int kTinyWaves = kTinyThreads / kWave;

// Sum over the workgroup; every thread returns the total.  `red` is
// kTinyWaves floats of LDS; the leading barrier protects its previous use.
__device__ float block_sum(float v, float* red) {
  v = group_sum<kWave>(v);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kTinyWaves; ++i) t += red[i];
  return t;
}

__device__ float dot_half_row(const __half* w, const float* x, int n) {
  float acc = 0.0f;
  for (int k = 0; k < n; ++k) acc += __half2float(w[k]) * x[k];
  return acc;
}

template <typename KV>
__global__ __launch_bounds__(kTinyThreads) void tiny_step_kernel(TinyStepArgs a) {
  __shared__ float h[kTinyMaxWidth];
  __shared__ float x[kTinyMaxWidth];
  __shared__ float qkv[kTinyMaxWidth];
  __shared__ float att[kTinyMaxWidth];
  __shared__ float act[kTinyMaxFfn];
  __shared__ float score[kTinyWaves][kTinyMaxContext];
  __shared__ float red[kTinyWaves];
  __shared__ float best_v[kTinyThreads];
  __shared__ int best_i[kTinyThreads];

  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int p = *a.pos;
  if (p < 0 || p >= a.capacity) {  // uniform over the block: nothing runs
    if (tid == 0) *a.err = 1;
    return;
  }
  const int H = a.hidden, D = a.d, Hq = a.hq, Hkv = a.hkv, F = a.f, V = a.vocab;
  const int qs = Hq * D, kvs = Hkv * D, R = qs + 2 * kvs, group = Hq / Hkv;
  int tok = a.seq[p];
  tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);  // the host validated every id it uploaded
  for (int i = tid; i < H; i += kTinyThreads) h[i] = __half2float(a.embed[static_cast<int64_t>(tok) * H + i]);
  __syncthreads();

  for (int l = 0; l < a.n_layers; ++l) {
    const TinyLayerPtrs L = a.layers[l];
    KV* kc = static_cast<KV*>(L.kcache);
    KV* vc = static_cast<KV*>(L.vcache);
    // input RMSNorm, x * (scale * w) (decoder_layer.cpp:32-42, :327)
    float ss = 0.0f;
    for (int i = tid; i < H; i += kTinyThreads) ss += h[i] * h[i];
    ss = block_sum(ss, red);
    float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + a.eps);
    for (int i = tid; i < H; i += kTinyThreads) x[i] = h[i] * (scale * L.input_norm[i]);
    __syncthreads();
    // fused q | k | v projection (:331-335)
    for (int r = tid; r < R; r += kTinyThreads) qkv[r] = dot_half_row(L.qkv + static_cast<int64_t>(r) * H, x, H);
    __syncthreads();
    // per-head RMSNorm of q and k, then rotate-half RoPE at position p (:342-352)
    for (int hh = tid; hh < Hq + Hkv; hh += kTinyThreads) {
      float* v = qkv + hh * D;
      const float* w = hh < Hq ? L.q_norm : L.k_norm;
      float s2 = 0.0f;
      for (int i = 0; i < D; ++i) s2 += v[i] * v[i];
      const float hs = 1.0f / sqrtf(s2 / static_cast<float>(D) + a.eps);
      for (int i = 0; i < D; ++i) v[i] = v[i] * (hs * w[i]);
      for (int i = 0; i < D / 2; ++i) {
        float sn, cs;
        sincosf(static_cast<float>(p) * a.inv_freq[i], &sn, &cs);
        const float x1 = v[i], x2 = v[i + D / 2];
        v[i] = x1 * cs - x2 * sn;
        v[i + D / 2] = x2 * cs + x1 * sn;
      }
    }
    __syncthreads();
    // append k, v at cache row p (:354-359); layout [kv_head][rows][d].  With
    // an fp16 cache the rounded values are what this and later steps read.
    for (int i = tid; i < kvs; i += kTinyThreads) {
      const int64_t idx = (static_cast<int64_t>(i / D) * a.rows + p) * D + i % D;
      kc[idx] = from_float<KV>(qkv[qs + i]);
      vc[idx] = from_float<KV>(qkv[qs + kvs + i]);
    }
    __syncthreads();
    // attention over p + 1 keys, one wave per query head (:184-234):
    // s_t = q.k_t / sqrt(d), softmax, sum of p_t v_t
    const int n = p + 1;
    const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(D));
    for (int hh = wave; hh < Hq; hh += kTinyWaves) {
      const int g = hh / group;
      const float* q = qkv + hh * D;
      float* s = score[wave];
      float m = -INFINITY;
      for (int t = lane; t < n; t += kWave) {
        const KV* kr = kc + (static_cast<int64_t>(g) * a.rows + t) * D;
        float dot = 0.0f;
        for (int i = 0; i < D; ++i) dot += q[i] * to_float<KV>(kr[i]);
        const float v = dot * inv_sqrt_d;
        s[t] = v;
        m = fmaxf(m, v);
      }
      m = group_max<kWave>(m);
      float den = 0.0f;
      for (int t = lane; t < n; t += kWave) {
        const float e = expf(s[t] - m);
        s[t] = e;
        den += e;
      }
      den = group_sum<kWave>(den);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float inv_den = 1.0f / den;
      for (int dd = lane; dd < D; dd += kWave) {
        float acc = 0.0f;
        for (int t = 0; t < n; ++t) acc += s[t] * to_float<KV>(vc[(static_cast<int64_t>(g) * a.rows + t) * D + dd]);
        att[hh * D + dd] = acc * inv_den;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();
    // o projection + residual (:362-367)
    for (int r = tid; r < H; r += kTinyThreads) h[r] = h[r] + dot_half_row(L.o + static_cast<int64_t>(r) * qs, att, qs);
    __syncthreads();
    // post-attention RMSNorm (:369)
    ss = 0.0f;
    for (int i = tid; i < H; i += kTinyThreads) ss += h[i] * h[i];
    ss = block_sum(ss, red);
    scale = 1.0f / sqrtf(ss / static_cast<float>(H) + a.eps);
    for (int i = tid; i < H; i += kTinyThreads) x[i] = h[i] * (scale * L.post_norm[i]);
    __syncthreads();
    // gate_up (rows interleaved gate_i, up_i) + SwiGLU (:392-394)
    for (int i = tid; i < F; i += kTinyThreads) {
      const float gv = dot_half_row(L.gate_up + static_cast<int64_t>(2 * i) * H, x, H);
      const float uv = dot_half_row(L.gate_up + static_cast<int64_t>(2 * i + 1) * H, x, H);
      act[i] = (gv / (1.0f + expf(-gv))) * uv;
    }
    __syncthreads();
    // down projection + residual (:400-405)
    for (int r = tid; r < H; r += kTinyThreads) h[r] = h[r] + dot_half_row(L.down + static_cast<int64_t>(r) * F, act, F);
    __syncthreads();
  }

  // final RMSNorm, (x * scale) * w (language_model.cpp:24-38)
  float ss = 0.0f;
  for (int i = tid; i < H; i += kTinyThreads) ss += h[i] * h[i];
  ss = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + a.eps);
  for (int i = tid; i < H; i += kTinyThreads) x[i] = (h[i] * scale) * a.final_norm[i];
  __syncthreads();
  // lm_head, logits, first index of the maximum (language_model.cpp:408-413)
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int v = tid; v < V; v += kTinyThreads) {
    const float lg = dot_half_row(a.lm_head + static_cast<int64_t>(v) * H, x, H);
    a.logits[v] = lg;
    if (argmax_better(lg, v, bv, bi)) {
      bv = lg;
      bi = v;
    }
  }
  best_v[tid] = bv;
  best_i[tid] = bi;
  __syncthreads();
  if (tid == 0) {
    float B = best_v[0];
    int I = best_i[0];
    for (int j = 1; j < kTinyThreads; ++j)
      if (argmax_better(best_v[j], best_i[j], B, I)) {
        B = best_v[j];
        I = best_i[j];
      }
    if (I >= V) I = 0;  // every logit NaN
    *a.token_out = I;
    const int np = p + 1;
    if (np < a.seq_len && np >= *a.prompt_len) a.seq[np] = I;
    *a.pos = np;
  }
}

}  // namespace

bool tiny_step_supported(int hidden, int hq, int hkv, int d, int f, int vocab, int capacity) {
  if (hidden <= 0 || hq <= 0 || hkv <= 0 || d <= 0 || f <= 0 || vocab <= 0 || capacity <= 0) return false;
  if (hq % hkv != 0 || d % 2 != 0 || d > kTinyMaxHeadDim) return false;
  if (hidden > kTinyMaxWidth || (hq + 2 * hkv) * d > kTinyMaxWidth || f > kTinyMaxFfn) return false;
  return capacity <= kTinyMaxContext;
}

hipError_t launch_tiny_step(const TinyStepArgs& a, KvDtype kv, hipStream_t stream) {
  if (kv == kKvF16) {
    tiny_step_kernel<__half><<<1, kTinyThreads, 0, stream>>>(a);
  } else {
    tiny_step_kernel<float><<<1, kTinyThreads, 0, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace mmr
