// batch.hip -- kernels specific to decoding a batch of independent sequences
// (the reference's DecoderState holds one sequence,
// language_model.h:22-25).  The projections of a batched step run on the
// prefill GEMM (M = batch) and the attention on the split kernel with a
// paged cache; these kernels cover the per-sequence token handling.
#include "attention_common.h"
#include "device_common.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace mmr {
namespace {

constexpr int kBatchThreads = 256;

// Embedding rows of each sequence's current token (language_model.cpp:67-77).
__global__ __launch_bounds__(kBatchThreads) void batch_embed_kernel(const __half* embed, const int32_t* seq,
                                                                    int seq_stride, const int32_t* pos, int vocab,
                                                                    int hidden, float* h) {
  const int b = blockIdx.y;
  int token = seq[static_cast<int64_t>(b) * seq_stride + pos[b]];
  token = token < 0 ? 0 : (token >= vocab ? vocab - 1 : token);
  const __half* row = embed + static_cast<int64_t>(token) * hidden;
  for (int i = blockIdx.x * kBatchThreads + threadIdx.x; i < hidden; i += gridDim.x * kBatchThreads)
    h[static_cast<int64_t>(b) * hidden + i] = __half2float(row[i]);
}

// First-index argmax of one sequence's logits (std::max_element,
// language_model.cpp:408-413) and the step bookkeeping.
__global__ __launch_bounds__(kBatchThreads) void batch_argmax_kernel(const float* logits, int vocab,
                                                                     int32_t* token_out, int32_t* seq, int seq_stride,
                                                                     int32_t* pos, const int32_t* prompt_len,
                                                                     int seq_len) {
  __shared__ float s_val[kBatchThreads / kWave];
  __shared__ int s_idx[kBatchThreads / kWave];
  const int b = blockIdx.x;
  const float* row = logits + static_cast<int64_t>(b) * vocab;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int i = threadIdx.x; i < vocab; i += kBatchThreads) {
    const float v = row[i];
    if (argmax_better(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  // Wave reduction with the same ordering (larger value, then lower index).
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_i, off);
    if (argmax_better(ov, oi, best, best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  if (threadIdx.x % kWave == 0) {
    s_val[threadIdx.x / kWave] = best;
    s_idx[threadIdx.x / kWave] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBatchThreads / kWave; ++w)
      if (argmax_better(s_val[w], s_idx[w], best, best_i)) {
        best = s_val[w];
        best_i = s_idx[w];
      }
    const int next = best_i < vocab ? best_i : 0;
    if (token_out) token_out[b] = next;
    if (pos) {
      const int p = pos[b];
      if (p + 1 < seq_len && p + 1 >= prompt_len[b]) seq[static_cast<int64_t>(b) * seq_stride + p + 1] = next;
      pos[b] = p + 1;
    }
  }
}

// Head of the batched step: logits[b] = sum_s part[s][b] (split order, at
// most kHeadParts partials, all loads issued first), then the first-index
// argmax and the same bookkeeping as batch_argmax_kernel.  One block of
// kHeadThreads per sequence, kHeadPer logits per thread per pass.
constexpr int kHeadThreads = 1024;
constexpr int kHeadPer = 8;
constexpr int kHeadParts = 4;

__global__ __launch_bounds__(kHeadThreads) void batch_head_kernel(const float* part, int splits, int batch, int vocab,
                                                                  float* logits, int32_t* token_out, int32_t* seq,
                                                                  int seq_stride, int32_t* pos,
                                                                  const int32_t* prompt_len, int seq_len) {
  __shared__ float s_val[kHeadThreads / kWave];
  __shared__ int s_idx[kHeadThreads / kWave];
  const int b = blockIdx.x;
  const int64_t sstride = static_cast<int64_t>(batch) * vocab;
  const float* src = part + static_cast<int64_t>(b) * vocab;
  float* row = logits + static_cast<int64_t>(b) * vocab;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int base = 0; base < vocab; base += kHeadThreads * kHeadPer) {  // block-uniform
    float pv[kHeadPer][kHeadParts];
#pragma unroll
    for (int e = 0; e < kHeadPer; ++e) {
      const int i = min(base + static_cast<int>(threadIdx.x) + e * kHeadThreads, vocab - 1);
#pragma unroll
      for (int sp = 0; sp < kHeadParts; ++sp) pv[e][sp] = src[min(sp, splits - 1) * sstride + i];
    }
#pragma unroll
    for (int e = 0; e < kHeadPer; ++e) {
      const int i = base + static_cast<int>(threadIdx.x) + e * kHeadThreads;
      float v = 0.0f;
#pragma unroll
      for (int sp = 0; sp < kHeadParts; ++sp)
        if (sp < splits) v += pv[e][sp];
      if (i < vocab) {
        row[i] = v;
        if (argmax_better(v, i, best, best_i)) {
          best = v;
          best_i = i;
        }
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_i, off);
    if (argmax_better(ov, oi, best, best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  if (threadIdx.x % kWave == 0) {
    s_val[threadIdx.x / kWave] = best;
    s_idx[threadIdx.x / kWave] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kHeadThreads / kWave; ++w)
      if (argmax_better(s_val[w], s_idx[w], best, best_i)) {
        best = s_val[w];
        best_i = s_idx[w];
      }
    const int next = best_i < vocab ? best_i : 0;
    if (token_out) token_out[b] = next;
    if (pos) {
      const int p = pos[b];
      if (p + 1 < seq_len && p + 1 >= prompt_len[b]) seq[static_cast<int64_t>(b) * seq_stride + p + 1] = next;
      pos[b] = p + 1;
    }
  }
}

// Split-K skinny GEMM (m <= 32 rows of A) on the fp16 matrix cores.
// Block = 4 waves x 16 rows of W (64 rows) x one K chunk [k0, k0 + 32 NB)
// (chunks tile K exactly).  The chunk of A is staged once in LDS as two fp16
// planes: with a power-of-two scale s per row (the row's chunk maximum maps
// into [2^14, 2^15)), hi = fp16(s a) and lo = fp16(s a - hi), so
// hi + lo carries ~22 significant bits of s a (fp32 has 24), and W (fp16) is
// exact.  Per 32-k block, lane l supplies W row n0 + 16 wave + l % 16 and A
// row 16 bt + l % 16 at the same 8 k positions 8 (l / 16) .. + 7, so one
// 16x16x32 MFMA per plane covers the block; the products are exact and
// accumulate in fp32, and the result is multiplied by 1 / s (exact).
// Output: part[split][m][n], every element written exactly once.
constexpr int kSplitRows = kSplitKRows;
constexpr int kSplitMaxKc = 256;
constexpr int kSplitMaxM = 32;

using f32x4 = float __attribute__((ext_vector_type(4)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f16x4 = _Float16 __attribute__((ext_vector_type(4)));

// A staging modes: plain rows; SwiGLU of the gate_up partials (at most
// kSwiGluParts, read with clamped indices and summed in split order, as
// batch_swiglu_kernel does); the attention output merged from at most 4 or 8
// split partials (log-sum-exp in split order).
constexpr int kAPlain = 0, kASwiGlu = 1, kACombine4 = 2, kACombine8 = 3;
constexpr int kSwiGluParts = 4;

template <int BT, int NB, int kAMode>
__global__ __launch_bounds__(256) void gemm_splitk_kernel(SplitKArgs g) {
  constexpr bool kSwiGlu = kAMode == kASwiGlu;
  constexpr int kCombine = kAMode == kACombine4 ? 4 : kAMode == kACombine8 ? 8 : 0;
  constexpr int KC = 32 * NB;
  constexpr int kLd = KC + 8;           // halves per LDS row (16-byte aligned rows)
  constexpr int kRowsPerWave = BT * 4;  // A rows staged by each wave: w, w + 4, ...
  constexpr int QR = KC / 4;            // float4 quads per A row
  // Rows per pass: short rows share a wave (QR consecutive lanes per row).
  constexpr int kRpp0 = kWave % QR == 0 ? kWave / QR : 1;
  constexpr int RPP = kRpp0 < kRowsPerWave ? kRpp0 : kRowsPerWave;
  constexpr int kPasses = kRowsPerWave / RPP;
  constexpr int GW = RPP > 1 ? QR : kWave;  // lanes reducing one row's maximum
  __shared__ __align__(16) _Float16 a_hi[BT * 16][kLd];
  __shared__ __align__(16) _Float16 a_lo[BT * 16][kLd];
  __shared__ float row_inv[BT * 16];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  // Block -> (W row block bx, K chunk by), the blocks of one K chunk on one
  // XCD where the chunk count allows (splitk_block_tile).
  const SplitKTile tile = splitk_block_tile(static_cast<int>(blockIdx.x + gridDim.x * blockIdx.y),
                                            static_cast<int>(gridDim.x), static_cast<int>(gridDim.y));
  const int bx = tile.row_block, by = tile.chunk;
  const int n0 = bx * kSplitRows + wave * 16;
  const int k0 = by * KC;
  // W: NB x 8 halves per lane (rows past n clamp to the last row).  Issued
  // right after the A operand's loads: vector loads complete in issue order,
  // so the A staging below waits for its own (small) loads, not for the W
  // stream behind them.
  const int wrow = min(n0 + lane % 16, g.n - 1);
  const __half* wsrc = g.w + static_cast<int64_t>(wrow) * g.k + k0 + 8 * (lane / 16);
  uint4 wv[NB];
  auto load_w = [&] {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < NB; ++i) wv[i] = *reinterpret_cast<const uint4*>(wsrc + 32 * i);
    asm volatile("" ::: "memory");
  };
  // A: pass p, lane -> row wave + 4 (p RPP + lane / QR), columns 4 (lane % QR) ..
  const int sub = lane / QR, q = lane % QR;
  const bool lane_on = lane < RPP * QR;
  float4 av[kPasses];
  if constexpr (kSwiGlu) {
    // All partial loads first: two float4 (four gate/up pairs) per part.
    float4 pv[kPasses][kSwiGluParts][2];
    const int64_t part_stride = static_cast<int64_t>(g.m) * 2 * g.k;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = wave + 4 * (p * RPP + sub);
      const bool on = lane_on && r < g.m;
      const float* row = g.gu + static_cast<int64_t>(on ? r : 0) * 2 * g.k + 2 * (k0 + 4 * (on ? q : 0));
#pragma unroll
      for (int s = 0; s < kSwiGluParts; ++s) {
        const float* src = row + min(s, g.gu_splits - 1) * part_stride;
        pv[p][s][0] = *reinterpret_cast<const float4*>(src);
        pv[p][s][1] = *reinterpret_cast<const float4*>(src + 4);
      }
    }
    load_w();
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      float gs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, us[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < kSwiGluParts; ++s) {
        if (s < g.gu_splits) {
          gs[0] += pv[p][s][0].x;
          us[0] += pv[p][s][0].y;
          gs[1] += pv[p][s][0].z;
          us[1] += pv[p][s][0].w;
          gs[2] += pv[p][s][1].x;
          us[2] += pv[p][s][1].y;
          gs[3] += pv[p][s][1].z;
          us[3] += pv[p][s][1].w;
        }
      }
      const int r = wave + 4 * (p * RPP + sub);
      float x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = silu_fast(gs[j]) * us[j];  // decoder_layer.cpp:175-182
      av[p] = (lane_on && r < g.m) ? make_float4(x[0], x[1], x[2], x[3]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  } else if constexpr (kCombine > 0) {
    // This lane's quad lies in one head (d is a multiple of 4): head kk / d,
    // dims kk % d .. + 3.  All split loads first, then the merge.
    const int R = g.hq / g.hkv;
    const int kk = k0 + 4 * q;
    const int head = kk / g.d, dd = kk % g.d;
    const int gq = head / R, hr = head % R;
    const int S = g.attn_splits;
    float2 ml[kPasses][kCombine];
    float4 ov[kPasses][kCombine];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = wave + 4 * (p * RPP + sub);
      const bool on = lane_on && r < g.m;
      const float* base = g.attn_part + static_cast<int64_t>(on ? r : 0) * g.attn_part_stride;
#pragma unroll
      for (int sp = 0; sp < kCombine; ++sp) {
        const int sc = min(sp, S - 1);
        ml[p][sp] = *reinterpret_cast<const float2*>(base + attn_ml_offset(gq, sc, hr, S, R, g.d, g.hkv));
        ov[p][sp] = *reinterpret_cast<const float4*>(base + attn_o_offset(gq, sc, hr, S, R, g.d) + dd);
      }
    }
    load_w();
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      float M = -INFINITY;
#pragma unroll
      for (int sp = 0; sp < kCombine; ++sp)
        if (sp < S) M = fmaxf(M, ml[p][sp].x);
      float L = 0.0f;
      float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int sp = 0; sp < kCombine; ++sp) {
        if (sp < S) {
          const float e = __builtin_amdgcn_exp2f((ml[p][sp].x - M) * 1.4426950408889634f);  // e^x = 2^(x log2 e)
          L = fmaf(ml[p][sp].y, e, L);
          o.x = fmaf(ov[p][sp].x, e, o.x);
          o.y = fmaf(ov[p][sp].y, e, o.y);
          o.z = fmaf(ov[p][sp].z, e, o.z);
          o.w = fmaf(ov[p][sp].w, e, o.w);
        }
      }
      const float inv = 1.0f / L;
      const int r = wave + 4 * (p * RPP + sub);
      av[p] = (lane_on && r < g.m) ? make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv)
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  } else {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = wave + 4 * (p * RPP + sub);
      av[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (lane_on && r < g.m)
        av[p] = *reinterpret_cast<const float4*>(g.a + static_cast<int64_t>(r) * g.lda + k0 + 4 * q);
    }
    load_w();
  }
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = wave + 4 * (p * RPP + sub);
    const float4 v = av[p];
    const float mx = group_max<GW>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    int e = 0;
    frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1); e = 0 for mx = 0
    e = max(e, -100);
    const float sc = ldexpf(1.0f, 15 - e);
    if (lane_on) {
      const float x[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
      f16x4 hi, lo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[j] = static_cast<_Float16>(x[j]);
        lo[j] = static_cast<_Float16>(x[j] - static_cast<float>(hi[j]));
      }
      *reinterpret_cast<f16x4*>(&a_hi[r][4 * q]) = hi;
      *reinterpret_cast<f16x4*>(&a_lo[r][4 * q]) = lo;
      if (q == 0) row_inv[r] = ldexpf(1.0f, e - 15);
    }
  }
  __syncthreads();
  f32x4 acc_hi[BT], acc_lo[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    acc_hi[bt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc_lo[bt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const f16x8 wh = __builtin_bit_cast(f16x8, wv[i]);
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      const int ar = bt * 16 + lane % 16, ac = 32 * i + 8 * (lane / 16);
      const f16x8 ah = *reinterpret_cast<const f16x8*>(&a_hi[ar][ac]);
      const f16x8 al = *reinterpret_cast<const f16x8*>(&a_lo[ar][ac]);
      acc_hi[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, ah, acc_hi[bt], 0, 0, 0);
      acc_lo[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, al, acc_lo[bt], 0, 0, 0);
    }
  }
  // lane holds D[n0 + 4 (lane / 16) + r][16 bt + lane % 16], r = 0..3
  const int nb = n0 + 4 * (lane / 16);
  const bool vec = (g.n % 4 == 0) && nb + 3 < g.n;
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int m = bt * 16 + lane % 16;
    if (m >= g.m) continue;
    const float inv = row_inv[m];
    float* dst = g.part + (static_cast<int64_t>(by) * g.m + m) * g.n + nb;
    const float o[4] = {(acc_hi[bt][0] + acc_lo[bt][0]) * inv, (acc_hi[bt][1] + acc_lo[bt][1]) * inv,
                        (acc_hi[bt][2] + acc_lo[bt][2]) * inv, (acc_hi[bt][3] + acc_lo[bt][3]) * inv};
    if (vec) {
      *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < g.n) dst[r] = o[r];
    }
  }
}

// Split-K partial sums, read with up to kPartLoads loads in flight per
// thread before any add: sum over s = s0, s0 + step, ... < splits of
// part4[s * sstride], in that order.
constexpr int kPartLoads = 8;

__device__ inline float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ inline float add4(float a, float b) { return a + b; }

template <typename T>
__device__ inline T sum_parts4(const T* part4, int64_t sstride, int s0, int step, int splits) {
  T acc{};
  for (int base = s0; base < splits; base += step * kPartLoads) {
    T v[kPartLoads];
#pragma unroll
    for (int u = 0; u < kPartLoads; ++u) v[u] = part4[min(base + step * u, splits - 1) * sstride];
    // Indices past the last split (clamped above) add zero: a select, not a
    // branch, which the compiler would turn into a reload of v[u] and a wait
    // inside the branch.
#pragma unroll
    for (int u = 0; u < kPartLoads; ++u) acc = add4(acc, base + step * u < splits ? v[u] : T{});
  }
  return acc;
}

// h[b] += sum_s part[s][b], then x[b] = RMSNorm(h[b]) with the layer
// association x * (scale * w) (decoder_layer.cpp:32-42) or the final one
// (x * scale) * w (language_model.cpp:24-38).  One block of kResThreads per
// row: kResThreads / 256 groups of 256 threads each sum every group-count-th
// split of a column chunk (float4 columns), then the groups' sums are added
// to h in group order.  splits == 0 normalizes h as it is.
// kResThreads: 1024 for a few rows (batched decode: more loads in flight per
// row), 256 for many (prefill: one group adds the splits in order).
constexpr int kResChunkQuads = 256;
constexpr int kResManyRows = 64;

// The pre-split planes of one row's 4 normalised columns at quad q (thread
// = 4 consecutive columns; the threads of a 128-column chunk reduce its
// maximum together, so every thread of the block must call this).
__device__ inline void write_split_quad(const float (&v)[4], bool live, int q, int64_t b, int cols, SplitPlanes sp) {
  const int nchunks = (cols + kSplitChunk - 1) / kSplitChunk;
  const float mx = group_max<kSplitChunk / 4>(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  if (!live) return;
  int e2 = 0;
  frexpf(mx, &e2);  // e2 = 0 for a zero chunk
  e2 = max(e2, -100);
  const float sc = ldexpf(1.0f, 15 - e2);
  uint16_t hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float xs = v[e] * sc;
    const _Float16 hh = static_cast<_Float16>(xs);
    const _Float16 ll = static_cast<_Float16>(xs - static_cast<float>(hh));
    __builtin_memcpy(&hi[e], &hh, 2);
    __builtin_memcpy(&lo[e], &ll, 2);
  }
  const int64_t off = b * cols + 4 * q;
  *reinterpret_cast<uint2*>(sp.hi + off) = make_uint2(hi[0] | (uint32_t{hi[1]} << 16), hi[2] | (uint32_t{hi[3]} << 16));
  *reinterpret_cast<uint2*>(sp.lo + off) = make_uint2(lo[0] | (uint32_t{lo[1]} << 16), lo[2] | (uint32_t{lo[3]} << 16));
  if (q % (kSplitChunk / 4) == 0) sp.inv[b * nchunks + q / (kSplitChunk / 4)] = ldexpf(1.0f, e2 - 15);
}

// batch_residual_norm_kernel for a row of at most kResChunkQuads quads: every
// load of the block goes out before any arithmetic (the split partials, the
// row of h and the norm gains, indices clamped: a guarded load is waited for
// where its branch joins), and group 0 keeps the updated row in registers
// for both writers, so the row costs one memory round trip instead of three.
// Same operations in the same order as the general path below.
template <bool kFinal, bool kSplit, int kResThreads>
__device__ inline void residual_norm_row(float4* h4, const float4* p4, int64_t sstride, int splits, int nq, int cols,
                                         int b, const float* w, float eps, float* x, SplitPlanes sp,
                                         float4 (&red)[kResThreads / 256][kResChunkQuads],
                                         float (&s_ss)[kResThreads / kWave]) {
  constexpr int kResGroups = kResThreads / 256;
  const int grp = threadIdx.x / 256, t = threadIdx.x % 256;
  const int qq = min(t, nq - 1);
  const bool live = grp == 0 && t < nq;
  const float4 hv = h4[qq];
  const float4 wv = reinterpret_cast<const float4*>(w)[qq];
  float4 ps = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (splits > 0) ps = sum_parts4(p4 + qq, sstride, grp, kResGroups, splits);
  float4 v = hv;
  if constexpr (kResGroups == 1) {  // the thread holds its column's whole sum: no LDS exchange
    if (splits > 0) {
      v = add4(v, ps);
      if (live) h4[t] = v;
    }
  } else {
    if (splits > 0) red[grp][t] = ps;
    __syncthreads();
    if (splits > 0) {
#pragma unroll
      for (int g2 = 0; g2 < kResGroups; ++g2) v = add4(v, red[g2][t]);
      if (live) h4[t] = v;
    }
  }
  float ss = live ? v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w : 0.0f;
  ss = group_sum<kWave>(ss);
  if (threadIdx.x % kWave == 0) s_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kResThreads / kWave; ++i) total += s_ss[i];
  const float scale = __builtin_amdgcn_rsqf(total / static_cast<float>(cols) + eps);  // v_rsq_f32, about 1 ulp
  const float hvv[4] = {v.x, v.y, v.z, v.w}, wvv[4] = {wv.x, wv.y, wv.z, wv.w};
  float xv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) xv[e] = kFinal ? (hvv[e] * scale) * wvv[e] : hvv[e] * (scale * wvv[e]);
  if (x && live) *reinterpret_cast<float4*>(x + static_cast<int64_t>(b) * cols + 4 * t) = make_float4(xv[0], xv[1], xv[2], xv[3]);
  if constexpr (kSplit) {
    float sv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) sv[e] = live ? xv[e] : 0.0f;
    write_split_quad(sv, live, t, b, cols, sp);
  }
}

template <bool kFinal, bool kSplit, int kResThreads>
__global__ __launch_bounds__(kResThreads) void batch_residual_norm_kernel(float* h, const float* part, int splits,
                                                                          int batch, int cols, const float* w,
                                                                          float eps, float* x, SplitPlanes sp,
                                                                          L2WarmSet warm) {
  constexpr int kResGroups = kResThreads / 256;
  __shared__ float4 red[kResGroups][kResChunkQuads];
  __shared__ float s_ss[kResThreads / kWave];
  // Blocks past the rows: padding up to a multiple of kXcds, then the
  // L2-warming blocks (their loads land in red, 1 KB per wave).
  static_assert(sizeof(red) >= kResThreads / kWave * kWave * 16, "a 1 KB landing zone per wave");
  if (static_cast<int>(blockIdx.x) >= batch) {
    const int first = (batch + kXcds - 1) / kXcds * kXcds;
    if (static_cast<int>(blockIdx.x) >= first)
      l2_warm<kResThreads>(warm, static_cast<int>(blockIdx.x) - first, &red[0][0]);
    return;
  }
  const int b = blockIdx.x;
  const int nq = cols / 4;
  const int grp = threadIdx.x / 256, t = threadIdx.x % 256;
  float4* h4 = reinterpret_cast<float4*>(h + static_cast<int64_t>(b) * cols);
  const float4* p4 = reinterpret_cast<const float4*>(part) + static_cast<int64_t>(b) * nq;
  const int64_t sstride = static_cast<int64_t>(batch) * nq;
  if (nq <= kResChunkQuads) {  // block-uniform
    residual_norm_row<kFinal, kSplit, kResThreads>(h4, p4, sstride, splits, nq, cols, b, w, eps, x, sp, red, s_ss);
    return;
  }
  float ss = 0.0f;
  for (int c0 = 0; c0 < nq; c0 += kResChunkQuads) {  // block-uniform
    const int q = c0 + t;
    if (splits > 0 && q < nq) red[grp][t] = sum_parts4(p4 + q, sstride, grp, kResGroups, splits);
    __syncthreads();
    if (grp == 0 && q < nq) {
      float4 v = h4[q];
      if (splits > 0) {
#pragma unroll
        for (int g2 = 0; g2 < kResGroups; ++g2) v = add4(v, red[g2][t]);
        h4[q] = v;
      }
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    __syncthreads();
  }
  ss = group_sum<kWave>(ss);
  if (threadIdx.x % kWave == 0) s_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kResThreads / kWave; ++i) total += s_ss[i];
  const float scale = __builtin_amdgcn_rsqf(total / static_cast<float>(cols) + eps);  // v_rsq_f32, about 1 ulp
  float* hr = h + static_cast<int64_t>(b) * cols;
  if (x) {
    float* xr = x + static_cast<int64_t>(b) * cols;
    for (int i = threadIdx.x; i < cols; i += kResThreads)
      xr[i] = kFinal ? (hr[i] * scale) * w[i] : hr[i] * (scale * w[i]);
  }
  if constexpr (kSplit) {
    // Thread = 4 consecutive columns; the threads of a chunk reduce its max
    // together (whole chunks per pass), then write the planes.
    const int nchunks = (cols + kSplitChunk - 1) / kSplitChunk;
    for (int q0 = 0; q0 < nchunks * (kSplitChunk / 4); q0 += kResThreads) {  // block-uniform
      const int q = q0 + static_cast<int>(threadIdx.x);
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (4 * q < cols) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * q + e;
          v[e] = kFinal ? (hr[i] * scale) * w[i] : hr[i] * (scale * w[i]);
        }
      }
      const float mx =
          group_max<kSplitChunk / 4>(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
      if (4 * q < cols) {
        int e2 = 0;
        frexpf(mx, &e2);  // e2 = 0 for a zero chunk
        e2 = max(e2, -100);
        const float sc = ldexpf(1.0f, 15 - e2);
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float xs = v[e] * sc;
          const _Float16 hh = static_cast<_Float16>(xs);
          const _Float16 ll = static_cast<_Float16>(xs - static_cast<float>(hh));
          __builtin_memcpy(&hi[e], &hh, 2);
          __builtin_memcpy(&lo[e], &ll, 2);
        }
        const int64_t off = static_cast<int64_t>(b) * cols + 4 * q;
        *reinterpret_cast<uint2*>(sp.hi + off) = make_uint2(hi[0] | (uint32_t{hi[1]} << 16), hi[2] | (uint32_t{hi[3]} << 16));
        *reinterpret_cast<uint2*>(sp.lo + off) = make_uint2(lo[0] | (uint32_t{lo[1]} << 16), lo[2] | (uint32_t{lo[3]} << 16));
        if (q % (kSplitChunk / 4) == 0) sp.inv[static_cast<int64_t>(b) * nchunks + q / (kSplitChunk / 4)] = ldexpf(1.0f, e2 - 15);
      }
    }
  }
}

// act[b][i] = silu(sum_s gu[s][b][2i]) * sum_s gu[s][b][2i + 1]
// (decoder_layer.cpp:175-182 on the interleaved gate/up rows); one float4
// (two gate/up pairs) per thread.
__global__ void batch_swiglu_kernel(const float* part, int splits, int batch, int f, float* act) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index: act[2i], act[2i + 1]
  if (2 * i >= f) return;
  const int64_t sstride = static_cast<int64_t>(batch) * f / 2;
  const float4 p = sum_parts4(reinterpret_cast<const float4*>(part) + static_cast<int64_t>(b) * f / 2 + i, sstride, 0, 1,
                              splits);
  float2 out;
  out.x = silu_fast(p.x) * p.y;
  out.y = silu_fast(p.z) * p.w;
  reinterpret_cast<float2*>(act + static_cast<int64_t>(b) * f)[i] = out;
}

// logits[b][v] = sum_s part[s][b][v] (the batch argmax then reads logits);
// T = float4 when n is a multiple of 4, else float.
template <typename T>
__global__ void batch_sum_parts_kernel(const float* part, int splits, int batch, int n, float* out) {
  constexpr int kW = sizeof(T) / sizeof(float);
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (kW * i >= n) return;
  const int64_t row = static_cast<int64_t>(n / kW);
  reinterpret_cast<T*>(out)[b * row + i] =
      sum_parts4(reinterpret_cast<const T*>(part) + b * row + i, static_cast<int64_t>(batch) * row, 0, 1, splits);
}

}  // namespace

hipError_t launch_batch_embed(const __half* embed, const int32_t* seq, int seq_stride, const int32_t* pos, int batch,
                              int vocab, int hidden, float* h, hipStream_t stream) {
  if (batch <= 0 || hidden <= 0) return hipErrorInvalidValue;
  const dim3 grid((hidden + kBatchThreads - 1) / kBatchThreads, batch);
  batch_embed_kernel<<<grid, kBatchThreads, 0, stream>>>(embed, seq, seq_stride, pos, vocab, hidden, h);
  return hipGetLastError();
}

hipError_t launch_batch_head(const float* part, int splits, int vocab, int batch, float* logits, int32_t* token_out,
                             int32_t* seq, int seq_stride, int32_t* pos, const int32_t* prompt_len, int seq_len,
                             hipStream_t stream) {
  if (batch <= 0 || vocab <= 0 || splits < 1) return hipErrorInvalidValue;
  if (splits > kHeadParts) {
    const hipError_t e = launch_batch_sum_parts(part, splits, batch, vocab, logits, stream);
    if (e != hipSuccess) return e;
    return launch_batch_argmax(logits, vocab, batch, token_out, seq, seq_stride, pos, prompt_len, seq_len, stream);
  }
  batch_head_kernel<<<batch, kHeadThreads, 0, stream>>>(part, splits, batch, vocab, logits, token_out, seq, seq_stride,
                                                       pos, prompt_len, seq_len);
  return hipGetLastError();
}

hipError_t launch_batch_argmax(const float* logits, int vocab, int batch, int32_t* token_out, int32_t* seq,
                               int seq_stride, int32_t* pos, const int32_t* prompt_len, int seq_len,
                               hipStream_t stream) {
  if (batch <= 0 || vocab <= 0) return hipErrorInvalidValue;
  batch_argmax_kernel<<<batch, kBatchThreads, 0, stream>>>(logits, vocab, token_out, seq, seq_stride, pos, prompt_len,
                                                           seq_len);
  return hipGetLastError();
}

int splitk_chunk(int n, int k) {
  // The largest chunk (fewest partial sums for the consumer) that tiles K
  // exactly and still gives at least kSplitMinBlocks blocks; else the chunk
  // with the most blocks.  (B = 32 to 4096 positions, per step: 128 blocks
  // 870.7 us, 192 blocks 866.0 us, 256 870.9 us, 64 922.4 us.)
  constexpr int kSplitMinBlocks = 192;
  if (k <= 0 || k % 32 != 0) return 0;
  const int nblocks = (n + kSplitRows - 1) / kSplitRows;
  int kc = 0;
  for (int nb = kSplitMaxKc / 32; nb >= 1; --nb) {
    if (k % (32 * nb) != 0) continue;
    kc = 32 * nb;  // block count grows as the chunk shrinks
    if (nblocks * (k / kc) >= kSplitMinBlocks) break;
  }
  return kc;
}

namespace {
// Staging passes of gemm_splitk_kernel (rows per wave / rows per pass).
constexpr int splitk_passes(int bt, int nb) {
  const int qr = 8 * nb, rows = 4 * bt;
  const int rpp0 = kWave % qr == 0 ? kWave / qr : 1;
  return rows / (rpp0 < rows ? rpp0 : rows);
}
// The SwiGLU staging holds passes x kSwiGluParts x 2 float4 per lane, the
// combine staging passes x (4 or 8) x (float4 + float2).
constexpr int kSwiGluMaxPasses = 4;
constexpr int kCombineMaxSlots = 16;  // passes x splits held
constexpr bool splitk_mode_fits(int bt, int nb, int mode) {
  return mode == kAPlain ? true
         : mode == kASwiGlu ? splitk_passes(bt, nb) <= kSwiGluMaxPasses
                            : splitk_passes(bt, nb) * (mode == kACombine4 ? 4 : 8) <= kCombineMaxSlots;
}
}  // namespace

bool splitk_swiglu_supported(int m, int kc, int gu_splits) {
  if (gu_splits < 1 || gu_splits > kSwiGluParts || m < 1 || m > kSplitMaxM || kc < 32 || kc % 32 != 0 ||
      kc > kSplitMaxKc)
    return false;
  return splitk_passes(m <= 16 ? 1 : 2, kc / 32) <= kSwiGluMaxPasses;
}

bool splitk_combine_supported(int m, int kc, int attn_splits, int d) {
  if (attn_splits < 1 || attn_splits > 8 || m < 1 || m > kSplitMaxM || kc < 32 || kc % 32 != 0 ||
      kc > kSplitMaxKc || d <= 0 || d % 4 != 0)
    return false;
  return splitk_passes(m <= 16 ? 1 : 2, kc / 32) * (attn_splits <= 4 ? 4 : 8) <= kCombineMaxSlots;
}

namespace {
template <int BT, int NB, int kAMode>
hipError_t launch_splitk_nb(const SplitKArgs& g, dim3 grid, hipStream_t stream) {
  if constexpr (!splitk_mode_fits(BT, NB, kAMode)) {
    return hipErrorInvalidValue;  // rejected by the *_supported checks; not instantiated
  } else {
    gemm_splitk_kernel<BT, NB, kAMode><<<grid, 256, 0, stream>>>(g);
    return hipGetLastError();
  }
}

template <int BT, int kAMode>
hipError_t launch_splitk_bt(const SplitKArgs& g, dim3 grid, hipStream_t stream) {
  switch (g.kc / 32) {
    case 1: return launch_splitk_nb<BT, 1, kAMode>(g, grid, stream);
    case 2: return launch_splitk_nb<BT, 2, kAMode>(g, grid, stream);
    case 3: return launch_splitk_nb<BT, 3, kAMode>(g, grid, stream);
    case 4: return launch_splitk_nb<BT, 4, kAMode>(g, grid, stream);
    case 5: return launch_splitk_nb<BT, 5, kAMode>(g, grid, stream);
    case 6: return launch_splitk_nb<BT, 6, kAMode>(g, grid, stream);
    case 7: return launch_splitk_nb<BT, 7, kAMode>(g, grid, stream);
    case 8: return launch_splitk_nb<BT, 8, kAMode>(g, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int kAMode>
hipError_t launch_splitk_mode(const SplitKArgs& g, dim3 grid, hipStream_t stream) {
  return g.m <= 16 ? launch_splitk_bt<1, kAMode>(g, grid, stream) : launch_splitk_bt<2, kAMode>(g, grid, stream);
}
}  // namespace

hipError_t launch_gemm_splitk(const SplitKArgs& g, hipStream_t stream) {
  if (g.m <= 0 || g.m > kSplitMaxM || g.n <= 0 || g.k <= 0 || g.kc <= 0 || g.kc % 32 != 0 || g.kc > kSplitMaxKc ||
      g.k % g.kc != 0)
    return hipErrorInvalidValue;
  const dim3 grid((g.n + kSplitRows - 1) / kSplitRows, g.k / g.kc);
  if (g.attn_part) {
    if (!splitk_combine_supported(g.m, g.kc, g.attn_splits, g.d) || g.hkv <= 0 || g.hq % g.hkv != 0 ||
        g.k != g.hq * g.d)
      return hipErrorInvalidValue;
    return g.attn_splits <= 4 ? launch_splitk_mode<kACombine4>(g, grid, stream)
                              : launch_splitk_mode<kACombine8>(g, grid, stream);
  }
  if (g.gu) {
    if (!splitk_swiglu_supported(g.m, g.kc, g.gu_splits)) return hipErrorInvalidValue;
    return launch_splitk_mode<kASwiGlu>(g, grid, stream);
  }
  if (g.lda < g.k || g.lda % 4 != 0) return hipErrorInvalidValue;
  return launch_splitk_mode<kAPlain>(g, grid, stream);
}

hipError_t launch_batch_residual_norm(float* h, const float* part, int splits, int batch, int cols, const float* w,
                                      float eps, float* x, bool final_norm, hipStream_t stream,
                                      const SplitPlanes* split, const L2WarmSet* warm) {
  if (batch <= 0 || cols <= 0 || cols % 4 != 0 || splits < 0) return hipErrorInvalidValue;
  if (split && (!split->hi || !split->lo || !split->inv)) return hipErrorInvalidValue;
  if (!x && !split) return hipErrorInvalidValue;
  if (warm && (warm->blocks < 0 || warm->blocks % kXcds != 0)) return hipErrorInvalidValue;
  // h, the gains and x are read and written as float4 rows.
  auto aligned16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  if (!aligned16(h) || !aligned16(w) || (x && !aligned16(x)) || (part && !aligned16(part))) return hipErrorInvalidValue;
  const SplitPlanes sp = split ? *split : SplitPlanes{};
  const L2WarmSet ws = warm ? *warm : L2WarmSet{};
  const int grid = ws.blocks > 0 ? (batch + kXcds - 1) / kXcds * kXcds + ws.blocks : batch;
  auto run = [&](auto threads) {
    constexpr int T = decltype(threads)::value;
    if (final_norm) {
      if (split) {
        batch_residual_norm_kernel<true, true, T><<<grid, T, 0, stream>>>(h, part, splits, batch, cols, w, eps, x, sp, ws);
      } else {
        batch_residual_norm_kernel<true, false, T><<<grid, T, 0, stream>>>(h, part, splits, batch, cols, w, eps, x, sp, ws);
      }
    } else if (split) {
      batch_residual_norm_kernel<false, true, T><<<grid, T, 0, stream>>>(h, part, splits, batch, cols, w, eps, x, sp, ws);
    } else {
      batch_residual_norm_kernel<false, false, T><<<grid, T, 0, stream>>>(h, part, splits, batch, cols, w, eps, x, sp, ws);
    }
  };
  if (batch >= kResManyRows) {
    run(std::integral_constant<int, 256>{});
  } else {
    run(std::integral_constant<int, 1024>{});
  }
  return hipGetLastError();
}

hipError_t launch_batch_swiglu(const float* part, int splits, int batch, int f, float* act, hipStream_t stream) {
  if (batch <= 0 || f <= 0 || f % 2 != 0 || splits <= 0) return hipErrorInvalidValue;
  batch_swiglu_kernel<<<dim3((f / 2 + 255) / 256, batch), 256, 0, stream>>>(part, splits, batch, f, act);
  return hipGetLastError();
}

hipError_t launch_batch_sum_parts(const float* part, int splits, int batch, int n, float* out, hipStream_t stream) {
  if (batch <= 0 || n <= 0 || splits <= 0) return hipErrorInvalidValue;
  if (n % 4 == 0) {
    batch_sum_parts_kernel<float4><<<dim3((n / 4 + 255) / 256, batch), 256, 0, stream>>>(part, splits, batch, n, out);
  } else {
    batch_sum_parts_kernel<float><<<dim3((n + 255) / 256, batch), 256, 0, stream>>>(part, splits, batch, n, out);
  }
  return hipGetLastError();
}

}  // namespace mmr
