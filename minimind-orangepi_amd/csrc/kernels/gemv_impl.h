// gemv_impl.h -- batch-1 fp16-weight GEMV family for gfx950.
//
// Replaces the reference's projection matvec (decoder_layer.cpp:65-90 on the
// CPU, aclnnMm through device_matmul at ascend_matmul.cpp:385-410) and the
// lm_head matvec + argmax (language_model.cpp:326-332, device_matmul_argmax at
// ascend_matmul.cpp:467-497).
//
// Design: the op is HBM-bound (about 1 FLOP per weight byte), so the kernel is
// built around getting every weight byte in flight at once.
//  * W is row-major [rows][k] fp16.  A group of G lanes (16/32/64) owns RPG
//    consecutive rows; lane j reads 16-byte chunks j, j+G, ... of each row, so
//    every load instruction of a group covers G*16 contiguous bytes.
//  * All RPG*CPL weight loads of a lane are issued before any arithmetic, so
//    one memory latency covers the whole tile.
//  * x (fp32) lives in registers: each lane only needs the chunks it multiplies.
//  * Fused prologues (RMSNorm, embedding gather, attention split combine) and
//    epilogues (residual add, SwiGLU over interleaved gate/up rows, per-block
//    first-index argmax) remove the separate elementwise launches of the
//    reference (K1, K4, K5, L2, L3).  No block ever waits for another.
#pragma once

#include "attention_common.h"
#include "device_common.h"
#include "kernels.h"

namespace mmr {
namespace gemv_detail {

template <int G, int RPG, int CPL, int PRO, int EPI>
__global__ __launch_bounds__(kGemvBlock) void gemv_kernel(GemvArgs a) {
  constexpr int kGroups = kGemvBlock / G;
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int k = a.k;
  const int kchunks = k >> 3;
  const int row0 = (blockIdx.x * kGroups + group) * RPG;

  // 1. Every load that does not depend on another goes out before any
  //    arithmetic, so one memory latency covers them all, in this order: the
  //    residual, the norm gains and the activations (x, or the attention
  //    split partials), then the weights.  Vector loads complete in order, so
  //    the prologue's arithmetic (RMSNorm, split merge) runs on the
  //    activations while the weights still stream in.  (The embedding
  //    prologue's row waits on two dependent scalar loads: its weights go
  //    before it.)  Compiler barriers keep this order, which the compiler,
  //    free to move these loads, would otherwise change (activations behind
  //    the weights, the residual sunk to its use at the end).  No load is
  //    guarded (a guard is a branch, with its own wait for the pointer it
  //    loads through): rows past N read the last row and are not stored,
  //    chunks past K read the last chunk and meet x = 0.
  uint4 wv[RPG][CPL];
  auto load_weights = [&] {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
      const int row = min(row0 + r, a.rows - 1);
      const uint4* wrow = reinterpret_cast<const uint4*>(a.w + static_cast<int64_t>(row) * k);
#pragma unroll
      for (int i = 0; i < CPL; ++i) wv[r][i] = wrow[min(lane + G * i, kchunks - 1)];
    }
    asm volatile("" ::: "memory");
  };
  // 1 / k for the RMSNorm mean, off the critical path (the mean is then one
  // fma with the epsilon instead of an IEEE divide after the reduction).
  const float inv_k = 1.0f / static_cast<float>(k);
  float res[RPG];
  if constexpr (EPI == kEpiResidual) {
#pragma unroll
    for (int r = 0; r < RPG; ++r) res[r] = a.residual[min(row0 + r, a.rows - 1)];
  }
  float nw[CPL][8];
  if constexpr (PRO == kProRmsNorm || PRO == kProRmsNormFinal || PRO == kProEmbedRmsNorm) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const float4* src = reinterpret_cast<const float4*>(a.norm_w + min(lane + G * i, kchunks - 1) * 8);
      const float4 lo = src[0];
      const float4 hi = src[1];
      nw[i][0] = lo.x; nw[i][1] = lo.y; nw[i][2] = lo.z; nw[i][3] = lo.w;
      nw[i][4] = hi.x; nw[i][5] = hi.y; nw[i][6] = hi.z; nw[i][7] = hi.w;
    }
  }

  // 2. x chunks owned by this lane (+ fused prologue).
  float xv[CPL][8];
  if constexpr (PRO == kProEmbedRmsNorm) {
    // The token at p = *pos: seq[p], or the argmax of the previous step's
    // lm_head partials (every block reduces them).  pos and seq[p] are read
    // through the scalar cache (no kernel writes them while this one runs,
    // except seq_out[p], stored by block 0 only when no block reads seq[p]),
    // so their dependent loads do not queue behind the vector loads.  The
    // partial loads go out before the weights: vector loads complete in
    // order, so the reduction waits for the partials alone.
    using cint = __attribute__((address_space(4))) const int32_t;
    const int p = *(cint*)a.pos;
    constexpr int kPrevPer = kGemvMaxPrevParts / kGemvBlock;
    const bool from_parts = a.prev_val != nullptr;
    float pv[kPrevPer];
    int pi[kPrevPer];
    if (from_parts) {
#pragma unroll
      for (int i = 0; i < kPrevPer; ++i) {
        const int j = min(static_cast<int>(threadIdx.x) + i * kGemvBlock, a.prev_parts - 1);
        pv[i] = a.prev_val[j];
        pi[i] = a.prev_idx[j];
      }
    }
    load_weights();
    int token;
    if (from_parts) {
      // (max, lowest index) is associative and commutative: the clamped
      // duplicates and the reduction order cannot change the result.
      float bv = pv[0];
      int bi = pi[0];
#pragma unroll
      for (int i = 1; i < kPrevPer; ++i)
        if (argmax_better(pv[i], pi[i], bv, bi)) {
          bv = pv[i];
          bi = pi[i];
        }
      wave_argmax(bv, bi);
      __shared__ float s_bv[kGemvBlock / kWave];
      __shared__ int s_bi[kGemvBlock / kWave];
      if (threadIdx.x % kWave == 0) {
        s_bv[threadIdx.x / kWave] = bv;
        s_bi[threadIdx.x / kWave] = bi;
      }
      __syncthreads();
      bv = s_bv[0];
      bi = s_bi[0];
#pragma unroll
      for (int w = 1; w < kGemvBlock / kWave; ++w)
        if (argmax_better(s_bv[w], s_bi[w], bv, bi)) {
          bv = s_bv[w];
          bi = s_bi[w];
        }
      const bool generated = p >= *(cint*)a.prompt_len;
      if (generated) {
        token = bi;
        if (blockIdx.x == 0 && threadIdx.x == 0 && p < a.seq_len) a.seq_out[p] = bi;
      } else {
        token = ((cint*)a.seq)[p];
      }
    } else {
      token = ((cint*)a.seq)[p];
    }
    token = token < 0 ? 0 : (token >= a.vocab ? a.vocab - 1 : token);
    const uint4* erow = reinterpret_cast<const uint4*>(a.embed + static_cast<int64_t>(token) * k);
    // Every chunk's load goes out before any is used (a use between them
    // would wait for the first before the second is issued).
    uint4 eraw[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) eraw[i] = erow[min(lane + G * i, kchunks - 1)];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      half8_to_float8(eraw[i], xv[i]);
      if (lane + G * i >= kchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
      }
    }
    if (blockIdx.x == 0 && group == 0) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + G * i;
        if (c < kchunks) {
          float4* dst = reinterpret_cast<float4*>(a.h_out + c * 8);
          dst[0] = make_float4(xv[i][0], xv[i][1], xv[i][2], xv[i][3]);
          dst[1] = make_float4(xv[i][4], xv[i][5], xv[i][6], xv[i][7]);
        }
      }
    }
  } else if constexpr (PRO == kProAttnCombine) {
    // Log-sum-exp merge of the attention split partials into LDS, computed by
    // every block (k = hq * head_dim <= 1024, splits <= 16, hq <= 16):
    //   M_h = max_s m[h][s],  e[h][s] = exp(m[h][s] - M_h),
    //   L_h = sum_s l[h][s] e[h][s],  x[h*d + i] = (sum_s o[h][s][i] e[h][s]) / L_h,
    // both sums in split order (attention_combine_kernel computes the same
    // quantity, summing over groups of splits: the two agree to rounding).
    __shared__ __align__(16) float s_x[kCombineMaxDim];
    __shared__ __align__(16) float s_e[kCombineMaxHeads][kCombineMaxSplits];
    __shared__ __align__(16) float s_l[kCombineMaxHeads][kCombineMaxSplits];
    const int S = a.splits, D = a.head_dim, R = a.hq / a.hkv;
    // Thread t owns x[4t, 4t + 4); its 16 float4 partial loads are
    // unconditional (split index clamped) so they issue back to back.  The
    // offsets are attn_o_offset / attn_ml_offset written as a per-lane base
    // plus a wave-uniform split term (scalar arithmetic), in 32 bits (the
    // partial buffer of at most kCombineMaxSplits splits is small), and the
    // lane's head and group come from small_quotient instead of divisions.
    const int t4 = min(static_cast<int>(threadIdx.x), k / 4 - 1);
    const int head = small_quotient(4 * t4, D), dim = 4 * t4 - head * D;
    const int g = small_quotient(head, R);
    const int obase = ((g * S) * R + (head - g * R)) * D + dim;  // attn_o_offset(g, 0, head % R, S, R, D) + dim
    // Lane (head, split) = (threadIdx / 16, threadIdx % 16): one 16-lane row
    // per head, so M_h is a row reduction.  Splits >= S get weight 0.  The
    // lane's (m, l) goes out first, then the o partials and the weights:
    // vector loads complete in issue order, so the weights' exponents below
    // wait for (m, l) alone.
    const int wh = min(static_cast<int>(threadIdx.x) / kCombineMaxSplits, a.hq - 1);
    const int ws = static_cast<int>(threadIdx.x) % kCombineMaxSplits;
    const int wg = small_quotient(wh, R);
    const float2 ml = *reinterpret_cast<const float2*>(
        a.part + a.hkv * S * R * D + ((wg * S + min(ws, S - 1)) * R + (wh - wg * R)) * 2);  // attn_ml_offset
    asm volatile("" ::: "memory");
    float4 ov[kCombineMaxSplits];
#pragma unroll
    for (int s = 0; s < kCombineMaxSplits; ++s)
      ov[s] = *reinterpret_cast<const float4*>(a.part + obase + min(s, S - 1) * (R * D));
    {
      load_weights();
      const bool live = ws < S;
      const float m = live ? ml.x : -INFINITY;
      const float M = group_max<kCombineMaxSplits>(m);
      s_e[threadIdx.x / kCombineMaxSplits][ws] = live ? expf(m - M) : 0.0f;
      s_l[threadIdx.x / kCombineMaxSplits][ws] = live ? ml.y : 0.0f;
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < k / 4) {
      float L = 0.0f;
      float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int s4 = 0; s4 < kCombineMaxSplits / 4; ++s4) {
        const float4 e4 = *reinterpret_cast<const float4*>(&s_e[head][4 * s4]);
        const float4 l4 = *reinterpret_cast<const float4*>(&s_l[head][4 * s4]);
        const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4& o = ov[4 * s4 + j];
          L = fmaf(lv[j], ev[j], L);
          x.x = fmaf(o.x, ev[j], x.x);
          x.y = fmaf(o.y, ev[j], x.y);
          x.z = fmaf(o.z, ev[j], x.z);
          x.w = fmaf(o.w, ev[j], x.w);
        }
      }
      const float inv = 1.0f / L;
      *reinterpret_cast<float4*>(&s_x[4 * threadIdx.x]) = make_float4(x.x * inv, x.y * inv, x.z * inv, x.w * inv);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + G * i;
      const int cc = min(c, kchunks - 1);
      const float4 lo = *reinterpret_cast<const float4*>(&s_x[cc * 8]);
      const float4 hi = *reinterpret_cast<const float4*>(&s_x[cc * 8 + 4]);
      const bool in = c < kchunks;
      xv[i][0] = in ? lo.x : 0.0f; xv[i][1] = in ? lo.y : 0.0f; xv[i][2] = in ? lo.z : 0.0f; xv[i][3] = in ? lo.w : 0.0f;
      xv[i][4] = in ? hi.x : 0.0f; xv[i][5] = in ? hi.y : 0.0f; xv[i][6] = in ? hi.z : 0.0f; xv[i][7] = in ? hi.w : 0.0f;
    }
  } else if (a.x_half != nullptr) {
    // fp16 x (BASELINE configs[1]'s input format): one 16-byte chunk per 8
    // elements, widened exactly to fp32 after the weight loads are out.
    uint4 xr[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) xr[i] = reinterpret_cast<const uint4*>(a.x_half)[min(lane + G * i, kchunks - 1)];
    load_weights();
#pragma unroll
    for (int i = 0; i < CPL; ++i) half8_to_float8(xr[i], xv[i]);
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      if (lane + G * i >= kchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
      }
  } else {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + G * i;
      const float4* src = reinterpret_cast<const float4*>(a.x + min(c, kchunks - 1) * 8);
      const float4 lo = src[0];
      const float4 hi = src[1];
      xv[i][0] = lo.x; xv[i][1] = lo.y; xv[i][2] = lo.z; xv[i][3] = lo.w;
      xv[i][4] = hi.x; xv[i][5] = hi.y; xv[i][6] = hi.z; xv[i][7] = hi.w;
    }
    load_weights();
    // Chunks past K meet x = 0 (after the weight loads are out: this reads x).
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      if (lane + G * i >= kchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
      }
  }

  // kEpiArgmax position bookkeeping, read once every load of the block is out
  // (a load under a branch is waited for where the branch joins), through the
  // scalar cache (its wait never covers the vector loads; the only write to
  // it in this kernel is block 0's own, at the end), and stored with the
  // block's partial.
  int advance_from = 0;
  if constexpr (EPI == kEpiArgmax) {
    if (a.advance_pos != nullptr && blockIdx.x == 0)
      advance_from = *(const __attribute__((address_space(4))) int32_t*)a.advance_pos;
  }

  if constexpr (PRO == kProRmsNorm || PRO == kProRmsNormFinal || PRO == kProEmbedRmsNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += xv[i][e] * xv[i][e];
    ss = group_sum<G>(ss);
    // 1 / sqrt as one v_rsq_f32 (about 1 ulp) instead of a correctly rounded
    // sqrt and an IEEE divide on the prologue's critical path.
    const float scale = __builtin_amdgcn_rsqf(fmaf(ss, inv_k, a.eps));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {  // chunks past K: x = 0, stays 0
        if constexpr (PRO == kProRmsNormFinal) {
          xv[i][e] = (xv[i][e] * scale) * nw[i][e];
        } else {
          xv[i][e] = xv[i][e] * (scale * nw[i][e]);
        }
      }
    }
  }

  // 3. Dot products, fp32 accumulation, butterfly reduce over the group.
  float acc[RPG];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      float wf[8];
      half8_to_float8(wv[r][i], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) s = fmaf(wf[e], xv[i][e], s);
    }
    acc[r] = group_sum<G>(s);
  }

  // 4. Epilogue.
  if constexpr (EPI == kEpiStore || EPI == kEpiResidual) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r;
        if (row < a.rows) {
          if constexpr (EPI == kEpiResidual) {
            a.y[row] = res[r] + acc[r];
          } else {
            a.y[row] = acc[r];
          }
        }
      }
    }
  } else if constexpr (EPI == kEpiSwiGlu) {
    static_assert(RPG % 2 == 0, "SwiGLU needs (gate, up) row pairs");
    if (lane == 0) {
#pragma unroll
      for (int p = 0; p < RPG / 2; ++p) {
        const int row = row0 + 2 * p;
        if (row + 1 < a.rows) {
          const float g = acc[2 * p];
          const float u = acc[2 * p + 1];
          a.y[row / 2] = silu_fast(g) * u;
        }
      }
    }
  } else {  // kEpiArgmax: per-block (max, first index) partial
    constexpr int kRowsPerBlock = kGroups * RPG;
    __shared__ float s_val[kRowsPerBlock];
    __shared__ int s_idx[kRowsPerBlock];
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r;
        const bool ok = row < a.rows;
        if (ok && a.y) a.y[row] = acc[r];
        s_val[group * RPG + r] = ok ? acc[r] : -INFINITY;
        s_idx[group * RPG + r] = ok ? row : 0x7fffffff;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = s_val[0];
      int bi = s_idx[0];
      for (int j = 1; j < kRowsPerBlock; ++j)
        if (argmax_better(s_val[j], s_idx[j], bv, bi)) {
          bv = s_val[j];
          bi = s_idx[j];
        }
      a.part_val[blockIdx.x] = bv;
      a.part_idx[blockIdx.x] = bi;
      if (a.advance_pos != nullptr && blockIdx.x == 0) *a.advance_pos = advance_from + 1;
    }
  }
}

template <int G, int RPG, int CPL>
hipError_t launch_shape(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, int blocks, hipStream_t s) {
  const dim3 grid(blocks), block(kGemvBlock);
#define MMR_GEMV_CASE(P, E)                                                           \
  if (pro == P && epi == E) {                                                         \
    gemv_kernel<G, RPG, CPL, P, E><<<grid, block, 0, s>>>(a);                         \
    return hipGetLastError();                                                         \
  }
  MMR_GEMV_CASE(kProPlain, kEpiStore)
  MMR_GEMV_CASE(kProPlain, kEpiResidual)
  MMR_GEMV_CASE(kProAttnCombine, kEpiResidual)
  MMR_GEMV_CASE(kProRmsNorm, kEpiStore)
  MMR_GEMV_CASE(kProEmbedRmsNorm, kEpiStore)
  MMR_GEMV_CASE(kProRmsNormFinal, kEpiArgmax)
  MMR_GEMV_CASE(kProPlain, kEpiArgmax)
  if constexpr (RPG % 2 == 0) {
    MMR_GEMV_CASE(kProRmsNorm, kEpiSwiGlu)
    MMR_GEMV_CASE(kProPlain, kEpiSwiGlu)
  }
#undef MMR_GEMV_CASE
  return hipErrorInvalidValue;
}

template <int G, int RPG>
hipError_t launch_cpl_impl(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, int cpl, int blocks,
                      hipStream_t s) {
  switch (cpl) {
    case 1: return launch_shape<G, RPG, 1>(a, pro, epi, blocks, s);
    case 2: return launch_shape<G, RPG, 2>(a, pro, epi, blocks, s);
    case 3: return launch_shape<G, RPG, 3>(a, pro, epi, blocks, s);
    case 4: return launch_shape<G, RPG, 4>(a, pro, epi, blocks, s);
    case 6: return launch_shape<G, RPG, 6>(a, pro, epi, blocks, s);
    case 8: return launch_shape<G, RPG, 8>(a, pro, epi, blocks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gemv_detail

// Defined in gemv_g16.hip / gemv_g32.hip / gemv_g64.hip (one TU per lane width).
template <int G, int RPG>
hipError_t launch_cpl(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, int cpl, int blocks, hipStream_t s);

}  // namespace mmr
