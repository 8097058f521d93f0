// gemv.hip -- launch planning and dispatch for the GEMV family (kernels in
// gemv_impl.h, instantiated per lane width in gemv_g16/g32/g64.hip).
#include "gemv_impl.h"

namespace mmr {
namespace {

int round_cpl(int needed) {
  static const int kAllowed[] = {1, 2, 3, 4, 6, 8};
  for (int c : kAllowed)
    if (c >= needed) return c;
  return -1;
}

}  // namespace

namespace {

// One block reduces the per-block argmax partials; thread 0 does the step
// bookkeeping.  (max, lowest index) is associative and commutative, so the
// lane exchanges and the wave order cannot change the result.
__global__ __launch_bounds__(kGemvBlock) void argmax_finalize_kernel(ArgmaxFinalizeArgs a) {
  constexpr int kWaves = kGemvBlock / kWave;
  __shared__ float w_val[kWaves];
  __shared__ int w_idx[kWaves];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = threadIdx.x; b < a.parts; b += kGemvBlock) {
    const float v = a.part_val[b];
    const int i = a.part_idx[b];
    if (argmax_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (argmax_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (threadIdx.x % kWave == 0) {
    w_val[threadIdx.x / kWave] = bv;
    w_idx[threadIdx.x / kWave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w)
      if (argmax_better(w_val[w], w_idx[w], bv, bi)) {
        bv = w_val[w];
        bi = w_idx[w];
      }
    const int32_t next = bi;
    if (a.token_out) *a.token_out = next;
    if (a.pos) {
      const int32_t p = *a.pos;
      if (p + 1 < a.seq_len && p + 1 >= *a.prompt_len) a.seq[p + 1] = next;
      *a.pos = p + 1;
    }
  }
}

}  // namespace

hipError_t launch_argmax_finalize(const ArgmaxFinalizeArgs& a, hipStream_t stream) {
  if (a.parts <= 0) return hipErrorInvalidValue;
  argmax_finalize_kernel<<<1, kGemvBlock, 0, stream>>>(a);
  return hipGetLastError();
}

bool gemv_plan(int rows, int k, GemvEpilogue epi, int lanes_per_row, int rows_per_group, GemvPlan* plan) {
  if (rows <= 0 || k <= 0 || k % 8 != 0) return false;
  const int kchunks = k / 8;
  int g = lanes_per_row;
  // Default lane width: 64 from k = 768 up (more, shorter blocks measured
  // faster in the decode step than fewer fully used lanes), else 32 / 16.
  if (g == 0) g = kchunks >= 96 ? 64 : (kchunks >= 48 ? 32 : 16);
  if (g != 16 && g != 32 && g != 64) return false;
  int rpg = rows_per_group;
  // Two rows per group for SwiGLU (the gate/up pair) and argmax (half the
  // partials for the finalize), one otherwise.
  if (rpg == 0) rpg = (epi == kEpiSwiGlu || epi == kEpiArgmax) ? 2 : 1;
  if (rpg != 1 && rpg != 2 && rpg != 4) return false;
  if (epi == kEpiSwiGlu && (rpg % 2 != 0 || rows % 2 != 0)) return false;
  const int cpl = round_cpl((kchunks + g - 1) / g);
  if (cpl < 0) return false;
  const int rows_per_block = (kGemvBlock / g) * rpg;
  plan->lanes_per_row = g;
  plan->rows_per_group = rpg;
  plan->chunks_per_lane = cpl;
  plan->blocks = (rows + rows_per_block - 1) / rows_per_block;
  return true;
}

hipError_t launch_gemv(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, const GemvPlan& p,
                       hipStream_t stream) {
  // The embedding prologue's token from the previous step's argmax partials.
  if (a.prev_val && (pro != kProEmbedRmsNorm || !a.prev_idx || !a.prompt_len || !a.seq_out || a.prev_parts < 1 ||
                     a.prev_parts > kGemvMaxPrevParts))
    return hipErrorInvalidValue;
  if (a.advance_pos && epi != kEpiArgmax) return hipErrorInvalidValue;
  const int cpl = p.chunks_per_lane;
#define MMR_GEMV_G(GV, RV)                                               \
  if (p.lanes_per_row == GV && p.rows_per_group == RV)                   \
    return launch_cpl<GV, RV>(a, pro, epi, cpl, p.blocks, stream);
  MMR_GEMV_G(16, 1)
  MMR_GEMV_G(16, 2)
  MMR_GEMV_G(16, 4)
  MMR_GEMV_G(32, 1)
  MMR_GEMV_G(32, 2)
  MMR_GEMV_G(32, 4)
  MMR_GEMV_G(64, 1)
  MMR_GEMV_G(64, 2)
  MMR_GEMV_G(64, 4)
#undef MMR_GEMV_G
  return hipErrorInvalidValue;
}

}  // namespace mmr
