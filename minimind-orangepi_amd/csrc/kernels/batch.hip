// batch.hip -- kernels specific to decoding a batch of independent sequences
// (the reference's DecoderState holds one sequence,
// language_model.h:22-25).  The projections of a batched step run on the
// prefill GEMM (M = batch) and the attention on the split kernel with a
// paged cache; these kernels cover the per-sequence token handling.
#include "device_common.h"
#include "kernels.h"

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

}  // namespace

hipError_t launch_batch_embed(const __half* embed, const int32_t* seq, int seq_stride, const int32_t* pos, int batch,
                              int vocab, int hidden, float* h, hipStream_t stream) {
  if (batch <= 0 || hidden <= 0) return hipErrorInvalidValue;
  const dim3 grid((hidden + kBatchThreads - 1) / kBatchThreads, batch);
  batch_embed_kernel<<<grid, kBatchThreads, 0, stream>>>(embed, seq, seq_stride, pos, vocab, hidden, h);
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

}  // namespace mmr
