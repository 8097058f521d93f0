// support.hip -- standalone elementwise ops of the reference operator surface.
//
// The fused decode step does not launch these (their work is folded into the
// GEMV prologues/epilogues and the attention kernel); they exist so that every
// entry point of the reference's device-op boundary has a drop-in:
//   device_rms_norm_rows  ascend_custom_ops.cpp:556-582 (K1)
//   device_add            ascend_custom_ops.cpp:535-554 (K5)
//   device_swiglu_rows    ascend_custom_ops.cpp:584-604 (K4)
//   device_embedding_gather ascend_custom_ops.cpp:737-767 (L3)
// All compute in fp32; RMSNorm honours the eps argument (the AscendC kernels
// hardcode 1e-5).
#include "device_common.h"
#include "kernels.h"

namespace mmr {
namespace {

constexpr int kRowThreads = 256;

// One block per row.  x * (scale * w) as decoder_layer.cpp:32-42, or with
// kFinal the final norm's (x * scale) * w (language_model.cpp:24-38).
template <bool kFinal>
__global__ __launch_bounds__(kRowThreads) void rms_norm_rows_kernel(const float* in, const float* w, float eps,
                                                                    int cols, float* out) {
  __shared__ float partial[kRowThreads / kWave];
  const float* x = in + static_cast<int64_t>(blockIdx.x) * cols;
  float* y = out + static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < cols; i += kRowThreads) ss += x[i] * x[i];
  ss = group_sum<kWave>(ss);
  if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kRowThreads / kWave; ++i) total += partial[i];
  const float scale = 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
  for (int i = threadIdx.x; i < cols; i += kRowThreads) y[i] = kFinal ? (x[i] * scale) * w[i] : x[i] * (scale * w[i]);
}

__global__ void add_kernel(const float* a, const float* b, int64_t n, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

// [rows][2*cols] gate|up halves -> [rows][cols] (decoder_layer.cpp:283-295).
__global__ void swiglu_rows_kernel(const float* gate_up, int rows, int cols, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(rows) * cols) return;
  const int64_t r = i / cols;
  const int64_t c = i % cols;
  const float g = gate_up[r * 2 * cols + c];
  const float u = gate_up[r * 2 * cols + cols + c];
  out[i] = (g / (1.0f + expf(-g))) * u;
}

// fp16 table row -> fp32 (language_model.cpp:67-77).  Out-of-range ids set
// *err and produce a zero row instead of reading outside the table.
__global__ void embedding_gather_kernel(const __half* table, const int32_t* ids, int vocab, int hidden, float* out,
                                        int32_t* err) {
  const int t = blockIdx.y;
  const int id = ids[t];
  const bool ok = id >= 0 && id < vocab;
  if (!ok && threadIdx.x == 0 && blockIdx.x == 0 && err) *err = 1;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    out[static_cast<int64_t>(t) * hidden + i] = ok ? __half2float(table[static_cast<int64_t>(id) * hidden + i]) : 0.0f;
}

}  // namespace

hipError_t launch_rms_norm_rows(const float* in, const float* w, float eps, int rows, int cols, float* out,
                                hipStream_t stream, bool final_norm) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (final_norm) {
    rms_norm_rows_kernel<true><<<rows, kRowThreads, 0, stream>>>(in, w, eps, cols, out);
  } else {
    rms_norm_rows_kernel<false><<<rows, kRowThreads, 0, stream>>>(in, w, eps, cols, out);
  }
  return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, int64_t n, float* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  add_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(a, b, n, out);
  return hipGetLastError();
}

hipError_t launch_swiglu_rows(const float* gate_up, int rows, int cols, float* out, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(rows) * cols;
  if (n <= 0) return hipSuccess;
  swiglu_rows_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(gate_up, rows, cols, out);
  return hipGetLastError();
}

hipError_t launch_embedding_gather(const __half* table, const int32_t* ids, int tokens, int vocab, int hidden,
                                   float* out, int32_t* err, hipStream_t stream) {
  if (tokens <= 0 || hidden <= 0) return hipSuccess;
  const dim3 grid((hidden + 255) / 256, tokens);
  embedding_gather_kernel<<<grid, 256, 0, stream>>>(table, ids, vocab, hidden, out, err);
  return hipGetLastError();
}

}  // namespace mmr
