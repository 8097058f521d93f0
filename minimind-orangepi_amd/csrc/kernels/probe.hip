// probe.hip -- launch-latency yardstick for the decode step's kernel chain.
//
// A decode step is a chain of dependent kernels replayed from one hipGraph, so
// every kernel pays the chain's per-launch floor before it moves any weight.
// measure_launch_floor captures `kernels` launches of one trivial kernel on a
// private stream, replays the graph `reps` times and reports the time per
// kernel: either an empty kernel, or one whose every thread loads one float its
// predecessor wrote and whose block stores one (a dependent round trip).
#include "kernels.h"

namespace mmr {
namespace {

__global__ void probe_empty_kernel() {}

__global__ void probe_load_store_kernel(const float* in, float* out, int n) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  const float v = in[i % n] * 0.5f + 1.0f;
  if (threadIdx.x == 0) out[blockIdx.x] = v;
}

}  // namespace

hipError_t measure_launch_floor(int kernels, int blocks, bool load_store, int reps, float* us_per_kernel) {
  if (kernels <= 0 || kernels > 4096 || blocks <= 0 || blocks > 65536 || reps <= 0 || !us_per_kernel)
    return hipErrorInvalidValue;
  constexpr int kThreads = 256;
  const int n = blocks * kThreads;
  float* buf = nullptr;
  hipStream_t s = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t st = hipMalloc(&buf, 2 * static_cast<size_t>(n) * sizeof(float));
  auto step = [&](hipError_t r) {
    if (st == hipSuccess) st = r;
    return st == hipSuccess;
  };
  if (step(st) && step(hipMemset(buf, 0, 2 * static_cast<size_t>(n) * sizeof(float))) &&
      step(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)) &&
      step(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal))) {
    for (int k = 0; k < kernels; ++k) {
      if (load_store) {
        probe_load_store_kernel<<<blocks, kThreads, 0, s>>>(buf + (k % 2) * n, buf + ((k + 1) % 2) * n, n);
      } else {
        probe_empty_kernel<<<blocks, kThreads, 0, s>>>();
      }
    }
    const hipError_t launch = hipGetLastError();
    const hipError_t end = hipStreamEndCapture(s, &graph);
    if (step(launch) && step(end) && step(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) &&
        step(hipEventCreate(&e0)) && step(hipEventCreate(&e1))) {
      for (int w = 0; w < 3 && step(hipGraphLaunch(exec, s)); ++w) {
      }
      float ms = 0.0f;
      if (step(hipStreamSynchronize(s)) && step(hipEventRecord(e0, s))) {
        for (int r = 0; r < reps && step(hipGraphLaunch(exec, s)); ++r) {
        }
        if (step(hipEventRecord(e1, s)) && step(hipEventSynchronize(e1)) && step(hipEventElapsedTime(&ms, e0, e1)))
          *us_per_kernel = ms * 1e3f / (static_cast<float>(reps) * static_cast<float>(kernels));
      }
    }
  }
  if (s) (void)hipStreamSynchronize(s);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  if (s) (void)hipStreamDestroy(s);
  if (buf) (void)hipFree(buf);
  return st;
}

}  // namespace mmr
