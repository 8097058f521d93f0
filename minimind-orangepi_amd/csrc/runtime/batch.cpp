// batch.cpp -- batched decode: B independent sequences advance one token per
// step, each at its own position, over a paged KV cache.
//
// The reference runtime decodes one sequence per DecoderState
// (language_model.h:22-25); each sequence of a batch computes exactly what
// LanguageModel::forward_next_token computes for it alone
// (language_model.cpp:310-333, decoder_layer.cpp:312-407), with the batch's
// projections as split-K GEMMs of B rows on the fp32 matrix cores, whose
// partial sums the next kernel adds in split order.  Step kernels:
//   embed rows of seq[b][pos[b]] -> input RMSNorm rows
//   per layer: QKV split-K -> paged split attention (sums the QKV partials;
//              q/k norm, RoPE at pos[b], K/V append) -> O split-K whose
//              staging merges the attention splits -> residual add + post
//              RMSNorm -> gate_up split-K -> down
//              split-K whose staging sums the gate_up partials and applies
//              SwiGLU -> residual add + next RMSNorm
//   lm_head split-K -> logits (sums the partials) + per-sequence argmax +
//   bookkeeping
// captured once per attention split count into a hipGraph.
//
// KV cache: per layer a pool of 64-token pages [page][Hkv][64][d]; sequence
// b's token t lives in page page_table[b][t / 64].  Pages are assigned at
// creation, interleaved across sequences (page p of sequence b is physical
// page p * B + b), so the attention reads every tile through the table.
#include "language_model.h"

#include "device.h"
#include "device_model.h"
#include "../kernels/kernels.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>

namespace minimind::model {

// Warming blocks per residual + norm launch (MMR_L2_WARM_BLOCKS sets them):
// none by default.  Since the split-K GEMMs stage A while their W fragments
// are still arriving, warming W costs more than it saves (B = 32, 256 -> 4096,
// same box: none 47.05k tok/s, p50 step 0.678 ms; 64 / 128 / 224 blocks
// 45.13k / 46.00k / 46.18k, 0.706 / 0.693 / 0.690 ms).  Before that change 128
// blocks measured best (892.9 -> 885.3 us per step).
constexpr int kBatchWarmBlocks = 0;
constexpr int64_t kBatchWarmMaxBytes = int64_t{16} << 20;  // half the 32 MB of L2

struct BatchDeviceState {
  std::shared_ptr<const DeviceModel> model;
  mmr::KvDtype kv = mmr::kKvF16;
  int64_t batch = 0;
  int64_t capacity = 0;       // positions per sequence
  int64_t pages_per_seq = 0;
  Arena arena;
  std::vector<void*> kpool, vpool;  // per layer [pages][Hkv][kKvPage][d]
  int32_t* page_table = nullptr;    // [batch][pages_per_seq]
  int32_t* seq = nullptr;           // [batch][capacity + 1]
  int32_t* pos = nullptr;           // [batch]
  int32_t* prompt_len = nullptr;    // [batch]
  int32_t* token_out = nullptr;     // [batch]
  int32_t* err = nullptr;
  float* h = nullptr;       // [batch][H]
  float* x = nullptr;       // [batch][H]
  float* qkv = nullptr;     // [batch][(Hq + 2 Hkv) d]
  float* attn = nullptr;    // [batch][Hq d]
  float* gu = nullptr;      // [batch][2F]
  float* act = nullptr;     // [batch][F]
  float* logits = nullptr;  // [batch][V]
  float* part = nullptr;    // attention partials, part_stride floats per sequence
  int64_t part_stride = 0;
  float* proj = nullptr;    // projection split-K partials [splits][batch][n] (one GEMM at a time)
  float* proj_gu = nullptr; // gate_up partials, read by the down projection's staging
  int32_t* staging = nullptr;  // pinned host
  int64_t staging_len = 0;
  hipStream_t stream = nullptr;
  std::map<int, hipGraphExec_t> graphs;
  bool use_graphs = true;
  // L2-warming blocks of the residual + norm launches (0 = none): the one
  // after the O projection loads gate_up and down, the one after down the
  // next layer's qkv (after the last layer the lm_head's).
  int warm_blocks = kBatchWarmBlocks;

  ~BatchDeviceState() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& g : graphs) (void)hipGraphExecDestroy(g.second);
    if (stream) (void)hipStreamDestroy(stream);
    if (staging) (void)hipHostFree(staging);
  }
};

BatchState::BatchState() = default;
BatchState::~BatchState() = default;
BatchState::BatchState(BatchState&&) noexcept = default;
BatchState& BatchState::operator=(BatchState&&) noexcept = default;
int64_t BatchState::batch() const { return device ? device->batch : 0; }
int64_t BatchState::capacity() const { return device ? device->capacity : 0; }
void* BatchState::stream() const { return device ? static_cast<void*>(device->stream) : nullptr; }

namespace {

// Attention splits per sequence: up to sixteen 64-token tiles per block (the
// next tile is prefetched while one is computed, so long per-block loops are
// cheap), raised while the context has the tiles until the launch has about
// one block per CU.  Fewer splits also leave fewer partials for the O
// projection's staging to merge, and past 8 the separate combine kernel runs.
// On the matrix-core attention at B = 32, 256 -> 4096 positions (aggregate
// tok/s, p50 step; same box): 16 tiles / 256 blocks (4 splits from 257
// positions on) 42.03k, 0.764 ms; 8 / 256 41.79k, 0.773; 8 / 512 (8 splits)
// 41.24k, 0.774; 8 / 128 41.58k, 0.773; 16 / 128 40.96k, 0.787; 4 / 512 and
// 8 / 1024 (16 splits, combine kernel) 38.8k / 37.5k, 0.869.
constexpr int kBatchMaxSplits = 64;
constexpr int kBatchTilesPerSplit = 16;
constexpr int64_t kBatchAttnBlocks = 256;

int batch_splits(int64_t n_keys, int tile, int64_t seq_heads) {
  const int64_t tiles = (n_keys + tile - 1) / tile;
  int s = 1;
  while (s < kBatchMaxSplits && s * kBatchTilesPerSplit < tiles) s *= 2;
  while (s < kBatchMaxSplits && 2 * s <= tiles && seq_heads * s < kBatchAttnBlocks) s *= 2;
  return s;
}

// K chunk of a projection's split-K launch (0: dense fallback, k not a
// multiple of 32); QKV partials are consumed by the attention prologue, which
// takes at most qkv_max_parts(k) of them.
int proj_chunk(int n, int k, int max_parts) {
  int kc = mmr::splitk_chunk(n, k);
  if (kc == 0 || max_parts <= 0 || k / kc <= max_parts) return kc;
  for (kc = 32; kc <= 256; kc += 32)  // the smallest chunk that tiles K in max_parts pieces
    if (k % kc == 0 && k / kc <= max_parts) return kc;
  return 0;
}

// Most QKV partials for a K of k: kAttnFewQkvParts where chunks of up to 256
// columns tile K in that many (the attention prologue's lighter variant),
// else kAttnMaxQkvParts.
int qkv_max_parts(int k) {
  for (int kc = 32; kc <= 256; kc += 32)
    if (k % kc == 0 && k / kc <= mmr::kAttnFewQkvParts) return mmr::kAttnFewQkvParts;
  return mmr::kAttnMaxQkvParts;
}

// out_parts[s][b][n] = partial products of x (batch rows, stride k) with W
// [n][k]; returns the number of splits (1 for the dense fallback).
int project(const BatchDeviceState& s, const float* x, const __half* w, int n, int k, int max_parts,
            float* out = nullptr) {
  if (!out) out = s.proj;
  const int B = static_cast<int>(s.batch);
  const int kc = B <= 32 ? proj_chunk(n, k, max_parts) : 0;
  if (kc > 0) {
    mmr::SplitKArgs g;
    g.a = x;
    g.lda = k;
    g.w = w;
    g.part = out;
    g.m = B;
    g.n = n;
    g.k = k;
    g.kc = kc;
    check_hip(mmr::launch_gemm_splitk(g, s.stream), "batch split-K gemm");
    return (k + kc - 1) / kc;
  }
  mmr::GemmArgs g;
  g.a = x;
  g.lda = k;
  g.w = w;
  g.c = out;
  g.ldc = n;
  g.m = B;
  g.n = n;
  g.k = k;
  check_hip(mmr::launch_gemm(g, s.stream), "batch gemm");
  return 1;
}

// The O projection of the attention output: the split-K staging merges the
// attention split partials itself where its registers allow (up to 8 splits),
// else the combine kernel writes attn first.
int project_combine(const BatchDeviceState& s, int splits, const __half* w, int n, int hq, int hkv, int d) {
  const int B = static_cast<int>(s.batch);
  const int k = hq * d;
  const int kc = B <= 32 ? proj_chunk(n, k, 0) : 0;
  if (kc > 0 && mmr::splitk_combine_supported(B, kc, splits, d)) {
    mmr::SplitKArgs g;
    g.attn_part = s.part;
    g.attn_splits = splits;
    g.attn_part_stride = s.part_stride;
    g.hq = hq;
    g.hkv = hkv;
    g.d = d;
    g.w = w;
    g.part = s.proj;
    g.m = B;
    g.n = n;
    g.k = k;
    g.kc = kc;
    check_hip(mmr::launch_gemm_splitk(g, s.stream), "batch split-K gemm (attention-combine input)");
    return k / kc;
  }
  check_hip(mmr::launch_attention_combine(s.part, hq, hkv, d, splits, s.attn, s.stream, B, s.part_stride),
            "batch attention combine");
  return project(s, s.attn, w, n, k, 0);
}

// The down projection of SwiGLU(gate_up partials): the split-K staging sums
// the partials and applies SwiGLU itself where its registers allow, else the
// SwiGLU kernel writes act first.
int project_swiglu(const BatchDeviceState& s, const float* gu, int gu_parts, const __half* w, int n, int f) {
  const int B = static_cast<int>(s.batch);
  const int kc = B <= 32 ? proj_chunk(n, f, 0) : 0;
  if (kc > 0 && mmr::splitk_swiglu_supported(B, kc, gu_parts)) {
    mmr::SplitKArgs g;
    g.gu = gu;
    g.gu_splits = gu_parts;
    g.w = w;
    g.part = s.proj;
    g.m = B;
    g.n = n;
    g.k = f;
    g.kc = kc;
    check_hip(mmr::launch_gemm_splitk(g, s.stream), "batch split-K gemm (SwiGLU input)");
    return f / kc;
  }
  check_hip(mmr::launch_batch_swiglu(gu, gu_parts, B, f, s.act, s.stream), "batch swiglu");
  return project(s, s.act, w, n, f, 0);
}

// The split-K launch of an n x k projection with chunk kc (grid
// (ceil(n / kSplitKRows), k / kc): block (x, y) reads a kc-column chunk of 64
// W rows) as an L2-warming region; unused for the dense fallback (kc = 0) or
// byte offsets past 32 bits.
mmr::L2Warm splitk_warm_region(const __half* w, int n, int k, int kc) {
  mmr::L2Warm r;
  const int64_t bytes = int64_t{n} * k * 2;
  if (kc <= 0 || bytes + int64_t{k} * 2 * mmr::kSplitKRows >= (int64_t{1} << 32)) return r;
  r.base = w;
  r.bytes = static_cast<uint32_t>(bytes);
  r.row_bytes = static_cast<uint32_t>(k * 2);
  r.seg_bytes = static_cast<uint32_t>(kc * 2);
  r.rows = mmr::kSplitKRows;
  r.units_x = (n + mmr::kSplitKRows - 1) / mmr::kSplitKRows;
  r.units_y = k / kc;
  return r;
}

// A warming set over the given regions when they fit the byte budget.
mmr::L2WarmSet warm_set(int blocks, std::initializer_list<mmr::L2Warm> regions) {
  mmr::L2WarmSet w;
  int64_t bytes = 0;
  int i = 0;
  for (const auto& r : regions) {
    if (i == mmr::kL2WarmRegions) break;
    w.region[i++] = r;
    bytes += r.bytes;
  }
  w.blocks = bytes > 0 && bytes <= kBatchWarmMaxBytes ? blocks : 0;
  return w;
}

void enqueue_batch_step_kernels(const BatchDeviceState& s, int splits) {
  const DeviceModel& m = *s.model;
  const auto& c = m.cfg;
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), Hkv = static_cast<int>(c.num_key_value_heads);
  const int F = static_cast<int>(c.intermediate_size), V = static_cast<int>(c.vocab_size);
  const int qkv_w = (Hq + 2 * Hkv) * D;
  const int B = static_cast<int>(s.batch);
  const int seq_stride = static_cast<int>(s.capacity + 1);
  const size_t L = m.layers.size();
  // K chunks of the split-K projections (as project / project_swiglu choose them).
  auto chunk = [&](int n, int k, int max_parts) { return B <= 32 ? proj_chunk(n, k, max_parts) : 0; };
  const int kc_qkv = chunk(qkv_w, H, qkv_max_parts(H)), kc_gu = chunk(2 * F, H, 0), kc_down = chunk(H, F, 0);
  const int kc_lm = chunk(V, H, 0);
  auto warm_qkv = [&](size_t l) {
    return warm_set(s.warm_blocks, {splitk_warm_region(m.layers[l].qkv, qkv_w, H, kc_qkv)});
  };
  check_hip(mmr::launch_batch_embed(m.embed, s.seq, seq_stride, s.pos, B, V, H, s.h, s.stream), "batch embed");
  const mmr::L2WarmSet warm0 = warm_qkv(0);
  check_hip(mmr::launch_batch_residual_norm(s.h, nullptr, 0, B, H, m.layers[0].input_norm, c.rms_norm_eps, s.x, false,
                                            s.stream, nullptr, &warm0),
            "batch input norm");
  for (size_t l = 0; l < L; ++l) {
    const LayerDev& Ld = m.layers[l];
    const int qkv_parts = project(s, s.x, Ld.qkv, qkv_w, H, qkv_max_parts(H));
    mmr::AttnArgs t;
    t.qkv = s.proj;
    t.qkv_stride = qkv_w;
    t.qkv_parts = qkv_parts;
    t.qkv_part_stride = static_cast<int64_t>(B) * qkv_w;
    t.q_norm = Ld.q_norm;
    t.k_norm = Ld.k_norm;
    t.eps = c.rms_norm_eps;
    t.inv_freq = m.inv_freq;
    t.pos = s.pos;
    t.kcache = s.kpool[l];
    t.vcache = s.vpool[l];
    t.capacity = static_cast<int>(s.capacity);
    t.rows = static_cast<int>(s.pages_per_seq * mmr::kKvPage);
    t.hq = Hq;
    t.hkv = Hkv;
    t.d = D;
    t.splits = splits;
    t.part = s.part;
    t.part_stride = s.part_stride;
    t.err = s.err;
    t.batch = B;
    t.page_table = s.page_table;
    t.pages_per_seq = static_cast<int>(s.pages_per_seq);
    t.page_interleave = B;  // the table's rule (set up in make_batch_state)
    check_hip(mmr::launch_attention(t, mmr::kAttnFused, s.kv, s.stream), "batch attention");
    const int o_parts = project_combine(s, splits, Ld.o, H, Hq, Hkv, D);
    const mmr::L2WarmSet warm_mlp = warm_set(s.warm_blocks, {splitk_warm_region(Ld.gate_up, 2 * F, H, kc_gu),
                                                             splitk_warm_region(Ld.down, H, F, kc_down)});
    check_hip(mmr::launch_batch_residual_norm(s.h, s.proj, o_parts, B, H, Ld.post_norm, c.rms_norm_eps, s.x, false,
                                              s.stream, nullptr, &warm_mlp),
              "batch residual + post norm");
    const int gu_parts = project(s, s.x, Ld.gate_up, 2 * F, H, 0, s.proj_gu);
    const int down_parts = project_swiglu(s, s.proj_gu, gu_parts, Ld.down, H, F);
    const bool last = l + 1 == L;
    const mmr::L2WarmSet warm_next =
        last ? warm_set(s.warm_blocks, {splitk_warm_region(m.lm_head, V, H, kc_lm)}) : warm_qkv(l + 1);
    check_hip(mmr::launch_batch_residual_norm(s.h, s.proj, down_parts, B, H,
                                              last ? m.final_norm : m.layers[l + 1].input_norm, c.rms_norm_eps, s.x,
                                              last, s.stream, nullptr, &warm_next),
              "batch residual + norm");
  }
  const int lm_parts = project(s, s.x, m.lm_head, V, H, 0);
  check_hip(mmr::launch_batch_head(s.proj, lm_parts, V, B, s.logits, s.token_out, s.seq, seq_stride, s.pos,
                                   s.prompt_len, seq_stride, s.stream),
            "batch logits + argmax");
}

// Floats of one projection's partial set: splits * batch * n.
int64_t parts_floats(int n, int k, int max_parts, int64_t batch) {
  const int kc = batch <= 32 ? proj_chunk(n, k, max_parts) : 0;
  const int64_t parts = kc > 0 ? (k + kc - 1) / kc : 1;
  return parts * batch * n;
}

// Floats of the projection partial buffer: the largest splits * batch * n of
// the step's projections.
int64_t proj_floats(const MiniMindConfig& c, int64_t batch) {
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int qkv_w = static_cast<int>((c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim);
  const int F = static_cast<int>(c.intermediate_size), V = static_cast<int>(c.vocab_size);
  const int qd = static_cast<int>(c.num_attention_heads) * D;
  const struct { int n, k, max_parts; } shapes[] = {
      {qkv_w, H, qkv_max_parts(H)}, {H, qd, 0}, {2 * F, H, 0}, {H, F, 0}, {V, H, 0}};
  int64_t most = 0;
  for (const auto& sh : shapes) most = std::max(most, parts_floats(sh.n, sh.k, sh.max_parts, batch));
  return most;
}

hipGraphExec_t capture_batch_step(BatchDeviceState& s, int splits) {
  hipGraph_t graph = nullptr;
  check_hip(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    enqueue_batch_step_kernels(s, splits);
  } catch (...) {
    (void)hipStreamEndCapture(s.stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    throw;
  }
  check_hip(hipStreamEndCapture(s.stream, &graph), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  check_hip(st, "hipGraphInstantiate");
  return exec;
}

}  // namespace

BatchState LanguageModel::make_batch_state(int64_t batch, int64_t capacity, KvCacheDtype kv) const {
  const auto& c = config_;
  const DeviceModel& m = *device_;
  if (batch < 1 || batch > 1024) throw std::invalid_argument("batch must be in [1, 1024]");
  if (capacity < 1 || capacity > c.max_position_embeddings)
    throw std::invalid_argument("batch capacity must be in [1, max_position_embeddings]");
  if (!m.gemm_prefill) throw std::invalid_argument("batched decode needs every projection's K to be a multiple of 8");
  auto s = std::make_unique<BatchDeviceState>();
  s->model = device_;
  s->kv = kv == KvCacheDtype::kFloat16 ? mmr::kKvF16 : mmr::kKvF32;
  s->batch = batch;
  s->capacity = capacity;
  s->pages_per_seq = (capacity + mmr::kKvPage - 1) / mmr::kKvPage;
  if (const char* wb = std::getenv("MMR_L2_WARM_BLOCKS"))
    s->warm_blocks = std::max(0, std::atoi(wb)) / mmr::kXcds * mmr::kXcds;
  const char* nog = std::getenv("MMR_NO_GRAPH");
  s->use_graphs = !(nog && nog[0] == '1');
  const int64_t H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
  const int64_t F = c.intermediate_size, V = c.vocab_size;
  const int64_t pages = batch * s->pages_per_seq;
  const std::size_t elem = s->kv == mmr::kKvF16 ? 2 : 4;
  const std::size_t pool_bytes = static_cast<std::size_t>(pages * Hkv * mmr::kKvPage * D) * elem;
  s->part_stride = static_cast<int64_t>(
      mmr::attention_partial_floats(static_cast<int>(Hq), static_cast<int>(Hkv), static_cast<int>(D), kBatchMaxSplits));
  Arena& ar = s->arena;
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    ar.plan(pool_bytes);
    ar.plan(pool_bytes);
  }
  ar.plan(pages * 4);
  ar.plan(batch * (capacity + 1) * 4);
  ar.plan(batch * 4 * 3 + 4);
  ar.plan(batch * H * 4 * 2);
  ar.plan(batch * (Hq + 2 * Hkv) * D * 4);
  ar.plan(batch * Hq * D * 4);
  ar.plan(batch * 2 * F * 4);
  ar.plan(batch * F * 4);
  ar.plan(batch * V * 4);
  ar.plan(batch * s->part_stride * 4);
  const int64_t proj = proj_floats(c, batch);
  ar.plan(proj * 4);
  const int64_t proj_gu = parts_floats(static_cast<int>(2 * c.intermediate_size), static_cast<int>(c.hidden_size), 0,
                                       batch);
  ar.plan(proj_gu * 4);
  ar.allocate();
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    s->kpool.push_back(ar.take<char>(pool_bytes));
    s->vpool.push_back(ar.take<char>(pool_bytes));
  }
  s->page_table = ar.take<int32_t>(pages);
  s->seq = ar.take<int32_t>(batch * (capacity + 1));
  int32_t* scalars = ar.take<int32_t>(batch * 3 + 1);
  s->pos = scalars;
  s->prompt_len = scalars + batch;
  s->token_out = scalars + 2 * batch;
  s->err = scalars + 3 * batch;
  float* hx = ar.take<float>(batch * H * 2);
  s->h = hx;
  s->x = hx + batch * H;
  s->qkv = ar.take<float>(batch * (Hq + 2 * Hkv) * D);
  s->attn = ar.take<float>(batch * Hq * D);
  s->gu = ar.take<float>(batch * 2 * F);
  s->act = ar.take<float>(batch * F);
  s->logits = ar.take<float>(batch * V);
  s->part = ar.take<float>(batch * s->part_stride);
  s->proj = ar.take<float>(proj);
  s->proj_gu = ar.take<float>(proj_gu);
  s->staging_len = std::max<int64_t>(pages, batch * (capacity + 1)) + 4 * batch + 8;
  check_hip(hipHostMalloc(reinterpret_cast<void**>(&s->staging), s->staging_len * sizeof(int32_t),
                          hipHostMallocDefault),
            "hipHostMalloc staging");
  check_hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
  // Page p of sequence b is physical page p * batch + b.
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t p = 0; p < s->pages_per_seq; ++p)
      s->staging[b * s->pages_per_seq + p] = static_cast<int32_t>(p * batch + b);
  check_hip(hipMemcpyAsync(s->page_table, s->staging, pages * sizeof(int32_t), hipMemcpyHostToDevice, s->stream),
            "hipMemcpyAsync page table");
  check_hip(hipMemsetAsync(scalars, 0, (batch * 3 + 1) * sizeof(int32_t), s->stream), "hipMemsetAsync");
  check_hip(hipMemsetAsync(s->seq, 0, batch * (capacity + 1) * sizeof(int32_t), s->stream), "hipMemsetAsync");
  check_hip(hipStreamSynchronize(s->stream), "batch state init");
  BatchState state;
  state.device = std::move(s);
  return state;
}

void LanguageModel::launch_batch_step(BatchState& state) const {
  BatchDeviceState& s = *state.device;
  if (state.steps >= s.capacity) throw std::length_error("KV cache capacity exhausted");
  const int splits = batch_splits(state.steps + 1, mmr::attention_tile_tokens(static_cast<int>(config_.head_dim)),
                                  s.batch * config_.num_key_value_heads);
  if (s.use_graphs) {
    auto it = s.graphs.find(splits);
    if (it == s.graphs.end()) it = s.graphs.emplace(splits, capture_batch_step(s, splits)).first;
    check_hip(hipGraphLaunch(it->second, s.stream), "hipGraphLaunch");
  } else {
    enqueue_batch_step_kernels(s, splits);
  }
  state.steps += 1;
}

void LanguageModel::enqueue_batch_prefill(BatchState& state, const std::vector<std::vector<int32_t>>& prompts) const {
  BatchDeviceState& s = *state.device;
  if (static_cast<int64_t>(prompts.size()) != s.batch) throw std::invalid_argument("one prompt per sequence");
  if (state.steps != 0) throw std::invalid_argument("batch prefill requires empty KV caches");
  int64_t longest = 0;
  for (const auto& p : prompts) {
    if (p.empty()) throw std::invalid_argument("prompt_tokens cannot be empty");
    for (int32_t t : p)
      if (t < 0 || t >= config_.vocab_size) throw std::out_of_range("token id out of vocabulary range");
    longest = std::max<int64_t>(longest, static_cast<int64_t>(p.size()));
  }
  if (longest > s.capacity) throw std::length_error("KV cache capacity exhausted");
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  const int64_t stride = s.capacity + 1;
  std::memset(s.staging, 0, static_cast<std::size_t>(s.batch * stride) * sizeof(int32_t));
  int32_t* lens = s.staging + s.batch * stride;
  for (int64_t b = 0; b < s.batch; ++b) {
    std::memcpy(s.staging + b * stride, prompts[b].data(), prompts[b].size() * sizeof(int32_t));
    lens[b] = static_cast<int32_t>(prompts[b].size());
  }
  check_hip(hipMemcpyAsync(s.seq, s.staging, s.batch * stride * sizeof(int32_t), hipMemcpyHostToDevice, s.stream),
            "hipMemcpyAsync prompts");
  check_hip(hipMemcpyAsync(s.prompt_len, lens, s.batch * sizeof(int32_t), hipMemcpyHostToDevice, s.stream),
            "hipMemcpyAsync prompt lengths");
  check_hip(hipMemsetAsync(s.pos, 0, s.batch * sizeof(int32_t), s.stream), "hipMemsetAsync pos");
  for (int64_t i = 0; i < longest; ++i) launch_batch_step(state);
}

void LanguageModel::enqueue_batch_decode(BatchState& state, int64_t n) const {
  BatchDeviceState& s = *state.device;
  if (n < 0) throw std::invalid_argument("step count cannot be negative");
  if (state.steps == 0) throw std::invalid_argument("batch decode needs prompts (enqueue_batch_prefill)");
  if (state.steps + n > s.capacity) throw std::length_error("KV cache capacity exhausted");
  for (int64_t i = 0; i < n; ++i) launch_batch_step(state);
}

void LanguageModel::synchronize(BatchState& state) const {
  BatchDeviceState& s = *state.device;
  int32_t* flag = s.staging + s.staging_len - 1;
  check_hip(hipMemcpyAsync(flag, s.err, sizeof(int32_t), hipMemcpyDeviceToHost, s.stream), "hipMemcpyAsync err");
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  if (*flag != 0) throw std::runtime_error("device kernel reported an out-of-range position");
}

std::vector<int32_t> LanguageModel::read_batch_sequence(BatchState& state, int64_t index, int64_t first,
                                                        int64_t count) const {
  BatchDeviceState& s = *state.device;
  if (index < 0 || index >= s.batch) throw std::out_of_range("sequence index");
  if (first < 0 || count < 0 || first + count > s.capacity + 1) throw std::out_of_range("sequence range");
  std::vector<int32_t> out(static_cast<size_t>(count));
  if (count == 0) return out;
  synchronize(state);
  check_hip(hipMemcpyAsync(s.staging, s.seq + index * (s.capacity + 1) + first, count * sizeof(int32_t),
                           hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync seq");
  synchronize(state);
  std::memcpy(out.data(), s.staging, count * sizeof(int32_t));
  return out;
}

std::vector<float> LanguageModel::read_batch_logits(BatchState& state, int64_t index) const {
  BatchDeviceState& s = *state.device;
  if (index < 0 || index >= s.batch) throw std::out_of_range("sequence index");
  std::vector<float> out(static_cast<size_t>(config_.vocab_size));
  synchronize(state);
  check_hip(hipMemcpyAsync(out.data(), s.logits + index * config_.vocab_size, out.size() * sizeof(float),
                           hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync logits");
  synchronize(state);
  return out;
}

}  // namespace minimind::model
