// language_model.cpp -- device-resident decode step and the reference-shaped
// model API on top of it.
//
// One decode step (language_model.cpp:310-333 + decoder_layer.cpp:312-407 of
// the reference) is 5 kernels per layer plus two for the head:
//   qkv   GEMV  RMSNorm prologue (layer 0: embedding gather of seq[pos])
//   attn        q/k RMSNorm + RoPE, K/V append at pos, split-context GQA
//               attention writing per-split (m, l, o) partials
//   o     GEMV  log-sum-exp combine of the partials in the prologue,
//               residual epilogue (h += W_o attn)
//   gu    GEMV  RMSNorm prologue, SwiGLU epilogue over interleaved gate/up rows
//   down  GEMV  residual epilogue  (h += W_down act)
//   head  GEMV  final RMSNorm prologue, per-block argmax partials, then the
//               finalize kernel writes seq[pos + 1] and advances pos
// Every kernel reads the position from device memory, so groups of 8 steps are
// captured once into a hipGraph (per attention split count) and replayed;
// inside a group the finalize runs after the last step only (the others fold
// it into the lm_head launch and the next step's layer-0 prologue), and the
// attention launch also warms the L2s with the layer's O, gate_up and down
// weights.
// Prompts run through the chunked prefill kernels (enqueue_prefill).
#include "language_model.h"

#include "device.h"
#include "decoder_layer.h"
#include "device_model.h"
#include "kv_store.h"
#include "prefill_layer.h"
#include "../kernels/kernels.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <map>
#include <stdexcept>

namespace minimind::model {

// L2 warming in the single-sequence step (the attention launch loads the
// layer's O, gate_up and down weights for the XCDs that will read them): the
// warming blocks fill the CUs the head blocks leave idle, up to kWarmBlocks
// (MiniMind2 at 768 keys, 128 head blocks: 96 or 128 warming blocks 255.2 us
// per step, 64: 261.4, none: 263.5); regions above half the 32 MB of L2 are
// not warmed.  Past 16 attention splits the split-merge launch carries them
// instead and takes every CU its 48 merge blocks leave idle (kMergeWarmBlocks:
// at 8,192 / 4,096 keys 208 blocks 341.5 / 312.9 us per step against 343.9 /
// 314.3 with 128, same box).  MMR_L2_WARM_BLOCKS overrides both caps.
constexpr int kWarmBlocks = 128;
constexpr int kMergeWarmBlocks = 1 << 20;  // no cap beyond the idle CUs
constexpr int64_t kWarmMaxBytes = int64_t{16} << 20;

struct DeviceState {
  std::shared_ptr<const DeviceModel> model;
  mmr::KvDtype kv = mmr::kKvF32;
  int64_t capacity = 0;
  Arena arena;
  // The KV cache: 64-token pages in doubling segments, backed as the context
  // grows (ensure_backed); the small-model kernel keeps [Hkv][capacity][d]
  // per layer in the arena instead (tiny_k / tiny_v).
  KvStore kv_store;
  std::vector<void*> tiny_k, tiny_v;
  int32_t* seq = nullptr;  // [capacity + 1]
  int32_t* pos = nullptr;
  int32_t* prompt_len = nullptr;
  int32_t* err = nullptr;
  int32_t* token_out = nullptr;
  float* h = nullptr;
  float* qkv = nullptr;
  float* attn = nullptr;
  float* act = nullptr;
  float* logits = nullptr;
  mmr::TinyLayerPtrs* tiny_layers = nullptr;  // small-model path: per-layer weights and caches
  float* attn_part = nullptr;  // split partials: o [Hkv][splits][R][d], then (m, l) [Hkv][splits][R][2]
  float* lm_part_val = nullptr;  // per-block argmax partials of the head GEMV
  int* lm_part_idx = nullptr;
  int32_t* staging = nullptr;        // pinned host [capacity + 8]
  // Prefill chunk buffers (rows = prompt tokens of one chunk, <= pf_chunk).
  int64_t pf_chunk = 0;
  float* pf_h = nullptr;    // [chunk][H] residual stream
  PrefillScratch pf;        // the layer's scratch for pf_chunk rows
  bool prefill_tokenwise = false;  // prefill through the decode step instead of the GEMM path
  hipStream_t stream = nullptr;
  std::map<std::pair<int, int>, hipGraphExec_t> graphs;  // (attention splits, steps) -> captured steps
  bool use_graphs = true;
  bool combine_kernel = false;  // merge attention splits in a separate kernel, not the O prologue
  // L2-warming blocks of the single-sequence attention launch (0 = none) and
  // the GPU's CU count, which bounds head blocks + warming blocks.
  int warm_blocks = kWarmBlocks;
  int merge_warm_blocks = kMergeWarmBlocks;  // the same for the split-merge launch
  int cus = 0;

  ~DeviceState() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
    if (stream) (void)hipStreamDestroy(stream);
    if (staging) (void)hipHostFree(staging);
  }
};

namespace {

// Attention split counts: the step graph is captured per split count, so the
// count only changes at bucket boundaries, and one tile per split up to
// kMaxSplits.  A split past the context's last tile still issues its
// speculative first-tile load (the kernel reads the position after its loads
// are out), so the buckets are kept close to the tile count: 8, 12, 16, then
// multiples of 8 (of 32 past 256 tiles).  Measured with FETCH_SIZE at 768
// keys (12 tiles): 16 splits fetched 1.54x the K/V bytes, 4 idle splits'
// loads being most of the excess.  Multiples of 8 rather than 16 from 129 to
// 256 tiles took the step at 8,192 keys from 345.1 to 343.6 us (136 splits
// against 144, same box).  The count never falls as the context grows
// (decode_attention_splits).
constexpr int kMaxSplits = 512;
// Prompt tokens per prefill chunk (GEMM rows); longer prompts run in chunks.
constexpr int64_t kPrefillChunk = 512;

void require_size(const std::vector<float>& v, int64_t expected, const std::string& name) {
  if (static_cast<int64_t>(v.size()) != expected) throw std::invalid_argument(name + " has invalid size");
}

// Up to kPrologueTiles tiles the step keeps 16 splits (two tiles for some
// blocks, the next one prefetched), so the O-projection prologue merges them
// and no combine kernel runs; beyond, one tile per split.  Measured per step
// (MiniMind2, f32 KV): 1024 keys 386 -> 368 us with the 16-split cap, 2048 keys
// 391 us with one tile per split against 405 us capped.
constexpr int64_t kPrologueTiles = 24;

// Decode steps per replayed graph in enqueue_decode.
constexpr int kGraphSteps = 8;

int choose_splits(int64_t n_keys, int tile) {
  const int64_t n_tiles = (n_keys + tile - 1) / tile;
  if (n_tiles <= 8) return 8;
  if (n_tiles <= 12) return 12;
  if (n_tiles <= kPrologueTiles) return mmr::kCombineMaxSplits;
  if (n_tiles >= kMaxSplits) return kMaxSplits;
  const int64_t step = n_tiles <= 256 ? 8 : 32;
  return static_cast<int>((n_tiles + step - 1) / step * step);
}

std::vector<uint16_t> to_half(const std::vector<float>& v) {
  std::vector<uint16_t> out(v.size());
  for (size_t i = 0; i < v.size(); ++i) out[i] = float_to_half(v[i]);
  return out;
}

template <typename T>
T* upload(Arena& arena, const void* host, std::size_t count) {
  T* dst = arena.take<T>(count);
  check_hip(hipMemcpy(dst, host, count * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy weights");
  return dst;
}


}  // namespace

// ------------------------------------------------------------------ state --

DecoderState::DecoderState() = default;
DecoderState::~DecoderState() = default;
DecoderState::DecoderState(DecoderState&&) noexcept = default;
DecoderState& DecoderState::operator=(DecoderState&&) noexcept = default;
int64_t DecoderState::capacity() const { return device ? device->capacity : 0; }
int64_t DecoderState::kv_backed() const {
  if (!device) return 0;
  return device->model->tiny ? device->capacity : std::min(device->capacity, device->kv_store.backed());
}
std::size_t DecoderState::kv_device_bytes() const {
  if (!device) return 0;
  if (!device->model->tiny) return device->kv_store.device_bytes();
  const auto& c = device->model->cfg;
  return static_cast<std::size_t>(2 * c.num_hidden_layers * c.num_key_value_heads * device->capacity * c.head_dim) *
         (device->kv == mmr::kKvF16 ? 2 : 4);
}
KvCacheDtype DecoderState::kv_dtype() const {
  return device && device->kv == mmr::kKvF16 ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32;
}
void* DecoderState::stream() const { return device ? static_cast<void*>(device->stream) : nullptr; }

// ------------------------------------------------------------------ model --

LanguageModel::LanguageModel(MiniMindConfig config, DenseModelWeights weights) : config_(std::move(config)) {
  const auto errors = validate_config(config_);
  if (!errors.empty()) throw std::invalid_argument("invalid MiniMind config: " + errors.front());
  const auto dev_errors = validate_device_config(config_);
  const auto& c = config_;
  // Shapes the GEMV / attention kernels do not take run through the
  // one-workgroup step kernel when they fit it (the reference's toy model).
  const bool tiny = !dev_errors.empty() && !c.use_moe &&
                    mmr::tiny_step_supported(static_cast<int>(c.hidden_size), static_cast<int>(c.num_attention_heads),
                                             static_cast<int>(c.num_key_value_heads), static_cast<int>(c.head_dim),
                                             static_cast<int>(c.intermediate_size), static_cast<int>(c.vocab_size), 1);
  if (!dev_errors.empty() && !tiny)
    throw std::invalid_argument("unsupported by the gfx950 runtime: " + dev_errors.front());
  const int64_t H = c.hidden_size, V = c.vocab_size, D = c.head_dim, F = c.intermediate_size;
  const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
  require_size(weights.embed_tokens, V * H, "embed_tokens");
  require_size(weights.final_norm, H, "final_norm");
  require_size(weights.lm_head, V * H, "lm_head");
  if (static_cast<int64_t>(weights.layers.size()) != c.num_hidden_layers)
    throw std::invalid_argument("layer weight count does not match config");
  for (const auto& L : weights.layers) check_layer_weights(c, L);

  auto dm = std::make_shared<DeviceModel>();
  dm->cfg = c;
  dm->tiny = tiny;
  const bool share_head = weights.lm_head == weights.embed_tokens;
  const int64_t half_d = D / 2;
  Arena& ar = dm->arena;
  ar.plan(V * H * 2);
  if (!share_head) ar.plan(V * H * 2);
  ar.plan(H * 4);
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) ar.plan(plan_layer_bytes(c));
  ar.plan(half_d * 4);
  ar.allocate();

  dm->embed = upload<__half>(ar, to_half(weights.embed_tokens).data(), V * H);
  dm->lm_head = share_head ? dm->embed : upload<__half>(ar, to_half(weights.lm_head).data(), V * H);
  dm->final_norm = upload<float>(ar, weights.final_norm.data(), H);
  std::size_t wbytes = V * H * 2 * (share_head ? 1 : 2) + H * 4;
  for (const auto& L : weights.layers) {
    dm->layers.push_back(upload_layer(ar, c, L));
    wbytes += 2 * H * 4 + 2 * D * 4 + ((qs + 2 * kvs) * H + H * qs + 2 * F * H + H * F) * 2;
  }
  // RoPE frequencies with the reference formula (decoder_layer.cpp:114); the
  // kernels evaluate cos/sin(float(pos) * inv_freq) on the device.
  {
    const std::vector<float> inv = rope_inv_freq(c);
    dm->inv_freq = upload<float>(ar, inv.data(), inv.size());
  }
  dm->weight_bytes = wbytes;
  if (tiny) {
    check_hip(hipDeviceSynchronize(), "weight upload");
    device_ = std::move(dm);
    return;
  }
  const LayerPlans lp = plan_layer(c);
  dm->plan_qkv = lp.qkv;
  dm->plan_o = lp.o;
  dm->plan_gu = lp.gate_up;
  dm->plan_down = lp.down;
  if (!mmr::gemv_plan(static_cast<int>(V), static_cast<int>(H), mmr::kEpiArgmax, 0, 0, &dm->plan_lm))
    throw std::invalid_argument("unsupported GEMV shape for lm_head");
  dm->gemm_prefill = mmr::gemm_supported(1, static_cast<int>(qs + 2 * kvs), static_cast<int>(H)) &&
                     mmr::gemm_supported(1, static_cast<int>(H), static_cast<int>(qs)) &&
                     mmr::gemm_supported(1, static_cast<int>(2 * F), static_cast<int>(H)) &&
                     mmr::gemm_supported(1, static_cast<int>(H), static_cast<int>(F));
  check_hip(hipDeviceSynchronize(), "weight upload");
  device_ = std::move(dm);
}

LanguageModel::~LanguageModel() = default;
LanguageModel::LanguageModel(LanguageModel&&) noexcept = default;
LanguageModel& LanguageModel::operator=(LanguageModel&&) noexcept = default;

std::size_t LanguageModel::device_weight_bytes() const { return device_->weight_bytes; }

int decode_attention_splits(int64_t n_keys, int tile) { return choose_splits(n_keys, tile); }

int64_t prefill_partial_floats(const MiniMindConfig& c, int64_t chunk_rows) {
  const int64_t H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
  const int64_t F = c.intermediate_size;
  const int64_t shapes[4][2] = {{(Hq + 2 * Hkv) * D, H}, {H, Hq * D}, {2 * F, H}, {H, F}};  // {N, K}
  int64_t most = 0;
  for (const auto& nk : shapes)
    for (int64_t r = 1; r <= chunk_rows; ++r) {
      const int splits = mmr::gemm_k_splits(static_cast<int>(r), static_cast<int>(nk[0]), static_cast<int>(nk[1]));
      most = std::max<int64_t>(most, int64_t{splits} * r * nk[0]);
    }
  return most;
}

DecoderState LanguageModel::make_state() const { return make_state(0, KvCacheDtype::kFloat32); }

DecoderState LanguageModel::make_state(int64_t capacity, KvCacheDtype kv) const {
  const auto& c = config_;
  // A small model's step kernel evaluates RoPE at any position, as the
  // reference CPU path does, so its states are bounded by the kernel's LDS
  // (kTinyMaxContext) rather than by max_position_embeddings (16 for the toy).
  const bool tiny = device_->tiny;
  const int64_t limit = tiny ? mmr::kTinyMaxContext : c.max_position_embeddings;
  if (capacity <= 0) capacity = limit;
  if (capacity > limit)
    throw std::invalid_argument(tiny ? "state capacity exceeds the small-model step kernel's 2048 positions"
                                     : "state capacity exceeds max_position_embeddings");
  auto s = std::make_unique<DeviceState>();
  s->model = device_;
  s->kv = kv == KvCacheDtype::kFloat16 ? mmr::kKvF16 : mmr::kKvF32;
  s->capacity = capacity;
  const char* nog = std::getenv("MMR_NO_GRAPH");
  s->use_graphs = !(nog && nog[0] == '1');
  const char* ck = std::getenv("MMR_COMBINE_KERNEL");
  s->combine_kernel = ck && ck[0] == '1';
  const char* pt = std::getenv("MMR_PREFILL_TOKENWISE");
  s->prefill_tokenwise = (pt && pt[0] == '1') || !device_->gemm_prefill;
  const char* rs = std::getenv("MMR_GEMM_REGISTER_STAGED");
  s->pf.register_staged = rs && rs[0] == '1';
  if (const char* wb = std::getenv("MMR_L2_WARM_BLOCKS"))
    s->warm_blocks = s->merge_warm_blocks = std::max(0, std::atoi(wb)) / mmr::kXcds * mmr::kXcds;
  {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    check_hip(hipDeviceGetAttribute(&s->cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
  }
  const int64_t H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
  const int64_t F = c.intermediate_size, V = c.vocab_size;
  const std::size_t kv_elem = s->kv == mmr::kKvF16 ? 2 : 4;
  // Small models: one [Hkv][capacity][d] block per layer for K and V.
  const std::size_t tiny_cache_bytes = tiny ? static_cast<std::size_t>(Hkv * capacity * D) * kv_elem : 0;
  Arena& ar = s->arena;
  for (int64_t l = 0; l < c.num_hidden_layers && tiny; ++l) {
    ar.plan(tiny_cache_bytes);
    ar.plan(tiny_cache_bytes);
  }
  const std::size_t part_floats =
      tiny ? 0 : mmr::attention_partial_floats(static_cast<int>(Hq), static_cast<int>(Hkv), static_cast<int>(D), kMaxSplits);
  const std::size_t tiny_bytes = tiny ? c.num_hidden_layers * sizeof(mmr::TinyLayerPtrs) : 0;
  ar.plan(tiny_bytes);
  ar.plan((capacity + 1) * 4);
  ar.plan(4 * 4);  // pos, prompt_len, err, token_out
  ar.plan(H * 4);
  ar.plan((Hq * D + 2 * Hkv * D) * 4);
  ar.plan(Hq * D * 4);
  ar.plan(F * 4);
  ar.plan(V * 4);
  ar.plan(part_floats * 4);
  ar.plan(device_->plan_lm.blocks * 4);
  ar.plan(device_->plan_lm.blocks * 4);
  int64_t chunk = kPrefillChunk;
  if (const char* pc = std::getenv("MMR_PREFILL_CHUNK")) chunk = std::max<int64_t>(1, std::atoll(pc));
  s->pf_chunk = s->prefill_tokenwise ? 0 : std::min<int64_t>(capacity, chunk);
  const int64_t C = s->pf_chunk;
  const std::size_t pf_bytes = C > 0 ? prefill_scratch_bytes(c, C) : 0;
  if (C > 0) {
    ar.plan(C * H * 4);
    ar.plan(pf_bytes);
  }
  ar.allocate();
  for (int64_t l = 0; l < c.num_hidden_layers && tiny; ++l) {
    s->tiny_k.push_back(ar.take<char>(tiny_cache_bytes));
    s->tiny_v.push_back(ar.take<char>(tiny_cache_bytes));
  }
  if (!tiny) {
    // Up front only the first segment (512 positions); later segments are
    // added as the context reaches them.
    s->kv_store = KvStore(c.num_hidden_layers, Hkv, D, s->kv, capacity);
    s->kv_store.reserve(std::min<int64_t>(capacity, mmr::kv_segment_tokens(0)));
  }
  s->seq = ar.take<int32_t>(capacity + 1);
  int32_t* scalars = ar.take<int32_t>(4);
  s->pos = scalars;
  s->prompt_len = scalars + 1;
  s->err = scalars + 2;
  s->token_out = scalars + 3;
  s->h = ar.take<float>(H);
  s->qkv = ar.take<float>(Hq * D + 2 * Hkv * D);
  s->attn = ar.take<float>(Hq * D);
  s->act = ar.take<float>(F);
  s->logits = ar.take<float>(V);
  s->attn_part = ar.take<float>(part_floats);
  s->lm_part_val = ar.take<float>(device_->plan_lm.blocks);
  s->lm_part_idx = ar.take<int>(device_->plan_lm.blocks);
  s->tiny_layers = tiny ? ar.take<mmr::TinyLayerPtrs>(static_cast<std::size_t>(c.num_hidden_layers)) : nullptr;
  if (C > 0) {
    s->pf_h = ar.take<float>(C * H);
    const bool staged = s->pf.register_staged;
    s->pf = carve_prefill_scratch(c, C, ar.take<char>(pf_bytes));
    s->pf.register_staged = staged;
  }
  if (tiny) {
    std::vector<mmr::TinyLayerPtrs> table(static_cast<std::size_t>(c.num_hidden_layers));
    for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
      const LayerDev& L = device_->layers[static_cast<std::size_t>(l)];
      auto& t = table[static_cast<std::size_t>(l)];
      t.input_norm = L.input_norm;
      t.post_norm = L.post_norm;
      t.q_norm = L.q_norm;
      t.k_norm = L.k_norm;
      t.qkv = L.qkv;
      t.o = L.o;
      t.gate_up = L.gate_up;
      t.down = L.down;
      t.kcache = s->tiny_k[static_cast<std::size_t>(l)];
      t.vcache = s->tiny_v[static_cast<std::size_t>(l)];
    }
    check_hip(hipMemcpy(s->tiny_layers, table.data(), tiny_bytes, hipMemcpyHostToDevice), "hipMemcpy layer table");
  }
  check_hip(hipHostMalloc(reinterpret_cast<void**>(&s->staging), (capacity + 8) * sizeof(int32_t),
                          hipHostMallocDefault),
            "hipHostMalloc staging");
  check_hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
  check_hip(hipMemsetAsync(scalars, 0, 4 * sizeof(int32_t), s->stream), "hipMemsetAsync");

  check_hip(hipMemsetAsync(s->seq, 0, (capacity + 1) * sizeof(int32_t), s->stream), "hipMemsetAsync");
  check_hip(hipStreamSynchronize(s->stream), "state init");
  DecoderState state;
  state.device = std::move(s);
  state.position = 0;
  return state;
}

namespace {

enum StepKernel : int { kQkv = 0, kAttention = 1, kOProj = 2, kGateUp = 3, kDown = 4, kHead = 5, kFinalize = 6 };

// One kernel (or, for kOProj with many splits, the combine + GEMV pair) of
// the decode step; `bookkeeping` (finalize only) lets it write seq[pos + 1]
// and advance the device position.
// The bytes each block of a GEMV launch with plan p reads (W fp16 [rows][k],
// rows in consecutive runs per block), as an L2-warming region; unused when
// the region's byte offsets do not fit 32 bits.
mmr::L2Warm gemv_warm_region(const __half* w, int rows, int k, const mmr::GemvPlan& p) {
  mmr::L2Warm r;
  const int64_t row_bytes = int64_t{k} * 2;
  const int64_t bytes = rows * row_bytes;
  const int rows_per_block = mmr::kGemvBlock / p.lanes_per_row * p.rows_per_group;
  if (bytes + rows_per_block * row_bytes >= (int64_t{1} << 32)) return r;
  r.base = w;
  r.bytes = static_cast<uint32_t>(bytes);
  r.row_bytes = static_cast<uint32_t>(row_bytes);
  r.seg_bytes = r.row_bytes;
  r.rows = rows_per_block;
  r.units_x = p.blocks;
  return r;
}

// Whether the O-projection GEMV's prologue merges the attention splits (else
// attention_combine_kernel runs first).
bool prologue_combines(const DeviceState& s, int splits) {
  const auto& c = s.model->cfg;
  const int64_t Hq = c.num_attention_heads;
  return !s.combine_kernel && splits <= mmr::kCombineMaxSplits && Hq <= mmr::kCombineMaxHeads &&
         Hq * c.head_dim <= mmr::kCombineMaxDim;
}

// L2 warming of layer L's O, gate_up and down weights by up to `cap` blocks
// on `idle_cus` CUs (rounded down to whole XCD rounds); none when the regions
// would pass kWarmMaxBytes (they must fit the L2s with room to spare).
mmr::L2WarmSet layer_warm_set(const DeviceState& s, const LayerDev& L, int idle_cus, int cap) {
  const DeviceModel& m = *s.model;
  const auto& c = m.cfg;
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), F = static_cast<int>(c.intermediate_size);
  mmr::L2WarmSet w;
  const int blocks = std::min(cap, std::max(0, idle_cus) / mmr::kXcds * mmr::kXcds);
  if (blocks <= 0) return w;
  w.region[0] = gemv_warm_region(L.o, H, Hq * D, m.plan_o);
  w.region[1] = gemv_warm_region(L.gate_up, 2 * F, H, m.plan_gu);
  w.region[2] = gemv_warm_region(L.down, H, F, m.plan_down);
  int64_t bytes = 0;
  for (const auto& r : w.region) bytes += r.bytes;
  if (bytes > kWarmMaxBytes) return mmr::L2WarmSet{};
  w.blocks = blocks;
  return w;
}

// A step's place in a replayed group of steps: inside a group the argmax
// finalize of every step but the last folds into the next step (its layer-0
// qkv prologue reduces the lm_head partials; the lm_head launch advances the
// position).
struct StepLink {
  bool token_from_partials = false;  // layer-0 qkv: token from the previous step's lm_head partials
  bool advance_in_head = false;      // lm_head: advance the position (no finalize follows)
};

void enqueue_kernel(const DeviceState& s, int kernel, size_t l, int splits, bool bookkeeping, StepLink link = {}) {
  const DeviceModel& m = *s.model;
  const auto& c = m.cfg;
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), Hkv = static_cast<int>(c.num_key_value_heads);
  const int F = static_cast<int>(c.intermediate_size), V = static_cast<int>(c.vocab_size);
  const int qkv_rows = (Hq + 2 * Hkv) * D;
  const LayerDev& L = m.layers[l];
  switch (kernel) {
    case kQkv: {
      mmr::GemvArgs a;
      a.w = L.qkv;
      a.rows = qkv_rows;
      a.k = H;
      a.x = s.h;
      a.norm_w = L.input_norm;
      a.eps = c.rms_norm_eps;
      a.y = s.qkv;
      mmr::GemvPrologue pro = mmr::kProRmsNorm;
      if (l == 0) {
        pro = mmr::kProEmbedRmsNorm;
        a.embed = m.embed;
        a.seq = s.seq;
        a.pos = s.pos;
        a.vocab = V;
        a.h_out = s.h;
        if (link.token_from_partials) {
          a.prev_val = s.lm_part_val;
          a.prev_idx = s.lm_part_idx;
          a.prev_parts = m.plan_lm.blocks;
          a.prompt_len = s.prompt_len;
          a.seq_out = s.seq;
          a.seq_len = static_cast<int>(s.capacity + 1);
        }
      }
      check_hip(mmr::launch_gemv(a, pro, mmr::kEpiStore, m.plan_qkv, s.stream), "qkv gemv");
      return;
    }
    case kAttention: {
      mmr::AttnArgs t;
      t.qkv = s.qkv;
      t.q_norm = L.q_norm;
      t.k_norm = L.k_norm;
      t.eps = c.rms_norm_eps;
      t.inv_freq = m.inv_freq;
      t.pos = s.pos;
      t.seg = s.kv_store.layer(static_cast<int64_t>(l));
      // Positions past the backed rows are flagged, never read (the launcher
      // backs every position a launch can reach before it captures or runs it).
      t.capacity = static_cast<int>(std::min(s.capacity, s.kv_store.backed()));
      t.rows = static_cast<int>(s.kv_store.backed());
      t.hq = Hq;
      t.hkv = Hkv;
      t.d = D;
      t.splits = splits;
      t.part = s.attn_part;
      t.err = s.err;
      // While the head blocks run on part of the GPU, extra blocks on the idle
      // CUs load this layer's O, gate_up and down weights into the L2s of the
      // XCDs whose blocks will read them.  (Past the prologue's splits the
      // combine launch warms instead.)
      if (prologue_combines(s, splits)) t.warm = layer_warm_set(s, L, s.cus - splits * Hq, s.warm_blocks);
      check_hip(mmr::launch_attention(t, mmr::kAttnFused, s.kv, s.stream), "attention");
      return;
    }
    case kOProj: {
      mmr::GemvArgs a;
      a.w = L.o;
      a.rows = H;
      a.k = Hq * D;
      a.y = s.h;
      a.residual = s.h;
      mmr::GemvPrologue pro = mmr::kProPlain;
      if (prologue_combines(s, splits)) {
        pro = mmr::kProAttnCombine;
        a.part = s.attn_part;
        a.splits = splits;
        a.hq = Hq;
        a.hkv = Hkv;
        a.head_dim = D;
      } else {
        const int merge_blocks = Hq * ((D + 15) / 16);  // one per head and 16-dimension slice
        const mmr::L2WarmSet warm = layer_warm_set(s, L, s.cus - merge_blocks, s.merge_warm_blocks);
        check_hip(mmr::launch_attention_combine(s.attn_part, Hq, Hkv, D, splits, s.attn, s.stream, 1, 0, &warm),
                  "attention combine");
        a.x = s.attn;
      }
      check_hip(mmr::launch_gemv(a, pro, mmr::kEpiResidual, m.plan_o, s.stream), "o gemv");
      return;
    }
    case kGateUp: {
      mmr::GemvArgs a;
      a.w = L.gate_up;
      a.rows = 2 * F;
      a.k = H;
      a.x = s.h;
      a.norm_w = L.post_norm;
      a.eps = c.rms_norm_eps;
      a.y = s.act;
      check_hip(mmr::launch_gemv(a, mmr::kProRmsNorm, mmr::kEpiSwiGlu, m.plan_gu, s.stream), "gate_up gemv");
      return;
    }
    case kDown: {
      mmr::GemvArgs a;
      a.w = L.down;
      a.rows = H;
      a.k = F;
      a.x = s.act;
      a.y = s.h;
      a.residual = s.h;
      check_hip(mmr::launch_gemv(a, mmr::kProPlain, mmr::kEpiResidual, m.plan_down, s.stream), "down gemv");
      return;
    }
    case kHead: {
      mmr::GemvArgs a;
      a.w = m.lm_head;
      a.rows = V;
      a.k = H;
      a.x = s.h;
      a.norm_w = m.final_norm;
      a.eps = c.rms_norm_eps;
      a.y = s.logits;
      a.part_val = s.lm_part_val;
      a.part_idx = s.lm_part_idx;
      if (link.advance_in_head) a.advance_pos = s.pos;
      check_hip(mmr::launch_gemv(a, mmr::kProRmsNormFinal, mmr::kEpiArgmax, m.plan_lm, s.stream), "lm_head gemv");
      return;
    }
    case kFinalize: {
      mmr::ArgmaxFinalizeArgs f;
      f.part_val = s.lm_part_val;
      f.part_idx = s.lm_part_idx;
      f.parts = m.plan_lm.blocks;
      f.token_out = s.token_out;
      if (bookkeeping) {
        f.seq = s.seq;
        f.pos = s.pos;
        f.prompt_len = s.prompt_len;
        f.seq_len = static_cast<int>(s.capacity + 1);
      }
      check_hip(mmr::launch_argmax_finalize(f, s.stream), "argmax finalize");
      return;
    }
    default:
      throw std::invalid_argument("unknown step kernel");
  }
}

// The whole step of a small model in one launch (tiny.hip).
void enqueue_tiny_step(const DeviceState& s) {
  const DeviceModel& m = *s.model;
  const auto& c = m.cfg;
  mmr::TinyStepArgs a;
  a.embed = m.embed;
  a.lm_head = m.lm_head;
  a.final_norm = m.final_norm;
  a.layers = s.tiny_layers;
  a.n_layers = static_cast<int>(c.num_hidden_layers);
  a.inv_freq = m.inv_freq;
  a.hidden = static_cast<int>(c.hidden_size);
  a.hq = static_cast<int>(c.num_attention_heads);
  a.hkv = static_cast<int>(c.num_key_value_heads);
  a.d = static_cast<int>(c.head_dim);
  a.f = static_cast<int>(c.intermediate_size);
  a.vocab = static_cast<int>(c.vocab_size);
  a.eps = c.rms_norm_eps;
  a.rows = static_cast<int>(s.capacity);
  a.capacity = static_cast<int>(s.capacity);
  a.seq = s.seq;
  a.pos = s.pos;
  a.prompt_len = s.prompt_len;
  a.seq_len = static_cast<int>(s.capacity + 1);
  a.err = s.err;
  a.token_out = s.token_out;
  a.logits = s.logits;
  check_hip(mmr::launch_tiny_step(a, s.kv, s.stream), "small-model step");
}

// One decode step; first / last: its place in a replayed group of steps.  The
// first step of a group reads its token from seq (the host may have written
// it); inside the group the finalize folds into the next step's kernels.
void enqueue_step_kernels(const DeviceState& s, int splits, bool first = true, bool last = true) {
  if (s.model->tiny) {
    enqueue_tiny_step(s);
    return;
  }
  const bool fold = s.model->plan_lm.blocks <= mmr::kGemvMaxPrevParts;
  for (size_t l = 0; l < s.model->layers.size(); ++l)
    for (int k = kQkv; k <= kDown; ++k) {
      StepLink link;
      link.token_from_partials = fold && !first && l == 0 && k == kQkv;
      enqueue_kernel(s, k, l, splits, false, link);
    }
  StepLink head;
  head.advance_in_head = fold && !last;
  enqueue_kernel(s, kHead, 0, splits, false, head);
  if (!head.advance_in_head) enqueue_kernel(s, kFinalize, 0, splits, true);
}

// One prefill chunk: prompt tokens at positions start .. start + n - 1 through
// every layer with batched kernels (the device prefill layer of
// decoder_layer.cpp:661-734, chunked): embedding rows -> per layer RMSNorm
// rows, qkv GEMM, q/k norm + RoPE + KV write, causal attention, O GEMM +
// residual, RMSNorm rows, gate_up GEMM, SwiGLU rows, down GEMM + residual.
// The residual stream of the chunk ends in s.pf_h.
void enqueue_prefill_chunk(const DeviceState& s, int64_t start, int64_t n) {
  const DeviceModel& m = *s.model;
  const auto& c = m.cfg;
  const int rows = static_cast<int>(n);
  check_hip(mmr::launch_embedding_gather(m.embed, s.seq + start, rows, static_cast<int>(c.vocab_size),
                                         static_cast<int>(c.hidden_size), s.pf_h, s.err, s.stream),
            "prefill embedding");
  // Layer 0's input norm; every later layer's comes from the previous
  // layer's residual consumer (after the last layer the final norm, whose
  // rows are not used: the head normalises the last row itself).
  enqueue_prefill_input_norm(c, s.pf, rows, s.pf_h, m.layers[0].input_norm, s.stream);
  const size_t L = m.layers.size();
  for (size_t l = 0; l < L; ++l) {
    PrefillKv kv;
    kv.seg = s.kv_store.layer(static_cast<int64_t>(l));
    kv.dtype = s.kv;
    kv.rope_start = static_cast<int>(start);
    kv.row0 = static_cast<int>(start);
    const bool last = l + 1 == L;
    enqueue_prefill_layer(c, m.layers[l], m.inv_freq, s.pf, kv, rows, s.pf_h,
                          last ? m.final_norm : m.layers[l + 1].input_norm, last, s.stream);
  }
}

// `steps` consecutive decode steps with one attention split count, as one
// graph: the steps read and advance the device position themselves.
hipGraphExec_t capture_steps(DeviceState& s, int splits, int steps) {
  hipGraph_t graph = nullptr;
  check_hip(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    for (int i = 0; i < steps; ++i) enqueue_step_kernels(s, splits, i == 0, i == steps - 1);
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

// Back every position a decode launch with `splits` attention splits can
// reach before it is captured or run: choose_splits gives that split count
// to contexts up to some length (the last bucket to all of the capacity), and
// a replayed graph keeps the segment table it was captured with.  Segments
// are never freed while the state lives, so every captured graph stays valid.
void ensure_backed_for_splits(DeviceState& s, int splits, int tile) {
  if (s.model->tiny || s.kv_store.backed() >= s.capacity) return;
  int64_t reach = s.capacity;
  if (splits < kMaxSplits) {
    int64_t tiles = 1;
    while (tiles * tile < s.capacity && choose_splits((tiles + 1) * tile, tile) <= splits) ++tiles;
    reach = std::min(s.capacity, tiles * tile);
  }
  if (s.kv_store.backed() < reach) s.kv_store.reserve(reach);
}

void check_token(const MiniMindConfig& c, int32_t token) {
  if (token < 0 || token >= c.vocab_size) throw std::out_of_range("token id out of vocabulary range");
}

}  // namespace

void LanguageModel::launch_step(DecoderState& state) const {
  DeviceState& s = *state.device;
  if (state.position >= s.capacity) throw std::length_error("KV cache capacity exhausted");
  const int tile = mmr::attention_tile_tokens(static_cast<int>(config_.head_dim));
  const int splits = choose_splits(state.position + 1, tile);
  ensure_backed_for_splits(s, splits, tile);
  if (s.use_graphs) {
    const auto key = std::make_pair(splits, 1);
    auto it = s.graphs.find(key);
    if (it == s.graphs.end()) it = s.graphs.emplace(key, capture_steps(s, splits, 1)).first;
    check_hip(hipGraphLaunch(it->second, s.stream), "hipGraphLaunch");
  } else {
    enqueue_step_kernels(s, splits);
  }
  state.position += 1;
}

void LanguageModel::synchronize(DecoderState& state) const {
  DeviceState& s = *state.device;
  check_hip(hipMemcpyAsync(s.staging + s.capacity + 4, s.err, sizeof(int32_t), hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync err");
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  if (s.staging[s.capacity + 4] != 0) throw std::runtime_error("device kernel reported an out-of-range position");
}

void LanguageModel::enqueue_decode(DecoderState& state, int64_t n, int32_t first_token) const {
  DeviceState& s = *state.device;
  if (n < 0) throw std::invalid_argument("step count cannot be negative");
  if (state.position + n > s.capacity) throw std::length_error("KV cache capacity exhausted");
  if (first_token >= 0) {
    check_token(config_, first_token);
    check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    s.staging[0] = first_token;
    check_hip(hipMemcpyAsync(s.seq + state.position, s.staging, sizeof(int32_t), hipMemcpyHostToDevice, s.stream),
              "hipMemcpyAsync token");
  }
  // While the attention splits merge in the O-projection prologue (short
  // contexts), whole groups of kGraphSteps steps replay as one graph, with
  // the split count of the group's last (longest) step: extra splits of the
  // earlier steps hold no tile and merge as neutral partials.  (At 4096 and
  // 8192 keys, with the separate combine kernel, grouped steps measured 1-3%
  // slower than single-step graphs, 308 -> 318 and 346 -> 354 us per step in
  // the latest same-box A/B; at 512 and 1024 keys 1.5% faster.)
  const int tile = mmr::attention_tile_tokens(static_cast<int>(config_.head_dim));
  int64_t i = 0;
  if (s.use_graphs) {
    for (; i + kGraphSteps <= n; i += kGraphSteps) {
      const int splits = choose_splits(state.position + kGraphSteps, tile);
      if (splits > mmr::kCombineMaxSplits) break;
      ensure_backed_for_splits(s, splits, tile);
      const auto key = std::make_pair(splits, kGraphSteps);
      auto it = s.graphs.find(key);
      if (it == s.graphs.end()) it = s.graphs.emplace(key, capture_steps(s, splits, kGraphSteps)).first;
      check_hip(hipGraphLaunch(it->second, s.stream), "hipGraphLaunch");
      state.position += kGraphSteps;
    }
  }
  for (; i < n; ++i) launch_step(state);
}

void LanguageModel::enqueue_prefill(DecoderState& state, const std::vector<int32_t>& prompt) const {
  DeviceState& s = *state.device;
  if (prompt.empty()) throw std::invalid_argument("prompt_tokens cannot be empty");
  for (int32_t t : prompt) check_token(config_, t);
  const int64_t n = static_cast<int64_t>(prompt.size());
  if (state.position + n > s.capacity) throw std::length_error("KV cache capacity exhausted");
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  std::memcpy(s.staging, prompt.data(), prompt.size() * sizeof(int32_t));
  s.staging[s.capacity + 1] = static_cast<int32_t>(state.position + n);
  check_hip(hipMemcpyAsync(s.seq + state.position, s.staging, prompt.size() * sizeof(int32_t),
                           hipMemcpyHostToDevice, s.stream),
            "hipMemcpyAsync prompt");
  check_hip(hipMemcpyAsync(s.prompt_len, s.staging + s.capacity + 1, sizeof(int32_t), hipMemcpyHostToDevice,
                           s.stream),
            "hipMemcpyAsync prompt_len");
  if (s.prefill_tokenwise) {
    for (int64_t i = 0; i < n; ++i) launch_step(state);
    return;
  }
  if (!device_->tiny) s.kv_store.reserve(state.position + n);  // the rows the chunks write
  // Chunked GEMM prefill; the head (final norm, lm_head, argmax) then runs on
  // the last prompt row with the device position at that row, so the
  // finalize kernel writes the prediction to seq[position + n] and advances
  // the position past the prompt, exactly as the last decode step would.
  const int64_t start = state.position;
  int64_t last_rows = 0;
  for (int64_t b = start; b < start + n; b += s.pf_chunk) {
    last_rows = std::min<int64_t>(s.pf_chunk, start + n - b);
    enqueue_prefill_chunk(s, b, last_rows);
  }
  s.staging[s.capacity + 2] = static_cast<int32_t>(start + n - 1);
  check_hip(hipMemcpyAsync(s.pos, s.staging + s.capacity + 2, sizeof(int32_t), hipMemcpyHostToDevice, s.stream),
            "hipMemcpyAsync pos");
  check_hip(hipMemcpyAsync(s.h, s.pf_h + (last_rows - 1) * config_.hidden_size, config_.hidden_size * sizeof(float),
                           hipMemcpyDeviceToDevice, s.stream),
            "hipMemcpyAsync last row");
  const int splits = choose_splits(start + n, mmr::attention_tile_tokens(static_cast<int>(config_.head_dim)));
  ::minimind::model::enqueue_kernel(s, kHead, 0, splits, false);
  ::minimind::model::enqueue_kernel(s, kFinalize, 0, splits, true);
  state.position += n;
}

void LanguageModel::enqueue_kernel(DecoderState& state, int kernel, int64_t layer, int64_t count) const {
  DeviceState& s = *state.device;
  if (device_->tiny) throw std::invalid_argument("a small model's step is one kernel: no per-kernel launches");
  const int64_t L = config_.num_hidden_layers;
  if (kernel < kQkv || kernel > kFinalize) throw std::invalid_argument("unknown step kernel");
  if (layer < 0 || layer >= L || count < 0) throw std::invalid_argument("layer / count out of range");
  if (kernel == kAttention && state.position >= s.capacity) throw std::length_error("KV cache capacity exhausted");
  const int tile = mmr::attention_tile_tokens(static_cast<int>(config_.head_dim));
  const int splits = choose_splits(state.position + 1, tile);
  ensure_backed_for_splits(s, splits, tile);
  for (int64_t i = 0; i < count; ++i)
    ::minimind::model::enqueue_kernel(s, kernel, static_cast<size_t>((layer + i) % L), splits, false);
}

double LanguageModel::time_kernel(DecoderState& state, int kernel, int64_t layer, int64_t count) const {
  DeviceState& s = *state.device;
  if (count <= 0) throw std::invalid_argument("count must be positive");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipGraphExec_t exec = nullptr;
  auto release = [&] {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
  };
  try {
    check_hip(hipEventCreate(&e0), "hipEventCreate");
    check_hip(hipEventCreate(&e1), "hipEventCreate");
    // Any KV segment the launches need is allocated now, not under capture.
    const int tile = mmr::attention_tile_tokens(static_cast<int>(config_.head_dim));
    ensure_backed_for_splits(s, choose_splits(state.position + 1, tile), tile);
    if (s.use_graphs) {
      hipGraph_t graph = nullptr;
      check_hip(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        enqueue_kernel(state, kernel, layer, count);
      } catch (...) {
        (void)hipStreamEndCapture(s.stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
      }
      check_hip(hipStreamEndCapture(s.stream, &graph), "hipStreamEndCapture");
      const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      check_hip(st, "hipGraphInstantiate");
      check_hip(hipGraphLaunch(exec, s.stream), "hipGraphLaunch");  // warm
      check_hip(hipEventRecord(e0, s.stream), "hipEventRecord");
      check_hip(hipGraphLaunch(exec, s.stream), "hipGraphLaunch");
    } else {
      enqueue_kernel(state, kernel, layer, 32);  // warm
      check_hip(hipEventRecord(e0, s.stream), "hipEventRecord");
      enqueue_kernel(state, kernel, layer, count);
    }
    check_hip(hipEventRecord(e1, s.stream), "hipEventRecord");
    check_hip(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.0f;
    check_hip(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    release();
    return static_cast<double>(ms) * 1e3 / static_cast<double>(count);
  } catch (...) {
    (void)hipStreamSynchronize(s.stream);
    release();
    throw;
  }
}

std::vector<int32_t> LanguageModel::read_sequence(DecoderState& state, int64_t first, int64_t count) const {
  DeviceState& s = *state.device;
  if (first < 0 || count < 0 || first + count > s.capacity + 1) throw std::out_of_range("sequence range");
  std::vector<int32_t> out(static_cast<size_t>(count));
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  if (count > 0) {
    check_hip(hipMemcpyAsync(s.staging, s.seq + first, count * sizeof(int32_t), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync seq");
    synchronize(state);
    std::memcpy(out.data(), s.staging, count * sizeof(int32_t));
  }
  return out;
}

std::vector<float> LanguageModel::read_logits(DecoderState& state) const {
  DeviceState& s = *state.device;
  std::vector<float> out(static_cast<size_t>(config_.vocab_size));
  check_hip(hipMemcpyAsync(out.data(), s.logits, out.size() * sizeof(float), hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync logits");
  synchronize(state);
  return out;
}

void LanguageModel::reset_state(DecoderState& state) const {
  DeviceState& s = *state.device;
  check_hip(hipMemsetAsync(s.pos, 0, 2 * sizeof(int32_t), s.stream), "hipMemsetAsync");
  check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
  state.position = 0;
}

void LanguageModel::reserve_kv(DecoderState& state, int64_t positions) const {
  DeviceState& s = *state.device;
  if (positions < 0) throw std::invalid_argument("positions cannot be negative");
  if (positions > s.capacity) throw std::length_error("KV cache capacity exhausted");
  if (!device_->tiny) s.kv_store.reserve(positions);
}

std::vector<float> LanguageModel::forward_token(int32_t token, DecoderState& state) const {
  check_token(config_, token);
  enqueue_decode(state, 1, token);
  return read_logits(state);
}

int32_t LanguageModel::forward_next_token(int32_t token, DecoderState& state) const {
  check_token(config_, token);
  const int64_t p = state.position;
  enqueue_decode(state, 1, token);
  DeviceState& s = *state.device;
  check_hip(hipMemcpyAsync(s.staging, s.seq + p + 1, sizeof(int32_t), hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync next");
  synchronize(state);
  return s.staging[0];
}

int32_t LanguageModel::prefill_next_token(const std::vector<int32_t>& prompt_tokens, DecoderState& state) const {
  if (prompt_tokens.empty()) throw std::invalid_argument("prompt_tokens cannot be empty");
  if (state.position != 0) throw std::invalid_argument("prefill layer requires an empty KV cache");
  enqueue_prefill(state, prompt_tokens);
  DeviceState& s = *state.device;
  check_hip(hipMemcpyAsync(s.staging, s.seq + state.position, sizeof(int32_t), hipMemcpyDeviceToHost, s.stream),
            "hipMemcpyAsync next");
  synchronize(state);
  return s.staging[0];
}

void LanguageModel::generate_stream(const std::vector<int32_t>& prompt_tokens, int64_t max_new_tokens,
                                    const std::function<void(int32_t)>& on_token) const {
  if (prompt_tokens.empty()) throw std::invalid_argument("prompt_tokens cannot be empty");
  if (max_new_tokens < 0) throw std::invalid_argument("max_new_tokens cannot be negative");
  const int64_t prompt_len = static_cast<int64_t>(prompt_tokens.size());
  const int64_t needed = prompt_len + std::max<int64_t>(max_new_tokens, 1) - 1;
  const int64_t limit = device_->tiny ? mmr::kTinyMaxContext : config_.max_position_embeddings;
  if (needed > limit) throw std::length_error("sequence exceeds max_position_embeddings");
  DecoderState state = make_state(std::max<int64_t>(needed, 1), KvCacheDtype::kFloat32);
  enqueue_prefill(state, prompt_tokens);
  // The prompt's last step predicts generated token 0 at seq[prompt_len].
  // Further steps run ahead in small chunks; tokens after an EOS are computed
  // but never emitted (language_model.cpp:389-395 stops after emitting EOS).
  constexpr int64_t kChunk = 8;
  int64_t emitted = 0;
  while (emitted < max_new_tokens) {
    const int64_t have = state.position - prompt_len + 1;  // generated ids present in seq
    const int64_t want = std::min(max_new_tokens, have);
    const auto ids = read_sequence(state, prompt_len + emitted, want - emitted);
    for (int32_t id : ids) {
      on_token(id);
      ++emitted;
      if (id == config_.eos_token_id) return;
    }
    if (emitted >= max_new_tokens) return;
    const int64_t steps = std::min<int64_t>(kChunk, max_new_tokens - emitted);
    enqueue_decode(state, steps);
  }
}

std::vector<int32_t> LanguageModel::generate(const std::vector<int32_t>& prompt_tokens, int64_t max_new_tokens) const {
  std::vector<int32_t> generated;
  generated.reserve(static_cast<size_t>(std::max<int64_t>(max_new_tokens, 0)));
  generate_stream(prompt_tokens, max_new_tokens, [&generated](int32_t t) { generated.push_back(t); });
  return generated;
}

int32_t argmax_token(const std::vector<float>& logits) {
  if (logits.empty()) throw std::invalid_argument("logits cannot be empty");
  return static_cast<int32_t>(std::distance(logits.begin(), std::max_element(logits.begin(), logits.end())));
}

std::pair<MiniMindConfig, DenseModelWeights> toy_model_weights() {
  MiniMindConfig c;  // struct defaults (rms_norm_eps 1e-6), then the toy's shape
  c.hidden_size = 4;
  c.num_hidden_layers = 1;
  c.use_moe = false;
  c.vocab_size = 8;
  c.bos_token_id = 1;
  c.eos_token_id = 2;
  c.num_attention_heads = 2;
  c.num_key_value_heads = 1;
  c.head_dim = 2;
  c.intermediate_size = 8;
  c.max_position_embeddings = 16;
  c.rope_theta = 10000.0F;
  c.tie_word_embeddings = false;
  c.moe_intermediate_size = 8;
  const int64_t H = c.hidden_size, V = c.vocab_size;
  // rows x cols with ones on the leading diagonal
  const auto eye = [](int64_t rows, int64_t cols) {
    std::vector<float> m(static_cast<size_t>(rows * cols), 0.0F);
    for (int64_t i = 0; i < std::min(rows, cols); ++i) m[static_cast<size_t>(i * cols + i)] = 1.0F;
    return m;
  };
  DenseModelWeights w;
  // Token 0 maps to zero; tokens 1..4 to the unit vectors e0..e3; tokens
  // 5..7 to e_j + e_(j+1).  lm_head row 0 is zero, rows 1..4 are 0.2 e_j,
  // rows 5..7 are 2 e_j + 0.1 e_(j+1): the tables of the reference toy.
  w.embed_tokens.assign(static_cast<size_t>(V * H), 0.0F);
  w.lm_head.assign(static_cast<size_t>(V * H), 0.0F);
  for (int64_t t = 1; t < V; ++t) {
    const int64_t j = t <= H ? t - 1 : t - H - 1;
    float* e = &w.embed_tokens[static_cast<size_t>(t * H)];
    float* o = &w.lm_head[static_cast<size_t>(t * H)];
    if (t <= H) {
      e[j] = 1.0F;
      o[j] = 0.2F;
    } else {
      e[j] = 1.0F;
      e[j + 1] = 1.0F;
      o[j] = 2.0F;
      o[j + 1] = 0.1F;
    }
  }
  w.final_norm.assign(static_cast<size_t>(H), 1.0F);
  DenseLayerWeights L;
  const int64_t qs = c.num_attention_heads * c.head_dim, kvs = c.num_key_value_heads * c.head_dim;
  L.input_norm.assign(static_cast<size_t>(H), 1.0F);
  L.post_attention_norm.assign(static_cast<size_t>(H), 1.0F);
  L.q_norm.assign(static_cast<size_t>(c.head_dim), 1.0F);
  L.k_norm.assign(static_cast<size_t>(c.head_dim), 1.0F);
  L.q_proj = eye(qs, H);
  L.k_proj = eye(kvs, H);
  L.v_proj = eye(kvs, H);
  L.o_proj = eye(H, qs);
  L.gate_proj = eye(c.intermediate_size, H);
  L.up_proj = eye(c.intermediate_size, H);
  L.down_proj = eye(H, c.intermediate_size);
  w.layers.push_back(std::move(L));
  return {c, std::move(w)};
}

LanguageModel make_toy_language_model() {
  auto cw = toy_model_weights();
  return LanguageModel(std::move(cw.first), std::move(cw.second));
}

bool has_runtime_language_model(const std::string& model_dir) {
  const std::filesystem::path dir(model_dir);
  return std::filesystem::exists(dir / "minimind_runtime_config.txt") && std::filesystem::exists(dir / "weights.bin");
}

LanguageModel load_runtime_language_model(const std::string& model_dir) {
  const std::filesystem::path dir(model_dir);
  MiniMindConfig config = config_from_file((dir / "minimind_runtime_config.txt").string());
  DenseModelWeights weights = read_weights(config, (dir / "weights.bin").string());
  return LanguageModel(std::move(config), std::move(weights));
}

}  // namespace minimind::model
