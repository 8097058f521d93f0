// decoder_layer.cpp -- one dense decoder layer's decode step on the device
// (reference decoder_layer.cpp:312-407 for the op order, :617-659 for the
// device twin this replaces).
#include "decoder_layer.h"

#include <cmath>
#include <stdexcept>
#include <string>

namespace minimind::model {

namespace {

void require_size(const std::vector<float>& v, int64_t expected, const std::string& name) {
  if (static_cast<int64_t>(v.size()) != expected) throw std::invalid_argument(name + " has invalid size");
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

mmr::GemvPlan plan_or_throw(int rows, int k, mmr::GemvEpilogue epi, int lanes, int rows_per_group,
                            const char* name) {
  mmr::GemvPlan p;
  if (!mmr::gemv_plan(rows, k, epi, lanes, rows_per_group, &p))
    throw std::invalid_argument(std::string("unsupported GEMV shape for ") + name);
  return p;
}

// Offsets (floats) of the scratch slices inside one call's workspace.
struct WorkspaceLayout {
  std::size_t qkv = 0, attn = 0, act = 0, part = 0, total = 0;
};

std::size_t round64(std::size_t n) { return (n + 63) / 64 * 64; }

WorkspaceLayout workspace_layout(const MiniMindConfig& c, int splits) {
  const int64_t D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
  WorkspaceLayout w;
  w.qkv = 0;
  w.attn = w.qkv + round64(static_cast<std::size_t>((Hq + 2 * Hkv) * D));
  w.act = w.attn + round64(static_cast<std::size_t>(Hq * D));
  w.part = w.act + round64(static_cast<std::size_t>(c.intermediate_size));
  w.total = w.part + round64(mmr::attention_partial_floats(static_cast<int>(Hq), static_cast<int>(Hkv),
                                                           static_cast<int>(D), splits));
  return w;
}

}  // namespace

LayerPlans plan_layer(const MiniMindConfig& c) {
  const int H = static_cast<int>(c.hidden_size), F = static_cast<int>(c.intermediate_size);
  const int qs = static_cast<int>(c.num_attention_heads * c.head_dim);
  const int qkv_rows = qs + 2 * static_cast<int>(c.num_key_value_heads * c.head_dim);
  LayerPlans p;
  // qkv from K = 768 up: 64-lane groups of two rows, 8 rows per block (144
  // blocks for MiniMind2 instead of 288 with one row).  Same-box step A/Bs:
  // 32-lane groups of one row (also 144 blocks) took the step from 249.7 to
  // 247.9 us, and the two-row 64-lane groups from there 251.8 -> 251.0 us on
  // another box.  O, down and gate_up measured slower with fewer, larger
  // blocks or other lane widths.
  p.qkv = plan_or_throw(qkv_rows, H, mmr::kEpiStore, 0, H / 8 >= 96 ? 2 : 0, "qkv_proj");
  p.o = plan_or_throw(H, qs, mmr::kEpiResidual, 0, 0, "o_proj");
  // gate_up keeps 32-lane groups: 64 measured slower for this kernel alone
  // and within noise for the step.
  p.gate_up = plan_or_throw(2 * F, H, mmr::kEpiSwiGlu, H / 8 >= 48 ? 32 : 0, 0, "gate_up_proj");
  p.down = plan_or_throw(H, F, mmr::kEpiResidual, 0, 0, "down_proj");
  return p;
}

std::vector<float> rope_inv_freq(const MiniMindConfig& c) {
  const int64_t D = c.head_dim;
  std::vector<float> inv(static_cast<size_t>(D / 2));
  for (int64_t i = 0; i < D / 2; ++i)
    inv[static_cast<size_t>(i)] = 1.0F / std::pow(c.rope_theta, static_cast<float>(i * 2) / static_cast<float>(D));
  return inv;
}

void check_layer_weights(const MiniMindConfig& c, const DenseLayerWeights& L) {
  const int64_t H = c.hidden_size, D = c.head_dim, F = c.intermediate_size;
  const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
  require_size(L.input_norm, H, "input_norm");
  require_size(L.post_attention_norm, H, "post_attention_norm");
  require_size(L.q_norm, D, "q_norm");
  require_size(L.k_norm, D, "k_norm");
  require_size(L.q_proj, qs * H, "q_proj");
  require_size(L.k_proj, kvs * H, "k_proj");
  require_size(L.v_proj, kvs * H, "v_proj");
  require_size(L.o_proj, H * qs, "o_proj");
  require_size(L.gate_proj, F * H, "gate_proj");
  require_size(L.up_proj, F * H, "up_proj");
  require_size(L.down_proj, H * F, "down_proj");
}

std::size_t plan_layer_bytes(const MiniMindConfig& c) {
  const int64_t H = c.hidden_size, D = c.head_dim, F = c.intermediate_size;
  const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
  return Arena::round_up(H * 4) * 2 + Arena::round_up(D * 4) * 2 + Arena::round_up((qs + 2 * kvs) * H * 2) +
         Arena::round_up(H * qs * 2) + Arena::round_up(2 * F * H * 2) + Arena::round_up(H * F * 2);
}

// Fused layout of language_model.cpp:95-119 (qkv = [q; k; v] rows), with the
// gate/up rows interleaved so one lane group of the GEMV owns a (gate, up)
// pair and applies SwiGLU in registers.
LayerDev upload_layer(Arena& ar, const MiniMindConfig& c, const DenseLayerWeights& L) {
  const int64_t H = c.hidden_size, D = c.head_dim, F = c.intermediate_size;
  const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
  LayerDev d;
  d.input_norm = upload<float>(ar, L.input_norm.data(), H);
  d.post_norm = upload<float>(ar, L.post_attention_norm.data(), H);
  d.q_norm = upload<float>(ar, L.q_norm.data(), D);
  d.k_norm = upload<float>(ar, L.k_norm.data(), D);
  std::vector<float> qkv;
  qkv.reserve(static_cast<size_t>((qs + 2 * kvs) * H));
  qkv.insert(qkv.end(), L.q_proj.begin(), L.q_proj.end());
  qkv.insert(qkv.end(), L.k_proj.begin(), L.k_proj.end());
  qkv.insert(qkv.end(), L.v_proj.begin(), L.v_proj.end());
  d.qkv = upload<__half>(ar, to_half(qkv).data(), qkv.size());
  d.o = upload<__half>(ar, to_half(L.o_proj).data(), L.o_proj.size());
  std::vector<uint16_t> gu(static_cast<size_t>(2 * F * H));
  for (int64_t r = 0; r < F; ++r)
    for (int64_t k = 0; k < H; ++k) {
      gu[static_cast<size_t>((2 * r) * H + k)] = float_to_half(L.gate_proj[static_cast<size_t>(r * H + k)]);
      gu[static_cast<size_t>((2 * r + 1) * H + k)] = float_to_half(L.up_proj[static_cast<size_t>(r * H + k)]);
    }
  d.gate_up = upload<__half>(ar, gu.data(), gu.size());
  d.down = upload<__half>(ar, to_half(L.down_proj).data(), L.down_proj.size());
  return d;
}

std::shared_ptr<DeviceLayerWeights> DeviceLayerWeights::upload(const MiniMindConfig& c, const DenseLayerWeights& host) {
  const auto errors = validate_config(c);
  if (!errors.empty()) throw std::invalid_argument("invalid MiniMind config: " + errors.front());
  const auto dev_errors = validate_device_config(c);
  if (!dev_errors.empty()) throw std::invalid_argument("unsupported by the gfx950 runtime: " + dev_errors.front());
  check_layer_weights(c, host);
  auto arena = std::make_shared<Arena>();
  arena->plan(plan_layer_bytes(c));
  arena->plan(static_cast<std::size_t>(c.head_dim / 2) * 4);
  arena->allocate();
  auto out = std::make_shared<DeviceLayerWeights>();
  out->cfg = c;
  out->plans = plan_layer(c);
  out->w = upload_layer(*arena, c, host);
  const auto inv = rope_inv_freq(c);
  float* f = arena->take<float>(inv.size());
  check_hip(hipMemcpy(f, inv.data(), inv.size() * 4, hipMemcpyHostToDevice), "hipMemcpy rope");
  out->inv_freq = f;
  check_hip(hipDeviceSynchronize(), "layer upload");
  out->owner = std::move(arena);
  return out;
}

std::shared_ptr<DeviceLayerWeights> DeviceLayerWeights::view(const std::shared_ptr<const DeviceModel>& model,
                                                             int64_t layer) {
  if (!model) throw std::invalid_argument("null model");
  if (layer < 0 || layer >= static_cast<int64_t>(model->layers.size()))
    throw std::out_of_range("layer index out of range");
  auto out = std::make_shared<DeviceLayerWeights>();
  out->cfg = model->cfg;
  out->w = model->layers[static_cast<size_t>(layer)];
  out->plans = LayerPlans{model->plan_qkv, model->plan_o, model->plan_gu, model->plan_down};
  out->inv_freq = model->inv_freq;
  out->owner = model;
  return out;
}

std::size_t decoder_layer_workspace_floats(const MiniMindConfig& c, int splits) {
  return workspace_layout(c, splits).total;
}

void enqueue_decoder_layer(const DeviceLayerWeights& W, const DecoderLayerIo& io, hipStream_t stream) {
  const auto& c = W.cfg;
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), Hkv = static_cast<int>(c.num_key_value_heads);
  const int F = static_cast<int>(c.intermediate_size);
  const WorkspaceLayout ws = workspace_layout(c, io.splits);
  float* qkv = io.workspace + ws.qkv;
  float* attn = io.workspace + ws.attn;
  float* act = io.workspace + ws.act;
  float* part = io.workspace + ws.part;

  // RMSNorm (:327) folded into the QKV projection (:331-335).
  mmr::GemvArgs a;
  a.w = W.w.qkv;
  a.rows = (Hq + 2 * Hkv) * D;
  a.k = H;
  a.x = io.hidden;
  a.norm_w = W.w.input_norm;
  a.eps = c.rms_norm_eps;
  a.y = qkv;
  check_hip(mmr::launch_gemv(a, mmr::kProRmsNorm, mmr::kEpiStore, W.plans.qkv, stream), "layer qkv gemv");

  // q/k norm + RoPE (:342-352), K/V append (:354-359) and attention (:361).
  mmr::AttnArgs t;
  t.qkv = qkv;
  t.q_norm = W.w.q_norm;
  t.k_norm = W.w.k_norm;
  t.eps = c.rms_norm_eps;
  t.inv_freq = W.inv_freq;
  t.pos = io.position;
  t.seg = io.seg;
  t.capacity = io.capacity;
  t.rows = io.rows;
  t.hq = Hq;
  t.hkv = Hkv;
  t.d = D;
  t.splits = io.splits;
  t.part = part;
  t.err = io.err;
  check_hip(mmr::launch_attention(t, mmr::kAttnFused, io.kv, stream), "layer attention");

  // O projection (:362) + residual (:364-367); the split partials merge in
  // the GEMV prologue while they fit it, else in the combine kernel first.
  mmr::GemvArgs o;
  o.w = W.w.o;
  o.rows = H;
  o.k = Hq * D;
  o.residual = io.hidden;
  o.y = io.out;
  mmr::GemvPrologue pro = mmr::kProPlain;
  if (io.splits <= mmr::kCombineMaxSplits && Hq <= mmr::kCombineMaxHeads && Hq * D <= mmr::kCombineMaxDim) {
    pro = mmr::kProAttnCombine;
    o.part = part;
    o.splits = io.splits;
    o.hq = Hq;
    o.hkv = Hkv;
    o.head_dim = D;
  } else {
    check_hip(mmr::launch_attention_combine(part, Hq, Hkv, D, io.splits, attn, stream), "layer attention combine");
    o.x = attn;
  }
  check_hip(mmr::launch_gemv(o, pro, mmr::kEpiResidual, W.plans.o, stream), "layer o gemv");

  // RMSNorm (:369) folded into gate_up (:392-393), SwiGLU (:394) in its epilogue.
  mmr::GemvArgs g;
  g.w = W.w.gate_up;
  g.rows = 2 * F;
  g.k = H;
  g.x = io.out;
  g.norm_w = W.w.post_norm;
  g.eps = c.rms_norm_eps;
  g.y = act;
  check_hip(mmr::launch_gemv(g, mmr::kProRmsNorm, mmr::kEpiSwiGlu, W.plans.gate_up, stream), "layer gate_up gemv");

  // down (:400) + residual (:403-405).
  mmr::GemvArgs dn;
  dn.w = W.w.down;
  dn.rows = H;
  dn.k = F;
  dn.x = act;
  dn.residual = io.out;
  dn.y = io.out;
  check_hip(mmr::launch_gemv(dn, mmr::kProPlain, mmr::kEpiResidual, W.plans.down, stream), "layer down gemv");
}

}  // namespace minimind::model
