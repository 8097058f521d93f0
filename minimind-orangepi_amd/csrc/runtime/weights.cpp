#include "weights.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <thread>

namespace minimind::model {

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ULL;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

// Draw n (1-based) of SplitMix64(seed): the state after n increments.
inline double uniform53(uint64_t seed, uint64_t n) {
  return static_cast<double>(mix64(seed + n * kGamma) >> 11) * 0x1.0p-53;
}

inline float normal_at(uint64_t seed, uint64_t i, double std) {
  const uint64_t p = i / 2;
  const double u1 = uniform53(seed, 2 * p + 1);
  const double u2 = uniform53(seed, 2 * p + 2);
  const double r = std::sqrt(-2.0 * std::log(1.0 - u1));
  const double t = 2.0 * M_PI * u2;
  const double z = (i % 2 == 0) ? r * std::cos(t) : r * std::sin(t);
  return static_cast<float>(std * z);
}

// One tensor record: u64 name length, name, u64 element count, payload of
// `count` little-endian fp32 (MMRTW001) or IEEE fp16 (MMRTH001) values.
std::vector<float> read_tensor(std::ifstream& in, const std::string& expected, int64_t count, bool half) {
  uint64_t len = 0;
  in.read(reinterpret_cast<char*>(&len), sizeof(len));
  if (!in || len > 4096) throw std::runtime_error("failed to read " + expected);
  std::string name(static_cast<size_t>(len), '\0');
  in.read(name.data(), static_cast<std::streamsize>(len));
  if (!in) throw std::runtime_error("failed to read " + expected);
  if (name != expected) throw std::runtime_error("expected tensor " + expected + ", got " + name);
  uint64_t n = 0;
  in.read(reinterpret_cast<char*>(&n), sizeof(n));
  if (!in) throw std::runtime_error("failed to read " + expected);
  if (static_cast<int64_t>(n) != count) throw std::runtime_error(expected + " has invalid size");
  std::vector<float> v(static_cast<size_t>(n));
  if (half) {
    std::vector<uint16_t> h(static_cast<size_t>(n));
    in.read(reinterpret_cast<char*>(h.data()), static_cast<std::streamsize>(n * sizeof(uint16_t)));
    if (!in) throw std::runtime_error("failed to read " + expected);
    for (size_t i = 0; i < h.size(); ++i) v[i] = half_to_float(h[i]);
  } else {
    in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(n * sizeof(float)));
    if (!in) throw std::runtime_error("failed to read " + expected);
  }
  return v;
}

void write_tensor(std::ofstream& out, const std::string& name, const float* data, uint64_t count) {
  const uint64_t len = name.size();
  out.write(reinterpret_cast<const char*>(&len), sizeof(len));
  out.write(name.data(), static_cast<std::streamsize>(len));
  out.write(reinterpret_cast<const char*>(&count), sizeof(count));
  out.write(reinterpret_cast<const char*>(data), static_cast<std::streamsize>(count * sizeof(float)));
}

struct TensorEntry {
  std::string name;
  int64_t count;
  bool drawn;  // false: norm gain (1.0) or tied lm_head (copy of embed)
};

std::vector<TensorEntry> tensor_order(const MiniMindConfig& c) {
  const int64_t H = c.hidden_size, V = c.vocab_size, D = c.head_dim, F = c.intermediate_size;
  const int64_t qs = c.num_attention_heads * D, kvs = c.num_key_value_heads * D;
  std::vector<TensorEntry> t;
  t.push_back({"model.embed_tokens.weight", V * H, true});
  t.push_back({"model.norm.weight", H, false});
  t.push_back({"lm_head.weight", V * H, !c.tie_word_embeddings});
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    t.push_back({p + "input_layernorm.weight", H, false});
    t.push_back({p + "post_attention_layernorm.weight", H, false});
    t.push_back({p + "self_attn.q_norm.weight", D, false});
    t.push_back({p + "self_attn.k_norm.weight", D, false});
    t.push_back({p + "self_attn.q_proj.weight", qs * H, true});
    t.push_back({p + "self_attn.k_proj.weight", kvs * H, true});
    t.push_back({p + "self_attn.v_proj.weight", kvs * H, true});
    t.push_back({p + "self_attn.o_proj.weight", H * qs, true});
    t.push_back({p + "mlp.gate_proj.weight", F * H, true});
    t.push_back({p + "mlp.up_proj.weight", F * H, true});
    t.push_back({p + "mlp.down_proj.weight", H * F, true});
  }
  return t;
}

}  // namespace

uint16_t float_to_half(float value) {
  uint32_t x;
  std::memcpy(&x, &value, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);
  if (a < 0x38800000u) {
    // Subnormal half: the unit is 2^-24; scale exactly and round to nearest even.
    float f;
    std::memcpy(&f, &a, 4);
    return static_cast<uint16_t>(sign | static_cast<uint32_t>(std::nearbyint(f * 16777216.0f)));
  }
  uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return static_cast<uint16_t>(sign | h);
}

float half_to_float(uint16_t value) {
  const uint32_t sign = (static_cast<uint32_t>(value) & 0x8000u) << 16;
  const uint32_t e = (value >> 10) & 0x1fu;
  const uint32_t m = value & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float f = static_cast<float>(m) * (1.0f / 16777216.0f);
    std::memcpy(&bits, &f, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

void synthesize_normals(uint64_t seed, uint64_t first, uint64_t count, double std, bool round_fp16, float* out) {
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const uint64_t min_chunk = uint64_t{1} << 18;
  const unsigned nthreads = static_cast<unsigned>(std::min<uint64_t>(hw, (count + min_chunk - 1) / min_chunk));
  auto work = [&](uint64_t b, uint64_t e) {
    for (uint64_t i = b; i < e; ++i) {
      float v = normal_at(seed, first + i, std);
      if (round_fp16) v = half_to_float(float_to_half(v));
      out[i] = v;
    }
  };
  if (nthreads <= 1) {
    work(0, count);
    return;
  }
  std::vector<std::thread> pool;
  const uint64_t per = (count + nthreads - 1) / nthreads;
  for (unsigned t = 0; t < nthreads; ++t) {
    const uint64_t b = t * per, e = std::min(count, b + per);
    if (b < e) pool.emplace_back(work, b, e);
  }
  for (auto& th : pool) th.join();
}

std::vector<int32_t> synthesize_prompt(uint64_t seed, int64_t count, int64_t vocab) {
  std::vector<int32_t> ids(static_cast<size_t>(std::max<int64_t>(count, 0)));
  for (int64_t j = 0; j < count; ++j)
    ids[static_cast<size_t>(j)] = static_cast<int32_t>(std::floor(uniform53(seed, static_cast<uint64_t>(j) + 1) *
                                                                  static_cast<double>(vocab)));
  return ids;
}

DenseModelWeights synthesize_weights(const MiniMindConfig& c, uint64_t seed, double std, bool round_fp16) {
  const auto order = tensor_order(c);
  std::vector<std::vector<float>> tensors;
  uint64_t cursor = 0;
  for (const auto& t : order) {
    std::vector<float> v(static_cast<size_t>(t.count), 1.0f);
    if (t.drawn) {
      synthesize_normals(seed, cursor, static_cast<uint64_t>(t.count), std, round_fp16, v.data());
      cursor += static_cast<uint64_t>(t.count);
    }
    tensors.push_back(std::move(v));
  }
  DenseModelWeights w;
  size_t i = 0;
  w.embed_tokens = std::move(tensors[i++]);
  w.final_norm = std::move(tensors[i++]);
  w.lm_head = std::move(tensors[i++]);
  if (c.tie_word_embeddings) w.lm_head = w.embed_tokens;
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    DenseLayerWeights L;
    L.input_norm = std::move(tensors[i++]);
    L.post_attention_norm = std::move(tensors[i++]);
    L.q_norm = std::move(tensors[i++]);
    L.k_norm = std::move(tensors[i++]);
    L.q_proj = std::move(tensors[i++]);
    L.k_proj = std::move(tensors[i++]);
    L.v_proj = std::move(tensors[i++]);
    L.o_proj = std::move(tensors[i++]);
    L.gate_proj = std::move(tensors[i++]);
    L.up_proj = std::move(tensors[i++]);
    L.down_proj = std::move(tensors[i++]);
    w.layers.push_back(std::move(L));
  }
  return w;
}

void write_config(const MiniMindConfig& c, const std::string& path) {
  std::ofstream out(path);
  if (!out) throw std::runtime_error("failed to write runtime config: " + path);
  char eps[64], theta[64];
  std::snprintf(eps, sizeof eps, "%.9g", static_cast<double>(c.rms_norm_eps));
  std::snprintf(theta, sizeof theta, "%.9g", static_cast<double>(c.rope_theta));
  out << "hidden_size=" << c.hidden_size << "\n"
      << "num_hidden_layers=" << c.num_hidden_layers << "\n"
      << "use_moe=" << (c.use_moe ? 1 : 0) << "\n"
      << "vocab_size=" << c.vocab_size << "\n"
      << "num_attention_heads=" << c.num_attention_heads << "\n"
      << "num_key_value_heads=" << c.num_key_value_heads << "\n"
      << "head_dim=" << c.head_dim << "\n"
      << "intermediate_size=" << c.intermediate_size << "\n"
      << "max_position_embeddings=" << c.max_position_embeddings << "\n"
      << "tie_word_embeddings=" << (c.tie_word_embeddings ? 1 : 0) << "\n"
      << "rms_norm_eps=" << eps << "\n"
      << "rope_theta=" << theta << "\n";
}

void write_synthetic_model(const std::string& dir, const MiniMindConfig& c, uint64_t seed, double std,
                           bool round_fp16) {
  std::filesystem::create_directories(dir);
  write_config(c, dir + "/minimind_runtime_config.txt");
  std::ofstream out(dir + "/weights.bin", std::ios::binary);
  if (!out) throw std::runtime_error("failed to write weights: " + dir);
  out.write("MMRTW001", 8);
  const auto order = tensor_order(c);
  std::vector<float> embed;
  uint64_t cursor = 0;
  for (const auto& t : order) {
    std::vector<float> v(static_cast<size_t>(t.count), 1.0f);
    if (t.drawn) {
      synthesize_normals(seed, cursor, static_cast<uint64_t>(t.count), std, round_fp16, v.data());
      cursor += static_cast<uint64_t>(t.count);
    }
    if (t.name == "model.embed_tokens.weight") embed = v;
    if (t.name == "lm_head.weight" && c.tie_word_embeddings) v = embed;
    write_tensor(out, t.name, v.data(), static_cast<uint64_t>(v.size()));
  }
  if (!out) throw std::runtime_error("failed to write weights: " + dir);
}

DenseModelWeights read_weights(const MiniMindConfig& c, const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("failed to open runtime weights: " + path);
  char magic[8]{};
  in.read(magic, 8);
  if (!in) throw std::runtime_error("failed to read magic");
  const std::string format(magic, 8);
  if (format != "MMRTW001" && format != "MMRTH001") throw std::runtime_error("unsupported runtime weight format");
  const bool half = format == "MMRTH001";
  if (c.use_moe) throw std::runtime_error("the gfx950 runtime implements the dense model only (use_moe=0)");
  const auto order = tensor_order(c);
  std::vector<std::vector<float>> tensors;
  for (const auto& t : order) tensors.push_back(read_tensor(in, t.name, t.count, half));
  DenseModelWeights w;
  size_t i = 0;
  w.embed_tokens = std::move(tensors[i++]);
  w.final_norm = std::move(tensors[i++]);
  w.lm_head = std::move(tensors[i++]);
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    DenseLayerWeights L;
    L.input_norm = std::move(tensors[i++]);
    L.post_attention_norm = std::move(tensors[i++]);
    L.q_norm = std::move(tensors[i++]);
    L.k_norm = std::move(tensors[i++]);
    L.q_proj = std::move(tensors[i++]);
    L.k_proj = std::move(tensors[i++]);
    L.v_proj = std::move(tensors[i++]);
    L.o_proj = std::move(tensors[i++]);
    L.gate_proj = std::move(tensors[i++]);
    L.up_proj = std::move(tensors[i++]);
    L.down_proj = std::move(tensors[i++]);
    w.layers.push_back(std::move(L));
  }
  return w;
}

void write_weights(const MiniMindConfig& c, const DenseModelWeights& w, const std::string& path) {
  std::ofstream out(path, std::ios::binary);
  if (!out) throw std::runtime_error("failed to write weights: " + path);
  out.write("MMRTW001", 8);
  const auto put = [&](const std::string& n, const std::vector<float>& v) {
    write_tensor(out, n, v.data(), static_cast<uint64_t>(v.size()));
  };
  put("model.embed_tokens.weight", w.embed_tokens);
  put("model.norm.weight", w.final_norm);
  put("lm_head.weight", w.lm_head);
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    const auto& L = w.layers[static_cast<size_t>(l)];
    put(p + "input_layernorm.weight", L.input_norm);
    put(p + "post_attention_layernorm.weight", L.post_attention_norm);
    put(p + "self_attn.q_norm.weight", L.q_norm);
    put(p + "self_attn.k_norm.weight", L.k_norm);
    put(p + "self_attn.q_proj.weight", L.q_proj);
    put(p + "self_attn.k_proj.weight", L.k_proj);
    put(p + "self_attn.v_proj.weight", L.v_proj);
    put(p + "self_attn.o_proj.weight", L.o_proj);
    put(p + "mlp.gate_proj.weight", L.gate_proj);
    put(p + "mlp.up_proj.weight", L.up_proj);
    put(p + "mlp.down_proj.weight", L.down_proj);
  }
  if (!out) throw std::runtime_error("failed to write weights: " + path);
}

}  // namespace minimind::model
