#include "config.h"

#include <cctype>
#include <cmath>
#include <fstream>
#include <stdexcept>
#include <unordered_map>

namespace minimind::model {

MiniMindConfig default_minimind_config() {
  MiniMindConfig config;
  config.head_dim = config.hidden_size / config.num_attention_heads;
  config.intermediate_size =
      static_cast<int64_t>(std::ceil(static_cast<double>(config.hidden_size) * 3.14159265358979323846 / 64.0)) * 64;
  config.moe_intermediate_size = config.intermediate_size;
  return config;
}

std::vector<std::string> validate_config(const MiniMindConfig& c) {
  std::vector<std::string> errors;
  const auto positive = [&](int64_t v, const char* name) {
    if (v <= 0) errors.push_back(std::string(name) + " must be positive");
  };
  positive(c.hidden_size, "hidden_size");
  positive(c.num_hidden_layers, "num_hidden_layers");
  positive(c.vocab_size, "vocab_size");
  positive(c.num_attention_heads, "num_attention_heads");
  positive(c.num_key_value_heads, "num_key_value_heads");
  positive(c.head_dim, "head_dim");
  positive(c.intermediate_size, "intermediate_size");
  positive(c.max_position_embeddings, "max_position_embeddings");
  if (c.hidden_size > 0 && c.num_attention_heads > 0) {
    if (c.hidden_size % c.num_attention_heads != 0)
      errors.push_back("hidden_size must be divisible by num_attention_heads");
    if (c.head_dim != c.hidden_size / c.num_attention_heads)
      errors.push_back("head_dim must equal hidden_size / num_attention_heads");
  }
  if (c.num_attention_heads > 0 && c.num_key_value_heads > 0 && c.num_attention_heads % c.num_key_value_heads != 0)
    errors.push_back("num_attention_heads must be divisible by num_key_value_heads");
  if (!(c.rope_theta > 0.0F)) errors.push_back("rope_theta must be positive");
  if (!(c.rms_norm_eps > 0.0F)) errors.push_back("rms_norm_eps must be positive");
  if (c.hidden_act != "silu") errors.push_back("only silu hidden_act is currently supported");
  if (c.use_moe) {
    positive(c.num_experts, "num_experts");
    positive(c.num_experts_per_tok, "num_experts_per_tok");
    positive(c.moe_intermediate_size, "moe_intermediate_size");
    if (c.num_experts_per_tok != 1) errors.push_back("only top-1 MoE routing is currently planned");
    if (c.num_experts_per_tok > c.num_experts) errors.push_back("num_experts_per_tok cannot exceed num_experts");
  }
  if (c.rope_scaling.enabled) {
    if (c.rope_scaling.type != "yarn") errors.push_back("only yarn rope scaling is supported");
    if (c.rope_scaling.factor <= 1.0F) errors.push_back("rope scaling factor must be greater than 1");
    if (c.rope_scaling.original_max_position_embeddings <= 0)
      errors.push_back("rope scaling original_max_position_embeddings must be positive");
  }
  return errors;
}

std::vector<std::string> validate_device_config(const MiniMindConfig& c) {
  std::vector<std::string> errors = validate_config(c);
  if (!errors.empty()) return errors;
  if (c.use_moe) errors.push_back("the gfx950 runtime implements the dense model only (use_moe=0)");
  const int64_t q_size = c.num_attention_heads * c.head_dim;
  const auto width = [&](int64_t v, const char* name) {
    if (v % 8 != 0 || v > 4096) errors.push_back(std::string(name) + " must be a multiple of 8 and <= 4096");
  };
  width(c.hidden_size, "hidden_size");
  width(q_size, "num_attention_heads * head_dim");
  width(c.intermediate_size, "intermediate_size");
  const int64_t d = c.head_dim;
  if (!(d == 16 || d == 32 || d == 64 || d == 96 || d == 128)) errors.push_back("head_dim must be 16, 32, 64, 96 or 128");
  if (c.num_attention_heads / c.num_key_value_heads > 8) errors.push_back("num_attention_heads / num_key_value_heads must be <= 8");
  if (c.vocab_size > (int64_t{1} << 30)) errors.push_back("vocab_size too large");
  if (c.max_position_embeddings > (int64_t{1} << 24)) errors.push_back("max_position_embeddings too large");
  return errors;
}

namespace {

std::string trim(const std::string& v) {
  size_t b = 0, e = v.size();
  while (b < e && std::isspace(static_cast<unsigned char>(v[b]))) ++b;
  while (e > b && std::isspace(static_cast<unsigned char>(v[e - 1]))) --e;
  return v.substr(b, e - b);
}

}  // namespace

MiniMindConfig config_from_file(const std::string& path) {
  std::ifstream in(path);
  if (!in) throw std::runtime_error("failed to open runtime config: " + path);
  std::unordered_map<std::string, std::string> kv;
  std::string line;
  while (std::getline(in, line)) {
    line = trim(line);
    if (line.empty() || line[0] == '#') continue;
    const size_t eq = line.find('=');
    if (eq == std::string::npos) throw std::runtime_error("invalid runtime config line: " + line);
    kv[trim(line.substr(0, eq))] = trim(line.substr(eq + 1));
  }
  const auto i64 = [&](const char* key, int64_t fallback) {
    const auto it = kv.find(key);
    return it == kv.end() ? fallback : static_cast<int64_t>(std::stoll(it->second));
  };
  const auto flag = [&](const char* key, bool fallback) {
    const auto it = kv.find(key);
    if (it == kv.end()) return fallback;
    return it->second == "1" || it->second == "true" || it->second == "True";
  };
  const auto f32 = [&](const char* key, float fallback) {
    const auto it = kv.find(key);
    return it == kv.end() ? fallback : std::stof(it->second);
  };
  MiniMindConfig c = default_minimind_config();
  c.hidden_size = i64("hidden_size", c.hidden_size);
  c.num_hidden_layers = i64("num_hidden_layers", c.num_hidden_layers);
  c.use_moe = flag("use_moe", false);
  c.vocab_size = i64("vocab_size", c.vocab_size);
  c.num_attention_heads = i64("num_attention_heads", c.num_attention_heads);
  c.num_key_value_heads = i64("num_key_value_heads", c.num_key_value_heads);
  c.head_dim = i64("head_dim", c.num_attention_heads > 0 ? c.hidden_size / c.num_attention_heads : 0);
  c.intermediate_size = i64("intermediate_size", c.intermediate_size);
  c.max_position_embeddings = i64("max_position_embeddings", c.max_position_embeddings);
  c.tie_word_embeddings = flag("tie_word_embeddings", c.tie_word_embeddings);
  c.num_experts = i64("num_experts", c.num_experts);
  c.num_experts_per_tok = i64("num_experts_per_tok", c.num_experts_per_tok);
  c.moe_intermediate_size = i64("moe_intermediate_size", c.intermediate_size);
  c.rms_norm_eps = f32("rms_norm_eps", c.rms_norm_eps);
  c.rope_theta = f32("rope_theta", c.rope_theta);
  return c;
}

}  // namespace minimind::model
