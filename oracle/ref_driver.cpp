// ref_driver.cpp -- harness around a build of the reference's own CPU path.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles the reference sources
// where they lie under /root/reference (unmodified) and links them with this
// file into oracle/_ref/ref_driver.  Nothing here restates reference math: it
// calls the reference's LanguageModel (language_model.h:27-49).
//
// Modes (all print one JSON object on stdout):
//   generate <dir> <prompt_csv> <max_new> [logits_out.bin] [logit_steps_csv]
//       Builds MiniMindConfig from the runtime config file, honouring the
//       rms_norm_eps / rope_theta keys (the reference loader leaves them at
//       their defaults, runtime_loader.cpp:71-88), reads weights.bin, runs
//       LanguageModel::generate (language_model.cpp:398-406) and, step by
//       step, LanguageModel::forward_token for the logits of each generated
//       token.  Logits of the generated-token indices in logit_steps_csv are
//       appended to logits_out.bin as float32.
//   stream <dir> <prompt_csv> <steps> [logits_out.bin] [logit_steps_csv]
//       Greedy forward_token/argmax_token loop of exactly <steps> tokens with
//       no EOS stop; per step the top-2 margin and the runner-up id.
//   loader <dir> <prompt_csv> <max_new>
//       load_runtime_language_model (runtime_loader.cpp:177-182) + generate.
//   bench <dir> <prompt_csv> <decode_steps>
//       bench_decode.cpp:86-113 timing, with the prompt fed token by token
//       (prefill_next_token needs Ascend, language_model.cpp:339-341).
#include "language_model.h"
#include "runtime_loader.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

using minimind::model::DenseLayerWeights;
using minimind::model::DenseModelWeights;
using minimind::model::LanguageModel;
using minimind::model::MiniMindConfig;

namespace {

std::vector<int32_t> parse_csv(const std::string& s) {
  std::vector<int32_t> out;
  std::stringstream ss(s);
  std::string item;
  while (std::getline(ss, item, ','))
    if (!item.empty()) out.push_back(static_cast<int32_t>(std::strtol(item.c_str(), nullptr, 10)));
  return out;
}

std::string strip(const std::string& v) {
  size_t b = v.find_first_not_of(" \t\r\n");
  size_t e = v.find_last_not_of(" \t\r\n");
  return b == std::string::npos ? std::string() : v.substr(b, e - b + 1);
}

MiniMindConfig read_config(const std::string& path) {
  std::ifstream in(path);
  if (!in) throw std::runtime_error("failed to open " + path);
  std::map<std::string, std::string> kv;
  std::string line;
  while (std::getline(in, line)) {
    line = strip(line);
    if (line.empty() || line[0] == '#') continue;
    auto eq = line.find('=');
    if (eq == std::string::npos) throw std::runtime_error("bad config line: " + line);
    kv[strip(line.substr(0, eq))] = strip(line.substr(eq + 1));
  }
  auto i64 = [&](const char* k, int64_t fb) { return kv.count(k) ? std::stoll(kv[k]) : fb; };
  auto b = [&](const char* k, bool fb) {
    if (!kv.count(k)) return fb;
    return kv[k] == "1" || kv[k] == "true" || kv[k] == "True";
  };
  MiniMindConfig c = minimind::model::default_minimind_config();
  c.hidden_size = i64("hidden_size", c.hidden_size);
  c.num_hidden_layers = i64("num_hidden_layers", c.num_hidden_layers);
  c.use_moe = b("use_moe", false);
  c.vocab_size = i64("vocab_size", c.vocab_size);
  c.num_attention_heads = i64("num_attention_heads", c.num_attention_heads);
  c.num_key_value_heads = i64("num_key_value_heads", c.num_key_value_heads);
  c.head_dim = i64("head_dim", c.hidden_size / c.num_attention_heads);
  c.intermediate_size = i64("intermediate_size", c.intermediate_size);
  c.max_position_embeddings = i64("max_position_embeddings", c.max_position_embeddings);
  c.tie_word_embeddings = b("tie_word_embeddings", c.tie_word_embeddings);
  if (kv.count("rms_norm_eps")) c.rms_norm_eps = std::strtof(kv["rms_norm_eps"].c_str(), nullptr);
  if (kv.count("rope_theta")) c.rope_theta = std::strtof(kv["rope_theta"].c_str(), nullptr);
  return c;
}

std::vector<float> read_tensor(std::ifstream& in, const std::string& name) {
  uint64_t len = 0;
  in.read(reinterpret_cast<char*>(&len), 8);
  std::string got(len, '\0');
  in.read(&got[0], static_cast<std::streamsize>(len));
  if (!in || got != name) throw std::runtime_error("expected tensor " + name);
  uint64_t count = 0;
  in.read(reinterpret_cast<char*>(&count), 8);
  std::vector<float> v(count);
  in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(count * 4));
  if (!in) throw std::runtime_error("short tensor " + name);
  return v;
}

LanguageModel build_model(const std::string& dir) {
  MiniMindConfig c = read_config(dir + "/minimind_runtime_config.txt");
  std::ifstream in(dir + "/weights.bin", std::ios::binary);
  char magic[8];
  in.read(magic, 8);
  if (!in || std::string(magic, 8) != "MMRTW001") throw std::runtime_error("bad weights magic");
  DenseModelWeights w;
  w.embed_tokens = read_tensor(in, "model.embed_tokens.weight");
  w.final_norm = read_tensor(in, "model.norm.weight");
  w.lm_head = read_tensor(in, "lm_head.weight");
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    DenseLayerWeights L;
    L.input_norm = read_tensor(in, p + "input_layernorm.weight");
    L.post_attention_norm = read_tensor(in, p + "post_attention_layernorm.weight");
    L.q_norm = read_tensor(in, p + "self_attn.q_norm.weight");
    L.k_norm = read_tensor(in, p + "self_attn.k_norm.weight");
    L.q_proj = read_tensor(in, p + "self_attn.q_proj.weight");
    L.k_proj = read_tensor(in, p + "self_attn.k_proj.weight");
    L.v_proj = read_tensor(in, p + "self_attn.v_proj.weight");
    L.o_proj = read_tensor(in, p + "self_attn.o_proj.weight");
    L.gate_proj = read_tensor(in, p + "mlp.gate_proj.weight");
    L.up_proj = read_tensor(in, p + "mlp.up_proj.weight");
    L.down_proj = read_tensor(in, p + "mlp.down_proj.weight");
    w.layers.push_back(std::move(L));
  }
  return LanguageModel(std::move(c), std::move(w));
}

void print_tokens(const char* key, const std::vector<int32_t>& t) {
  std::printf("\"%s\": [", key);
  for (size_t i = 0; i < t.size(); ++i) std::printf("%s%d", i ? ", " : "", t[i]);
  std::printf("]");
}

int run_generate(const std::string& dir, const std::vector<int32_t>& prompt, int64_t max_new, const char* logits_path,
                 const std::vector<int32_t>& logit_steps) {
  LanguageModel model = build_model(dir);
  const auto generated = model.generate(prompt, max_new);

  // Step-by-step replay through forward_token for the logits that produced
  // each generated token (the CPU forward_next_token takes argmax of the same
  // logits, language_model.cpp:332).
  auto state = model.make_state();
  std::vector<float> logits;
  for (int32_t t : prompt) logits = model.forward_token(t, state);
  std::vector<int32_t> replay;
  std::vector<double> margin, lsum, lsq;
  std::FILE* lf = logits_path ? std::fopen(logits_path, "wb") : nullptr;
  for (int64_t i = 0; i < static_cast<int64_t>(generated.size()); ++i) {
    const int32_t next = minimind::model::argmax_token(logits);
    replay.push_back(next);
    std::vector<float> sorted(logits);
    std::partial_sort(sorted.begin(), sorted.begin() + 2, sorted.end(), std::greater<float>());
    margin.push_back(static_cast<double>(sorted[0]) - static_cast<double>(sorted[1]));
    double s = 0, q = 0;
    for (float v : logits) {
      s += v;
      q += static_cast<double>(v) * v;
    }
    lsum.push_back(s);
    lsq.push_back(q);
    if (lf && std::find(logit_steps.begin(), logit_steps.end(), static_cast<int32_t>(i)) != logit_steps.end())
      std::fwrite(logits.data(), 4, logits.size(), lf);
    if (i + 1 < static_cast<int64_t>(generated.size())) logits = model.forward_token(next, state);
  }
  if (lf) std::fclose(lf);
  std::printf("{");
  print_tokens("generated", generated);
  std::printf(", ");
  print_tokens("replay", replay);
  std::printf(", \"margin\": [");
  for (size_t i = 0; i < margin.size(); ++i) std::printf("%s%.9g", i ? ", " : "", margin[i]);
  std::printf("], \"logit_sum\": [");
  for (size_t i = 0; i < lsum.size(); ++i) std::printf("%s%.17g", i ? ", " : "", lsum[i]);
  std::printf("], \"logit_sumsq\": [");
  for (size_t i = 0; i < lsq.size(); ++i) std::printf("%s%.17g", i ? ", " : "", lsq[i]);
  std::printf("], \"eps\": %.9g, \"theta\": %.9g}\n", static_cast<double>(model.config().rms_norm_eps),
              static_cast<double>(model.config().rope_theta));
  return 0;
}

// Greedy continuation with no EOS stop (the device loop and the batched step
// decode a fixed number of steps): forward_token + argmax_token per step, as
// forward_next_token does (language_model.cpp:310-333).  Per step it records
// the top-2 margin and the runner-up id, so a GPU run that parts ways at a
// near-tie can be told apart from a wrong result.
int run_stream(const std::string& dir, const std::vector<int32_t>& prompt, int64_t steps, const char* logits_path,
               const std::vector<int32_t>& logit_steps) {
  LanguageModel model = build_model(dir);
  auto state = model.make_state();
  std::vector<float> logits;
  for (int32_t t : prompt) logits = model.forward_token(t, state);
  std::vector<int32_t> tokens, runner_up;
  std::vector<double> margin;
  std::FILE* lf = logits_path ? std::fopen(logits_path, "wb") : nullptr;
  for (int64_t i = 0; i < steps; ++i) {
    const int32_t next = minimind::model::argmax_token(logits);
    int32_t second = -1;
    for (int32_t j = 0; j < static_cast<int32_t>(logits.size()); ++j)
      if (j != next && (second < 0 || logits[j] > logits[second])) second = j;
    tokens.push_back(next);
    runner_up.push_back(second);
    margin.push_back(static_cast<double>(logits[next]) - static_cast<double>(logits[second]));
    if (lf && std::find(logit_steps.begin(), logit_steps.end(), static_cast<int32_t>(i)) != logit_steps.end())
      std::fwrite(logits.data(), 4, logits.size(), lf);
    if (i + 1 < steps) logits = model.forward_token(next, state);
  }
  if (lf) std::fclose(lf);
  std::printf("{");
  print_tokens("generated", tokens);
  std::printf(", ");
  print_tokens("runner_up", runner_up);
  std::printf(", \"margin\": [");
  for (size_t i = 0; i < margin.size(); ++i) std::printf("%s%.9g", i ? ", " : "", margin[i]);
  std::printf("], \"eps\": %.9g, \"theta\": %.9g}\n", static_cast<double>(model.config().rms_norm_eps),
              static_cast<double>(model.config().rope_theta));
  return 0;
}

int run_loader(const std::string& dir, const std::vector<int32_t>& prompt, int64_t max_new) {
  LanguageModel model = minimind::model::load_runtime_language_model(dir);
  const auto generated = model.generate(prompt, max_new);
  std::printf("{");
  print_tokens("generated", generated);
  std::printf(", \"eps\": %.9g}\n", static_cast<double>(model.config().rms_norm_eps));
  return 0;
}

int run_bench(const std::string& dir, const std::vector<int32_t>& prompt, int64_t decode_tokens) {
  LanguageModel model = build_model(dir);
  auto state = model.make_state();
  const auto p0 = std::chrono::steady_clock::now();
  int32_t next = 0;
  for (int32_t t : prompt) next = model.forward_next_token(t, state);
  const auto p1 = std::chrono::steady_clock::now();
  std::vector<int32_t> generated;
  const auto d0 = std::chrono::steady_clock::now();
  for (int64_t i = 0; i < decode_tokens; ++i) {
    generated.push_back(next);
    if (i + 1 < decode_tokens) next = model.forward_next_token(next, state);
  }
  const auto d1 = std::chrono::steady_clock::now();
  const double ps = std::chrono::duration<double>(p1 - p0).count();
  const double ds = std::chrono::duration<double>(d1 - d0).count();
  const int64_t steps = std::max<int64_t>(0, decode_tokens - 1);
  std::printf("{\"prefill_tokens\": %zu, \"prefill_seconds\": %.6f, \"decode_steps\": %lld, \"decode_seconds\": %.6f, "
              "\"decode_tokens_per_second\": %.6f, ",
              prompt.size(), ps, static_cast<long long>(steps), ds, ds > 0 ? steps / ds : 0.0);
  print_tokens("generated", generated);
  std::printf("}\n");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc < 5) {
      std::fprintf(stderr, "usage: ref_driver generate|loader|bench <dir> <prompt_csv> <n> [...]\n");
      return 2;
    }
    const std::string mode = argv[1];
    const std::string dir = argv[2];
    const auto prompt = parse_csv(argv[3]);
    const int64_t n = std::strtoll(argv[4], nullptr, 10);
    if (mode == "generate")
      return run_generate(dir, prompt, n, argc > 5 ? argv[5] : nullptr,
                          argc > 6 ? parse_csv(argv[6]) : std::vector<int32_t>{});
    if (mode == "stream")
      return run_stream(dir, prompt, n, argc > 5 ? argv[5] : nullptr,
                        argc > 6 ? parse_csv(argv[6]) : std::vector<int32_t>{});
    if (mode == "loader") return run_loader(dir, prompt, n);
    if (mode == "bench") return run_bench(dir, prompt, n);
    std::fprintf(stderr, "unknown mode %s\n", mode.c_str());
    return 2;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_driver error: %s\n", e.what());
    return 1;
  }
}
