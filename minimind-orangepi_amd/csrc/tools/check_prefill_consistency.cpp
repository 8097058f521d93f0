// check_prefill_consistency -- the batched prompt path must agree with feeding
// the prompt one token at a time (bench/check_prefill_consistency.cpp:9-57 of
// the reference, same usage and output):
//   check_prefill_consistency <model-dir> [tokens] [--kv f16|f32]
// The probe prompt is token ids (i % 1000) + 1.  Both states then take four
// more greedy steps; next tokens and positions must match at every point.
// Prints "prefill consistency ok" and exits 0, or the first disagreement on
// stderr and exits 1.
#include "../runtime/language_model.h"
#include "tool_support.h"

#include <iostream>
#include <string>
#include <vector>

int main(int argc, char** argv) {
  using namespace minimind::model;
  if (argc < 2 || std::string(argv[1]).rfind("--", 0) == 0) {
    std::cerr << "usage: check_prefill_consistency <model-dir> [tokens] [--kv f16|f32]\n";
    return 1;
  }
  try {
    const int64_t n = argc >= 3 && std::string(argv[2]).rfind("--", 0) != 0 ? std::strtoll(argv[2], nullptr, 10) : 8;
    if (n <= 0) {
      std::cerr << "tokens must be positive\n";
      return 1;
    }
    const std::string kv_name = mmr_tools::Argv(argc, argv).text("--kv", "f32");
    const KvCacheDtype kv = kv_name == "f16" ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32;
    const LanguageModel model = load_runtime_language_model(argv[1]);
    std::vector<int32_t> prompt(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) prompt[static_cast<size_t>(i)] = static_cast<int32_t>(i % 1000 + 1);

    const int64_t capacity = n + 4;
    DecoderState stepwise = model.make_state(capacity, kv);
    DecoderState batched = model.make_state(capacity, kv);
    int32_t a = 0;
    for (int32_t t : prompt) a = model.forward_next_token(t, stepwise);
    int32_t b = model.prefill_next_token(prompt, batched);
    const auto report = [&](const char* where, int step) {
      std::cerr << where;
      if (step >= 0) std::cerr << " step=" << step;
      std::cerr << " token_by_token=" << a << " prefill=" << b << " token_by_token_pos=" << stepwise.position
                << " prefill_pos=" << batched.position << '\n';
      return 1;
    };
    if (a != b || stepwise.position != batched.position) return report("after the prompt:", -1);
    for (int step = 0; step < 4; ++step) {
      a = model.forward_next_token(a, stepwise);
      b = model.forward_next_token(b, batched);
      if (a != b || stepwise.position != batched.position) return report("follow-up", step);
    }
    std::cout << "prefill consistency ok\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "check_prefill_consistency: " << e.what() << '\n';
    return 1;
  }
}
