// bench_decode -- prefill/decode timing with the reference's flags and output
// keys (bench/bench_decode.cpp:117-151):
//   --model DIR --prompt TEXT --input-tokens 1,2 --tokens N --warmup W
// decode_steps = tokens - 1 as in the reference.  Without a runtime model
// directory it times the reference's toy model (bench_decode.cpp:124-126).
// --kv f16|f32 picks the KV cache dtype (default f16, the reference device
// cache's).  The reference times
// forward_next_token calls that each synchronise; --device-loop 1 instead
// enqueues the steps back to back with the token fed forward on the device
// and synchronises once (the runtime's throughput mode).
#include "../runtime/language_model.h"
#include "cli_args.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <iostream>

namespace {

using namespace minimind::model;

struct Timing {
  double prefill_seconds = 0, decode_seconds = 0;
  int64_t prefill_tokens = 0, decode_steps = 0;
};

Timing run(const LanguageModel& model, const std::vector<int32_t>& prompt, int64_t decode_tokens, bool device_loop,
           KvCacheDtype kv, std::vector<int32_t>& generated) {
  const int64_t cap = static_cast<int64_t>(prompt.size()) + std::max<int64_t>(decode_tokens, 1);
  DecoderState state = model.make_state(cap, kv);
  Timing t;
  const auto p0 = std::chrono::steady_clock::now();
  int32_t next = model.prefill_next_token(prompt, state);
  const auto p1 = std::chrono::steady_clock::now();
  generated.clear();
  const auto d0 = std::chrono::steady_clock::now();
  if (device_loop) {
    if (decode_tokens > 1) model.enqueue_decode(state, decode_tokens - 1);
    model.synchronize(state);
    const auto d1 = std::chrono::steady_clock::now();
    t.decode_seconds = std::chrono::duration<double>(d1 - d0).count();
    generated = model.read_sequence(state, static_cast<int64_t>(prompt.size()), std::max<int64_t>(decode_tokens, 0));
  } else {
    for (int64_t i = 0; i < decode_tokens; ++i) {
      generated.push_back(next);
      if (i + 1 < decode_tokens) next = model.forward_next_token(next, state);
    }
    const auto d1 = std::chrono::steady_clock::now();
    t.decode_seconds = std::chrono::duration<double>(d1 - d0).count();
  }
  t.prefill_seconds = std::chrono::duration<double>(p1 - p0).count();
  t.prefill_tokens = static_cast<int64_t>(prompt.size());
  t.decode_steps = std::max<int64_t>(0, decode_tokens - 1);
  return t;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const std::string model_dir = mmr_cli::arg_value(argc, argv, "--model", "");
    const std::string prompt = mmr_cli::arg_value(argc, argv, "--prompt", "hello");
    const std::string explicit_tokens = mmr_cli::arg_value(argc, argv, "--input-tokens", "");
    const int64_t decode_tokens = mmr_cli::int_arg_value(argc, argv, "--tokens", 16);
    const int64_t warmup = mmr_cli::int_arg_value(argc, argv, "--warmup", 1);
    const bool device_loop = mmr_cli::int_arg_value(argc, argv, "--device-loop", 0) != 0;
    const std::string kv_name = mmr_cli::arg_value(argc, argv, "--kv", "f16");
    if (kv_name != "f16" && kv_name != "f32") {
      std::cerr << "bench_decode: --kv must be f16 or f32\n";
      return 2;
    }
    const KvCacheDtype kv = kv_name == "f16" ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32;
    LanguageModel model = !model_dir.empty() && has_runtime_language_model(model_dir)
                              ? load_runtime_language_model(model_dir)
                              : make_toy_language_model();
    auto tokens = explicit_tokens.empty() ? std::vector<int32_t>{} : mmr_cli::parse_token_ids(explicit_tokens);
    if (tokens.empty()) tokens = mmr_cli::byte_prompt(prompt, model.config().vocab_size, model.config().bos_token_id);
    std::vector<int32_t> generated;
    for (int64_t i = 0; i < warmup; ++i) (void)run(model, tokens, decode_tokens, device_loop, kv, generated);
    const Timing t = run(model, tokens, decode_tokens, device_loop, kv, generated);
    const double dtps = t.decode_steps == 0 || t.decode_seconds == 0.0 ? 0.0 : t.decode_steps / t.decode_seconds;
    const double ptps = t.prefill_tokens == 0 || t.prefill_seconds == 0.0 ? 0.0 : t.prefill_tokens / t.prefill_seconds;
    std::cout << "prompt_tokens=" << tokens.size() << '\n';
    std::cout << "generated_tokens=" << generated.size() << '\n';
    std::cout << "prefill_tokens=" << t.prefill_tokens << '\n';
    std::cout << "prefill_seconds=" << t.prefill_seconds << '\n';
    std::cout << "prefill_tokens_per_second=" << ptps << '\n';
    std::cout << "decode_steps=" << t.decode_steps << '\n';
    std::cout << "decode_seconds=" << t.decode_seconds << '\n';
    std::cout << "decode_tokens_per_second=" << dtps << '\n';
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "bench_decode: " << e.what() << '\n';
    return 1;
  }
}
