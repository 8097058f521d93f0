// bench_decode -- prefill and decode timing of one greedy run.
//
// Interface of the reference tool (bench/bench_decode.cpp:117-151):
//   --model DIR  --prompt TEXT (default "hello")  --input-tokens 1,2
//   --tokens N (default 16, ids collected)  --warmup W (default 1)
// stdout: eight key=value lines, prompt_tokens, generated_tokens,
// prefill_tokens, prefill_seconds, prefill_tokens_per_second, decode_steps,
// decode_seconds, decode_tokens_per_second.  Timing semantics kept from the
// reference: W untimed runs on fresh states, then one timed run on a fresh
// state; the prefill clock covers prefill_next_token, the decode clock covers
// the N-1 greedy steps that produce ids 2..N; decode_steps = N - 1; a rate is 0
// when its count or time is 0.  Without a runtime model directory the toy model
// runs (bench_decode.cpp:124-126).
//
// Added here:
//   --kv f16|f32      KV cache dtype (default f16, the reference device cache's)
//   --device-loop 1   enqueue the N-1 steps back to back with the token fed
//                     forward on the device and one synchronisation at the end
//                     (the runtime's throughput mode); 0 (default) makes one
//                     synchronous forward_next_token call per step, as the
//                     reference does.
#include "tool_support.h"

#include <algorithm>
#include <chrono>
#include <iostream>
#include <sstream>
#include <string>
#include <utility>

namespace {

using minimind::model::DecoderState;
using minimind::model::KvCacheDtype;
using minimind::model::LanguageModel;

template <class Work>
double seconds_spent(Work&& work) {
  const auto begin = std::chrono::steady_clock::now();
  work();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - begin).count();
}

double rate(double count, double seconds) { return count == 0.0 || seconds == 0.0 ? 0.0 : count / seconds; }

// Counts print as integers, times and rates in the stream's default format.
std::string as_text(int64_t count) { return std::to_string(count); }
std::string as_text(double number) {
  std::ostringstream out;
  out << number;
  return out.str();
}

struct Settings {
  int64_t wanted = 16;  // ids to collect: the prefill's prediction plus wanted-1 steps
  int64_t warmup = 1;
  bool device_loop = false;
  KvCacheDtype kv = KvCacheDtype::kFloat16;
};

struct Measured {
  std::vector<int32_t> ids;
  double prefill_s = 0.0;
  double decode_s = 0.0;
};

Measured measure_once(const LanguageModel& model, const std::vector<int32_t>& prompt, const Settings& s) {
  const int64_t prompt_len = static_cast<int64_t>(prompt.size());
  const int64_t steps = std::max<int64_t>(s.wanted - 1, 0);
  DecoderState state = model.make_state(prompt_len + steps + 1, s.kv);
  Measured m;
  int32_t last = 0;
  m.prefill_s = seconds_spent([&] { last = model.prefill_next_token(prompt, state); });
  if (s.wanted <= 0) return m;
  if (s.device_loop) {
    m.decode_s = seconds_spent([&] {
      if (steps > 0) model.enqueue_decode(state, steps);
      model.synchronize(state);
    });
    m.ids = model.read_sequence(state, prompt_len, s.wanted);
  } else {
    m.ids.reserve(static_cast<size_t>(s.wanted));
    m.decode_s = seconds_spent([&] {
      m.ids.push_back(last);
      for (int64_t i = 0; i < steps; ++i) m.ids.push_back(last = model.forward_next_token(last, state));
    });
  }
  return m;
}

int bench(const mmr_tools::Argv& args) {
  Settings s;
  const std::string kv = args.text("--kv", "f16");
  if (kv != "f16" && kv != "f32") {
    std::cerr << "bench_decode: --kv must be f16 or f32\n";
    return 2;
  }
  s.kv = kv == "f16" ? KvCacheDtype::kFloat16 : KvCacheDtype::kFloat32;
  s.wanted = args.integer("--tokens", 16);
  s.warmup = args.integer("--warmup", 1);
  s.device_loop = args.integer("--device-loop", 0) != 0;

  const LanguageModel model = mmr_tools::open_model(args.text("--model", ""));
  const std::vector<int32_t> prompt = mmr_tools::prompt_ids(args, "--input-tokens", "hello", model.config(), false);
  for (int64_t i = 0; i < s.warmup; ++i) (void)measure_once(model, prompt, s);
  const Measured m = measure_once(model, prompt, s);

  const int64_t prompt_len = static_cast<int64_t>(prompt.size());
  const int64_t steps = std::max<int64_t>(s.wanted - 1, 0);
  const std::pair<const char*, std::string> rows[] = {
      {"prompt_tokens", as_text(prompt_len)},
      {"generated_tokens", as_text(static_cast<int64_t>(m.ids.size()))},
      {"prefill_tokens", as_text(prompt_len)},
      {"prefill_seconds", as_text(m.prefill_s)},
      {"prefill_tokens_per_second", as_text(rate(static_cast<double>(prompt_len), m.prefill_s))},
      {"decode_steps", as_text(steps)},
      {"decode_seconds", as_text(m.decode_s)},
      {"decode_tokens_per_second", as_text(rate(static_cast<double>(steps), m.decode_s))},
  };
  for (const auto& [key, text] : rows) std::cout << key << '=' << text << '\n';
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return bench(mmr_tools::Argv(argc, argv));
  } catch (const std::exception& e) {
    std::cerr << "bench_decode: " << e.what() << '\n';
    return 1;
  }
}
