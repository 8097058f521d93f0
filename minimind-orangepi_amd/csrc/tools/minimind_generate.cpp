// minimind_generate -- greedy generation CLI with the reference's flags and
// stdout protocol (src/csrc/tools/minimind_generate.cpp:77-111):
//   --model DIR --prompt TEXT --tokens 1,2,3 --max-new-tokens N [--stream]
// prints "prompt_tokens: ...", optional "token: N" lines, "generated_tokens: ...".
// Without a runtime model directory it runs the reference's built-in toy model
// (minimind_generate.cpp:84-86), on the GPU like any other model.
#include "../runtime/language_model.h"
#include "cli_args.h"

#include <iostream>
#include <stdexcept>

int main(int argc, char** argv) {
  using namespace minimind::model;
  try {
    const std::string prompt = mmr_cli::arg_value(argc, argv, "--prompt", "MiniMind");
    const std::string explicit_tokens = mmr_cli::arg_value(argc, argv, "--tokens", "");
    const std::string model_dir = mmr_cli::arg_value(argc, argv, "--model", "");
    const int64_t max_new = mmr_cli::int_arg_value(argc, argv, "--max-new-tokens", 8);
    const bool stream = mmr_cli::has_arg(argc, argv, "--stream");
    LanguageModel model = !model_dir.empty() && has_runtime_language_model(model_dir)
                              ? load_runtime_language_model(model_dir)
                              : make_toy_language_model();
    auto tokens = explicit_tokens.empty() ? std::vector<int32_t>{} : mmr_cli::parse_token_ids(explicit_tokens);
    if (tokens.empty()) tokens = mmr_cli::byte_prompt(prompt, model.config().vocab_size, model.config().bos_token_id);
    for (int32_t t : tokens)
      if (t < 0 || t >= model.config().vocab_size) throw std::out_of_range("input token id is out of vocabulary range");
    std::cout << "prompt_tokens:";
    for (int32_t t : tokens) std::cout << ' ' << t;
    std::cout << '\n';
    std::vector<int32_t> generated;
    if (stream) {
      std::cout << std::flush;
      model.generate_stream(tokens, max_new, [&generated](int32_t t) {
        generated.push_back(t);
        std::cout << "token: " << t << '\n' << std::flush;
      });
    } else {
      generated = model.generate(tokens, max_new);
    }
    std::cout << "generated_tokens:";
    for (int32_t t : generated) std::cout << ' ' << t;
    std::cout << '\n' << std::flush;
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "minimind_generate: " << e.what() << '\n';
    return 1;
  }
}
