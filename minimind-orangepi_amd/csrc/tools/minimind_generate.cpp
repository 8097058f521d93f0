// minimind_generate -- greedy generation from the command line.
//
// Interface of the reference tool (src/csrc/tools/minimind_generate.cpp:77-111):
//   --model DIR  --prompt TEXT (default "MiniMind")  --tokens 1,2,3
//   --max-new-tokens N (default 8)  --stream
// stdout: "prompt_tokens: ...", with --stream one "token: N" line per id as it
// is produced, then "generated_tokens: ...".  With no runtime model directory
// the reference's built-in toy model runs, on the GPU like any other model.
//
// Every id goes through one sink that records it and, when streaming, echoes
// it at once; the blocking and streaming modes differ only in that echo.
#include "tool_support.h"

#include <iostream>

namespace {

class IdSink {
 public:
  IdSink(std::ostream& out, bool echo) : out_(out), echo_(echo) {}
  void operator()(int32_t id) {
    ids_.push_back(id);
    if (echo_) out_ << "token: " << id << std::endl;  // one flushed line per id
  }
  const std::vector<int32_t>& ids() const { return ids_; }

 private:
  std::ostream& out_;
  bool echo_;
  std::vector<int32_t> ids_;
};

void generate_to(std::ostream& out, const mmr_tools::Argv& args) {
  const minimind::model::LanguageModel model = mmr_tools::open_model(args.text("--model", ""));
  const std::vector<int32_t> prompt = mmr_tools::prompt_ids(args, "--tokens", "MiniMind", model.config(), true);
  const int64_t budget = args.integer("--max-new-tokens", 8);
  const bool streaming = args.has("--stream");

  mmr_tools::write_id_line(out, "prompt_tokens", prompt);
  if (streaming) out.flush();  // the prompt line reaches a reader before the first id
  IdSink sink(out, streaming);
  model.generate_stream(prompt, budget, [&sink](int32_t id) { sink(id); });
  mmr_tools::write_id_line(out, "generated_tokens", sink.ids());
  out.flush();
}

}  // namespace

int main(int argc, char** argv) {
  try {
    generate_to(std::cout, mmr_tools::Argv(argc, argv));
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "minimind_generate: " << e.what() << '\n';
    return 1;
  }
}
