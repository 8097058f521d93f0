// tool_support.h -- what the three CLI tools share: an argv index, the model
// choice (runtime directory or the built-in toy), prompt ids and id lines.
//
// The command-line conventions are the reference tools' interface and are kept:
// `--name value` options where the first occurrence wins and a name in the last
// position has no value; bare switches such as `--stream`; token lists written
// `1,2,3` with empty fields skipped; a text prompt becomes one id per byte,
// folded into the vocabulary, and an empty prompt becomes [bos]
// (src/csrc/tools/minimind_generate.cpp:53-74 of the reference).
#pragma once

#include "../runtime/language_model.h"

#include <cstdint>
#include <cstdlib>
#include <optional>
#include <ostream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace mmr_tools {

// Every argv word after the program name, indexed by its first position.
class Argv {
 public:
  Argv(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) words_.emplace_back(argv[i]);
    for (size_t i = words_.size(); i-- > 0;) first_[words_[i]] = i;  // walking back leaves the first position
  }

  bool has(const std::string& name) const { return first_.count(name) != 0; }

  // The word after the first `name`, if there is one.
  std::optional<std::string> value(const std::string& name) const {
    const auto hit = first_.find(name);
    if (hit == first_.end() || hit->second + 1 >= words_.size()) return std::nullopt;
    return words_[hit->second + 1];
  }

  std::string text(const std::string& name, const std::string& fallback) const {
    return value(name).value_or(fallback);
  }

  // strtoll semantics (leading integer, 0 for none); an absent or empty value gives `fallback`.
  int64_t integer(const std::string& name, int64_t fallback) const {
    const auto v = value(name);
    return v && !v->empty() ? std::strtoll(v->c_str(), nullptr, 10) : fallback;
  }

  // i-th word that is not an option name or an option's value, given which names take values.
  std::optional<std::string> positional(size_t index, const std::vector<std::string>& valued) const {
    size_t seen = 0;
    for (size_t i = 0; i < words_.size(); ++i) {
      const std::string& w = words_[i];
      if (w.rfind("--", 0) == 0) {
        for (const auto& name : valued)
          if (w == name) ++i;  // skip its value too
        continue;
      }
      if (seen++ == index) return w;
    }
    return std::nullopt;
  }

 private:
  std::vector<std::string> words_;
  std::unordered_map<std::string, size_t> first_;
};

// `1,2,,3` -> {1, 2, 3}; each field converted like strtol.
inline std::vector<int32_t> split_ids(const std::string& list) {
  std::vector<int32_t> ids;
  for (size_t at = 0; at < list.size();) {
    size_t comma = list.find(',', at);
    if (comma == std::string::npos) comma = list.size();
    if (comma > at) ids.push_back(static_cast<int32_t>(std::strtol(list.substr(at, comma - at).c_str(), nullptr, 10)));
    at = comma + 1;
  }
  return ids;
}

// Explicit ids when the list option names any, else the bytes of the text
// prompt modulo the vocabulary, else [bos].  With `check_range`, an id outside
// [0, vocab) raises std::out_of_range (minimind_generate's behaviour).
inline std::vector<int32_t> prompt_ids(const Argv& args, const std::string& list_option,
                                       const std::string& default_text, const minimind::model::MiniMindConfig& cfg,
                                       bool check_range) {
  std::vector<int32_t> ids = split_ids(args.text(list_option, ""));
  if (ids.empty()) {
    const std::string text = args.text("--prompt", default_text);
    ids.reserve(text.size());
    for (unsigned char byte : text) ids.push_back(static_cast<int32_t>(byte % cfg.vocab_size));
  }
  if (ids.empty()) ids.push_back(cfg.bos_token_id);
  if (check_range)
    for (int32_t id : ids)
      if (id < 0 || id >= cfg.vocab_size) throw std::out_of_range("input token id is out of vocabulary range");
  return ids;
}

// The runtime model in `dir` when it holds one, else the reference's toy model.
inline minimind::model::LanguageModel open_model(const std::string& dir) {
  using namespace minimind::model;
  if (!dir.empty() && has_runtime_language_model(dir)) return load_runtime_language_model(dir);
  return make_toy_language_model();
}

// "label: 1 2 3" and a newline.
inline void write_id_line(std::ostream& out, const char* label, const std::vector<int32_t>& ids) {
  std::string line(label);
  line += ':';
  for (int32_t id : ids) (line += ' ') += std::to_string(id);
  out << line << '\n';
}

}  // namespace mmr_tools
