// cli_args.h -- flag parsing shared by the CLI tools (same conventions as the
// reference tools: `--name value`, comma-separated token lists).
#pragma once

#include <cstdint>
#include <cstdlib>
#include <sstream>
#include <string>
#include <vector>

namespace mmr_cli {

inline std::string arg_value(int argc, char** argv, const std::string& name, const std::string& fallback) {
  for (int i = 1; i + 1 < argc; ++i)
    if (argv[i] == name) return argv[i + 1];
  return fallback;
}

inline bool has_arg(int argc, char** argv, const std::string& name) {
  for (int i = 1; i < argc; ++i)
    if (argv[i] == name) return true;
  return false;
}

inline int64_t int_arg_value(int argc, char** argv, const std::string& name, int64_t fallback) {
  const std::string v = arg_value(argc, argv, name, "");
  return v.empty() ? fallback : std::strtoll(v.c_str(), nullptr, 10);
}

inline std::vector<int32_t> parse_token_ids(const std::string& value) {
  std::vector<int32_t> tokens;
  std::stringstream stream(value);
  std::string item;
  while (std::getline(stream, item, ','))
    if (!item.empty()) tokens.push_back(static_cast<int32_t>(std::strtol(item.c_str(), nullptr, 10)));
  return tokens;
}

// Byte-level tokenizer of the reference CLI (tokenizer.cpp:7-14): one id per
// byte, folded into the vocabulary with `% vocab`; empty prompt -> [bos].
inline std::vector<int32_t> byte_prompt(const std::string& text, int64_t vocab, int32_t bos) {
  std::vector<int32_t> tokens;
  for (unsigned char b : text) tokens.push_back(static_cast<int32_t>(b) % static_cast<int32_t>(vocab));
  if (tokens.empty()) tokens.push_back(bos);
  return tokens;
}

}  // namespace mmr_cli
