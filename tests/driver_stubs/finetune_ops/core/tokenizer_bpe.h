// Declarations of the reference's BPE tokenizers (GPT-2, Qwen2), for
// compiling the reference drivers' sources in tests/test_driver_sources.py.
// Tokenizers are outside this build; nothing is defined here.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace ops {

struct BPEConfig {
  static BPEConfig from_pretrained(const std::string& dir);
};
class GPT2BPETokenizer {
 public:
  explicit GPT2BPETokenizer(const BPEConfig& cfg);
  void load();
  std::vector<int32_t> encode(const std::string& text) const;
  std::string decode(const std::vector<int32_t>& ids) const;
};

struct QwenTokenizerConfig {
  int eos_token_id = 151643;
  static QwenTokenizerConfig from_pretrained(const std::string& dir);
};
class QwenBPETokenizer {
 public:
  explicit QwenBPETokenizer(const QwenTokenizerConfig& cfg);
  void load();
  std::vector<int32_t> encode(const std::string& text) const;
};

}  // namespace ops
