// Declarations of the reference's Gemma tokenizer, for compiling the
// reference drivers' sources in tests/test_driver_sources.py.  Tokenizers are
// outside this build; nothing is defined here.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace ops {

struct GemmaTokenizerConfig {
  static GemmaTokenizerConfig from_pretrained(const std::string& dir);
};
class GemmaTokenizer {
 public:
  explicit GemmaTokenizer(const GemmaTokenizerConfig& cfg);
  void load();
  std::vector<int> encode(const std::string& text, bool add_bos, int max_len, bool truncate) const;
  int get_eos_token_id() const;
  int get_pad_token_id() const;
};

}  // namespace ops
