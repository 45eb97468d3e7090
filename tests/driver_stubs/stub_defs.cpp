// Definitions for the data-layer and tokenizer declarations in this folder,
// so the reference drivers' objects link into executables against
// libfinetune_ops.so in tests/test_driver_sources.py (the link shows that
// every operators-API symbol a driver references is defined by the library).
// These parts are outside this build: every function throws if called.
#include <stdexcept>

#include "finetune_ops/core/tokenizer_bpe.h"
#include "finetune_ops/core/tokenizer_gemma.h"
#include "finetune_ops/data/wikitext2_dataset.h"

namespace ops {
namespace {
[[noreturn]] void outside(const char* what) {
  throw std::runtime_error(std::string(what) + " is outside this build (data layer / tokenizers)");
}
}  // namespace

BPEConfig BPEConfig::from_pretrained(const std::string&) { outside("BPEConfig::from_pretrained"); }
GPT2BPETokenizer::GPT2BPETokenizer(const BPEConfig&) { outside("GPT2BPETokenizer"); }
void GPT2BPETokenizer::load() { outside("GPT2BPETokenizer::load"); }
std::vector<int32_t> GPT2BPETokenizer::encode(const std::string&) const { outside("GPT2BPETokenizer::encode"); }
std::string GPT2BPETokenizer::decode(const std::vector<int32_t>&) const { outside("GPT2BPETokenizer::decode"); }

QwenTokenizerConfig QwenTokenizerConfig::from_pretrained(const std::string&) {
  outside("QwenTokenizerConfig::from_pretrained");
}
QwenBPETokenizer::QwenBPETokenizer(const QwenTokenizerConfig&) { outside("QwenBPETokenizer"); }
void QwenBPETokenizer::load() { outside("QwenBPETokenizer::load"); }
std::vector<int32_t> QwenBPETokenizer::encode(const std::string&) const { outside("QwenBPETokenizer::encode"); }

GemmaTokenizerConfig GemmaTokenizerConfig::from_pretrained(const std::string&) {
  outside("GemmaTokenizerConfig::from_pretrained");
}
GemmaTokenizer::GemmaTokenizer(const GemmaTokenizerConfig&) { outside("GemmaTokenizer"); }
void GemmaTokenizer::load() { outside("GemmaTokenizer::load"); }
std::vector<int> GemmaTokenizer::encode(const std::string&, bool, int, bool) const {
  outside("GemmaTokenizer::encode");
}
int GemmaTokenizer::get_eos_token_id() const { outside("GemmaTokenizer::get_eos_token_id"); }
int GemmaTokenizer::get_pad_token_id() const { outside("GemmaTokenizer::get_pad_token_id"); }

WikiText2Dataset::WikiText2Dataset(const WT2Config&, GPT2BPETokenizer*) { outside("WikiText2Dataset"); }
WikiText2Dataset::WikiText2Dataset(const WT2Config&, EncodeFn) { outside("WikiText2Dataset"); }
void WikiText2Dataset::load(Split) { outside("WikiText2Dataset::load"); }
size_t WikiText2Dataset::num_sequences() const { outside("WikiText2Dataset::num_sequences"); }
void WikiText2Dataset::reset_cursor() { outside("WikiText2Dataset::reset_cursor"); }
WT2Batch WikiText2Dataset::next_batch(int, bool) { outside("WikiText2Dataset::next_batch"); }
std::vector<int32_t> WikiText2Dataset::peek_tokens(size_t) const { outside("WikiText2Dataset::peek_tokens"); }

}  // namespace ops
