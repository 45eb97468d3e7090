// Declarations of the reference's data layer (WikiText2Dataset, WT2Config),
// for compiling the reference drivers' sources against this build's headers
// in tests/test_driver_sources.py.  The data layer is outside this build
// (the benchmark feeds synthetic token ids), so only the names, members and
// signatures the drivers use are declared here; nothing is defined.
#pragma once
#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {

class GPT2BPETokenizer;

enum class Split { Train, Valid, Test };

struct WT2Config {
  std::string train_path, valid_path, test_path;
  std::string jsonl_train, jsonl_valid, jsonl_test;
  std::string pretokenized_path, pretokenized_meta;
  int seq_len = 128;
  int stride = -1;
  int eos_id = -1;
  int pad_id = 0;
  uint64_t seed = 42;
  bool streaming_mode = true;
  bool shuffle_train = true;
  bool drop_last = true;
  bool insert_eos_between_lines = false;
  float data_fraction = 1.0f;
};

struct WT2Batch {
  TensorPtr input_ids, attention_mask, labels;
};

class WikiText2Dataset {
 public:
  using EncodeFn = std::function<std::vector<int32_t>(const std::string&)>;
  WikiText2Dataset(const WT2Config& cfg, GPT2BPETokenizer* tokenizer);
  WikiText2Dataset(const WT2Config& cfg, EncodeFn encode);
  void load(Split split);
  size_t num_sequences() const;
  void reset_cursor();
  WT2Batch next_batch(int batch_size, bool loop = true);
  std::vector<int32_t> peek_tokens(size_t n) const;
};

}  // namespace ops
