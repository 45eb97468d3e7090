// finetune_ops/graph/safetensors_loader.h — checkpoint reading and writing in
// the safetensors format.
//
// Replaces graph/safetensors_loader.h of the reference (absent), as the
// drivers use it:
//   SafeTensorsReader reader(dir + "/model.safetensors");
//   reader.parse_header();
//   auto map = GPT2KeyMapper::generate_gpt2_mapping(cfg.n_layer);
//   SafeTensorsLoadOptions opts; opts.transpose_linear = false;
//   for (auto& kv : reader.load_tensors_mapped(map, opts)) model.assign_weight(kv.first, kv.second);
// (gpt2_small_lora_finetune/src/main.cpp:207-219, qwen_lora_finetune/src/wikitext_main.cpp:67-74,
// gemma_3_270m_lora_finetune/src/main.cpp:332-340) and reader.load_tensor(hf_key, transpose)
// (gpt2_medium_lora_finetune/src/eval_mmlu.cpp:84).
//
// File format: 8-byte little-endian header length N, N bytes of JSON
// {name: {"dtype", "shape", "data_offsets": [begin, end)}, "__metadata__": {str: str}},
// then the tensor bytes (offsets relative to the end of the header).
// F32 and F16 load as kFloat32 / kFloat16 tensors, BF16 widens exactly to
// kFloat32; other dtypes are rejected.  A mapping is internal name → HF key;
// a key absent from the file is also looked up with a "transformer.",
// "model." or "language_model." prefix added or removed, and a key found
// under none of them throws.  With transpose_linear, every 2-D tensor except
// the embeddings is transposed from HF's Linear [out, in] to [in, out].
//
// The host layer (read_host / read_mapped_host / write_safetensors) touches
// no device memory; load_tensor / load_tensors_mapped copy its result into
// GPU tensors.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {

struct SafeTensorsLoadOptions {
  bool transpose_linear = true;  // HF Linear [out, in] → [in, out] for 2-D non-embedding tensors
  bool verbose = true;           // one line per loaded tensor
};

struct SafeTensorInfo {
  std::string dtype;  // "F32", "F16", "BF16", ...
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte range within the data section
};

// A tensor in host memory, after dtype widening and optional transposition.
struct HostTensor {
  std::string name;
  DType dtype = kFloat32;
  std::vector<int64_t> shape;
  std::vector<uint8_t> bytes;
};

class SafeTensorsReader {
 public:
  explicit SafeTensorsReader(const std::string& path);
  // Reads and validates the header (called on first use if not called).
  void parse_header();

  std::vector<std::string> get_tensor_names();
  bool has_tensor(const std::string& key);
  const SafeTensorInfo& tensor_info(const std::string& key);
  const std::map<std::string, std::string>& metadata();

  // Host layer.
  HostTensor read_host(const std::string& key, bool transpose);
  std::vector<HostTensor> read_mapped_host(const std::unordered_map<std::string, std::string>& internal_to_hf,
                                           const SafeTensorsLoadOptions& opts);

  // GPU tensors.
  TensorPtr load_tensor(const std::string& key, bool transpose = false);
  std::unordered_map<std::string, TensorPtr> load_tensors_mapped(
      const std::unordered_map<std::string, std::string>& internal_to_hf, const SafeTensorsLoadOptions& opts = {});

 private:
  std::string resolve(const std::string& key);  // the key as stored in the file, or throws
  std::string path_;
  bool parsed_ = false;
  uint64_t data_start_ = 0, data_len_ = 0;
  std::map<std::string, SafeTensorInfo> tensors_;
  std::map<std::string, std::string> metadata_;
};

// One tensor to write: raw little-endian bytes of `dtype` ("F32", "F16", "BF16").
struct SafeTensorsEntry {
  std::string name;
  std::string dtype;
  std::vector<int64_t> shape;
  const void* data = nullptr;
  size_t nbytes = 0;
};

// Writes `entries` in the given order, data offsets back to back, the header
// padded with spaces so the data section starts 8-byte aligned.  Creates the
// parent directory.  Throws on a size that does not match dtype × shape.
void write_safetensors(const std::string& path, const std::vector<SafeTensorsEntry>& entries,
                       const std::map<std::string, std::string>& metadata = {});

// Internal parameter name → HF checkpoint key.
struct GPT2KeyMapper {
  // Internal names are the reference's: wte.weight, wpe.weight,
  // blocks.{i}.{ln_1,attn.qkv,attn.proj,ln_2,mlp.fc_in,mlp.fc_out}.{weight,bias},
  // ln_f.{weight,bias} (gpt2_small_lora_finetune/src/main_full.cpp:122-151);
  // HF keys h.{i}.attn.c_attn.weight, ... (GPT-2 Conv1D weights are [in, out]).
  static std::unordered_map<std::string, std::string> generate_gpt2_mapping(int n_layer);
};
struct QwenKeyMapper {
  // embed_tokens.weight, layers.{i}.{input_layernorm, self_attn.{q,k,v,o}_proj,
  // post_attention_layernorm, mlp.{gate,up,down}_proj}.*, norm.weight → "model." + name.
  static std::unordered_map<std::string, std::string> generate_qwen_mapping(int n_layer);
};
struct GemmaKeyMapper {
  // As Qwen2 without biases, plus self_attn.{q,k}_norm and the
  // pre/post_feedforward_layernorm of Gemma-3 decoder layers.
  static std::unordered_map<std::string, std::string> generate_gemma_mapping(int n_layer);
};

}  // namespace ops
