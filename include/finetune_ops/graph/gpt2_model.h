// finetune_ops/graph/gpt2_model.h — GPT-2 with LoRA on the MI355X backend.
//
// Replaces graph/gpt2_model.h of the reference (absent): GPT2Config (with
// from_pretrained(config.json)), GPT2Model{tie_weights, print_model_info,
// assign_weight, init_lora_modules, get_block(i).{qkv_lin, proj_lin,
// fc_in_lin, fc_out_lin}->clear_lora(), get_lora_parameters, parameters,
// forward(ids, mask), config} as driven by
// gpt2_small_lora_finetune/src/main.cpp:202-276 and main_full.cpp:122-151.
// Linear weights are [in, out] (HF Conv1D layout, main.cpp:211-214); the LM
// head is the tied token embedding.  Parameter names are the HF ones without
// the "transformer." prefix (which is also accepted): wte, wpe,
// h.{i}.ln_1.weight, h.{i}.attn.c_attn.weight / .bias / .lora_A / .lora_B,
// h.{i}.attn.c_proj.*, h.{i}.ln_2.*, h.{i}.mlp.c_fc.*, h.{i}.mlp.c_proj.*,
// ln_f.weight / .bias.  The reference's internal names (wte.weight,
// blocks.{i}.attn.qkv.weight, blocks.{i}.attn.proj.*, blocks.{i}.mlp.fc_in.*,
// blocks.{i}.mlp.fc_out.*, main_full.cpp:122-151) are accepted as aliases.
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "finetune_ops/graph/engine_model.h"

namespace ops {

struct GPT2Config {
  int vocab_size = 50257;
  int n_positions = 1024;
  int n_embd = 768;
  int n_layer = 12;
  int n_head = 12;
  int n_inner = 0;  // 0 → 4·n_embd
  float layer_norm_epsilon = 1e-5f;
  // Reads the numeric fields of a HF GPT-2 config.json.
  static GPT2Config from_pretrained(const std::string& config_json_path);
};

// One LoRA-capable linear of a block (a handle into the model).
class LoraSlot {
 public:
  LoraSlot(EngineModel* m, int bit) : model_(m), bit_(bit) {}
  bool has_lora() const;
  // Detaches this linear's adapter; the next LoraInjector::inject re-attaches
  // adapters for the targets it names.
  void clear_lora();

 private:
  EngineModel* model_;
  int bit_;
};

struct GPT2Block {
  std::shared_ptr<LoraSlot> qkv_lin, proj_lin, fc_in_lin, fc_out_lin;
};

class GPT2Model : public EngineModel {
 public:
  explicit GPT2Model(const GPT2Config& cfg);
  void tie_weights() {}  // the LM head always reads the token embedding
  void print_model_info() const;
  void init_lora_modules() {}  // adapters attach in LoraInjector::inject
  GPT2Block& get_block(int i);
  const GPT2Config& config() const { return cfg_; }
  void clear_lora_bits(int bits);

 protected:
  std::string normalise_name(const std::string& name) const override;

 private:
  GPT2Config cfg_;
  std::vector<GPT2Block> blocks_;
};

}  // namespace ops
