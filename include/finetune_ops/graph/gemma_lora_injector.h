// finetune_ops/graph/gemma_lora_injector.h — LoRA adapters for GemmaModel.
//
// Replaces graph/gemma_lora_injector.h of the reference (absent), driven as
// GemmaLoraSpec::full_attn_mlp() / attention_only() / attention_light(),
// optionally with target_modules overridden, then
// GemmaLoraInjector().inject(model, spec); print_info()
// (gemma_3_270m_lora_finetune/src/main.cpp:3,357-376; target names from
// pytorch_alignment/gemma_lora_finetune.py:144-151).
#pragma once
#include <string>
#include <vector>

#include "finetune_ops/graph/gemma_model.h"

namespace ops {

struct GemmaLoraSpec {
  int rank = 8;
  float alpha = 32.0f;
  // Dropout on the LoRA branch's input in training forwards (PEFT's
  // lora_dropout).  The presets leave it at 0, the benchmark setting; the
  // reference's preset value is not in the published tree.
  float dropout = 0.0f;
  std::vector<std::string> target_modules;  // q_proj k_proj v_proj o_proj gate_proj up_proj down_proj
  static GemmaLoraSpec full_attn_mlp();
  static GemmaLoraSpec attention_only();
  static GemmaLoraSpec attention_light();  // q_proj, v_proj
};

class GemmaLoraInjector {
 public:
  void inject(GemmaModel& model, const GemmaLoraSpec& spec);
  void print_info() const;
  const GemmaLoraSpec& spec() const { return last_; }

 private:
  GemmaLoraSpec last_;
};

}  // namespace ops
