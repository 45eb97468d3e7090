// finetune_ops/graph/lora_injector.h — LoRA attachment for GPT-2.
//
// Replaces graph/lora_injector.h of the reference (absent): LoraSpec{rank,
// alpha, dropout, split_qkv, targets} with LoraTarget::{AttnQKV, AttnProj,
// MlpFcIn, MlpFcOut}, applied by LoraInjector().inject(model, spec)
// (gpt2_small_lora_finetune/src/main.cpp:264-276).  Adapters are A [r, in]
// and B [out, r] (PEFT layout, README.md:282,296) with scale alpha / r;
// dropout is PEFT's lora_dropout on the adapter input in training forwards
// (autograd enabled); split_qkv=false (the fused c_attn carries one adapter,
// as PEFT does).
#pragma once
#include <vector>

#include "finetune_ops/graph/gpt2_model.h"

namespace ops {

enum class LoraTarget { AttnQKV = 0, AttnProj = 1, MlpFcIn = 2, MlpFcOut = 3 };

struct LoraSpec {
  int rank = 8;
  float alpha = 16.0f;
  float dropout = 0.0f;
  bool split_qkv = false;
  std::vector<LoraTarget> targets = {LoraTarget::AttnQKV, LoraTarget::AttnProj};
};

class LoraInjector {
 public:
  void inject(GPT2Model& model, const LoraSpec& spec);
  void print_info() const;

 private:
  LoraSpec last_;
  int n_targets_ = 0;
};

}  // namespace ops
