// finetune_ops/graph/lora_saver.h — LoRA adapters to and from safetensors.
//
// Replaces graph/lora_saver.h of the reference (absent), as the drivers use it:
//   LoraSaver::save_safetensors(path, model, active_lora_spec);          // main.cpp:585-606
//   auto st = LoraSaver::load_safetensors(path);                          // main.cpp:244-262
//   if (st.compatible_with(model)) LoraSaver::attach_from_state(model, st);   // eval_ppl.cpp:112-123
//   spec.rank = st.rank; spec.alpha = st.alpha; spec.targets = st.targets; ...
//
// Files are PEFT adapters ("PEFT-compatible SafeTensors format", README.md:282):
//   base_model.model.<HF module path>.lora_A.weight  [r, in]   F32
//   base_model.model.<HF module path>.lora_B.weight  [out, r]  F32
// with the module path transformer.h.{i}.attn.c_attn (GPT-2) or
// model.layers.{i}.self_attn.q_proj (Qwen2, Gemma3), and string metadata
// lora_rank, lora_alpha, lora_dropout, split_qkv, targets (GPT-2 LoraTarget
// names) / target_modules.  Saving to a file named adapter_model.safetensors
// also writes PEFT's adapter_config.json beside it.  Loading reads rank from
// lora_A's shape and alpha from the metadata, else from an
// adapter_config.json beside the file, else alpha = rank.
#pragma once
#include <string>
#include <unordered_map>
#include <vector>

#include "finetune_ops/core/tensor.h"
#include "finetune_ops/graph/engine_model.h"
#include "finetune_ops/graph/gemma_lora_injector.h"
#include "finetune_ops/graph/lora_injector.h"

namespace ops {

struct LoraState {
  int rank = 0;
  float alpha = 0.f;
  float dropout = 0.f;
  bool split_qkv = false;
  std::vector<LoraTarget> targets;          // GPT-2 adapters
  std::vector<std::string> target_modules;  // Qwen2 / Gemma3 adapters (q_proj, ..., down_proj)
  int arch = -1;                            // 0 GPT-2, 1 HF-style decoder (Qwen2 / Gemma3)
  int n_layer = 0;                          // 1 + the largest layer index present
  std::unordered_map<std::string, TensorPtr> tensors;  // PEFT key → GPU tensor

  // Same architecture family, every layer index inside the model, and
  // every adapter's shape equal to what the model's linear needs at this rank.
  bool compatible_with(const EngineModel& model) const;
};

class LoraSaver {
 public:
  static void save_safetensors(const std::string& path, EngineModel& model, const LoraSpec& spec);
  static void save_safetensors(const std::string& path, EngineModel& model, const GemmaLoraSpec& spec);
  // Alpha and dropout from the model's attached adapters.
  static void save_safetensors(const std::string& path, EngineModel& model);
  static LoraState load_safetensors(const std::string& path);
  // Attaches adapters with the state's rank, alpha and targets (replacing
  // any present) and copies its tensors in.  Throws when !compatible_with.
  static void attach_from_state(EngineModel& model, const LoraState& state);
};

}  // namespace ops
