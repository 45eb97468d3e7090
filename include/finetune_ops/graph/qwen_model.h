// finetune_ops/graph/qwen_model.h — Qwen2 with LoRA on the MI355X backend.
//
// Replaces the reference's QwenConfig / QwenModel (absent), driven as
// QwenConfig::from_pretrained(dir + "/config.json"), QwenModel(cfg),
// assign_weight(name, t) with W transposed to [in, out] at load,
// init_lora(r, alpha, dropout[, qv_only]), freeze_base(), get_lora_parameters()
// (qwen_lora_finetune/src/wikitext_main.cpp:63-79, mmlu_main.cpp:125,145,217).
// dropout is PEFT's lora_dropout on the adapter inputs in training forwards
// (autograd enabled); the WikiText driver's default is 0.05 (:26).
// Adapters on q/k/v/o (q/v only with qv_only).  RMSNorm, SwiGLU MLP, RoPE,
// grouped KV heads, q/k/v biases.  Names are HF's without the "model."
// prefix (also accepted): embed_tokens.weight,
// layers.{i}.self_attn.{q,k,v,o}_proj.weight / .bias / .lora_A / .lora_B,
// layers.{i}.mlp.{gate,up,down}_proj.weight,
// layers.{i}.{input,post_attention}_layernorm.weight, norm.weight.
#pragma once
#include <string>

#include "finetune_ops/graph/engine_model.h"

namespace ops {

struct QwenConfig {
  int vocab_size = 151936;
  int hidden_size = 896;
  int intermediate_size = 4864;
  int num_hidden_layers = 24;
  int num_attention_heads = 14;
  int num_key_value_heads = 2;
  int max_position_embeddings = 32768;
  float rms_norm_eps = 1e-6f;
  double rope_theta = 1000000.0;
  static QwenConfig from_pretrained(const std::string& config_json_path);
};

class QwenModel : public EngineModel {
 public:
  explicit QwenModel(const QwenConfig& cfg);
  void init_lora(int rank, float alpha, float dropout, bool qv_only = false);
  void freeze_base() {}  // base weights are never trainable on this backend
  const QwenConfig& config() const { return cfg_; }

 protected:
  std::string normalise_name(const std::string& name) const override;

 private:
  QwenConfig cfg_;
};

}  // namespace ops
