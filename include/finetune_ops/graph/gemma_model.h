// finetune_ops/graph/gemma_model.h — Gemma-3 with LoRA on the MI355X backend.
//
// Replaces the reference's GemmaTextConfig / GemmaModel / GemmaLoraSpec /
// GemmaLoraInjector (absent), driven as GemmaTextConfig::from_pretrained(dir),
// GemmaModel(cfg), assign_weight, GemmaLoraSpec::full_attn_mlp() /
// attention_only() / attention_light() with target_modules, then
// GemmaLoraInjector().inject(model, spec) (gemma_3_270m_lora_finetune/src/
// main.cpp:326-379; target names from pytorch_alignment/
// gemma_lora_finetune.py:144-151).  RMSNorm with (1 + w), √d embedding
// scale, q/k RMSNorm, GeGLU MLP, grouped KV heads, local (sliding-window,
// rope_local_base_freq) and global layers.  Names are HF's without the
// "model." / "language_model.model." prefixes (both accepted).
#pragma once
#include <string>
#include <vector>

#include "finetune_ops/graph/engine_model.h"

namespace ops {

struct GemmaTextConfig {
  int vocab_size = 262144;
  int hidden_size = 640;
  int intermediate_size = 2048;
  int num_hidden_layers = 18;
  int num_attention_heads = 4;
  int num_key_value_heads = 1;
  int head_dim = 256;
  int max_position_embeddings = 32768;
  int sliding_window = 512;
  int sliding_window_pattern = 6;  // every 6th layer global
  float rms_norm_eps = 1e-6f;
  double rope_theta = 1000000.0;
  double rope_local_base_freq = 10000.0;
  float query_pre_attn_scalar = 256.f;
  bool weights_fp16 = false;  // store frozen W and the embedding as fp16
  static GemmaTextConfig from_pretrained(const std::string& model_dir);
};

class GemmaModel : public EngineModel {
 public:
  explicit GemmaModel(const GemmaTextConfig& cfg);
  const GemmaTextConfig& config() const { return cfg_; }
  void set_debug_retain_grads(bool) {}

 protected:
  std::string normalise_name(const std::string& name) const override;

 private:
  GemmaTextConfig cfg_;
};

struct GemmaLoraSpec {
  int rank = 8;
  float alpha = 32.0f;
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

 private:
  GemmaLoraSpec last_;
};

}  // namespace ops
