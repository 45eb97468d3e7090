// finetune_ops/graph/gemma_model.h — Gemma-3 with LoRA on the MI355X backend.
//
// Replaces the reference's GemmaTextConfig / GemmaModel / GemmaLoraSpec /
// GemmaLoraInjector (absent), driven as GemmaTextConfig::from_pretrained(dir),
// GemmaModel(cfg), assign_weight, get_block(i), the alignment-dump hooks
// (gemma_3_270m_lora_finetune/src/main.cpp:326-416,455-666); the LoRA spec
// and injector are in graph/gemma_lora_injector.h.  RMSNorm with (1 + w), √d embedding
// scale, q/k RMSNorm, GeGLU MLP, grouped KV heads, local (sliding-window,
// rope_local_base_freq) and global layers.  Names are HF's without the
// "model." / "language_model.model." prefixes (both accepted).
#pragma once
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "finetune_ops/graph/engine_model.h"
#include "finetune_ops/nn/lora_linear.h"

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

// LoRA linears of one decoder layer, as handles on the model's own
// parameters (frozen W and the adapter views): blk.q_proj_lora->debug_params()
// and friends (gemma_3_270m_lora_finetune/src/main.cpp:382-416,535-537).
// A handle without an adapter has no debug params.
struct GemmaBlock {
  std::shared_ptr<LoRALinear> q_proj_lora, k_proj_lora, v_proj_lora, o_proj_lora;
  std::shared_ptr<LoRALinear> gate_proj_lora, up_proj_lora, down_proj_lora;
};

class GemmaModel : public EngineModel {
 public:
  explicit GemmaModel(const GemmaTextConfig& cfg);
  const GemmaTextConfig& config() const { return cfg_; }
  // Whether the alignment dump (enable_debug_dump) also keeps the gradients
  // of the dumped layers' activations for debug_tensors()[...]->grad(); on
  // by default, as in the reference (main.cpp:328-330 turns it off).
  void set_debug_retain_grads(bool on);
  // Handles on layer i's LoRA linears (rebuilt when the adapters change).
  GemmaBlock& get_block(int i);

  // Alignment dumps (gemma_3_270m_lora_finetune/src/main.cpp:455-666).
  // enable_debug_dump: after every later forward, the activations the engine
  // keeps for `layers` (all when empty) are written to `dir` as float32 .npy
  // files named <activation>_l<layer>.npy (hidden_states_emb.npy for the
  // scaled embedding), shaped [B, S, C] without a leading batch of one.
  void enable_debug_dump(const std::string& dir, const std::vector<int>& layers);
  // The same activations of the last forward as tensors (valid until the
  // next forward), keyed as the dumps are named without ".npy": token-major
  // [B, S, C], q/k norm and RoPE outputs head-major [B, H, S, hd],
  // attn_scores / attn_probs [B, Hq, S, S].  While gradients are retained,
  // q/k before RoPE, gate_act and the scores / probabilities exist too, and
  // after a backward every tensor carries its gradient in grad().
  std::unordered_map<std::string, TensorPtr> debug_tensors();
  // Writes layer i's norm weights (input_layernorm, post_attention_layernorm,
  // pre_feedforward_layernorm, post_feedforward_layernorm, q_norm, k_norm) to
  // dir as float32 .npy files named layer<i>_<norm>.npy.
  void dump_layer_norm_weights(int layer, const std::string& dir);

 protected:
  std::string normalise_name(const std::string& name) const override;

 private:
  GemmaTextConfig cfg_;
  std::vector<GemmaBlock> blocks_;
  const void* blocks_engine_ = nullptr;  // engine the handles were built on
  std::string dump_dir_;
  std::vector<int> dump_layers_;
  bool dump_ = false;
  bool retain_grads_ = true;
  void before_forward() override;
  void after_forward() override;
};

}  // namespace ops
