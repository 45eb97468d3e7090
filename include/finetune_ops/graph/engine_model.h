// finetune_ops/graph/engine_model.h — common base of the GPU model classes.
//
// GPT2Model, QwenModel and GemmaModel keep the reference's model API
// (assign_weight, forward(ids, mask) → logits, get_lora_parameters,
// parameters; gpt2_small_lora_finetune/src/main.cpp:202-276,
// qwen_lora_finetune/src/wikitext_main.cpp:63-79,
// gemma_3_270m_lora_finetune/src/main.cpp:326-379) over one device-resident
// model of libmft_hip's step engine (mft_engine.h): the whole forward and
// backward run as fused kernels, and the autograd tape sees the model as one
// node from the LoRA parameters to the logits.  Weights assigned before the
// LoRA adapters are attached are held until the engine is built.
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {

struct EngineState;  // owns the engine model (see engine_model.cpp)

struct EngineModelConfig {
  int arch = 0;  // 0 GPT-2, 1 Qwen2, 2 Gemma3
  int n_layer = 0, d = 0, n_head = 0, n_kv_head = 0, head_dim = 0, d_ff = 0, max_pos = 0;
  int64_t vocab = 0;
  float norm_eps = 1e-5f;
  double rope_theta = 10000.0, rope_local_theta = 10000.0;
  int sliding_pattern = 0, sliding_window = 0;
  float attn_scale = 0.f;
  bool w_fp16 = false;
};

class EngineModel {
 public:
  explicit EngineModel(const EngineModelConfig& cfg);
  virtual ~EngineModel();
  EngineModel(const EngineModel&) = delete;
  EngineModel& operator=(const EngineModel&) = delete;

  // Copies `t` into the parameter `name` (after name normalisation by the
  // subclass); fp32 values are rounded to fp16 where the model stores W as
  // fp16.  Shapes must match exactly.
  void assign_weight(const std::string& name, const TensorPtr& t);
  // Tokens one forward may hold (activations are sized for it); default 4096.
  void set_max_tokens(int64_t n);
  // Deterministic on-device init (synthetic runs): W, E, biases N(0, std),
  // norms identity, LoRA A N(0, a_std), B N(0, b_std).
  void init_weights(uint64_t seed, float std, float a_std, float b_std);

  // input_ids [B, S] int32, attention_mask [B, S] float (nullable, 1 =
  // token).  Returns logits [B, S, V], a view of the model's logits buffer
  // valid until the next forward.  With autograd enabled and LoRA attached,
  // lm_cross_entropy(logits, ...)->backward() accumulates the LoRA grads.
  TensorPtr forward(const TensorPtr& input_ids, const TensorPtr& attention_mask);

  std::vector<TensorPtr> get_lora_parameters();
  std::vector<TensorPtr> parameters();
  std::vector<std::string> parameter_names();
  TensorPtr get_parameter(const std::string& name);
  bool has_lora() const { return lora_r_ > 0 && lora_mask_ != 0; }
  // Attaches (or re-attaches) LoRA with rank r, alpha and a target bit mask
  // (GPT-2: bit0 c_attn, bit1 attn c_proj, bit2 mlp c_fc, bit3 mlp c_proj;
  // Qwen2 / Gemma3: bits 0..6 q, k, v, o, gate, up, down); frozen weights
  // carry over, and mask 0 or r 0 removes the adapters.
  void set_lora(int rank, float alpha, int target_mask) { attach_lora(rank, alpha, target_mask); }
  // Dropout probability on every LoRA linear's input in training forwards
  // (forwards with autograd enabled) and the seed of its counter-based mask
  // stream (each training forward draws fresh masks from seed and a forward
  // counter); takes effect at the next set_lora.
  static constexpr uint64_t kDefaultDropoutSeed = 0x5EED0000ull;
  void set_lora_dropout(float p, uint64_t seed = kDefaultDropoutSeed);
  float lora_dropout() const { return lora_dropout_; }
  uint64_t lora_dropout_seed() const { return dropout_seed_; }
  const EngineModelConfig& engine_config() const { return ecfg_; }
  int lora_rank() const { return lora_r_; }
  float lora_alpha() const { return lora_alpha_; }
  int lora_mask() const { return lora_mask_; }

 protected:
  void attach_lora(int r, float alpha, int mask);
  virtual std::string normalise_name(const std::string& name) const { return name; }
  // Called at the start (engine settings for this forward) and at the end
  // (debug dumps) of every forward.
  virtual void before_forward() {}
  virtual void after_forward() {}
  void ensure_engine();

  EngineModelConfig ecfg_;
  int lora_r_ = 0, lora_mask_ = 0;
  float lora_alpha_ = 0.f;
  float lora_dropout_ = 0.f;
  uint64_t dropout_seed_ = kDefaultDropoutSeed;
  int64_t max_tokens_ = 4096;
  int last_S_ = 0;  // sequence length of the last forward
  std::shared_ptr<EngineState> st_;
  std::vector<TensorPtr> views_, grad_views_;  // parameter / gradient views, created on demand
  std::shared_ptr<MirrorGroup> lora_pg_, lora_gg_;  // host mirrors of the LoRA parameter / gradient arenas
  std::map<std::string, TensorPtr> pending_;  // assigned before the engine exists
};

}  // namespace ops
