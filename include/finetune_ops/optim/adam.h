// finetune_ops/optim/adam.h — Adam on the trainable (LoRA) parameters.
//
// Replaces optim/adam.h of the reference (absent): configured through
// AdamConfig{learning_rate, beta1, beta2, epsilon, weight_decay,
// clip_grad_norm} and driven as set_learning_rate(lr); step(params, grads)
// (gpt2_small_lora_finetune/src/main.cpp:341-348,493-502).  Bias-corrected
// Adam (Kingma & Ba) with decoupled weight decay; the moments live in HBM
// beside the parameters and the update runs in one kernel per tensor.  The
// driver clips the gradients itself before step() (main.cpp:384-409), so
// clip_grad_norm is kept for source compatibility and not applied here.
#pragma once
#include <memory>
#include <unordered_map>
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {

struct AdamConfig {
  float learning_rate = 1e-3f;
  float beta1 = 0.9f;
  float beta2 = 0.999f;
  float epsilon = 1e-8f;
  float weight_decay = 0.0f;
  float clip_grad_norm = 0.0f;
};

class Adam {
 public:
  explicit Adam(const AdamConfig& cfg = AdamConfig());
  ~Adam();
  void set_learning_rate(float lr) { cfg_.learning_rate = lr; }
  float get_learning_rate() const { return cfg_.learning_rate; }
  // One update of every params[i] with grads[i] (null grads are skipped);
  // the step count advances once per call.
  void step(const std::vector<TensorPtr>& params, const std::vector<TensorPtr>& grads);
  int step_count() const { return t_; }

 private:
  struct State;
  struct GroupState;
  AdamConfig cfg_;
  int t_ = 0;
  std::unordered_map<const Tensor*, std::unique_ptr<State>> state_;
  // moments of parameters that tile a mirror group (a model's LoRA arena)
  // live in one arena per group: per-tensor states are views into it, and a
  // step over every member of the group is one launch
  std::unordered_map<const MirrorGroup*, std::unique_ptr<GroupState>> gstate_;
};

}  // namespace ops
