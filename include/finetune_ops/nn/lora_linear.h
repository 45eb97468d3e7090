// finetune_ops/nn/lora_linear.h — a LoRA-augmented linear layer as a module.
//
// Replaces nn/LoRALinear of the reference (absent; used through the model
// blocks, gpt2_small_lora_finetune/src/main.cpp:231-232, and
// gemma_3_270m_lora_finetune/src/main.cpp:411-414):
//   y = x·W + b + (alpha/r)·(x·Aᵀ)·Bᵀ,  W [in, out] frozen, A [r, in], B [out, r].
// forward() records one autograd node whose backward gives dX, dA and dB
// (ops::lora_linear).  W may be float16 (widened in the GEMM tile load).
#pragma once
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "finetune_ops/core/ops.h"

namespace ops {

class LoRALinear {
 public:
  LoRALinear(TensorPtr W, TensorPtr bias) : W_(std::move(W)), b_(std::move(bias)) {}
  // Attaches A, B (trainable) with scale alpha / rank.
  void attach_lora(TensorPtr A, TensorPtr B, float alpha) {
    A_ = std::move(A);
    B_ = std::move(B);
    A_->set_requires_grad(true);
    B_->set_requires_grad(true);
    scale_ = alpha / (float)A_->shape()[0];
  }
  void clear_lora() {
    A_.reset();
    B_.reset();
    scale_ = 0.f;
  }
  bool has_lora() const { return A_ != nullptr; }
  TensorPtr forward(const TensorPtr& x) const { return lora_linear(x, W_, b_, A_, B_, scale_); }
  std::vector<TensorPtr> lora_parameters() const {
    return A_ ? std::vector<TensorPtr>{A_, B_} : std::vector<TensorPtr>{};
  }
  const TensorPtr& weight() const { return W_; }
  const TensorPtr& bias() const { return b_; }
  float scale() const { return scale_; }
  // Module path of the layer (e.g. "layers.3.self_attn.q_proj"), used to
  // name its adapters in debug_params().
  void set_name(std::string name) { name_ = std::move(name); }
  const std::string& name() const { return name_; }
  // (name, tensor) of the adapter: PEFT's state-dict keys
  // <module path>.lora_A.weight / .lora_B.weight with '.' written as '_'
  // (the Gemma driver prefixes "base_model_model_model_" to name its .npy
  // dumps, gemma_3_270m_lora_finetune/src/main.cpp:384-386,536-537).  The
  // tensors are the live parameters: host writes through data<float>() reach
  // the model.  Empty without an adapter.
  std::vector<std::pair<std::string, TensorPtr>> debug_params() const {
    if (!A_) return {};
    std::string base = name_;
    for (auto& ch : base)
      if (ch == '.') ch = '_';
    return {{base + "_lora_A_weight", A_}, {base + "_lora_B_weight", B_}};
  }

 private:
  TensorPtr W_, b_, A_, B_;
  float scale_ = 0.f;
  std::string name_;
};

}  // namespace ops
