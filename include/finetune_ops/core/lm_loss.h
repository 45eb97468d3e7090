// finetune_ops/core/lm_loss.h — causal-LM cross-entropy.
//
// Replaces lm_cross_entropy / perplexity_from_loss of the reference's
// core/lm_loss.h (absent), called as lm_cross_entropy(logits, labels, -100,
// "mean") (gpt2_small_lora_finetune/src/main.cpp:475) and restated in closed
// form at gemma_3_270m_lora_finetune/src/main.cpp:100-133: position s
// predicts labels[s+1] (HF shift), targets equal to ignore_index are
// skipped, NLL = logsumexp(row) − row[label] summed in double; "mean"
// divides by the number of valid targets, "sum" does not.
#pragma once
#include <cmath>
#include <string>

#include "finetune_ops/core/tensor.h"

namespace ops {

// logits [B, S, V] float32, labels [B, S] int32.  Returns a one-element
// float32 tensor; backward gives dlogits = g·(softmax − onehot)/norm.
TensorPtr lm_cross_entropy(const TensorPtr& logits, const TensorPtr& labels, int ignore_index = -100,
                           const std::string& reduction = "mean");
float perplexity_from_loss(float loss);

}  // namespace ops
