// finetune_ops/core/ops.h — differentiable operators on the LoRA hot path.
//
// Replaces the free functions of the reference's operators library (absent)
// that the drivers call on the training path:
//   mul(T, float)            gpt2_small_lora_finetune/src/main.cpp:483
//   linear(x, W, b)          README.md:260 (W stored [in, out], main.cpp:211-214)
//   reshape / flatten        gemma_3_270m_lora_finetune/src/main.cpp:616-651,
//                            gpt2_medium_lora_finetune/src/mmlu/mmlu_runner.cpp:159
// plus the fused LoRA linear of LoRALinear (nn/lora_linear.h) and the causal
// GQA attention that the model graphs compose from matmul/softmax/
// repeat_kv_heads (gemma_3_270m_lora_finetune/src/main.cpp:615-657).
// Every op runs in libmft_hip's kernels; float32 tensors only.
#pragma once
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {

// y = s·a
TensorPtr mul(const TensorPtr& a, float s);
// y = a + b (same shape)
TensorPtr add(const TensorPtr& a, const TensorPtr& b);
// y = x·W + b, x [..., in], W [in, out] frozen (no dW: base weights are
// frozen on the LoRA path, qwen_lora_finetune/src/wikitext_main.cpp:78),
// b [out] or nullptr.
TensorPtr linear(const TensorPtr& x, const TensorPtr& W, const TensorPtr& b);
// y = x·W + b + scale·(x·Aᵀ)·Bᵀ; A [r, in], B [out, r]; gradients for x, A, B.
// W may be float16 (widened inside the GEMM tile load).
TensorPtr lora_linear(const TensorPtr& x, const TensorPtr& W, const TensorPtr& b, const TensorPtr& A,
                      const TensorPtr& B, float scale);
// Causal softmax attention with grouped KV heads: q [B, S, Hq, hd],
// k/v [B, S, Hkv, hd], out [B, S, Hq, hd]; query head h reads KV head
// h / (Hq / Hkv) (the repeat_kv_heads mapping).  window > 0 limits each query
// to the last `window` keys; key_mask [B, S] (nullable, 1 = present).
TensorPtr causal_attention(const TensorPtr& q, const TensorPtr& k, const TensorPtr& v, float scale,
                           int window = 0, const TensorPtr& key_mask = nullptr);
// Views with a new shape over the same (contiguous) storage.
TensorPtr reshape(const TensorPtr& x, const std::vector<int64_t>& shape);
TensorPtr flatten(const TensorPtr& x, int start_dim, int end_dim);

// Layout and analysis ops the Gemma driver applies to dumped gradients in
// its alignment mode (gemma_3_270m_lora_finetune/src/main.cpp:626-651).
// They return new contiguous float32 tensors computed on the GPU and record
// no autograd node (the driver uses them on gradients, after backward()).
// permute: out dimension i is x's dimension dims[i] (negative dims count
// from the end).
TensorPtr permute(const TensorPtr& x, const std::vector<int64_t>& dims);
// Swaps two dimensions (e.g. transpose(t, -2, -1)).
TensorPtr transpose(const TensorPtr& x, int64_t dim0, int64_t dim1);
// [B, Hkv, S, D] → [B, Hkv·n_rep, S, D]: head h of the result is head
// h / n_rep of x (HF repeat_kv).
TensorPtr repeat_kv_heads(const TensorPtr& x, int n_rep);
// Batched matrix product over the last two dimensions: a [..., M, K],
// b [..., K, N] with equal leading dimensions (or b 2-D, shared) → [..., M, N].
TensorPtr matmul(const TensorPtr& a, const TensorPtr& b);

}  // namespace ops
