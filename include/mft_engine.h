/*
 * mft_engine.h — C-ABI of the device-resident LoRA training step
 * (libmft_hip.so).
 *
 * One model object owns every parameter, LoRA optimizer state and saved
 * activation in HBM and runs the training step of the reference drivers:
 *   for each micro-batch: model.forward → lm_cross_entropy →
 *   mul(loss, 1/accum)->backward()   (gpt2_small_lora_finetune/src/main.cpp:471-487)
 *   clip_and_get_grad_norm → Adam::step → zero_grad   (main.cpp:489-505)
 * for three graph families: GPT-2 (GPT2Model, main.cpp:202-276), Qwen2
 * (QwenModel, qwen_lora_finetune/src/wikitext_main.cpp:63-79) and Gemma3
 * (GemmaModel, gemma_3_270m_lora_finetune/src/main.cpp:326-379).  All
 * arithmetic runs in libmft_hip's kernels; the host only launches.
 *
 * Status codes and mft_last_error() are those of mft_hip.h.
 */
#ifndef MFT_ENGINE_H
#define MFT_ENGINE_H
#include <stdint.h>

#include "mft_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

enum mft_arch { MFT_ARCH_GPT2 = 0, MFT_ARCH_QWEN2 = 1, MFT_ARCH_GEMMA3 = 2 };

/* LoRA target bits.  GPT-2: bit0 attn.c_attn, bit1 attn.c_proj, bit2 mlp.c_fc,
 * bit3 mlp.c_proj (LoraTarget::AttnQKV/AttnProj, main.cpp:271-272).
 * Qwen2/Gemma3: bits 0..6 = q, k, v, o, gate, up, down
 * (pytorch_alignment/gemma_lora_finetune.py:144-151). */
typedef struct {
  int arch, n_layer, d, n_head, n_kv_head, head_dim, d_ff, max_pos;
  int64_t vocab;
  int lora_r;
  float lora_alpha;
  int lora_mask;
  float norm_eps;
  double rope_theta, rope_local_theta;
  int sliding_pattern; /* Gemma3: layer i is local iff (i+1) % pattern != 0 */
  int sliding_window;  /* key window of local layers (0 = none) */
  float attn_scale;    /* 0 → 1/sqrt(head_dim) */
  int w_fp16;          /* frozen linear + embedding weights stored as fp16 */
  /* PEFT's lora_dropout on every LoRA linear's input in training forwards
   * (QwenModel::init_lora(r, alpha, dropout), qwen_lora_finetune/src/
   * wikitext_main.cpp:26,77; LoraSpec.dropout).  Masks come from a counter
   * hash of (dropout_seed, training-forward count, layer·8 + target,
   * element) — the same stream the CPU oracle restates.  0 = off. */
  float lora_dropout;
  uint64_t dropout_seed;
  /* Shard store (ParameterSharder's require() streaming, README.md:302-329):
   * > 0 keeps the frozen linear weights and the token embedding in pinned
   * host memory (fp16 when w_fp16, as --shard_fp16_disk) and streams them
   * into an HBM pool of this many bytes on demand, least recently used
   * evicted, the next tensor of the previous step's order prefetched on a
   * copy stream while the current one is in use.  Must be at least the
   * largest such tensor (scripts/benchmark/test_sharding_aggressive.sh:
   * 58-65).  LoRA linears then take the rank-r panel path.  0 = all
   * parameters resident in HBM. */
  int64_t shard_budget;
} mft_model_cfg;

typedef struct mft_model_s* mft_model;

/* Shard store statistics since creation: tensors copied host→HBM (loads),
 * uses served by a resident copy (hits), and the pool size.  All zero when
 * the model is not sharded. */
int mft_model_shard_stats(mft_model m, int64_t* loads, int64_t* hits, int64_t* budget);
/* Drops every HBM copy of a streamed tensor (after the host copies were
 * written through mft_model_param_info's data pointers).  A no-op when the
 * model is not sharded. */
int mft_model_shard_reset(mft_model m);

/* max_tokens: capacity in tokens of one fused fwd/bwd pass (activations are
 * sized for it).  stream: hipStream_t or NULL. */
int mft_model_create(mft_model* out, const mft_model_cfg* cfg,
                     int64_t max_tokens, void* stream);
int mft_model_destroy(mft_model m);
/* Training (default) or evaluation mode of the forwards that keep
 * activations for a backward (mft_model_fwd_bwd, mft_model_forward_train,
 * mft_model_train_step): only training forwards apply LoRA dropout, as
 * PEFT's module.train() / eval() do.  mft_model_forward never does. */
int mft_model_set_training(mft_model m, int training);
int mft_model_num_params(mft_model m);
/* Parameter i: name, shape, trainable flag, storage dtype, device pointers
 * (grad is NULL for frozen parameters). */
int mft_model_param_info(mft_model m, int i, const char** name, int* ndim,
                         int64_t* dims, int* trainable, int* is_f16,
                         void** data, float** grad);
/* Deterministic on-device init: linear/embedding weights
 * and biases N(0, std); LayerNorm γ=1, β=0; Qwen RMSNorm w=1; Gemma RMSNorm
 * stored w=0 (the (1+w) form); LoRA A N(0, a_std), B N(0, b_std). */
int mft_model_init_params(mft_model m, uint64_t seed, float std, float a_std,
                          float b_std);
/* Forward + CE + backward over n_micro micro-batches of seqs_per_micro
 * sequences of length S, processed as one fused pass of
 * n_micro*seqs_per_micro sequences.  Each micro-batch's CE is normalised by
 * its own valid-target count and scaled by `upstream` (1/accum under the
 * driver's loss scaling), so LoRA gradients equal those of running the
 * micro-batches one after another.  ids/labels [n_micro*seqs*S] int32 and
 * mask (nullable, float, 1 = token present) are DEVICE pointers.  LoRA grads
 * accumulate until mft_model_opt_step.  Asynchronous. */
int mft_model_fwd_bwd(mft_model m, const int32_t* ids, const float* mask,
                      const int32_t* labels, int n_micro, int seqs_per_micro,
                      int S, float upstream);
/* Forward only: logits [tokens, V] into `logits` (device, nullable) and the
 * per-micro-batch loss statistics.  Asynchronous. */
int mft_model_forward(mft_model m, const int32_t* ids, const float* mask,
                      const int32_t* labels, int n_micro, int seqs_per_micro,
                      int S, float* logits);
/* Split points of the step for an operator-level host API whose autograd
 * tape runs model.forward → lm_cross_entropy → mul(loss, 1/accum) →
 * backward() one call at a time (gpt2_small_lora_finetune/src/main.cpp:
 * 471-487).  mft_model_forward_train runs the forward of nseq sequences of
 * length S and keeps every activation; mft_model_logits gives the device
 * logits buffer [nseq*S rows, row pitch ld ≥ vocab].  mft_model_ce adds the
 * summed NLL and the valid-target count of that forward's logits to the
 * DEVICE scalars loss_sum / n_valid (labels: device int32 [nseq*S], HF shift,
 * ignore_index); with backward = 1 it also overwrites the logits with
 * dlogits = upstream·(softmax − onehot)/norm (norm = norm_count if > 0, else
 * the valid count), after which mft_model_backward accumulates the LoRA
 * gradients.  backward = 2 forms those dlogits in a second buffer of the
 * logits' size (allocated at the first such call) and keeps the logits; a
 * later backward = 1 call for the same forward with the same upstream and
 * NULL loss_sum / n_valid then adopts them without a second pass (the two
 * buffers trade places: mft_model_logits afterwards returns the other one).
 * loss_sum and n_valid may both be NULL (dlogits only; nothing is summed).
 * Asynchronous. */
int mft_model_forward_train(mft_model m, const int32_t* ids, const float* mask,
                            int nseq, int S);
int mft_model_logits(mft_model m, float** logits, int64_t* ld);
int mft_model_ce(mft_model m, const int32_t* labels, int nseq, int S,
                 int ignore_index, float upstream, int64_t norm_count,
                 int backward, double* loss_sum, int64_t* n_valid);
int mft_model_backward(mft_model m, const float* mask, int nseq, int S);
/* Global grad-norm clip + Adam on the LoRA parameters + zero_grad, entirely
 * on the device (no host round trip). */
int mft_model_opt_step(mft_model m, float lr, float b1, float b2, float eps,
                       float wd, float clip);
/* One complete optimizer step: mft_model_fwd_bwd + mft_model_opt_step with
 * the loss statistics reset first.  use_graph != 0 captures the whole step
 * (every kernel of forward, CE, backward, clip and Adam) into a HIP graph on
 * the first call and replays it on later calls with the same buffers and
 * shapes; the learning rate and the other Adam scalars are uploaded before
 * each replay, so a schedule can change them per step.  The caller's
 * stream is ordered before and after the replay by events. */
int mft_model_train_step(mft_model m, const int32_t* ids, const float* mask,
                         const int32_t* labels, int n_micro,
                         int seqs_per_micro, int S, float upstream, float lr,
                         float b1, float b2, float eps, float wd, float clip,
                         int use_graph);
/* Synchronises, returns the mean over micro-batches of the micro-batch mean
 * loss since the last call (the driver's accum_loss / accum), the number of
 * valid targets and the last pre-clip grad norm; resets the loss statistics.
 * Returns MFT_EINVAL (after filling the outputs) when a token id or a label
 * (other than ignore_index) outside [0, vocab) reached a step since the last
 * call: such ids embed as zero rows, such labels count as ignored. */
int mft_model_read_stats(mft_model m, float* mean_loss, int64_t* n_valid,
                         float* grad_norm);

/* Saved forward activation of the last forward, for debugging dumps (the
 * Gemma driver's alignment mode, gemma_3_270m_lora_finetune/src/main.cpp:
 * 455-666): device pointer to `rows` token rows of `cols` floats, rows `ld`
 * apart; valid until the next forward or backward.  layer -1: "embed" (the
 * scaled embedding, layer 0's input), "final_norm".  Per layer: "x" (layer
 * input), "norm1", "q", "k", "v" (as attention reads them: after Gemma's
 * q/k norms and RoPE), "attn" (attention output), "mid" (residual stream
 * after the attention block), "norm2", "gate" (GPT-2: c_fc pre-activation),
 * "up" (Qwen2/Gemma3), "act" (MLP activation), "out" (layer output); Gemma3
 * also "q_proj", "k_proj" (before the q/k norms), "o_proj", "down_proj"
 * (before the post-norms).  MFT_EINVAL for a name the model does not keep. */
int mft_model_activation(mft_model m, int layer, const char* name,
                         const float** ptr, int64_t* rows, int64_t* cols,
                         int64_t* ld);

/* Alignment-dump debug mode (the Gemma driver's --align_dump_grads,
 * gemma_3_270m_lora_finetune/src/main.cpp:547-657; the reference model
 * retains these gradients by default, main.cpp:328-330): with bit l of
 * layer_mask set, later forwards also keep layer l's "q_normed", "k_normed"
 * (q/k after Gemma3's norms, before RoPE), "gate_act" (GELU(gate)), "scores"
 * and "probs" (the attention's scaled scores, −FLT_MAX where masked, and
 * softmax, [B·Hq·S rows, S]) for mft_model_activation, and later backwards
 * keep the gradients of every named activation of the layer (those of
 * mft_model_activation, layer −1 "embed" for layer 0's input) for
 * mft_model_activation_grad, until the next forward.  Costs extra launches
 * and memory; 0 (the default) turns it off.  Gemma3 models only; not while
 * a step graph is captured. */
int mft_model_set_retain(mft_model m, uint64_t layer_mask);
/* A retained activation gradient: device pointer to `rows` rows of `cols`
 * floats, `ld` apart, valid until the next forward.  MFT_EINVAL when the
 * last backward kept none of that name. */
int mft_model_activation_grad(mft_model m, int layer, const char* name, const float** ptr, int64_t* rows,
                              int64_t* cols, int64_t* ld);

/* ---- measurement ----------------------------------------------------------
 * When enabled, HIP events are recorded on the model's stream around every
 * launch of a kernel class; mft_model_timing returns the summed duration
 * (ms), algorithmic FLOPs or bytes, and launch count since the last reset.
 * class 0 = linear GEMMs (LoRA and frozen projections, fwd + dX; a GEMM's
 * time includes its split-K reduction, where the plan splits K),
 * 1 = LM-head GEMMs (likewise), 2 = attention kernels (fwd + bwd; work =
 * 2·B·H·S²·hd forward and 4·B·H·S²·hd backward, causal), 3 = cross-entropy
 * (work in HBM bytes: read logits, write dlogits), 4 = rank-r LoRA kernels
 * (work in HBM bytes: the W_eff merge and the rank-r projections and outer
 * products). */
int mft_model_set_timing(mft_model m, int enable);
int mft_model_timing(mft_model m, int cls, double* ms, double* work,
                     int64_t* launches);
int mft_model_reset_timing(mft_model m);

#ifdef __cplusplus
}
#endif
#endif
