// finetune_ops/optim/gemma_trainer.h — the Gemma LoRA training loop.
//
// Replaces optim/gemma_trainer.h of the reference (absent), driven as
//   GemmaTrainerConfig cfg; cfg.learning_rate = ...; ...
//   GemmaLoRATrainer trainer(model, injector, train_data, eval_data, cfg);
//   trainer.train();
//   trainer.save_lora(cfg.output_dir + "/gemma_lora.safetensors");
// (gemma_3_270m_lora_finetune/src/main.cpp:678-699).  Its semantics follow the
// PyTorch mirror of that loop (pytorch_alignment/gemma_lora_finetune.py:
// 154-166,288-350):
//   total_steps = max_steps if > 0, else ceil(ceil(sequences / micro_batch)
//                 / grad_accum) · num_epochs;  warmup = int(total · warmup_ratio)
//   lr(step)    = lr · step / warmup          for 1-indexed step ≤ warmup,
//                 lr · (1 − clamp((step − warmup) / max(1, total − warmup)))
//                 after (linear decay);
//   per step: zero grads; grad_accum micro-batches of forward →
//   lm_cross_entropy (mean) → (loss / grad_accum).backward(); global
//   grad-norm clip to max_grad_norm (> 0); AdamW (bias-corrected, decoupled
//   weight_decay) at lr(step);
//   log line "[Step N] Loss=<mean micro loss> PPL=<exp(loss)> LR=<lr>
//   GradNorm=<pre-clip norm> Tokens=<attention-mask sum>" — the prefix that
//   scripts/Finetune/plot_loss_curve.py:18 and
//   scripts/Finetune/run_gemma_270m_grad_accum_test.sh:102,177-178 parse.
// Every logging_steps steps a line is printed; every eval_steps (> 0) the
// eval set's perplexity; every save_every (> 0) steps the adapter is written
// to output_dir/checkpoint-<step>/gemma_lora.safetensors.
//
// The data layer (WikiText2Dataset) is outside this build; the trainer reads
// any dataset type with next_batch(int batch, bool loop) returning a batch
// with input_ids / attention_mask / labels tensors, plus num_sequences() and
// reset_cursor().
#pragma once
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "finetune_ops/core/tensor.h"
#include "finetune_ops/graph/gemma_lora_injector.h"
#include "finetune_ops/graph/gemma_model.h"

namespace ops {

struct GemmaTrainerConfig {
  float learning_rate = 2e-4f;
  int num_epochs = 1;
  int micro_batch_size = 1;
  int grad_accum_steps = 1;
  std::string output_dir = "./gemma_lora";
  int max_steps = -1;       // > 0 overrides the epoch count
  int eval_steps = 0;       // 0 = no periodic evaluation
  int eval_batches = 16;    // micro-batches per evaluation
  int logging_steps = 1;
  int save_every = 0;       // 0 = no periodic checkpoints
  float warmup_ratio = 0.03f;
  float max_grad_norm = 1.0f;
  float weight_decay = 0.0f;
  float adam_beta1 = 0.9f, adam_beta2 = 0.999f, adam_eps = 1e-8f;
  // Embedding dump (gemma_3_270m_lora_finetune/src/main.cpp:205-207,
  // 283-284, 688-690): at step dump_embedding_step (1-indexed) the trainer
  // writes the first micro-batch's scaled token embeddings (the model's
  // hidden_states_emb, [B, S, hidden], a leading 1 dropped) and its token ids
  // as embedding_step<N>.npy and input_ids_step<N>.npy into
  // dump_embedding_dir ("./debug" when empty).
  bool dump_embedding = false;
  int dump_embedding_step = 1;
  std::string dump_embedding_dir;
};

// One micro-batch as the trainer consumes it.
struct TrainerBatch {
  TensorPtr input_ids, attention_mask, labels;
};

// What the trainer needs from a dataset (adapters wrap the caller's type).
class BatchSource {
 public:
  virtual ~BatchSource() = default;
  virtual TrainerBatch next_batch(int batch_size, bool loop) = 0;
  virtual size_t num_sequences() const = 0;
  virtual void reset_cursor() = 0;
};

template <class DS>
class DatasetSource : public BatchSource {
 public:
  explicit DatasetSource(DS& ds) : ds_(ds) {}
  TrainerBatch next_batch(int batch_size, bool loop) override {
    auto b = ds_.next_batch(batch_size, loop);
    return {b.input_ids, b.attention_mask, b.labels};
  }
  size_t num_sequences() const override { return static_cast<size_t>(ds_.num_sequences()); }
  void reset_cursor() override { ds_.reset_cursor(); }

 private:
  DS& ds_;
};

struct TrainerStepLog {
  int step = 0;
  float loss = 0.f, lr = 0.f, grad_norm = 0.f;
  int64_t tokens = 0;
};

class GemmaLoRATrainer {
 public:
  template <class TrainDS, class EvalDS>
  GemmaLoRATrainer(GemmaModel& model, GemmaLoraInjector& injector, TrainDS& train_data, EvalDS& eval_data,
                   const GemmaTrainerConfig& cfg)
      : GemmaLoRATrainer(model, injector, std::make_unique<DatasetSource<TrainDS>>(train_data),
                         std::make_unique<DatasetSource<EvalDS>>(eval_data), cfg) {}
  GemmaLoRATrainer(GemmaModel& model, GemmaLoraInjector& injector, std::unique_ptr<BatchSource> train,
                   std::unique_ptr<BatchSource> eval, const GemmaTrainerConfig& cfg);
  ~GemmaLoRATrainer();

  void train();
  // Mean loss and perplexity over up to max_batches eval micro-batches (no
  // gradients).
  float evaluate(int max_batches);
  void save_lora(const std::string& path);

  int total_steps() const;
  int warmup_steps() const;
  float lr_at(int step) const;  // 1-indexed step
  const std::vector<TrainerStepLog>& history() const { return history_; }

 private:
  void dump_embedding_output(int step, const TrainerBatch& b);
  GemmaModel& model_;
  GemmaLoraInjector& injector_;
  std::unique_ptr<BatchSource> train_, eval_;
  GemmaTrainerConfig cfg_;
  std::vector<TrainerStepLog> history_;
};

}  // namespace ops
