// trainer.cpp — GemmaLoRATrainer: the Gemma driver's training loop
// (warmup + linear decay schedule, gradient accumulation, global-norm clip,
// AdamW, the "[Step N] Loss= PPL=" log) over the GPU model and operators.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "finetune_ops/core/autograd_engine.h"
#include "finetune_ops/core/lm_loss.h"
#include "finetune_ops/core/ops.h"
#include "finetune_ops/graph/lora_saver.h"
#include "finetune_ops/optim/adam.h"
#include "finetune_ops/optim/gemma_trainer.h"
#include "internal.h"

namespace ops {

using detail::hip_check;
using detail::mft_check;

namespace {

int64_t mask_tokens(const TrainerBatch& b) {
  if (!b.attention_mask) return b.input_ids ? b.input_ids->numel() : 0;
  const float* m = static_cast<const Tensor&>(*b.attention_mask).data<float>();
  int64_t n = 0;
  for (int64_t i = 0; i < b.attention_mask->numel(); ++i) n += m[i] > 0.5f;
  return n;
}

// Global L2 norm of the gradients (fp64 sum of squares on the device).
float grad_norm(const std::vector<TensorPtr>& grads) {
  Tensor acc(std::vector<int64_t>{2}, kFloat32, kGPU);  // one zeroed double
  double* d = static_cast<double*>(acc.device_data());
  for (const auto& g : grads)
    if (g && g->numel() > 0)
      mft_check(mft_sumsq(detail::handle(), static_cast<const float*>(g->device_data()), g->numel(), d), "mft_sumsq");
  double ss = 0.0;
  hip_check(hipMemcpy(&ss, d, sizeof(double), hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return (float)std::sqrt(ss);
}

}  // namespace

GemmaLoRATrainer::GemmaLoRATrainer(GemmaModel& model, GemmaLoraInjector& injector, std::unique_ptr<BatchSource> train,
                                   std::unique_ptr<BatchSource> eval, const GemmaTrainerConfig& cfg)
    : model_(model), injector_(injector), train_(std::move(train)), eval_(std::move(eval)), cfg_(cfg) {
  if (!train_) throw std::invalid_argument("GemmaLoRATrainer: training data required");
  if (cfg_.micro_batch_size < 1 || cfg_.grad_accum_steps < 1)
    throw std::invalid_argument("GemmaLoRATrainer: micro_batch_size and grad_accum_steps must be >= 1");
}

GemmaLoRATrainer::~GemmaLoRATrainer() = default;

int GemmaLoRATrainer::total_steps() const {
  if (cfg_.max_steps > 0) return cfg_.max_steps;
  const int64_t n = (int64_t)train_->num_sequences();
  const int64_t micro = (n + cfg_.micro_batch_size - 1) / cfg_.micro_batch_size;
  const int64_t per_epoch = (micro + cfg_.grad_accum_steps - 1) / cfg_.grad_accum_steps;
  return (int)(per_epoch * std::max(1, cfg_.num_epochs));
}

int GemmaLoRATrainer::warmup_steps() const { return (int)(total_steps() * cfg_.warmup_ratio); }

// pytorch_alignment/gemma_lora_finetune.py:154-166 (linear mode), step 1-indexed.
float GemmaLoRATrainer::lr_at(int step) const {
  const int total = total_steps(), warm = warmup_steps();
  const double base = cfg_.learning_rate;
  if (warm > 0 && step <= warm) return (float)(base * step / std::max(1, warm));
  double progress = (double)(step - warm) / (double)std::max(1, total - warm);
  progress = std::min(1.0, std::max(0.0, progress));
  return (float)(base * (1.0 - progress));
}

void GemmaLoRATrainer::dump_embedding_output(int step, const TrainerBatch& b) {
  const std::string dir = cfg_.dump_embedding_dir.empty() ? std::string("./debug") : cfg_.dump_embedding_dir;
  auto acts = model_.debug_tensors();
  auto it = acts.find("hidden_states_emb");
  if (it == acts.end() || !it->second) throw std::runtime_error("dump_embedding: the model kept no embedding output");
  const TensorPtr& e = it->second;
  std::vector<int64_t> shp = e->shape();
  if (!shp.empty() && shp[0] == 1) shp.erase(shp.begin());
  const std::string tag = "_step" + std::to_string(step) + ".npy";
  detail::write_npy(dir + "/embedding" + tag, static_cast<const Tensor&>(*e).data<float>(), shp, false);
  std::vector<int64_t> ishp = b.input_ids->shape();
  if (!ishp.empty() && ishp[0] == 1) ishp.erase(ishp.begin());
  detail::write_npy(dir + "/input_ids" + tag, static_cast<const Tensor&>(*b.input_ids).data<int32_t>(), ishp, true);
  std::printf("[Trainer] step %d: embedding dump written to %s\n", step, dir.c_str());
}

void GemmaLoRATrainer::train() {
  auto params = model_.get_lora_parameters();
  if (params.empty()) throw std::runtime_error("GemmaLoRATrainer::train: the model has no LoRA adapters (inject first)");
  AdamConfig acfg;
  acfg.learning_rate = cfg_.learning_rate;
  acfg.beta1 = cfg_.adam_beta1;
  acfg.beta2 = cfg_.adam_beta2;
  acfg.epsilon = cfg_.adam_eps;
  acfg.weight_decay = cfg_.weight_decay;
  Adam opt(acfg);
  const int total = total_steps();
  const int accum = cfg_.grad_accum_steps;
  std::printf("[Trainer] steps=%d warmup=%d micro_batch=%d grad_accum=%d lr=%g wd=%g clip=%g\n", total,
              warmup_steps(), cfg_.micro_batch_size, accum, cfg_.learning_rate, cfg_.weight_decay,
              cfg_.max_grad_norm);
  autograd::Engine::instance().set_enabled(true);
  train_->reset_cursor();
  history_.clear();
  for (int step = 1; step <= total; ++step) {
    for (auto& p : params) p->zero_grad();
    double loss_sum = 0.0;
    int64_t tokens = 0;
    for (int a = 0; a < accum; ++a) {
      TrainerBatch b = train_->next_batch(cfg_.micro_batch_size, true);
      if (!b.input_ids) throw std::runtime_error("GemmaLoRATrainer::train: the training data yielded no batch");
      auto logits = model_.forward(b.input_ids, b.attention_mask);
      if (cfg_.dump_embedding && step == cfg_.dump_embedding_step && a == 0) dump_embedding_output(step, b);
      auto loss = lm_cross_entropy(logits, b.labels, -100, "mean");
      loss_sum += loss->data<float>()[0];
      mul(loss, 1.0f / (float)accum)->backward();
      tokens += mask_tokens(b);
    }
    std::vector<TensorPtr> grads;
    for (auto& p : params) grads.push_back(p->grad());
    const float norm = grad_norm(grads);
    if (cfg_.max_grad_norm > 0.f && norm > cfg_.max_grad_norm) {  // torch clip_grad_norm_
      const float sc = cfg_.max_grad_norm / (norm + 1e-6f);
      for (auto& g : grads) {
        float* d = static_cast<float*>(g->device_data());
        mft_check(mft_scale(detail::handle(), d, g->numel(), sc, d), "mft_scale");
        g->mark_device_written();
      }
    }
    const float lr = lr_at(step);
    opt.set_learning_rate(lr);
    opt.step(params, grads);
    TrainerStepLog rec;
    rec.step = step;
    rec.loss = (float)(loss_sum / accum);
    rec.lr = lr;
    rec.grad_norm = norm;
    rec.tokens = tokens;
    history_.push_back(rec);
    if (cfg_.logging_steps > 0 && step % cfg_.logging_steps == 0)
      std::printf("[Step %d] Loss=%.4f PPL=%.2f LR=%.6g GradNorm=%.4f Tokens=%lld\n", step, rec.loss,
                  std::exp(rec.loss), lr, norm, (long long)tokens);
    if (cfg_.eval_steps > 0 && step % cfg_.eval_steps == 0 && eval_) {
      const float el = evaluate(cfg_.eval_batches);
      std::printf("[Eval] step %d valid_loss=%.4f valid_ppl=%.2f\n", step, el, std::exp(el));
    }
    if (cfg_.save_every > 0 && step % cfg_.save_every == 0)
      save_lora(cfg_.output_dir + "/checkpoint-" + std::to_string(step) + "/gemma_lora.safetensors");
    std::fflush(stdout);
  }
}

float GemmaLoRATrainer::evaluate(int max_batches) {
  if (!eval_) throw std::runtime_error("GemmaLoRATrainer::evaluate: no eval data");
  const bool was = autograd::Engine::instance().is_enabled();
  autograd::Engine::instance().set_enabled(false);
  eval_->reset_cursor();
  double sum = 0.0;
  int n = 0;
  for (int i = 0; i < max_batches; ++i) {
    TrainerBatch b = eval_->next_batch(cfg_.micro_batch_size, false);
    if (!b.input_ids) break;
    auto logits = model_.forward(b.input_ids, b.attention_mask);
    sum += lm_cross_entropy(logits, b.labels, -100, "mean")->data<float>()[0];
    ++n;
  }
  autograd::Engine::instance().set_enabled(was);
  return n > 0 ? (float)(sum / n) : 0.f;
}

void GemmaLoRATrainer::save_lora(const std::string& path) {
  detail::make_parent_dirs(path);
  LoraSaver::save_safetensors(path, model_, injector_.spec());
}

}  // namespace ops
