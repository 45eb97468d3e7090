// api_bench — throughput of the operators API (libfinetune_ops.so) driven the
// way the reference's GPT-2 driver drives its operators
// (gpt2_small_lora_finetune/src/main.cpp:456-505): per micro-batch
//   logits = model.forward(ids, mask); loss = lm_cross_entropy(logits, labels,
//   -100, "mean"); loss->data<float>() (the logged value);
//   mul(loss, 1/accum)->backward();
// then the driver's host-side clip over p->grad()->data<float>()
// (main.cpp:384-409), Adam::step(trainable, grads) and zero_grad().
// Synthetic token ids, random-init weights (EngineModel::init_weights).
//
// usage: api_bench [B S accum steps warmup rank alpha]   (defaults: GPT-2
// small, 4 128 1 20 3 8 16).  Prints one JSON line.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "finetune_ops/core/lm_loss.h"
#include "finetune_ops/core/ops.h"
#include "finetune_ops/graph/gpt2_model.h"
#include "finetune_ops/graph/lora_injector.h"
#include "finetune_ops/optim/adam.h"

using namespace ops;

static float clip_and_get_grad_norm(const std::vector<TensorPtr>& trainable, float max_norm) {
  double norm_sq = 0.0;
  for (const auto& p : trainable) {
    auto grad = p->grad();
    if (!grad) continue;
    const float* g = grad->data<float>();
    for (int64_t i = 0; i < grad->numel(); ++i) norm_sq += double(g[i]) * double(g[i]);
  }
  float norm = float(std::sqrt(norm_sq));
  if (max_norm > 0.0f && norm > max_norm) {
    const float scale = max_norm / (norm + 1e-6f);
    for (const auto& p : trainable) {
      auto grad = p->grad();
      if (!grad) continue;
      float* g = grad->data<float>();
      for (int64_t i = 0; i < grad->numel(); ++i) g[i] *= scale;
    }
    norm = max_norm;
  }
  return norm;
}

int main(int argc, char** argv) {
  const int B = argc > 1 ? std::atoi(argv[1]) : 4;
  const int S = argc > 2 ? std::atoi(argv[2]) : 128;
  const int accum = argc > 3 ? std::atoi(argv[3]) : 1;
  const int steps = argc > 4 ? std::atoi(argv[4]) : 20;
  const int warmup = argc > 5 ? std::atoi(argv[5]) : 3;
  const int rank = argc > 6 ? std::atoi(argv[6]) : 8;
  const float alpha = argc > 7 ? (float)std::atof(argv[7]) : 16.f;
  try {
    GPT2Config cfg;  // GPT-2 small
    GPT2Model model(cfg);
    model.tie_weights();
    model.set_max_tokens((int64_t)B * S);
    model.init_lora_modules();
    LoraSpec spec;
    spec.rank = rank;
    spec.alpha = alpha;
    spec.targets = {LoraTarget::AttnQKV, LoraTarget::AttnProj};
    LoraInjector injector;
    injector.inject(model, spec);
    model.init_weights(1235, 0.02f, 1.f / rank, 0.02f);
    std::vector<TensorPtr> trainable = model.get_lora_parameters();
    AdamConfig oc;
    oc.learning_rate = 2e-4f;
    oc.clip_grad_norm = 1.0f;
    Adam optimizer(oc);
    std::mt19937 rng(1235);
    std::vector<int32_t> ids((size_t)B * S);
    std::vector<float> mask((size_t)B * S, 1.f);
    double loss_sum = 0.0;
    auto one_step = [&]() {
      for (int a = 0; a < accum; ++a) {
        for (auto& t : ids) t = (int32_t)(rng() % (uint32_t)cfg.vocab_size);
        auto ids_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, ids.data(), kInt32, kCPU);
        auto mask_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, mask.data(), kFloat32, kCPU);
        auto logits = model.forward(ids_t, mask_t);
        auto loss = lm_cross_entropy(logits, ids_t, -100, "mean");
        loss_sum += loss->data<float>()[0];
        mul(loss, 1.0f / float(accum))->backward();
      }
      clip_and_get_grad_norm(trainable, 1.0f);
      std::vector<TensorPtr> grads;
      for (const auto& p : trainable) grads.push_back(p->grad());
      optimizer.step(trainable, grads);
      for (auto& p : trainable) p->zero_grad();
    };
    for (int i = 0; i < warmup; ++i) one_step();
    // The step's last host access (the clip loop's reads, Adam on the device
    // views) leaves nothing queued that the next step would not wait for, so
    // wall time over the loop is the step time.
    loss_sum = 0.0;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) one_step();
    trainable[0]->data<float>();  // waits for the last optimizer step
    const double sec = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const double tokens = (double)B * S * accum;
    std::printf("{\"path\": \"operators API (libfinetune_ops.so), driver loop\", \"tokens_per_s\": %.1f, "
                "\"ms_per_step\": %.4f, \"steps\": %d, \"tokens_per_step\": %.0f, \"mean_loss\": %.5f}\n",
                tokens * steps / sec, 1000.0 * sec / steps, steps, tokens, loss_sum / (steps * accum));
  } catch (const std::exception& e) {
    std::fprintf(stderr, "api_bench: %s\n", e.what());
    return 1;
  }
  return 0;
}
