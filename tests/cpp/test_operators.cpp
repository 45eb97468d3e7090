// test_operators.cpp — parity of the finetune_ops C++ API (GPU) against the
// CPU oracle, plus checkpoint round trips (frozen weights through
// SafeTensorsReader + the key mappers, adapters through LoraSaver) into a
// fresh model whose logits must equal the trained model's, driven the way the reference drivers drive their operators:
//   logits = model.forward(ids, mask); loss = lm_cross_entropy(logits, labels,
//   -100, "mean"); mul(loss, 1/accum)->backward();  then the host-side clip
//   over p->grad()->data<float>(), optimizer.step(trainable, grads) and
//   zero_grad()   (gpt2_small_lora_finetune/src/main.cpp:471-505, 384-409).
// Also the standalone operator chain lora_linear → causal_attention →
// lm_cross_entropy → backward against the oracle's per-op functions.
//
// Exit status = number of failed checks.  Tolerances:
// loss and gradients ≤ 1e-4 relative L2, parameters after Adam ≤ 1e-5.
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <iterator>
#include <fstream>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <functional>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "finetune_ops/core/autograd_engine.h"
#include "finetune_ops/core/lm_loss.h"
#include "finetune_ops/core/memory_manager.h"
#include "finetune_ops/core/ops.h"
#include "finetune_ops/graph/gemma_lora_injector.h"
#include "finetune_ops/graph/gpt2_model.h"
#include "finetune_ops/graph/lora_injector.h"
#include "finetune_ops/graph/lora_saver.h"
#include "finetune_ops/graph/qwen_model.h"
#include "finetune_ops/graph/safetensors_loader.h"
#include "finetune_ops/optim/adam.h"
#include "finetune_ops/optim/gemma_trainer.h"
#include "oracle.h"

using namespace ops;

static int g_fail = 0;

// Minimal .npy (format 1.0, little-endian) readers for the dumps the API writes.
static std::vector<char> npy_payload(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return {};
  std::vector<char> all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (all.size() < 10) return {};
  const size_t hlen = (size_t)(unsigned char)all[8] | ((size_t)(unsigned char)all[9] << 8);
  return std::vector<char>(all.begin() + 10 + (std::ptrdiff_t)hlen, all.end());
}
static std::vector<float> read_npy_f32(const std::string& path) {
  const auto p = npy_payload(path);
  std::vector<float> v(p.size() / 4);
  std::memcpy(v.data(), p.data(), v.size() * 4);
  return v;
}
static std::vector<int32_t> read_npy_i32(const std::string& path) {
  const auto p = npy_payload(path);
  std::vector<int32_t> v(p.size() / 4);
  std::memcpy(v.data(), p.data(), v.size() * 4);
  return v;
}

static double rel_l2(const float* a, const float* b, int64_t n) {
  double num = 0, den = 0;
  for (int64_t i = 0; i < n; ++i) {
    num += (double)(a[i] - b[i]) * (a[i] - b[i]);
    den += (double)b[i] * b[i];
  }
  return den > 0 ? std::sqrt(num / den) : std::sqrt(num);
}

static void check(const std::string& what, double err, double tol) {
  const bool ok = err <= tol && std::isfinite(err);
  std::printf("%s %s err=%.3e tol=%.0e\n", ok ? "PASS" : "FAIL", what.c_str(), err, tol);
  if (!ok) ++g_fail;
}

// Copies seeded values into every parameter of both models (same names).
static void init_both(EngineModel& gm, orc_model* om, uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> nd(0.f, 1.f);
  const int n = orc_model_num_params(om);
  for (int i = 0; i < n; ++i) {
    const char* name = nullptr;
    int ndim = 0, tr = 0, f16 = 0;
    int64_t dims[2] = {0, 0};
    const int64_t numel = orc_model_param_info(om, i, &name, &ndim, dims, &tr, &f16);
    const std::string nm = name;
    std::vector<float> v(numel);
    const bool norm = nm.find("norm") != std::string::npos || nm.find("ln_") != std::string::npos;
    for (auto& x : v) {
      if (nm.size() > 7 && nm.compare(nm.size() - 7, 7, ".lora_A") == 0) x = nd(rng) / 8.f;
      else if (norm && nm.find("weight") != std::string::npos && nm.find("ln_") != std::string::npos) x = 1.f + 0.1f * nd(rng);
      else x = (norm ? 0.1f : 0.02f) * nd(rng);
    }
    std::vector<int64_t> shape(dims, dims + ndim);
    gm.assign_weight(nm, std::make_shared<Tensor>(shape, v.data(), kFloat32, kCPU));
    if (f16) {  // the oracle model stores fp16 bits; give it the same rounding
      std::vector<uint16_t> h(numel);
      orc_f32_to_f16(v.data(), h.data(), numel);
      std::memcpy(orc_model_param_data(om, i), h.data(), numel * 2);
    } else {
      std::memcpy(orc_model_param_data(om, i), v.data(), numel * 4);
    }
  }
}

// The driver's clip_and_get_grad_norm (main.cpp:384-409), verbatim in effect.
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
    float scale = max_norm / (norm + 1e-6f);
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

static int oracle_index(orc_model* om, const std::string& name) {
  const int n = orc_model_num_params(om);
  for (int i = 0; i < n; ++i) {
    const char* nm = nullptr;
    int ndim, tr, f16;
    int64_t dims[2];
    orc_model_param_info(om, i, &nm, &ndim, dims, &tr, &f16);
    if (name == nm) return i;
  }
  return -1;
}

// Runs `steps` optimizer steps of `accum` micro-batches through the C++ API
// and the oracle; compares loss per micro-batch, every LoRA gradient before
// the clip and every LoRA parameter after Adam.
static void driver_loop(const std::string& tag, EngineModel& model, orc_model* om, int B, int S, int64_t V, int steps,
                        int accum, bool pad, float clip, float lr) {
  std::vector<TensorPtr> trainable = model.get_lora_parameters();
  for (auto& p : trainable) p->zero_grad();
  std::vector<std::string> names;
  for (auto& nm : model.parameter_names())
    if (nm.find(".lora_") != std::string::npos) names.push_back(nm);
  if (names.size() != trainable.size()) {
    std::printf("FAIL %s trainable count %zu vs %zu\n", tag.c_str(), trainable.size(), names.size());
    ++g_fail;
    return;
  }
  AdamConfig oc;
  oc.learning_rate = lr;
  oc.clip_grad_norm = clip;
  Adam optimizer(oc);
  std::mt19937 rng(99);
  for (int step = 0; step < steps; ++step) {
    for (int acc = 0; acc < accum; ++acc) {
      std::vector<int32_t> ids(B * S), labels(B * S);
      std::vector<float> mask(B * S, 1.f);
      for (int i = 0; i < B * S; ++i) ids[i] = labels[i] = (int32_t)(rng() % V);
      if (pad)  // right padding of the last sequence: mask 0, label ignored
        for (int s = S - 3; s < S; ++s) {
          mask[(B - 1) * S + s] = 0.f;
          labels[(B - 1) * S + s] = -100;
        }
      auto ids_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, ids.data(), kInt32, kCPU);
      auto lab_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, labels.data(), kInt32, kCPU);
      auto mask_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, mask.data(), kFloat32, kCPU);

      auto logits = model.forward(ids_t, mask_t);
      auto loss = lm_cross_entropy(logits, lab_t, -100, "mean");
      float loss_val = loss->data<float>()[0];
      {
        float inv_accum = 1.0f / float(accum);
        auto scaled_loss = mul(loss, inv_accum);
        scaled_loss->backward();
      }
      const float ol = orc_model_fwd_bwd(om, ids.data(), mask.data(), labels.data(), B, S, 1.0f / accum);
      check(tag + " step" + std::to_string(step) + " micro" + std::to_string(acc) + " loss",
            std::fabs(loss_val - ol) / std::fabs(ol), 1e-4);
    }
    double gerr = 0;
    std::vector<std::vector<float>> og(names.size());
    for (size_t i = 0; i < names.size(); ++i) {
      const int oi = oracle_index(om, names[i]);
      const float* g = trainable[i]->grad()->data<float>();
      const float* o = orc_model_param_grad(om, oi);
      og[i].assign(o, o + trainable[i]->numel());
      gerr = std::max(gerr, rel_l2(g, o, trainable[i]->numel()));
    }
    check(tag + " step" + std::to_string(step) + " LoRA grads (max over tensors)", gerr, 1e-4);

    const float gn = clip_and_get_grad_norm(trainable, clip);
    optimizer.set_learning_rate(lr);
    std::vector<TensorPtr> grads;
    for (const auto& p : trainable) grads.push_back(p->grad());
    optimizer.step(trainable, grads);
    for (auto& p : trainable) p->zero_grad();
    const float on = orc_model_opt_step(om, lr, 0.9f, 0.999f, 1e-8f, 0.f, clip);
    check(tag + " step" + std::to_string(step) + " clipped grad norm", std::fabs(gn - on) / std::fabs(on), 1e-4);

    // Adam's first steps move each element by lr·g/(|g|+eps): for an element
    // whose gradient is near zero that ratio is set by fp32 summation-order
    // noise (~1e-5 of the tensor's rms here), so elements below 1e-4 of the
    // tensor's rms gradient are left out of the parameter comparison.
    double perr = 0, covered = 0, total = 0;
    for (size_t i = 0; i < names.size(); ++i) {
      const int oi = oracle_index(om, names[i]);
      const float* p = trainable[i]->data<float>();
      const float* o = static_cast<const float*>(orc_model_param_data(om, oi));
      double ss = 0;
      for (float x : og[i]) ss += (double)x * x;
      const float grms = (float)std::sqrt(ss / og[i].size());
      std::vector<float> a, b;
      for (int64_t j = 0; j < trainable[i]->numel(); ++j)
        if (std::fabs(og[i][j]) > 1e-4f * grms) {
          a.push_back(p[j]);
          b.push_back(o[j]);
        }
      covered += a.size();
      total += trainable[i]->numel();
      if (!a.empty()) perr = std::max(perr, rel_l2(a.data(), b.data(), (int64_t)a.size()));
      const float* g = trainable[i]->grad()->data<float>();
      for (int64_t j = 0; j < trainable[i]->numel(); ++j)
        if (g[j] != 0.f) {
          std::printf("FAIL %s zero_grad left a nonzero gradient\n", tag.c_str());
          ++g_fail;
          break;
        }
    }
    check(tag + " step" + std::to_string(step) + " LoRA params after Adam", perr, 1e-5);
    check(tag + " step" + std::to_string(step) + " params compared (share left out)", 1.0 - covered / total, 1e-2);
    // Next step starts from the oracle's parameters (written through the host
    // view, which the next forward copies back to the device), so each step's
    // gradients are compared from identical weights.
    for (size_t i = 0; i < names.size(); ++i) {
      const float* o = static_cast<const float*>(orc_model_param_data(om, oracle_index(om, names[i])));
      std::memcpy(trainable[i]->data<float>(), o, trainable[i]->numel() * sizeof(float));
    }
  }
  // Host edits of the gradients, then zero_grad() of one member only: the
  // fill must not lose the other members' edits (they reach the device
  // first), while a zero_grad() of every member needs no upload.
  if (trainable.size() >= 2) {
    for (size_t i = 0; i < trainable.size(); ++i) {
      float* g = trainable[i]->grad()->data<float>();
      for (int64_t j = 0; j < trainable[i]->numel(); ++j) g[j] = 0.25f * (float)(i + 1) + 1e-3f * (float)(j % 97);
    }
    trainable[0]->zero_grad();
    auto dev_scaled = mul(trainable[1]->grad(), 2.f);  // reads the device copy
    const float* d = dev_scaled->data<float>();
    const float* h = trainable[1]->grad()->data<float>();
    const float* z = trainable[0]->grad()->data<float>();
    double e = 0;
    for (int64_t j = 0; j < trainable[1]->numel(); ++j) {
      const float want = 0.5f + 1e-3f * (float)(j % 97);
      e = std::max(e, (double)std::fabs(h[j] - want) + std::fabs(d[j] - 2.f * want));
    }
    for (int64_t j = 0; j < trainable[0]->numel(); ++j) e = std::max(e, (double)std::fabs(z[j]));
    check(tag + " partial zero_grad keeps host edits", e, 0.0);
    for (auto& p : trainable) p->zero_grad();
  }
}


static std::vector<float> host_copy(const TensorPtr& t) {
  const float* p = static_cast<const Tensor&>(*t).data<float>();
  return std::vector<float>(p, p + t->numel());
}

// Writes `trained`'s frozen weights as an HF checkpoint (nn.Linear weights
// back in [out, in] when `hf_linear`), saves its adapters with `save`, then
// loads both into `fresh` the way the drivers do (main.cpp:207-219,
// 244-262) and compares logits and adapters.
static void checkpoint_roundtrip(const std::string& tag, EngineModel& trained, EngineModel& fresh, bool hf_linear,
                                 const std::unordered_map<std::string, std::string>& mapping,
                                 const std::function<void(const std::string&)>& save, int B, int S) {
  const std::string dir = "/tmp/mft_ckpt_" + tag + "_" + std::to_string(getpid());
  std::vector<std::vector<float>> keep;
  keep.reserve(mapping.size());
  std::vector<SafeTensorsEntry> entries;
  for (const auto& kv : mapping) {
    TensorPtr t = trained.get_parameter(kv.first);
    std::vector<float> v = host_copy(t);
    std::vector<int64_t> shape = t->shape();
    if (hf_linear && shape.size() == 2 && kv.first.find("embed") == std::string::npos) {
      std::vector<float> tr(v.size());
      for (int64_t r = 0; r < shape[0]; ++r)
        for (int64_t c = 0; c < shape[1]; ++c) tr[c * shape[0] + r] = v[r * shape[1] + c];
      v.swap(tr);
      std::swap(shape[0], shape[1]);
    }
    keep.push_back(std::move(v));
    entries.push_back({kv.second, "F32", shape, keep.back().data(), keep.back().size() * 4});
  }
  write_safetensors(dir + "/model.safetensors", entries);
  save(dir + "/adapter_model.safetensors");

  SafeTensorsReader reader(dir + "/model.safetensors");
  reader.parse_header();
  SafeTensorsLoadOptions opts;
  opts.transpose_linear = hf_linear;
  opts.verbose = false;
  for (auto& kv : reader.load_tensors_mapped(mapping, opts)) fresh.assign_weight(kv.first, kv.second);
  LoraState st = LoraSaver::load_safetensors(dir + "/adapter_model.safetensors");
  check(tag + " checkpoint adapters compatible", st.compatible_with(fresh) ? 0.0 : 1.0, 0.0);
  check(tag + " checkpoint rank/alpha", std::fabs(st.rank - trained.lora_rank()) + std::fabs(st.alpha - trained.lora_alpha()),
        0.0);
  check(tag + " checkpoint adapter_config.json written",
        std::filesystem::exists(dir + "/adapter_config.json") ? 0.0 : 1.0, 0.0);
  LoraSaver::attach_from_state(fresh, st);

  double worst = 0;
  for (const auto& name : trained.parameter_names()) {
    const auto a = host_copy(trained.get_parameter(name)), b = host_copy(fresh.get_parameter(name));
    worst = std::max(worst, rel_l2(b.data(), a.data(), (int64_t)a.size()));
  }
  check(tag + " checkpoint every parameter restored", worst, 0.0);

  std::mt19937 rng(5);
  std::vector<int32_t> ids(B * S);
  for (auto& x : ids) x = (int32_t)(rng() % 50);
  auto ids_t = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, ids.data(), kInt32, kCPU);
  autograd::Engine::instance().set_enabled(false);
  const auto la = host_copy(trained.forward(ids_t, nullptr));
  const auto lb = host_copy(fresh.forward(ids_t, nullptr));
  autograd::Engine::instance().set_enabled(true);
  check(tag + " checkpoint logits equal", rel_l2(lb.data(), la.data(), (int64_t)la.size()), 0.0);
  std::filesystem::remove_all(dir);
}

static void test_gpt2() {
  GPT2Config cfg;
  cfg.vocab_size = 101;
  cfg.n_positions = 32;
  cfg.n_embd = 128;
  cfg.n_layer = 2;
  cfg.n_head = 2;
  GPT2Model model(cfg);
  model.tie_weights();
  model.init_lora_modules();
  LoraSpec spec;
  spec.rank = 4;
  spec.alpha = 8.f;
  spec.targets = {LoraTarget::AttnQKV, LoraTarget::AttnProj};
  LoraInjector injector;
  injector.inject(model, spec);

  orc_model_cfg oc{};
  oc.arch = ORC_GPT2;
  oc.n_layer = 2;
  oc.d = 128;
  oc.n_head = 2;
  oc.n_kv_head = 2;
  oc.head_dim = 64;
  oc.d_ff = 512;
  oc.max_pos = 32;
  oc.vocab = 101;
  oc.lora_r = 4;
  oc.lora_alpha = 8.f;
  oc.lora_mask = 0b0011;
  oc.norm_eps = 1e-5f;
  orc_model* om = orc_model_create(&oc);
  init_both(model, om, 11);
  driver_loop("gpt2", model, om, 2, 16, 101, 2, 2, false, 0.05f, 1e-3f);
  orc_model_destroy(om);
  GPT2Model fresh(cfg);
  checkpoint_roundtrip("gpt2", model, fresh, false, GPT2KeyMapper::generate_gpt2_mapping(cfg.n_layer),
                       [&](const std::string& p) { LoraSaver::save_safetensors(p, model, spec); }, 2, 16);
}

static void test_qwen() {
  QwenConfig cfg;
  cfg.vocab_size = 97;
  cfg.hidden_size = 128;
  cfg.intermediate_size = 96;
  cfg.num_hidden_layers = 2;
  cfg.num_attention_heads = 2;
  cfg.num_key_value_heads = 1;
  cfg.max_position_embeddings = 64;
  cfg.rms_norm_eps = 1e-6f;
  cfg.rope_theta = 1e6;
  QwenModel model(cfg);
  model.init_lora(8, 16.f, 0.f);
  model.freeze_base();

  orc_model_cfg oc{};
  oc.arch = ORC_QWEN2;
  oc.n_layer = 2;
  oc.d = 128;
  oc.n_head = 2;
  oc.n_kv_head = 1;
  oc.head_dim = 64;
  oc.d_ff = 96;
  oc.max_pos = 64;
  oc.vocab = 97;
  oc.lora_r = 8;
  oc.lora_alpha = 16.f;
  oc.lora_mask = 0b1111;
  oc.norm_eps = 1e-6f;
  oc.rope_theta = 1e6;
  oc.rope_local_theta = 1e6;
  orc_model* om = orc_model_create(&oc);
  init_both(model, om, 12);
  driver_loop("qwen2", model, om, 2, 12, 97, 2, 1, true, 1.0f, 1e-3f);
  orc_model_destroy(om);
  QwenModel fresh(cfg);
  checkpoint_roundtrip("qwen2", model, fresh, true, QwenKeyMapper::generate_qwen_mapping(cfg.num_hidden_layers),
                       [&](const std::string& p) { LoraSaver::save_safetensors(p, model); }, 2, 12);
}

// LoRA dropout p = 0.1 through QwenModel::init_lora: each micro-batch's
// training forward draws the oracle's masks (same seed, same forward counter).
static void test_qwen_dropout() {
  QwenConfig cfg;
  cfg.vocab_size = 89;
  cfg.hidden_size = 128;
  cfg.intermediate_size = 160;
  cfg.num_hidden_layers = 2;
  cfg.num_attention_heads = 2;
  cfg.num_key_value_heads = 1;
  cfg.max_position_embeddings = 64;
  cfg.rms_norm_eps = 1e-6f;
  cfg.rope_theta = 1e6;
  QwenModel model(cfg);
  model.init_lora(8, 16.f, 0.1f);
  model.freeze_base();

  orc_model_cfg oc{};
  oc.arch = ORC_QWEN2;
  oc.n_layer = 2;
  oc.d = 128;
  oc.n_head = 2;
  oc.n_kv_head = 1;
  oc.head_dim = 64;
  oc.d_ff = 160;
  oc.max_pos = 64;
  oc.vocab = 89;
  oc.lora_r = 8;
  oc.lora_alpha = 16.f;
  oc.lora_mask = 0b1111;
  oc.norm_eps = 1e-6f;
  oc.rope_theta = 1e6;
  oc.rope_local_theta = 1e6;
  oc.lora_dropout = 0.1f;
  oc.dropout_seed = EngineModel::kDefaultDropoutSeed;
  orc_model* om = orc_model_create(&oc);
  init_both(model, om, 21);
  driver_loop("qwen2-dropout", model, om, 2, 12, 89, 2, 2, false, 1.0f, 1e-3f);
  orc_model_destroy(om);
}

static void test_gemma(bool fp16) {
  GemmaTextConfig cfg;
  cfg.vocab_size = 89;
  cfg.hidden_size = 64;
  cfg.intermediate_size = 96;
  cfg.num_hidden_layers = 6;
  cfg.num_attention_heads = 4;
  cfg.num_key_value_heads = 1;
  cfg.head_dim = 64;
  cfg.max_position_embeddings = 64;
  cfg.sliding_window = 5;
  cfg.sliding_window_pattern = 6;
  cfg.rms_norm_eps = 1e-6f;
  cfg.rope_theta = 1e6;
  cfg.rope_local_base_freq = 1e4;
  cfg.query_pre_attn_scalar = 16.f;
  cfg.weights_fp16 = fp16;
  GemmaModel model(cfg);
  GemmaLoraSpec spec = GemmaLoraSpec::full_attn_mlp();
  GemmaLoraInjector injector;
  injector.inject(model, spec);

  orc_model_cfg oc{};
  oc.arch = ORC_GEMMA3;
  oc.n_layer = 6;
  oc.d = 64;
  oc.n_head = 4;
  oc.n_kv_head = 1;
  oc.head_dim = 64;
  oc.d_ff = 96;
  oc.max_pos = 64;
  oc.vocab = 89;
  oc.lora_r = 8;
  oc.lora_alpha = 32.f;
  oc.lora_mask = 0x7f;
  oc.norm_eps = 1e-6f;
  oc.rope_theta = 1e6;
  oc.rope_local_theta = 1e4;
  oc.sliding_pattern = 6;
  oc.sliding_window = 5;
  oc.attn_scale = 1.f / std::sqrt(16.f);
  oc.w_fp16 = fp16 ? 1 : 0;
  orc_model* om = orc_model_create(&oc);
  init_both(model, om, 13);
  driver_loop(fp16 ? "gemma3-fp16w" : "gemma3", model, om, 2, 12, 89, 2, 2, false, 1.0f, 1e-3f);
  orc_model_destroy(om);
}

// A tiny Gemma-3 config shared by the trainer and debug-API tests.
static GemmaTextConfig tiny_gemma() {
  GemmaTextConfig cfg;
  cfg.vocab_size = 89;
  cfg.hidden_size = 64;
  cfg.intermediate_size = 96;
  cfg.num_hidden_layers = 3;
  cfg.num_attention_heads = 4;
  cfg.num_key_value_heads = 1;
  cfg.head_dim = 64;
  cfg.max_position_embeddings = 64;
  cfg.sliding_window = 5;
  cfg.sliding_window_pattern = 3;
  cfg.rms_norm_eps = 1e-6f;
  cfg.rope_theta = 1e6;
  cfg.rope_local_base_freq = 1e4;
  cfg.query_pre_attn_scalar = 16.f;
  return cfg;
}

static orc_model* tiny_gemma_oracle(int lora_mask) {
  orc_model_cfg oc{};
  oc.arch = ORC_GEMMA3;
  oc.n_layer = 3;
  oc.d = 64;
  oc.n_head = 4;
  oc.n_kv_head = 1;
  oc.head_dim = 64;
  oc.d_ff = 96;
  oc.max_pos = 64;
  oc.vocab = 89;
  oc.lora_r = 8;
  oc.lora_alpha = 32.f;
  oc.lora_mask = lora_mask;
  oc.norm_eps = 1e-6f;
  oc.rope_theta = 1e6;
  oc.rope_local_theta = 1e4;
  oc.sliding_pattern = 3;
  oc.sliding_window = 5;
  oc.attn_scale = 1.f / std::sqrt(16.f);
  return orc_model_create(&oc);
}

// A dataset with the reference data layer's interface over a fixed pool of
// seeded sequences (the trainer binds any such type).
struct SyntheticLM {
  struct Batch {
    TensorPtr input_ids, attention_mask, labels;
  };
  int S = 12, V = 89;
  std::vector<std::vector<int32_t>> seqs;
  size_t cursor = 0;
  SyntheticLM(int n, uint64_t seed) {
    std::mt19937_64 rng(seed);
    for (int i = 0; i < n; ++i) {
      std::vector<int32_t> s(S);
      for (auto& t : s) t = (int32_t)(rng() % V);
      seqs.push_back(s);
    }
  }
  size_t num_sequences() const { return seqs.size(); }
  void reset_cursor() { cursor = 0; }
  // the sequences of the next batch, as the trainer will see them
  std::vector<int32_t> take(int bs, bool loop) {
    std::vector<int32_t> ids;
    for (int b = 0; b < bs; ++b) {
      if (cursor >= seqs.size()) {
        if (!loop) return {};
        cursor = 0;
      }
      ids.insert(ids.end(), seqs[cursor].begin(), seqs[cursor].end());
      ++cursor;
    }
    return ids;
  }
  Batch next_batch(int bs, bool loop) {
    auto ids = take(bs, loop);
    if (ids.empty()) return {};
    std::vector<float> mask(ids.size(), 1.f);
    Batch b;
    b.input_ids = std::make_shared<Tensor>(std::vector<int64_t>{bs, S}, ids.data(), kInt32, kCPU);
    b.attention_mask = std::make_shared<Tensor>(std::vector<int64_t>{bs, S}, mask.data(), kFloat32, kCPU);
    b.labels = std::make_shared<Tensor>(std::vector<int64_t>{bs, S}, ids.data(), kInt32, kCPU);
    return b;
  }
};

// GemmaLoRATrainer against the oracle driven through the same schedule:
// 10 sequences, micro-batch 2, grad_accum 2, one epoch → 3 steps, warmup
// int(3·0.34) = 1, linear decay, clip 0.5, AdamW with weight decay 0.01.
static void test_gemma_trainer() {
  const GemmaTextConfig cfg = tiny_gemma();
  GemmaModel model(cfg);
  GemmaLoraInjector injector;
  injector.inject(model, GemmaLoraSpec::full_attn_mlp());
  orc_model* om = tiny_gemma_oracle(0x7f);
  init_both(model, om, 21);
  SyntheticLM train(10, 5), eval(4, 6);
  GemmaTrainerConfig tc;
  tc.learning_rate = 1e-3f;
  tc.num_epochs = 1;
  tc.micro_batch_size = 2;
  tc.grad_accum_steps = 2;
  tc.warmup_ratio = 0.34f;
  tc.max_grad_norm = 0.5f;
  tc.weight_decay = 0.01f;
  tc.eval_steps = 3;
  tc.eval_batches = 2;
  tc.output_dir = "/tmp/mft_trainer_test";
  tc.dump_embedding = true;  // step 2's first micro-batch
  tc.dump_embedding_step = 2;
  tc.dump_embedding_dir = tc.output_dir + "/emb";
  GemmaLoRATrainer trainer(model, injector, train, eval, tc);
  check("gemma trainer total steps", std::abs(trainer.total_steps() - 3), 0);
  check("gemma trainer warmup steps", std::abs(trainer.warmup_steps() - 1), 0);
  const float want_lr[3] = {1e-3f, 5e-4f, 0.f};  // warmup 1/1, then decay over 2 steps
  for (int s = 1; s <= 3; ++s) check("gemma trainer lr step" + std::to_string(s), std::abs(trainer.lr_at(s) - want_lr[s - 1]), 1e-9);
  trainer.train();
  const auto& hist = trainer.history();
  check("gemma trainer ran 3 steps", std::abs((int)hist.size() - 3), 0);
  // oracle replay
  SyntheticLM replay(10, 5);
  std::vector<float> mask(2 * 12, 1.f);
  for (int step = 1; step <= 3 && step <= (int)hist.size(); ++step) {
    double loss = 0;
    for (int a = 0; a < 2; ++a) {
      auto ids = replay.take(2, true);
      loss += orc_model_fwd_bwd(om, ids.data(), mask.data(), ids.data(), 2, 12, 0.5f);
    }
    // the oracle returns the norm after clipping (clip_and_get_grad_norm's
    // value); the trainer logs the norm before it
    const float norm = orc_model_opt_step(om, trainer.lr_at(step), 0.9f, 0.999f, 1e-8f, 0.01f, 0.5f);
    const float clipped = std::min(hist[step - 1].grad_norm, 0.5f);
    check("gemma trainer step" + std::to_string(step) + " loss", std::abs(hist[step - 1].loss - loss / 2) / (loss / 2), 1e-4);
    check("gemma trainer step" + std::to_string(step) + " clipped grad norm", std::abs(clipped - norm) / norm, 1e-4);
  }
  // parameters after the three AdamW steps
  std::vector<float> got, want;
  for (auto& name : model.parameter_names()) {
    if (name.find(".lora_") == std::string::npos) continue;
    auto t = model.get_parameter(name);
    const float* g = static_cast<const Tensor&>(*t).data<float>();
    const float* o = static_cast<const float*>(orc_model_param_data(om, oracle_index(om, name)));
    got.insert(got.end(), g, g + t->numel());
    want.insert(want.end(), o, o + t->numel());
  }
  check("gemma trainer LoRA params after 3 steps", rel_l2(got.data(), want.data(), (int64_t)got.size()), 1e-5);
  {
    // the embedding dump of step 2: sequences 4 and 5 of the stream (steps
    // take 2 micro-batches of 2), each row wte[id]·√hidden (HF Gemma3's
    // scaled embedding; the table is frozen, so it is the initial one)
    SyntheticLM again(10, 5);
    (void)again.take(4, true);
    const std::vector<int32_t> ids = again.take(2, true);
    const std::vector<float> emb = read_npy_f32(tc.dump_embedding_dir + "/embedding_step2.npy");
    const std::vector<int32_t> got_ids = read_npy_i32(tc.dump_embedding_dir + "/input_ids_step2.npy");
    const int d = cfg.hidden_size;
    auto wte = model.get_parameter("embed_tokens.weight");
    const float* w = static_cast<const Tensor&>(*wte).data<float>();
    const float sc = std::sqrt((float)d);
    std::vector<float> want_e(ids.size() * (size_t)d);
    for (size_t r = 0; r < ids.size(); ++r)
      for (int c = 0; c < d; ++c) want_e[r * d + c] = w[(size_t)ids[r] * d + c] * sc;
    check("gemma trainer embedding dump ids", got_ids == ids ? 0.0 : 1.0, 0);
    check("gemma trainer embedding dump size", std::abs((double)emb.size() - (double)want_e.size()), 0);
    if (emb.size() == want_e.size())
      check("gemma trainer embedding dump values", rel_l2(emb.data(), want_e.data(), (int64_t)emb.size()), 0);
  }
  trainer.save_lora(tc.output_dir + "/gemma_lora.safetensors");
  std::ifstream saved(tc.output_dir + "/gemma_lora.safetensors", std::ios::binary);
  check("gemma trainer adapter written", saved.good() ? 0.0 : 1.0, 0);
  orc_model_destroy(om);
}

// Checkpoint and resume as the reference drivers do them (main.cpp:143-150,
// 241-262): a run writes checkpoint-<step> every save_every steps; a run that
// stops after the step-2 save is restarted from that file — base weights
// from the model files, LoRA A/B through load_safetensors +
// attach_from_state, a fresh optimizer and schedule.  The restored adapters
// must equal the ones the first run held at the save bit for bit, and two
// further trainer steps from them must match the oracle started from the
// same adapters with a fresh AdamW.
static void test_gemma_resume() {
  const GemmaTextConfig cfg = tiny_gemma();
  const std::string dir = "/tmp/mft_resume_" + std::to_string(getpid());
  std::vector<std::string> names;
  std::vector<std::vector<float>> at_save;
  {
    GemmaModel model(cfg);
    GemmaLoraInjector injector;
    injector.inject(model, GemmaLoraSpec::full_attn_mlp());
    orc_model* om = tiny_gemma_oracle(0x7f);
    init_both(model, om, 33);
    orc_model_destroy(om);
    SyntheticLM train(8, 9), eval(2, 10);
    GemmaTrainerConfig tc;
    tc.learning_rate = 1e-3f;
    tc.micro_batch_size = 2;
    tc.max_steps = 2;
    tc.save_every = 2;
    tc.warmup_ratio = 0.f;
    tc.output_dir = dir;
    GemmaLoRATrainer trainer(model, injector, train, eval, tc);
    trainer.train();
    for (auto& name : model.parameter_names())
      if (name.find(".lora_") != std::string::npos) {
        names.push_back(name);
        at_save.push_back(host_copy(model.get_parameter(name)));
      }
  }  // the first run ends after its step-2 save
  const std::string ckpt = dir + "/checkpoint-2/gemma_lora.safetensors";
  check("resume checkpoint-2 written", std::filesystem::exists(ckpt) ? 0.0 : 1.0, 0.0);
  GemmaModel model(cfg);
  GemmaLoraInjector injector;
  injector.inject(model, GemmaLoraSpec::full_attn_mlp());
  orc_model* om = tiny_gemma_oracle(0x7f);
  init_both(model, om, 33);  // the base weights, as loaded from the model files
  LoraState st = LoraSaver::load_safetensors(ckpt);
  check("resume checkpoint compatible", st.compatible_with(model) ? 0.0 : 1.0, 0.0);
  LoraSaver::attach_from_state(model, st);
  double worst = 0;
  for (size_t i = 0; i < names.size(); ++i) {
    const auto got = host_copy(model.get_parameter(names[i]));
    worst = std::max(worst, rel_l2(got.data(), at_save[i].data(), (int64_t)got.size()));
    std::memcpy(orc_model_param_data(om, oracle_index(om, names[i])), at_save[i].data(), at_save[i].size() * 4);
  }
  check("resume adapters restored bit for bit", worst, 0.0);
  SyntheticLM train(8, 9), eval(2, 10), replay(8, 9);
  GemmaTrainerConfig tc;
  tc.learning_rate = 1e-3f;
  tc.micro_batch_size = 2;
  tc.max_steps = 2;
  tc.warmup_ratio = 0.5f;
  tc.output_dir = dir;
  GemmaLoRATrainer trainer(model, injector, train, eval, tc);
  trainer.train();
  const auto& hist = trainer.history();
  check("resumed run ran 2 steps", std::abs((int)hist.size() - 2), 0);
  std::vector<float> mask(2 * 12, 1.f);
  for (int step = 1; step <= (int)hist.size(); ++step) {
    auto ids = replay.take(2, true);
    const float loss = orc_model_fwd_bwd(om, ids.data(), mask.data(), ids.data(), 2, 12, 1.f);
    orc_model_opt_step(om, trainer.lr_at(step), 0.9f, 0.999f, 1e-8f, 0.f, 1.f);
    check("resumed step" + std::to_string(step) + " loss", std::abs(hist[step - 1].loss - loss) / loss, 1e-4);
  }
  std::vector<float> got, want;
  for (auto& name : names) {
    const auto g = host_copy(model.get_parameter(name));
    const float* o = static_cast<const float*>(orc_model_param_data(om, oracle_index(om, name)));
    got.insert(got.end(), g.begin(), g.end());
    want.insert(want.end(), o, o + g.size());
  }
  check("resumed LoRA params after 2 more steps", rel_l2(got.data(), want.data(), (int64_t)got.size()), 1e-5);
  orc_model_destroy(om);
  std::filesystem::remove_all(dir);
}

// The Gemma driver's alignment-mode API: block handles and debug_params,
// dumps, dlogits through retain_grad, and the layout ops it applies.
// The align dump's gradients (gemma_3_270m_lora_finetune/src/main.cpp:547-657)
// after forward + lm_cross_entropy + backward on `ids` ([1, S]): every dumped
// tensor's grad() against the oracle's retained intermediates of the same
// step (oracle.h: orc_model_set_retain), and the driver's analytical
// attention gradients (dMat = dScores·scale, dQ = dMat·repeat_kv(K),
// dK = dMatᵀ·Q, dV = Pᵀ·dContext) against the oracle's d(q), d(k), d(v).
static void check_align_grads(GemmaModel& model, orc_model* om,
                              std::unordered_map<std::string, TensorPtr>& dbg, const std::vector<int32_t>& ids,
                              const GemmaTextConfig& cfg) {
  const int S = (int)ids.size(), H = cfg.num_attention_heads, Hk = cfg.num_key_value_heads, hd = cfg.head_dim;
  orc_model_set_retain(om, (1ull << 0) | (1ull << 2));
  std::vector<float> mask(S, 1.f);
  orc_model_fwd_bwd(om, ids.data(), mask.data(), ids.data(), 1, S, 1.f);
  // token-major [S, H·hd] oracle rows → head-major [H, S, hd]
  auto head = [&](const float* t, int heads) {
    std::vector<float> o((size_t)heads * S * hd);
    for (int s = 0; s < S; ++s)
      for (int h = 0; h < heads; ++h)
        for (int e = 0; e < hd; ++e) o[((size_t)h * S + s) * hd + e] = t[((size_t)s * heads + h) * hd + e];
    return o;
  };
  const char* keys[][3] = {{"hidden_before_attn", "x", "T"},      {"hidden_after_attn_norm", "norm1", "T"},
                           {"q_proj_out", "q_proj", "T"},         {"k_proj_out", "k_proj", "T"},
                           {"v_proj_out", "v", "T"},              {"q_norm_out", "q_normed", "Q"},
                           {"k_norm_out_pre_rope", "k_normed", "K"}, {"q_rotary_out", "q", "Q"},
                           {"k_rotary_out", "k", "K"},            {"attn_context", "attn", "T"},
                           {"attn_scores", "scores", "A"},        {"attn_probs", "probs", "A"},
                           {"attn_out_raw", "o_proj", "T"},       {"hidden_after_attn", "mid", "T"},
                           {"hidden_after_mlp_norm", "norm2", "T"}, {"gate_proj_out", "gate", "T"},
                           {"gate_act", "gate_act", "T"},         {"up_proj_out", "up", "T"},
                           {"mlp_prod", "act", "T"},              {"down_proj_out", "down_proj", "T"},
                           {"hidden_after_mlp", "out", "T"}};
  for (int layer : {0, 2}) {
    const std::string L = "_l" + std::to_string(layer);
    for (const auto& k : keys) {
      auto it = dbg.find(k[0] + L);
      int64_t n = 0;
      const float* ref = orc_model_retained(om, layer, k[1], 1, &n);
      if (it == dbg.end() || !it->second->grad() || !ref) {
        check(std::string("align grad present ") + k[0] + L, 1.0, 0);
        continue;
      }
      std::vector<float> want(ref, ref + n);
      if (k[2][0] == 'Q') want = head(ref, H);
      if (k[2][0] == 'K') want = head(ref, Hk);
      auto g = it->second->grad();
      check(std::string("align grad ") + k[0] + L,
            g->numel() == (int64_t)want.size() ? rel_l2(g->data<float>(), want.data(), want.size()) : 1.0, 1e-4);
    }
  }
  {
    int64_t n = 0;
    const float* ref = orc_model_retained(om, -1, "embed", 1, &n);
    auto e = dbg["hidden_states_emb"];
    check("align grad hidden_states_emb",
          ref && e->grad() ? rel_l2(e->grad()->data<float>(), ref, (size_t)n) : 1.0, 1e-4);
  }
  // the driver's analytical attention gradients (main.cpp:599-657)
  for (int layer : {0, 2}) {
    const std::string L = "_l" + std::to_string(layer);
    const float qk_scale = std::pow(cfg.query_pre_attn_scalar, -0.5f);
    auto dMat = mul(dbg["attn_scores" + L]->grad(), qk_scale);
    auto k_full = repeat_kv_heads(dbg["k_rotary_out" + L], H / Hk);
    auto dQ = matmul(dMat, k_full);                            // [1, H, S, hd]
    auto dK = matmul(transpose(dMat, -2, -1), dbg["q_rotary_out" + L]);  // per query head
    auto G = dbg["attn_context" + L]->grad();                  // [1, S, H·hd]
    auto Gh = permute(reshape(G, {1, S, H, hd}), {0, 2, 1, 3});
    auto dV = matmul(transpose(dbg["attn_probs" + L], -2, -1), Gh);
    int64_t n = 0;
    auto want_q = head(orc_model_retained(om, layer, "q", 1, &n), H);
    check("align analytical dq" + L, rel_l2(dQ->data<float>(), want_q.data(), want_q.size()), 1e-4);
    for (const char* which : {"k", "v"}) {
      auto want = head(orc_model_retained(om, layer, which, 1, &n), Hk);
      const float* per = (which[0] == 'k' ? dK : dV)->data<float>();  // [H, S, hd]: sum each KV head's group
      std::vector<float> sum(want.size(), 0.f);
      for (int h = 0; h < H; ++h)
        for (size_t i = 0; i < (size_t)S * hd; ++i) sum[(size_t)(h / (H / Hk)) * S * hd + i] += per[(size_t)h * S * hd + i];
      check(std::string("align analytical d") + which + L, rel_l2(sum.data(), want.data(), want.size()), 1e-4);
    }
  }
}

static void test_gemma_debug_api() {
  const GemmaTextConfig cfg = tiny_gemma();
  GemmaModel model(cfg);
  GemmaLoraInjector injector;
  injector.inject(model, GemmaLoraSpec::attention_only());
  orc_model* om = tiny_gemma_oracle(0x0f);
  init_both(model, om, 22);
  auto& blk = model.get_block(1);
  auto dp = blk.q_proj_lora->debug_params();
  check("gemma debug_params names", dp.size() == 2 && dp[0].first == "layers_1_self_attn_q_proj_lora_A_weight" &&
                                            dp[1].first == "layers_1_self_attn_q_proj_lora_B_weight" ? 0.0 : 1.0, 0);
  check("gemma no adapter on gate_proj", blk.gate_proj_lora->debug_params().empty() ? 0.0 : 1.0, 0);
  // a host write through the handle reaches the model (the align mode's LoRA-A load)
  auto A = dp[0].second;
  float* a = A->data<float>();
  for (int64_t i = 0; i < A->numel(); ++i) a[i] = 0.01f * (float)((i % 7) - 3);
  const float* back = static_cast<const Tensor&>(*model.get_parameter("layers.1.self_attn.q_proj.lora_A")).data<float>();
  check("gemma debug_params write-through", std::abs(back[5] - 0.01f * 2.f), 0);
  {  // the oracle gets the same LoRA-A, for the gradient checks below
    const int oi = oracle_index(om, "layers.1.self_attn.q_proj.lora_A");
    std::memcpy(orc_model_param_data(om, oi), a, A->numel() * 4);
  }
  const std::string dir = "/tmp/mft_align_dump";
  model.enable_debug_dump(dir, {0, 2});
  model.dump_layer_norm_weights(0, dir);
  std::vector<int32_t> ids(12);
  for (int i = 0; i < 12; ++i) ids[i] = (i * 37 + 5) % 89;
  auto tids = std::make_shared<Tensor>(std::vector<int64_t>{1, 12}, ids.data(), kInt32, kCPU);
  auto logits = model.forward(tids, nullptr);
  logits->set_requires_grad(true);
  logits->retain_grad();
  std::vector<float> lg(static_cast<const Tensor&>(*logits).data<float>(),
                        static_cast<const Tensor&>(*logits).data<float>() + 12 * 89);
  auto loss = lm_cross_entropy(logits, tids, -100, "mean");
  loss->backward();
  std::vector<float> dl_ref(12 * 89), nll(12);
  double ls = 0;
  orc_ce_fwd_bwd(lg.data(), ids.data(), 1, 12, 89, -100, 1.f, 0, &ls, dl_ref.data(), nll.data());
  check("gemma retain_grad dlogits", logits->grad() ? rel_l2(logits->grad()->data<float>(), dl_ref.data(), 12 * 89) : 1.0, 1e-5);
  auto dbg = model.debug_tensors();
  check("gemma debug tensors present",
        dbg.count("q_rotary_out_l0") && dbg.count("attn_context_l2") && dbg.count("hidden_states_emb") &&
                dbg.count("attn_scores_l0") && dbg.count("attn_probs_l2") && dbg.count("q_norm_out_pre_rope_l0") &&
                dbg.count("gate_act_l2") && !dbg.count("q_rotary_out_l1") ? 0.0 : 1.0, 0);
  check_align_grads(model, om, dbg, ids, cfg);
  for (const char* f : {"/hidden_states_emb.npy", "/q_rotary_out_l0.npy", "/mlp_prod_l2.npy", "/layer0_q_norm.npy"}) {
    std::ifstream in(dir + f, std::ios::binary);
    char magic[6] = {0};
    in.read(magic, 6);
    check(std::string("gemma dump ") + f, in.good() && magic[1] == 'N' && magic[5] == 'Y' ? 0.0 : 1.0, 0);
  }
  // hidden_states_emb = E[ids]·sqrt(d), against the frozen table
  {
    auto emb = dbg["hidden_states_emb"];
    const float* e = static_cast<const Tensor&>(*emb).data<float>();
    const float* E = static_cast<const Tensor&>(*model.get_parameter("embed_tokens.weight")).data<float>();
    std::vector<float> want(12 * 64);
    for (int t = 0; t < 12; ++t)
      for (int c = 0; c < 64; ++c) want[t * 64 + c] = E[ids[t] * 64 + c] * std::sqrt(64.f);
    check("gemma hidden_states_emb", rel_l2(e, want.data(), 12 * 64), 1e-6);
  }
  // layout ops against host loops
  std::vector<float> x(2 * 3 * 4 * 5);
  for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i * 0.5f - 7.f;
  auto tx = std::make_shared<Tensor>(std::vector<int64_t>{2, 3, 4, 5}, x.data(), kFloat32, kCPU);
  auto tp = permute(tx, {0, 2, 1, 3});
  auto tt = transpose(tx, -2, -1);
  auto tr = repeat_kv_heads(tx, 2);
  auto y = std::make_shared<Tensor>(std::vector<int64_t>{2, 3, 5, 6}, x.data(), kFloat32, kCPU);  // reuse values
  std::vector<float> yv(2 * 3 * 5 * 6);
  for (size_t i = 0; i < yv.size(); ++i) yv[i] = std::sin((float)i);
  y = std::make_shared<Tensor>(std::vector<int64_t>{2, 3, 5, 6}, yv.data(), kFloat32, kCPU);
  auto mm = matmul(tx, y);
  double e_p = 0, e_t = 0, e_r = 0, e_m = 0;
  const float* pp = tp->data<float>();
  const float* pt = tt->data<float>();
  const float* pr = tr->data<float>();
  const float* pm = mm->data<float>();
  for (int b = 0; b < 2; ++b)
    for (int h = 0; h < 3; ++h)
      for (int s2 = 0; s2 < 4; ++s2)
        for (int d = 0; d < 5; ++d) {
          const float v = x[((b * 3 + h) * 4 + s2) * 5 + d];
          e_p += std::abs(pp[((b * 4 + s2) * 3 + h) * 5 + d] - v);
          e_t += std::abs(pt[((b * 3 + h) * 5 + d) * 4 + s2] - v);
          for (int r = 0; r < 2; ++r) e_r += std::abs(pr[((b * 6 + h * 2 + r) * 4 + s2) * 5 + d] - v);
        }
  for (int b = 0; b < 2; ++b)
    for (int h = 0; h < 3; ++h)
      for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 6; ++j) {
          double acc = 0;
          for (int k = 0; k < 5; ++k) acc += (double)x[((b * 3 + h) * 4 + i) * 5 + k] * yv[((b * 3 + h) * 5 + k) * 6 + j];
          e_m += std::abs(pm[((b * 3 + h) * 4 + i) * 6 + j] - acc) / (1 + std::abs(acc));
        }
  check("layout permute", e_p, 0);
  check("layout transpose", e_t, 0);
  check("layout repeat_kv_heads", e_r, 0);
  check("layout matmul", e_m, 1e-4);
  check("layout shapes", tp->shape() == std::vector<int64_t>{2, 4, 3, 5} && tt->shape() == std::vector<int64_t>{2, 3, 5, 4} &&
                             tr->shape() == std::vector<int64_t>{2, 6, 4, 5} && mm->shape() == std::vector<int64_t>{2, 3, 4, 6}
                         ? 0.0 : 1.0, 0);
  orc_model_destroy(om);
}

// lora_linear → causal_attention (q, k, v views of one projection output) →
// lm_cross_entropy, backward to x, A, B; against the oracle's functions.
static void test_ops_chain() {
  const int B = 2, S = 8, H = 2, hd = 64, D = H * hd, K = 24, V = D;
  const int r = 4;
  const float scale = 2.f, att_scale = 0.25f;
  std::mt19937_64 rng(5);
  std::normal_distribution<float> nd(0.f, 1.f);
  auto randv = [&](size_t n, float s) {
    std::vector<float> v(n);
    for (auto& x : v) x = s * nd(rng);
    return v;
  };
  const int M = B * S;
  auto x = randv(M * K, 1.f), Wq = randv(K * D, 0.2f), Wk = randv(K * D, 0.2f), Wv = randv(K * D, 0.2f);
  auto A = randv(r * K, 0.25f), Bm = randv(D * r, 0.1f), bq = randv(D, 0.1f);
  std::vector<int32_t> labels(M);
  for (auto& l : labels) l = (int32_t)(rng() % V);
  labels[3] = -100;

  // GPU through the API
  auto xt = std::make_shared<Tensor>(std::vector<int64_t>{B, S, K}, x.data(), kFloat32, kCPU);
  xt->set_requires_grad(true);
  auto Wqt = std::make_shared<Tensor>(std::vector<int64_t>{K, D}, Wq.data(), kFloat32, kCPU);
  auto Wkt = std::make_shared<Tensor>(std::vector<int64_t>{K, D}, Wk.data(), kFloat32, kCPU);
  auto Wvt = std::make_shared<Tensor>(std::vector<int64_t>{K, D}, Wv.data(), kFloat32, kCPU);
  auto bqt = std::make_shared<Tensor>(std::vector<int64_t>{D}, bq.data(), kFloat32, kCPU);
  auto At = std::make_shared<Tensor>(std::vector<int64_t>{r, K}, A.data(), kFloat32, kCPU);
  auto Bt = std::make_shared<Tensor>(std::vector<int64_t>{D, r}, Bm.data(), kFloat32, kCPU);
  At->set_requires_grad(true);
  Bt->set_requires_grad(true);
  auto lt = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, labels.data(), kInt32, kCPU);
  auto q = reshape(lora_linear(xt, Wqt, bqt, At, Bt, scale), {B, S, H, hd});
  auto k = reshape(linear(xt, Wkt, nullptr), {B, S, H, hd});
  auto v = reshape(linear(xt, Wvt, nullptr), {B, S, H, hd});
  auto o = causal_attention(q, k, v, att_scale);
  auto logits = reshape(o, {B, S, V});
  auto loss = lm_cross_entropy(logits, lt, -100, "mean");
  const float lv = loss->data<float>()[0];
  mul(loss, 0.5f)->backward();

  // oracle
  std::vector<float> qo(M * D), ko(M * D), vo(M * D), xa(M * r), oo(M * D), lse(B * H * S);
  orc_lora_linear_fwd(x.data(), M, K, Wq.data(), D, bq.data(), A.data(), Bm.data(), r, scale, qo.data(), xa.data());
  orc_lora_linear_fwd(x.data(), M, K, Wk.data(), D, nullptr, nullptr, nullptr, 0, 0.f, ko.data(), nullptr);
  orc_lora_linear_fwd(x.data(), M, K, Wv.data(), D, nullptr, nullptr, nullptr, 0, 0.f, vo.data(), nullptr);
  orc_attn_fwd(qo.data(), D, ko.data(), D, vo.data(), D, B, H, H, S, hd, att_scale, 1, 0, nullptr, oo.data(), D,
               lse.data());
  std::vector<float> dlog(M * V), nll(M);
  double ls = 0;
  const int64_t nv = orc_ce_fwd_bwd(oo.data(), labels.data(), B, S, V, -100, 0.5f, 0, &ls, dlog.data(), nll.data());
  check("ops chain loss", std::fabs(lv - (float)(ls / nv)) / std::fabs((float)(ls / nv)), 1e-4);
  std::vector<float> dq(M * D), dk(M * D), dv(M * D), dx(M * K, 0.f), dx1(M * K), dA(r * K, 0.f), dB(D * r, 0.f);
  orc_attn_bwd(qo.data(), D, ko.data(), D, vo.data(), D, oo.data(), D, dlog.data(), D, lse.data(), B, H, H, S, hd,
               att_scale, 1, 0, nullptr, dq.data(), D, dk.data(), D, dv.data(), D);
  orc_lora_linear_bwd(dq.data(), x.data(), Wq.data(), A.data(), Bm.data(), xa.data(), M, K, D, r, scale, dx1.data(),
                      dA.data(), dB.data(), 0);
  for (int i = 0; i < M * K; ++i) dx[i] += dx1[i];
  orc_lora_linear_bwd(dk.data(), x.data(), Wk.data(), nullptr, nullptr, nullptr, M, K, D, 0, 0.f, dx1.data(), nullptr,
                      nullptr, 0);
  for (int i = 0; i < M * K; ++i) dx[i] += dx1[i];
  orc_lora_linear_bwd(dv.data(), x.data(), Wv.data(), nullptr, nullptr, nullptr, M, K, D, 0, 0.f, dx1.data(), nullptr,
                      nullptr, 0);
  for (int i = 0; i < M * K; ++i) dx[i] += dx1[i];
  check("ops chain dX (three consumers summed)", rel_l2(xt->grad()->data<float>(), dx.data(), M * K), 1e-4);
  check("ops chain dA", rel_l2(At->grad()->data<float>(), dA.data(), r * K), 1e-4);
  check("ops chain dB", rel_l2(Bt->grad()->data<float>(), dB.data(), D * r), 1e-4);

  // A second backward through a fresh graph accumulates (grads add up).
  auto q2 = reshape(lora_linear(xt, Wqt, bqt, At, Bt, scale), {B, S, H, hd});
  auto o2 = causal_attention(q2, k, v, att_scale);
  lm_cross_entropy(reshape(o2, {B, S, V}), lt, -100, "mean")->backward();
  std::vector<float> dA2(dA);
  for (auto& z : dA2) z *= 3.f;  // 0.5·g + 1·g with the first graph's k, v reused
  // k and v saved by the first graph were built from the same x: dA depends
  // only on the q path, so the total is 1.5× the first backward's (which was
  // scaled by 0.5): 3× dA of scale 0.5.
  check("ops chain dA accumulates across backward calls", rel_l2(At->grad()->data<float>(), dA2.data(), r * K), 1e-4);
}

int main() {
  orc_set_blas(0);
  try {
    test_ops_chain();
    test_gpt2();
    test_qwen();
    test_qwen_dropout();
    test_gemma(false);
    test_gemma(true);
    test_gemma_trainer();
    test_gemma_resume();
    test_gemma_debug_api();
    MemoryManager::instance().force_cleanup();
  } catch (const std::exception& e) {
    std::printf("FAIL exception: %s\n", e.what());
    ++g_fail;
  }
  std::printf("%s: %d failed checks\n", g_fail ? "FAILED" : "OK", g_fail);
  return g_fail;
}
