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

#include <cmath>
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
#include "finetune_ops/graph/gemma_model.h"
#include "finetune_ops/graph/gpt2_model.h"
#include "finetune_ops/graph/lora_injector.h"
#include "finetune_ops/graph/lora_saver.h"
#include "finetune_ops/graph/qwen_model.h"
#include "finetune_ops/graph/safetensors_loader.h"
#include "finetune_ops/optim/adam.h"
#include "oracle.h"

using namespace ops;

static int g_fail = 0;

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
    test_gemma(false);
    test_gemma(true);
    MemoryManager::instance().force_cleanup();
  } catch (const std::exception& e) {
    std::printf("FAIL exception: %s\n", e.what());
    ++g_fail;
  }
  std::printf("%s: %d failed checks\n", g_fail ? "FAILED" : "OK", g_fail);
  return g_fail;
}
