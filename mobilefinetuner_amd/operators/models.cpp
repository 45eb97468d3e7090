// models.cpp — GPT2Model / QwenModel / GemmaModel over libmft_hip's step
// engine, their config readers and LoRA injectors, and the autograd node
// that joins lm_cross_entropy on a model's logits to the engine's backward.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <unordered_map>

#include "finetune_ops/core/autograd_engine.h"
#include "finetune_ops/graph/gemma_lora_injector.h"
#include "finetune_ops/graph/gpt2_model.h"
#include "finetune_ops/graph/lora_injector.h"
#include "finetune_ops/graph/qwen_model.h"
#include "internal.h"
#include "mft_engine.h"

namespace ops {

using detail::hip_check;
using detail::mft_check;

// ------------------------------------------------------------ engine state --

struct EngineState {
  mft_model m = nullptr;
  struct Rec {
    std::string name;
    std::vector<int64_t> shape;
    bool trainable = false, f16 = false;
    void* data = nullptr;
    float* grad = nullptr;
  };
  std::vector<Rec> recs;
  std::unordered_map<std::string, int> index;
  // views handed out (the model object holds the strong references; a
  // strong one here would be a cycle through the views' owner pointer)
  std::vector<std::weak_ptr<Tensor>> views, grad_views;
  uint64_t generation = 0;                   // forwards run so far
  // Pinned (Σ NLL, count) slots the loss launch adds into, read once the
  // stream has drained: no fill or copy launch around the loss read-back.
  void* loss_host = nullptr;
  void* loss_dev = nullptr;  // loss_host as kernels address it
  // upstream gradient of the last loss backward: the factor the next loss
  // forms its dlogits with beside the logits (the drivers' 1/accum repeats)
  float last_up = 1.f;
  ~EngineState() {
    if (m) (void)mft_model_destroy(m);
    if (loss_host) (void)hipHostFree(loss_host);
  }
};

namespace {

// Logits views handed out by forward(), with what their loss needs.
struct LogitsCtx {
  std::weak_ptr<EngineState> st;
  uint64_t generation = 0;
  int B = 0, S = 0;
  TensorPtr ids, mask;
  bool trainable = false;
};
std::unordered_map<const Tensor*, LogitsCtx>& logits_registry() {
  static std::unordered_map<const Tensor*, LogitsCtx> r;
  return r;
}

const int32_t* labels_ptr(const TensorPtr& labels) { return static_cast<const int32_t*>(labels->device_data()); }

// Summed NLL and valid count of the engine's current logits (slots zeroed
// first, read back after the launch).  mode: 0 loss only, 1 dlogits in place
// of the logits, 2 the loss and the dlogits for `upstream` beside the logits
// (taken up by the mode-1 call of the backward when its factor matches).
void model_ce(EngineState* st, const LogitsCtx& c, const TensorPtr& labels, int ignore, float upstream, bool sum,
              int mode, double* ls, int64_t* nv) {
  if (!ls && !nv) {  // dlogits only: no loss slots to clear or read
    mft_check(mft_model_ce(st->m, labels_ptr(labels), c.B, c.S, ignore, upstream, sum ? 1 : 0, mode, nullptr,
                           nullptr),
              "mft_model_ce");
    return;
  }
  if (!st->loss_host) {
    hip_check(hipHostMalloc(&st->loss_host, 16, hipHostMallocDefault), "hipHostMalloc");
    if (hipHostGetDevicePointer(&st->loss_dev, st->loss_host, 0) != hipSuccess) {
      st->loss_dev = nullptr;
      (void)hipGetLastError();
    }
  }
  if (st->loss_dev) {
    // the previous read-back drained the stream, so no launch still writes the slots
    std::memset(st->loss_host, 0, 16);
    char* p = static_cast<char*>(st->loss_dev);
    mft_check(mft_model_ce(st->m, labels_ptr(labels), c.B, c.S, ignore, upstream, sum ? 1 : 0, mode,
                           reinterpret_cast<double*>(p), reinterpret_cast<int64_t*>(p + 8)),
              "mft_model_ce");
    hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
    if (ls) std::memcpy(ls, st->loss_host, 8);
    if (nv) std::memcpy(nv, static_cast<const char*>(st->loss_host) + 8, 8);
    return;
  }
  auto stats = std::make_shared<Tensor>(std::vector<int64_t>{4}, kFloat32, kGPU);
  char* p = static_cast<char*>(stats->device_data());
  mft_check(mft_model_ce(st->m, labels_ptr(labels), c.B, c.S, ignore, upstream, sum ? 1 : 0, mode,
                         reinterpret_cast<double*>(p), reinterpret_cast<int64_t*>(p + 8)),
            "mft_model_ce");
  char buf[16];  // loss sum and count are adjacent: one read-back
  hip_check(hipMemcpy(buf, p, 16, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  if (ls) std::memcpy(ls, buf, 8);
  if (nv) std::memcpy(nv, buf + 8, 8);
}

// loss = lm_cross_entropy(model.forward(...)); its backward turns the
// logits into dlogits (scaled by the incoming gradient) and runs the
// engine's backward, which accumulates into the LoRA gradient arena.
struct ModelLossNode : autograd::Node {
  std::shared_ptr<EngineState> st;
  LogitsCtx ctx;
  std::weak_ptr<Tensor> logits;
  TensorPtr labels;
  int ignore = -100;
  bool sum = false;
  const char* name() const override { return "ModelLmLossBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    if (st->generation != ctx.generation)
      throw std::runtime_error("backward: the model ran another forward since this loss was computed");
    const float up = detail::read_scalar(g);
    st->last_up = up;
    model_ce(st.get(), ctx, labels, ignore, up, sum, 1, nullptr, nullptr);  // the loss was read at the forward
    // logits->retain_grad(): the gradient the CE just wrote over the logits
    // buffer is copied out before the backward consumes it
    if (auto lg = logits.lock())
      if (lg->retains_grad()) {
        float* dl = nullptr;
        int64_t ld = 0;
        mft_check(mft_model_logits(st->m, &dl, &ld), "mft_model_logits");
        const int64_t V = lg->shape().back(), rows = lg->numel() / V;
        auto g = std::make_shared<Tensor>(lg->shape(), kFloat32, kGPU);
        hip_check(hipMemcpy2D(g->device_data(), V * 4, dl, ld * 4, V * 4, rows, hipMemcpyDeviceToDevice),
                  "hipMemcpy2D");
        autograd::accumulate_grad(lg, g);
      }
    // gradients edited through host views go back before the backward adds to them
    for (auto& w : st->grad_views)
      if (auto gv = w.lock()) (void)gv->device_data();
    mft_check(mft_model_backward(st->m, ctx.mask ? static_cast<const float*>(ctx.mask->device_data()) : nullptr, ctx.B,
                                 ctx.S),
              "mft_model_backward");
    for (auto& w : st->grad_views)
      if (auto gv = w.lock()) gv->mark_device_written();
    // the drivers read the gradients next (their clip loop): queue the copy
    // to the host now, behind the backward
    for (auto& w : st->grad_views)
      if (auto gv = w.lock()) {
        detail::prefetch_host(gv);
        break;  // one group holds them all
      }
    return {};
  }
};

}  // namespace

namespace detail {

ModelLoss model_loss_hook(const TensorPtr& logits) {
  auto& reg = logits_registry();
  auto it = reg.find(logits.get());
  if (it == reg.end()) return nullptr;
  LogitsCtx ctx = it->second;
  auto st = ctx.st.lock();
  if (!st) return nullptr;
  return [st, ctx, logits](const TensorPtr& labels, int ignore, bool sum) -> TensorPtr {
    if (st->generation != ctx.generation)
      throw std::runtime_error("lm_cross_entropy: these logits were overwritten by a later forward of the model");
    if (labels->numel() != (int64_t)ctx.B * ctx.S) throw std::invalid_argument("lm_cross_entropy: labels must be [B, S]");
    double ls;
    int64_t nv;
    // a loss the tape records is most likely backpropagated: its dlogits are
    // formed in the same pass over the logits, for the factor the last
    // backward brought (the backward recomputes them if its factor differs)
    const bool recorded = ctx.trainable && autograd::Engine::instance().is_enabled();
    model_ce(st.get(), ctx, labels, ignore, recorded ? st->last_up : 1.f, sum, recorded ? 2 : 0, &ls, &nv);
    auto loss = make_loss(ls, nv, sum);
    if (recorded) {
      auto n = std::make_shared<ModelLossNode>();
      n->st = st;
      n->ctx = ctx;
      n->labels = labels;
      n->ignore = ignore;
      n->sum = sum;
      n->logits = logits;
      for (size_t i = 0; i < st->recs.size(); ++i)
        if (st->recs[i].trainable)
          if (auto v = st->views[i].lock()) n->inputs.push_back(v);
      if (n->inputs.empty()) n->inputs.push_back(logits);  // keeps the node recordable
      logits->set_requires_grad(true);
      autograd::Engine::instance().record(loss, n);
    }
    return loss;
  };
}

}  // namespace detail

// ------------------------------------------------------------- EngineModel --

EngineModel::EngineModel(const EngineModelConfig& cfg) : ecfg_(cfg) {}
EngineModel::~EngineModel() {
  auto& reg = logits_registry();
  for (auto it = reg.begin(); it != reg.end();)
    it = it->second.st.expired() || it->second.st.lock() == st_ ? reg.erase(it) : std::next(it);
}

void EngineModel::set_max_tokens(int64_t n) {
  if (n <= 0) throw std::invalid_argument("set_max_tokens: positive count required");
  if (n == max_tokens_) return;
  max_tokens_ = n;
  if (st_) attach_lora(lora_r_, lora_alpha_, lora_mask_);  // rebuild with the new capacity
}

void EngineModel::ensure_engine() {
  if (st_) return;
  mft_model_cfg c{};
  c.arch = ecfg_.arch;
  c.n_layer = ecfg_.n_layer;
  c.d = ecfg_.d;
  c.n_head = ecfg_.n_head;
  c.n_kv_head = ecfg_.n_kv_head;
  c.head_dim = ecfg_.head_dim;
  c.d_ff = ecfg_.d_ff;
  c.max_pos = ecfg_.max_pos;
  c.vocab = ecfg_.vocab;
  c.lora_r = has_lora() ? lora_r_ : 0;
  c.lora_alpha = lora_alpha_;
  c.lora_mask = has_lora() ? lora_mask_ : 0;
  c.norm_eps = ecfg_.norm_eps;
  c.rope_theta = ecfg_.rope_theta;
  c.rope_local_theta = ecfg_.rope_local_theta;
  c.sliding_pattern = ecfg_.sliding_pattern;
  c.sliding_window = ecfg_.sliding_window;
  c.attn_scale = ecfg_.attn_scale;
  c.w_fp16 = ecfg_.w_fp16 ? 1 : 0;
  c.lora_dropout = has_lora() ? lora_dropout_ : 0.f;
  c.dropout_seed = dropout_seed_;
  auto st = std::make_shared<EngineState>();
  mft_check(mft_model_create(&st->m, &c, max_tokens_, nullptr), "mft_model_create");
  const int n = mft_model_num_params(st->m);
  for (int i = 0; i < n; ++i) {
    const char* name = nullptr;
    int ndim = 0, tr = 0, f16 = 0;
    int64_t dims[2] = {0, 0};
    void* data = nullptr;
    float* grad = nullptr;
    mft_check(mft_model_param_info(st->m, i, &name, &ndim, dims, &tr, &f16, &data, &grad), "mft_model_param_info");
    EngineState::Rec r;
    r.name = name;
    r.shape.assign(dims, dims + ndim);
    r.trainable = tr != 0;
    r.f16 = f16 != 0;
    r.data = data;
    r.grad = grad;
    st->index[r.name] = i;
    st->recs.push_back(r);
  }
  st->views.assign(n, {});
  st->grad_views.assign(n, {});
  views_.assign(n, nullptr);
  grad_views_.assign(n, nullptr);
  lora_pg_.reset();
  lora_gg_.reset();
  st_ = st;
  // LoRA adapters not assigned below start as PEFT does: A small random, B zero.
  std::mt19937 rng(1234);
  for (auto& r : st_->recs) {
    if (!r.trainable || pending_.count(r.name)) continue;
    const bool is_a = r.name.size() > 7 && r.name.compare(r.name.size() - 7, 7, ".lora_A") == 0;
    int64_t numel = 1;
    for (auto d : r.shape) numel *= d;
    std::vector<float> v(numel, 0.f);
    if (is_a) {
      const float bound = 1.f / std::sqrt((float)r.shape[1]);
      std::uniform_real_distribution<float> u(-bound, bound);
      for (auto& x : v) x = u(rng);
    }
    hip_check(hipMemcpy(r.data, v.data(), numel * 4, hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  auto pend = std::move(pending_);
  pending_.clear();
  for (auto& kv : pend) {
    // adapters of targets this engine does not carry are dropped
    if (kv.first.find(".lora_") != std::string::npos && !st_->index.count(kv.first)) continue;
    assign_weight(kv.first, kv.second);
  }
}

void EngineModel::set_lora_dropout(float p, uint64_t seed) {
  if (!(p >= 0.f && p < 1.f)) throw std::invalid_argument("LoRA dropout must lie in [0, 1)");
  lora_dropout_ = p;
  dropout_seed_ = seed;
}

void EngineModel::attach_lora(int r, float alpha, int mask) {
  if (r != 0 && r != 4 && r != 8 && r != 16 && r != 32) throw std::invalid_argument("LoRA rank must be 4, 8, 16 or 32");
  if (st_) {
    // Carry every parameter of the old engine over (device copies).
    for (size_t i = 0; i < st_->recs.size(); ++i) {
      const auto& rec = st_->recs[i];
      auto t = std::make_shared<Tensor>(rec.shape, rec.f16 ? kFloat16 : kFloat32, kGPU);
      int64_t numel = t->numel();
      hip_check(hipMemcpy(t->device_data(), rec.data, numel * (rec.f16 ? 2 : 4), hipMemcpyDeviceToDevice),
                "hipMemcpy D2D");
      if (!pending_.count(rec.name)) pending_[rec.name] = t;
    }
    // LoRA tensors whose rank changes cannot carry over.
    if (r != lora_r_)
      for (auto it = pending_.begin(); it != pending_.end();)
        it = it->first.find(".lora_") != std::string::npos ? pending_.erase(it) : std::next(it);
    st_.reset();
    views_.clear();
    grad_views_.clear();
    lora_pg_.reset();
    lora_gg_.reset();
  }
  lora_r_ = r;
  lora_alpha_ = alpha;
  lora_mask_ = mask;
  ensure_engine();
}

void EngineModel::assign_weight(const std::string& raw, const TensorPtr& t) {
  if (!t) throw std::invalid_argument("assign_weight: null tensor");
  const std::string name = normalise_name(raw);
  if (name.empty()) return;  // a key this backend has no use for (tied head, attention buffers)
  if (!st_) {
    pending_[name] = t;
    return;
  }
  auto it = st_->index.find(name);
  if (it == st_->index.end()) {
    if (name.find(".lora_") != std::string::npos && !has_lora()) {  // adapters come with inject
      pending_[name] = t;
      return;
    }
    throw std::invalid_argument("assign_weight: unknown parameter " + raw);
  }
  const auto& r = st_->recs[it->second];
  int64_t numel = 1;
  for (auto d : r.shape) numel *= d;
  if (t->numel() != numel) throw std::invalid_argument("assign_weight: size mismatch for " + raw);
  if (!t->contiguous()) throw std::invalid_argument("assign_weight: contiguous tensor required for " + raw);
  if (r.f16) {
    if (t->dtype() == kFloat16) {
      hip_check(hipMemcpy(r.data, t->device_data(), numel * 2, hipMemcpyDeviceToDevice), "hipMemcpy D2D");
    } else if (t->dtype() == kFloat32) {  // rounded to nearest even, as the fp16 shard store does
      mft_check(mft_quant_f16(detail::handle(), static_cast<const float*>(t->device_data()),
                              static_cast<uint16_t*>(r.data), numel),
                "mft_quant_f16");
    } else {
      throw std::invalid_argument("assign_weight: float tensor required for " + raw);
    }
  } else {
    if (t->dtype() == kFloat32) {
      hip_check(hipMemcpy(r.data, t->device_data(), numel * 4, hipMemcpyDeviceToDevice), "hipMemcpy D2D");
    } else if (t->dtype() == kFloat16) {
      mft_check(mft_dequant_f16(detail::handle(), static_cast<const uint16_t*>(t->device_data()),
                                static_cast<float*>(r.data), numel),
                "mft_dequant_f16");
    } else {
      throw std::invalid_argument("assign_weight: float tensor required for " + raw);
    }
  }
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  if (views_[it->second]) views_[it->second]->mark_device_written();
}

void EngineModel::init_weights(uint64_t seed, float std, float a_std, float b_std) {
  ensure_engine();
  mft_check(mft_model_init_params(st_->m, seed, std, a_std, b_std), "mft_model_init_params");
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  for (auto& v : views_)
    if (v) v->mark_device_written();
}

TensorPtr EngineModel::forward(const TensorPtr& ids, const TensorPtr& mask) {
  ensure_engine();
  if (!ids || ids->dtype() != kInt32 || ids->dim() != 2) throw std::invalid_argument("forward: input_ids must be int32 [B, S]");
  const int B = (int)ids->shape()[0], S = (int)ids->shape()[1];
  if (mask && (mask->dtype() != kFloat32 || mask->numel() != (int64_t)B * S))
    throw std::invalid_argument("forward: attention_mask must be float32 [B, S]");
  detail::check_ids(ids, ecfg_.vocab, "forward");
  // Parameters edited through host views are copied back before the forward.
  for (auto& v : views_)
    if (v) (void)v->device_data();
  // training forward (LoRA dropout) iff gradients are being recorded
  mft_check(mft_model_set_training(st_->m, autograd::Engine::instance().is_enabled() ? 1 : 0),
            "mft_model_set_training");
  before_forward();
  mft_check(mft_model_forward_train(st_->m, static_cast<const int32_t*>(ids->device_data()),
                                    mask ? static_cast<const float*>(mask->device_data()) : nullptr, B, S),
            "mft_model_forward_train");
  st_->generation++;
  last_S_ = S;
  float* lg = nullptr;
  int64_t ld = 0;
  mft_check(mft_model_logits(st_->m, &lg, &ld), "mft_model_logits");
  auto logits = Tensor::view({B, S, ecfg_.vocab}, kFloat32, lg, ld, st_);
  LogitsCtx ctx;
  ctx.st = st_;
  ctx.generation = st_->generation;
  ctx.B = B;
  ctx.S = S;
  ctx.ids = ids;
  ctx.mask = mask;
  ctx.trainable = has_lora();
  auto& reg = logits_registry();
  for (auto it = reg.begin(); it != reg.end();)  // drop entries of earlier forwards
    it = it->second.st.lock() == st_ || it->second.st.expired() ? reg.erase(it) : std::next(it);
  reg[logits.get()] = ctx;
  after_forward();
  return logits;
}

std::vector<TensorPtr> EngineModel::parameters() {
  ensure_engine();
  std::vector<TensorPtr> out;
  // The LoRA parameters and their gradients each tile one device arena: each
  // arena gets one host mirror, so the drivers' host loops over
  // p->grad()->data<float>() cost one copy each way per step, not one per tensor.
  if (!lora_pg_) {
    char *plo = nullptr, *phi = nullptr, *glo = nullptr, *ghi = nullptr;
    for (const auto& r : st_->recs) {
      if (!r.trainable) continue;
      size_t b = 4;
      for (int64_t d : r.shape) b *= (size_t)d;
      char* pd = static_cast<char*>(r.data);
      char* gd = reinterpret_cast<char*>(r.grad);
      if (!plo || pd < plo) plo = pd;
      if (!phi || pd + b > phi) phi = pd + b;
      if (!glo || gd < glo) glo = gd;
      if (!ghi || gd + b > ghi) ghi = gd + b;
    }
    if (plo) {
      lora_pg_ = Tensor::mirror_group(plo, (size_t)(phi - plo));
      lora_gg_ = Tensor::mirror_group(glo, (size_t)(ghi - glo));
    }
  }
  for (size_t i = 0; i < st_->recs.size(); ++i) {
    if (!views_[i]) {
      const auto& r = st_->recs[i];
      const int64_t last = r.shape.empty() ? 1 : r.shape.back();
      views_[i] = r.trainable ? Tensor::view(r.shape, kFloat32, r.data, st_, lora_pg_)
                              : Tensor::view(r.shape, r.f16 ? kFloat16 : kFloat32, r.data, last, st_);
      st_->views[i] = views_[i];
      if (r.trainable) {
        grad_views_[i] = Tensor::view(r.shape, kFloat32, r.grad, st_, lora_gg_);
        st_->grad_views[i] = grad_views_[i];
        views_[i]->set_requires_grad(true);
        views_[i]->set_grad(grad_views_[i]);
      }
    }
    out.push_back(views_[i]);
  }
  return out;
}

std::vector<TensorPtr> EngineModel::get_lora_parameters() {
  auto all = parameters();
  std::vector<TensorPtr> out;
  for (size_t i = 0; i < all.size(); ++i)
    if (st_->recs[i].trainable) out.push_back(all[i]);
  return out;
}

std::vector<std::string> EngineModel::parameter_names() {
  ensure_engine();
  std::vector<std::string> out;
  for (auto& r : st_->recs) out.push_back(r.name);
  return out;
}

TensorPtr EngineModel::get_parameter(const std::string& raw) {
  auto all = parameters();
  auto it = st_->index.find(normalise_name(raw));
  if (it == st_->index.end()) throw std::invalid_argument("get_parameter: unknown parameter " + raw);
  return all[it->second];
}

// ------------------------------------------------------- config.json reading --

namespace {

std::string slurp(const std::string& path) {
  std::ifstream f(path);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

// Value of a top-level numeric key (the first occurrence), or `def`.
double json_num(const std::string& js, const std::string& key, double def) {
  const std::string pat = "\"" + key + "\"";
  size_t p = js.find(pat);
  if (p == std::string::npos) return def;
  p = js.find(':', p + pat.size());
  if (p == std::string::npos) return def;
  ++p;
  while (p < js.size() && (js[p] == ' ' || js[p] == '\t' || js[p] == '\n' || js[p] == '\r')) ++p;
  if (p < js.size() && (js[p] == 'n')) return def;  // null
  char* end = nullptr;
  const double v = std::strtod(js.c_str() + p, &end);
  return end == js.c_str() + p ? def : v;
}

bool strip(std::string& s, const std::string& prefix) {
  if (s.compare(0, prefix.size(), prefix) != 0) return false;
  s = s.substr(prefix.size());
  return true;
}

bool ends_with(const std::string& s, const std::string& suf) {
  return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

}  // namespace

GPT2Config GPT2Config::from_pretrained(const std::string& path) {
  const std::string js = slurp(path);
  GPT2Config c;
  c.vocab_size = (int)json_num(js, "vocab_size", c.vocab_size);
  c.n_positions = (int)json_num(js, "n_positions", c.n_positions);
  c.n_embd = (int)json_num(js, "n_embd", c.n_embd);
  c.n_layer = (int)json_num(js, "n_layer", c.n_layer);
  c.n_head = (int)json_num(js, "n_head", c.n_head);
  c.n_inner = (int)json_num(js, "n_inner", 0);
  c.layer_norm_epsilon = (float)json_num(js, "layer_norm_epsilon", c.layer_norm_epsilon);
  return c;
}

QwenConfig QwenConfig::from_pretrained(const std::string& path) {
  const std::string js = slurp(path);
  QwenConfig c;
  c.vocab_size = (int)json_num(js, "vocab_size", c.vocab_size);
  c.hidden_size = (int)json_num(js, "hidden_size", c.hidden_size);
  c.intermediate_size = (int)json_num(js, "intermediate_size", c.intermediate_size);
  c.num_hidden_layers = (int)json_num(js, "num_hidden_layers", c.num_hidden_layers);
  c.num_attention_heads = (int)json_num(js, "num_attention_heads", c.num_attention_heads);
  c.num_key_value_heads = (int)json_num(js, "num_key_value_heads", c.num_key_value_heads);
  c.max_position_embeddings = (int)json_num(js, "max_position_embeddings", c.max_position_embeddings);
  c.rms_norm_eps = (float)json_num(js, "rms_norm_eps", c.rms_norm_eps);
  c.rope_theta = json_num(js, "rope_theta", c.rope_theta);
  return c;
}

GemmaTextConfig GemmaTextConfig::from_pretrained(const std::string& dir) {
  const std::string js = slurp(dir + "/config.json");
  GemmaTextConfig c;
  c.vocab_size = (int)json_num(js, "vocab_size", c.vocab_size);
  c.hidden_size = (int)json_num(js, "hidden_size", c.hidden_size);
  c.intermediate_size = (int)json_num(js, "intermediate_size", c.intermediate_size);
  c.num_hidden_layers = (int)json_num(js, "num_hidden_layers", c.num_hidden_layers);
  c.num_attention_heads = (int)json_num(js, "num_attention_heads", c.num_attention_heads);
  c.num_key_value_heads = (int)json_num(js, "num_key_value_heads", c.num_key_value_heads);
  c.head_dim = (int)json_num(js, "head_dim", c.head_dim);
  c.max_position_embeddings = (int)json_num(js, "max_position_embeddings", c.max_position_embeddings);
  c.sliding_window = (int)json_num(js, "sliding_window", c.sliding_window);
  c.sliding_window_pattern = (int)json_num(js, "sliding_window_pattern", c.sliding_window_pattern);
  c.rms_norm_eps = (float)json_num(js, "rms_norm_eps", c.rms_norm_eps);
  c.rope_theta = json_num(js, "rope_theta", c.rope_theta);
  c.rope_local_base_freq = json_num(js, "rope_local_base_freq", c.rope_local_base_freq);
  c.query_pre_attn_scalar = (float)json_num(js, "query_pre_attn_scalar", c.query_pre_attn_scalar);
  return c;
}

// --------------------------------------------------------------------- GPT-2 --

namespace {

EngineModelConfig gpt2_ecfg(const GPT2Config& c) {
  EngineModelConfig e;
  e.arch = MFT_ARCH_GPT2;
  e.n_layer = c.n_layer;
  e.d = c.n_embd;
  e.n_head = c.n_head;
  e.n_kv_head = c.n_head;
  e.head_dim = c.n_head ? c.n_embd / c.n_head : 0;
  e.d_ff = c.n_inner > 0 ? c.n_inner : 4 * c.n_embd;
  e.max_pos = c.n_positions;
  e.vocab = c.vocab_size;
  e.norm_eps = c.layer_norm_epsilon;
  return e;
}

}  // namespace

bool LoraSlot::has_lora() const { return model_->has_lora() && ((model_->lora_mask() >> bit_) & 1); }

void LoraSlot::clear_lora() {
  if (auto* g = dynamic_cast<GPT2Model*>(model_)) g->clear_lora_bits(1 << bit_);
}

GPT2Model::GPT2Model(const GPT2Config& cfg) : EngineModel(gpt2_ecfg(cfg)), cfg_(cfg) {
  blocks_.resize(cfg.n_layer);
  for (auto& b : blocks_) {
    b.qkv_lin = std::make_shared<LoraSlot>(this, 0);
    b.proj_lin = std::make_shared<LoraSlot>(this, 1);
    b.fc_in_lin = std::make_shared<LoraSlot>(this, 2);
    b.fc_out_lin = std::make_shared<LoraSlot>(this, 3);
  }
}

GPT2Block& GPT2Model::get_block(int i) {
  if (i < 0 || i >= (int)blocks_.size()) throw std::out_of_range("get_block: layer index");
  return blocks_[i];
}

void GPT2Model::clear_lora_bits(int bits) {
  // Adapters are attached model-wide per target, so clearing one block's
  // slot clears that target everywhere; the drivers clear all blocks.
  const int mask = lora_mask_ & ~bits;
  if (mask != lora_mask_) attach_lora(mask ? lora_r_ : 0, lora_alpha_, mask);
}

void GPT2Model::print_model_info() const {
  std::printf("GPT2Model: n_layer=%d n_embd=%d n_head=%d vocab=%d n_positions=%d (MI355X engine)\n", cfg_.n_layer,
              cfg_.n_embd, cfg_.n_head, cfg_.vocab_size, cfg_.n_positions);
}

std::string GPT2Model::normalise_name(const std::string& raw) const {
  std::string n = raw;
  strip(n, "transformer.");
  if (n == "lm_head.weight" || ends_with(n, ".attn.bias") || ends_with(n, ".attn.masked_bias")) return "";
  if (n == "wte.weight") return "wte";
  if (n == "wpe.weight") return "wpe";
  // The reference's internal names, blocks.{i}.attn.qkv.weight and so on
  // (gpt2_small_lora_finetune/src/main_full.cpp:122-151).
  if (strip(n, "blocks.")) {
    n = "h." + n;
    static const char* const kRef[4][2] = {
        {".attn.qkv.", ".attn.c_attn."}, {".attn.proj.", ".attn.c_proj."},
        {".mlp.fc_in.", ".mlp.c_fc."}, {".mlp.fc_out.", ".mlp.c_proj."}};
    for (const auto& r : kRef) {
      const size_t pos = n.find(r[0]);
      if (pos != std::string::npos) {
        n.replace(pos, std::string(r[0]).size(), r[1]);
        break;
      }
    }
  }
  return n;
}

void LoraInjector::inject(GPT2Model& model, const LoraSpec& spec) {
  if (spec.split_qkv) throw std::invalid_argument("LoraInjector: split_qkv is not supported (one adapter on c_attn)");
  int mask = 0;
  for (auto t : spec.targets) mask |= 1 << (int)t;
  model.set_lora_dropout(spec.dropout);
  model.set_lora(spec.rank, spec.alpha, mask);
  last_ = spec;
  n_targets_ = model.config().n_layer * (int)spec.targets.size();
}

void LoraInjector::print_info() const {
  std::printf("LoRA: rank=%d alpha=%.1f targets=%d linears\n", last_.rank, last_.alpha, n_targets_);
}

// ---------------------------------------------------------------------- Qwen --

namespace {

EngineModelConfig qwen_ecfg(const QwenConfig& c) {
  EngineModelConfig e;
  e.arch = MFT_ARCH_QWEN2;
  e.n_layer = c.num_hidden_layers;
  e.d = c.hidden_size;
  e.n_head = c.num_attention_heads;
  e.n_kv_head = c.num_key_value_heads;
  e.head_dim = c.num_attention_heads ? c.hidden_size / c.num_attention_heads : 0;
  e.d_ff = c.intermediate_size;
  e.max_pos = c.max_position_embeddings;
  e.vocab = c.vocab_size;
  e.norm_eps = c.rms_norm_eps;
  e.rope_theta = c.rope_theta;
  e.rope_local_theta = c.rope_theta;
  return e;
}

}  // namespace

QwenModel::QwenModel(const QwenConfig& cfg) : EngineModel(qwen_ecfg(cfg)), cfg_(cfg) {}

void QwenModel::init_lora(int rank, float alpha, float dropout, bool qv_only) {
  set_lora_dropout(dropout);
  attach_lora(rank, alpha, qv_only ? 0b0101 : 0b1111);
}

std::string QwenModel::normalise_name(const std::string& raw) const {
  std::string n = raw;
  strip(n, "model.");
  if (n == "lm_head.weight") return "";
  return n;
}

// --------------------------------------------------------------------- Gemma --

namespace {

EngineModelConfig gemma_ecfg(const GemmaTextConfig& c) {
  EngineModelConfig e;
  e.arch = MFT_ARCH_GEMMA3;
  e.n_layer = c.num_hidden_layers;
  e.d = c.hidden_size;
  e.n_head = c.num_attention_heads;
  e.n_kv_head = c.num_key_value_heads;
  e.head_dim = c.head_dim;
  e.d_ff = c.intermediate_size;
  e.max_pos = c.max_position_embeddings;
  e.vocab = c.vocab_size;
  e.norm_eps = c.rms_norm_eps;
  e.rope_theta = c.rope_theta;
  e.rope_local_theta = c.rope_local_base_freq;
  e.sliding_pattern = c.sliding_window_pattern;
  e.sliding_window = c.sliding_window;
  e.attn_scale = 1.f / std::sqrt(c.query_pre_attn_scalar);
  e.w_fp16 = c.weights_fp16;
  return e;
}

const char* kGemmaTargets[7] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};

}  // namespace

GemmaModel::GemmaModel(const GemmaTextConfig& cfg) : EngineModel(gemma_ecfg(cfg)), cfg_(cfg) {}

std::string GemmaModel::normalise_name(const std::string& raw) const {
  std::string n = raw;
  if (!strip(n, "language_model.model.")) strip(n, "model.");
  if (n == "lm_head.weight") return "";
  return n;
}

GemmaBlock& GemmaModel::get_block(int i) {
  if (i < 0 || i >= cfg_.num_hidden_layers) throw std::out_of_range("get_block: layer index");
  ensure_engine();
  if (blocks_engine_ != st_.get() || blocks_.empty()) {
    blocks_.assign(cfg_.num_hidden_layers, GemmaBlock{});
    for (int l = 0; l < cfg_.num_hidden_layers; ++l) {
      GemmaBlock& b = blocks_[l];
      std::shared_ptr<LoRALinear>* slots[7] = {&b.q_proj_lora,    &b.k_proj_lora,  &b.v_proj_lora,
                                               &b.o_proj_lora,    &b.gate_proj_lora, &b.up_proj_lora,
                                               &b.down_proj_lora};
      for (int t = 0; t < 7; ++t) {
        const std::string mod = std::string("layers.") + std::to_string(l) +
                                (t < 4 ? ".self_attn." : ".mlp.") + kGemmaTargets[t];
        auto lin = std::make_shared<LoRALinear>(get_parameter(mod + ".weight"), nullptr);
        lin->set_name(mod);
        if (has_lora() && ((lora_mask() >> t) & 1))
          lin->attach_lora(get_parameter(mod + ".lora_A"), get_parameter(mod + ".lora_B"), lora_alpha());
        *slots[t] = lin;
      }
    }
    blocks_engine_ = st_.get();
  }
  return blocks_[i];
}

namespace {
// (dump name, engine activation name, layout) of a Gemma layer's debug
// tensors: token-major [B, S, C] (T), head-major [B, H, S, hd] of the query
// (Q) or key (K) heads, or [B, Hq, S, S] (A).  The norm / RoPE outputs are
// head-major as the driver's analytical gradients multiply them with the
// [B, H, S, S] score gradients (main.cpp:615-651).  q/k before RoPE, GELU(gate),
// scores and probabilities exist while the dump retains gradients.
struct DumpKey {
  const char* dump;
  const char* act;
  char layout;
};
const DumpKey kGemmaDumps[] = {
    {"hidden_before_attn", "x", 'T'},       {"hidden_after_attn_norm", "norm1", 'T'},
    {"q_proj_out", "q_proj", 'T'},          {"k_proj_out", "k_proj", 'T'},
    {"v_proj_out", "v", 'T'},               {"q_norm_out", "q_normed", 'Q'},
    {"k_norm_out", "k_normed", 'K'},        {"q_norm_out_pre_rope", "q_normed", 'Q'},
    {"k_norm_out_pre_rope", "k_normed", 'K'}, {"q_rotary_out", "q", 'Q'},
    {"k_rotary_out", "k", 'K'},             {"attn_context", "attn", 'T'},
    {"attn_scores", "scores", 'A'},         {"attn_probs", "probs", 'A'},
    {"attn_out_raw", "o_proj", 'T'},        {"hidden_after_attn", "mid", 'T'},
    {"hidden_before_mlp_norm", "mid", 'T'}, {"hidden_after_mlp_norm", "norm2", 'T'},
    {"gate_proj_out", "gate", 'T'},         {"gate_act", "gate_act", 'T'},
    {"up_proj_out", "up", 'T'},             {"mlp_prod", "act", 'T'},
    {"down_proj_out", "down_proj", 'T'},    {"hidden_after_mlp", "out", 'T'}};
}  // namespace

void GemmaModel::set_debug_retain_grads(bool on) { retain_grads_ = on; }

void GemmaModel::before_forward() {
  uint64_t mask = 0;
  if (dump_ && retain_grads_) {
    const int n = std::min(cfg_.num_hidden_layers, 64);
    if (dump_layers_.empty()) mask = n == 64 ? ~0ull : (1ull << n) - 1;
    for (int l : dump_layers_)
      if (l >= 0 && l < 64) mask |= 1ull << l;
  }
  mft_check(mft_model_set_retain(st_->m, mask), "mft_model_set_retain");
}

std::unordered_map<std::string, TensorPtr> GemmaModel::debug_tensors() {
  std::unordered_map<std::string, TensorPtr> out;
  if (!st_) return out;
  const int64_t S = last_S_;
  const int64_t hd = cfg_.head_dim;
  // engine rows [rows, cols] (rows ld apart) as a tensor of the key's layout
  auto shaped = [&](const float* p, int64_t rows, int64_t cols, int64_t ld, char layout) -> TensorPtr {
    const int64_t s = S > 0 ? S : rows;
    if (layout == 'A') return Tensor::view({rows / (cfg_.num_attention_heads * s), cfg_.num_attention_heads, s, s},
                                           kFloat32, const_cast<float*>(p), ld, st_);
    if (layout == 'T') return Tensor::view({rows / s, s, cols}, kFloat32, const_cast<float*>(p), ld, st_);
    // [B, S, H, hd] rows → a head-major [B, H, S, hd] copy
    const int64_t B = rows / s, H = cols / hd;
    auto t = std::make_shared<Tensor>(std::vector<int64_t>{B, H, s, hd}, kFloat32, kGPU);
    const int64_t shape[4] = {B, H, s, hd}, strides[4] = {s * ld, hd, ld, 1};
    mft_check(mft_strided_copy(detail::handle(), p, static_cast<float*>(t->device_data()), 4, shape, strides),
              "mft_strided_copy");
    return t;
  };
  auto add = [&](const std::string& key, int layer, const char* act, char layout) {
    const float* p = nullptr;
    int64_t rows = 0, cols = 0, ld = 0;
    if (mft_model_activation(st_->m, layer, act, &p, &rows, &cols, &ld) != 0) return;
    TensorPtr t = shaped(p, rows, cols, ld, layout);
    if (mft_model_activation_grad(st_->m, layer, act, &p, &rows, &cols, &ld) == 0)
      t->set_grad(shaped(p, rows, cols, ld, layout));
    out[key] = t;
  };
  add("hidden_states_emb", -1, "embed", 'T');
  for (int l = 0; l < cfg_.num_hidden_layers; ++l) {
    if (!dump_layers_.empty() && std::find(dump_layers_.begin(), dump_layers_.end(), l) == dump_layers_.end())
      continue;
    for (const auto& d : kGemmaDumps) add(std::string(d.dump) + "_l" + std::to_string(l), l, d.act, d.layout);
  }
  return out;
}

void GemmaModel::enable_debug_dump(const std::string& dir, const std::vector<int>& layers) {
  dump_dir_ = dir;
  dump_layers_ = layers;
  dump_ = true;
}

void GemmaModel::after_forward() {
  if (!dump_) return;
  for (auto& kv : debug_tensors()) {
    const TensorPtr& t = kv.second;
    std::vector<int64_t> shp = t->shape();
    if (!shp.empty() && shp[0] == 1) shp.erase(shp.begin());
    detail::write_npy(dump_dir_ + "/" + kv.first + ".npy", t->data<float>(), shp, false);
  }
}

void GemmaModel::dump_layer_norm_weights(int layer, const std::string& dir) {
  if (layer < 0 || layer >= cfg_.num_hidden_layers) throw std::out_of_range("dump_layer_norm_weights: layer index");
  static const char* const kNorms[6] = {"input_layernorm",           "post_attention_layernorm",
                                        "pre_feedforward_layernorm", "post_feedforward_layernorm",
                                        "self_attn.q_norm",          "self_attn.k_norm"};
  for (const char* n : kNorms) {
    const std::string name = "layers." + std::to_string(layer) + "." + n + ".weight";
    auto t = get_parameter(name);
    std::string file = n;
    const size_t dot = file.find('.');
    if (dot != std::string::npos) file = file.substr(dot + 1);
    detail::write_npy(dir + "/layer" + std::to_string(layer) + "_" + file + ".npy", t->data<float>(), t->shape(),
                      false);
  }
}

GemmaLoraSpec GemmaLoraSpec::full_attn_mlp() {
  GemmaLoraSpec s;
  s.target_modules = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};
  return s;
}
GemmaLoraSpec GemmaLoraSpec::attention_only() {
  GemmaLoraSpec s;
  s.target_modules = {"q_proj", "k_proj", "v_proj", "o_proj"};
  return s;
}
GemmaLoraSpec GemmaLoraSpec::attention_light() {
  GemmaLoraSpec s;
  s.target_modules = {"q_proj", "v_proj"};
  return s;
}

void GemmaLoraInjector::inject(GemmaModel& model, const GemmaLoraSpec& spec) {
  int mask = 0;
  for (const auto& t : spec.target_modules) {
    int bit = -1;
    for (int i = 0; i < 7; ++i)
      if (t == kGemmaTargets[i]) bit = i;
    if (bit < 0) throw std::invalid_argument("GemmaLoraInjector: unknown target module " + t);
    mask |= 1 << bit;
  }
  model.set_lora_dropout(spec.dropout);
  model.set_lora(spec.rank, spec.alpha, mask);
  last_ = spec;
}

void GemmaLoraInjector::print_info() const {
  std::printf("Gemma LoRA: rank=%d alpha=%.1f targets=%zu modules per layer\n", last_.rank, last_.alpha,
              last_.target_modules.size());
}

}  // namespace ops
