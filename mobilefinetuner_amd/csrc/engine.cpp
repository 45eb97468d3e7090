// engine.cpp — device-resident LoRA training step for GPT-2, Qwen2 and
// Gemma3 graphs (C-ABI in include/mft_engine.h).
//
// Memory layout in HBM:
//   * frozen parameters: one arena, each tensor 256-byte aligned, fp32 or
//     (w_fp16) IEEE fp16 for linear weights and the embedding;
//   * LoRA parameters: four flat fp32 arrays (value, grad, Adam m, Adam v)
//     with every A/B tensor at a 64-float-aligned offset, so grad-norm and
//     Adam are single launches over one contiguous range;
//   * activations: one arena sized for `max_tokens`, holding what the
//     backward needs per layer (inputs of every linear, attention output and
//     lse, norm statistics, MLP pre-activations), plus per-pass scratch;
//   * logits [tokens, V] — dlogits overwrite them in place.
// The step never returns to the host: CE normalisation, grad-norm, clip
// factor and Adam all read device scalars.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.h"
#include "mft_engine.h"

namespace mft {
namespace {

enum InitKind { INIT_NORMAL, INIT_ONE, INIT_ZERO, INIT_LORA_A, INIT_LORA_B };
enum { T_Q = 0, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_MAX };
enum { G_ATTN = 0, G_PROJ, G_FC, G_FC2 };
enum { CLS_LINEAR = 0, CLS_LMHEAD, CLS_ATTN, CLS_CE, CLS_RANK, CLS_MAX };

struct Param {
  std::string name;
  int ndim = 1;
  int64_t dims[2] = {0, 0};
  int64_t numel = 0;
  bool trainable = false, f16 = false;
  InitKind init = INIT_NORMAL;
  bool streamable = false;  // a linear weight or the token embedding (shard store)
  int shard = -1;           // its shard store entry when the model is sharded
  size_t offset = 0;  // bytes in the frozen arena (or the host store), or floats in the LoRA arrays
  void* data = nullptr;
  float* grad = nullptr;
};

struct Linear {
  int W = -1, b = -1, A = -1, B = -1;
  int K = 0, N = 0;
  float* weff = nullptr;  // merged weight W + s·Aᵀ·Bᵀ [K, N] fp32 (LoRA linears), rows weff_ld apart
  int weff_ld = 0;
  int lid = 0;            // LoRA dropout stream: layer·8 + target
  float* xd = nullptr;    // LoRA input after dropout [M, K] (training forwards with dropout)
  // rank-r panel path: batched launch run before this linear's forward GEMM
  // (every xa of its input group) and before its dX GEMM (every U of its
  // gradient group); -1 when another linear of the group runs it
  int xa_batch = -1, u_batch = -1;
  float* u = nullptr;  // U = dY·B of this linear (panel path)
  // row scales of this linear's GEMM input (x forward, dY backward) for the
  // fp16 matrix-core GEMM, written by the batched rank-r launches (panel path)
  const float* rs_fwd = nullptr;
  const float* rs_bwd = nullptr;
};


struct Layer {
  int n1w = -1, n1b = -1, n2w = -1, n2b = -1, qn = -1, kn = -1, pan = -1, pfn = -1;
  Linear lin[T_MAX];
};

struct Acts {
  float *x, *n1, *mean1, *rstd1;
  float *q, *k, *v, *qraw, *kraw, *qrs, *krs;
  int64_t qs, ks, vs;
  float* xa[T_MAX];
  float* U[T_MAX];   // dY·B of each LoRA linear (kept for dA at the end of the backward)
  float* DY[T_MAX];  // dY of each LoRA linear, kept until the end of the backward
  int64_t dy_ld[T_MAX];  // row pitch of DY[t] (N, or the fused q|k|v width)
  float *qkv, *dyqkv;    // fused q|k|v projection output and its gradient (fuse_qkv)
  float *gu, *dygu;      // fused gate|up projection output [M, 2·ff] and its gradient (fuse_gu)
  float *att, *lse, *o, *ors, *hmid, *n2, *mean2, *rstd2;
  float *gate, *up, *act, *mo, *mrs;
};

struct Bump {
  char* base = nullptr;
  size_t cap = 0, used = 0;
  void* take(size_t bytes) {
    size_t b = (bytes + 255) & ~size_t(255);
    if (used + b > cap) throw Error(MFT_ENOMEM, "activation arena exhausted");
    void* p = base + used;
    used += b;
    return p;
  }
  float* f(int64_t n) { return reinterpret_cast<float*>(take((size_t)n * sizeof(float))); }
};

struct TimedLaunch {
  int cls;
  double work;
  hipEvent_t a, b;
  hipEvent_t c = nullptr, d = nullptr;  // a second interval (a GEMM's split-K reduction), or null
};

}  // namespace
}  // namespace mft

using namespace mft;

// Frozen weights streamed from pinned host memory into an HBM pool
// (ParameterSharder's require(), README.md:302-329).  Every use takes the
// tensor's pool copy (loading it first when absent: least recently used
// entries are evicted until a first-fit block is free), makes the compute
// stream wait for the copy, and records a use event after the launch, which
// the copy stream waits on before it overwrites the block.  After each use
// the tensor that followed it in the previous pass is prefetched.
struct ShardStore {
  int64_t budget = 0;
  char* pool = nullptr;  // device, budget bytes
  char* host = nullptr;  // pinned host memory holding every streamed tensor
  hipStream_t copy = nullptr;
  struct Entry {
    int param = -1;
    size_t bytes = 0;
    int64_t off = -1;  // pool offset while resident
    uint64_t last = 0;  // LRU clock of the last use or prefetch
    bool held = false;  // in use by a launch being enqueued
    bool used_valid = false, ready_valid = false;
    hipEvent_t ready = nullptr, used = nullptr;
  };
  std::vector<Entry> ents;
  std::map<int64_t, int64_t> free_blocks;  // pool offset → bytes
  uint64_t clock = 0;
  std::vector<int> seq, prev;  // entries in use order: this pass and the previous one
  int64_t loads = 0, hits = 0;
  // error of a prefetch issued from a use's release (reported by the next use)
  int deferred_code = 0;
  std::string deferred;
};

// Loss and count slots of a step: 64 doubles then 64 int64 (8-byte words).
constexpr int kStatWords = 128;
static_assert(sizeof(double) == 8 && sizeof(int64_t) == 8, "stat slots");

struct mft_model_s {
  mft_model_cfg c{};
  ShardStore sh;
  hipStream_t stream = nullptr;
  int64_t max_tokens = 0;
  std::vector<Param> P;
  std::vector<Layer> L;
  int wte = -1, wpe = -1, nfw = -1, nfb = -1;
  // arenas
  void* frozen = nullptr;
  size_t frozen_bytes = 0;
  float *lora_p = nullptr, *lora_g = nullptr, *lora_m = nullptr, *lora_v = nullptr;
  int64_t lora_n = 0;
  void* act_mem = nullptr;
  Bump act;
  std::vector<Acts> A;
  float *h_final = nullptr, *hf = nullptr, *fmean = nullptr, *frstd = nullptr;
  float* logits = nullptr;
  int64_t ldv = 0;  // logits row stride: vocab rounded up to 4 (zeroed padding)
  // Per-row softmax statistics of the logits, one (max, Σ) pair per 64
  // columns, written by the LM head's GEMM for vocabularies too wide for the
  // cross-entropy to hold a row in registers; stats_fresh says the last
  // forward wrote them for the logits now in place.
  float2* row_stats = nullptr;
  int64_t stats_ld = 0;
  bool stats_fresh = false;
  // dh, dh2: residual-stream gradients entering a layer's MLP and attention
  // blocks (alternating, so norm backward passes run out of place)
  float *dh = nullptr, *dh2 = nullptr, *dtmp = nullptr, *dn = nullptr, *datt = nullptr;
  float *dq = nullptr, *dk = nullptr, *dv = nullptr, *dqkv = nullptr;
  float *dact = nullptr, *dgate = nullptr, *dup = nullptr;
  float *dtq = nullptr, *dtk = nullptr;
  float* row_nll = nullptr;
  // RoPE angle tables (cos, sin) for positions [0, max_tokens): global θ and
  // (Gemma3) the local layers' θ
  float2* rope_tab[2] = {nullptr, nullptr};
  Scratch ws;
  // Merged LoRA weights and batched rank-r work.  With `merged`, every LoRA
  // linear multiplies by W_eff = W + s·Aᵀ·Bᵀ (rebuilt by one launch at the
  // start of each forward), its dY is written to a buffer of its own and kept,
  // and the gradients dA = s·Uᵀ·x, dB = s·dYᵀ·xa (U = dY·B, xa = x·Aᵀ) come
  // from three table-driven launches: all xa at the start of the backward,
  // all U and dB after the last layer, then all dA.
  bool merged = false;
  // Rank-r panel path (LoRA linears over fp16-stored W, which a fp32 W_eff
  // would double): every LoRA linear multiplies the frozen W, widened in the
  // GEMM's tile load, and adds s·xa·Bᵀ (forward) or s·U·A (dX) as one more
  // MFMA K-panel of depth r.  xa and U come from one batched launch per
  // input / gradient group of a layer (q|k|v, o, gate|up, down); dB and dA
  // from two whole-model launches at the end of the backward.
  bool panel = false;
  // Alignment-dump debug mode: layers whose activations and activation
  // gradients are retained (bit l = layer l), and the retained copies keyed
  // by (layer, name): activations a forward does not keep as they are
  // (q/k before RoPE, GELU(gate), attention scores and probabilities) and
  // every activation gradient the backward forms.
  uint64_t retain = 0;
  struct Kept {
    float* p = nullptr;
    int64_t rows = 0, cols = 0;
    size_t cap = 0;
  };
  std::map<std::pair<int, std::string>, Kept> kept_act, kept_grad;
  // Row scales for the fp16 matrix-core GEMMs of fp16-stored W: one
  // [max_tokens] slot per linear of a layer (written by the batched rank-r
  // launches, read by the GEMMs that follow them), then one for GEMMs whose
  // input no batched launch reads.
  float* rscale = nullptr;
  // row scales of the dlogits, written by the CE backward for the LM head's
  // dH GEMM on the fp16 path (fresh until that GEMM reads them)
  float* dl_rscale = nullptr;
  bool dl_rs_fresh = false;
  void* weff_mem = nullptr;
  void* tables = nullptr;  // device: MergeJob[n_merge], then RankJob[]
  const MergeJob* d_merge = nullptr;
  int n_merge = 0, merge_tiles_total = 0;
  struct Batch {
    const RankJob* jobs;
    int njobs, nproj, outer_blocks;
    double work_per_row;  // HBM bytes per token row (timing)
    ProjJobs pj;          // pj.n > 0: the same projections by value (one launch of rank_proj_jobs)
  };
  std::vector<Batch> batches;
  int xa_batch = -1, udb_batch = -1, da_batch = -1, db_batch = -1;
  // device scalars: [0..63] per-micro loss sums (double), counts (int64)
  double* d_loss = nullptr;
  int64_t* d_cnt = nullptr;
  int64_t* d_tmpcnt = nullptr;
  double* d_sumsq = nullptr;
  double* d_partials = nullptr;  // kOptBlocks Σg² partials of the optimizer
  bool zero_pending = false;      // the loss/count slots are cleared by the next forward's first launch
  float* d_clip = nullptr;  // [0] scale, [1] norm
  float* d_hp = nullptr;    // {lr, b1, b2, eps, wd, max_norm}
  int* d_t = nullptr;       // Adam step count (advanced on the device)
  // input error bits set by kernels: 1 = a token id outside [0, vocab)
  // (its embedding row is zeros), 2 = a label outside [0, vocab) that is not
  // ignore_index (counted as ignored); reported by mft_model_read_stats
  int* d_err = nullptr;
  int* d_drop_step = nullptr;  // training forwards run (LoRA dropout stream)
  bool training = true;        // training forwards apply LoRA dropout
  bool fwd_dropout = false;    // the last forward applied it (its backward must too)
  int drop_n_fwd = 1;          // micro-batch forwards the last forward launch covered
  int64_t drop_rows = 0;       // rows per micro-batch forward
  int n_micro_pending = 0;
  int adam_t = 0;
  // Qwen2 / Gemma3 with LoRA on q, k and v (merged path): one GEMM for
  // q|k|v forward and one for its dX, over a W_eff block [d, nqkv]
  bool fuse_qkv = false;
  int nqkv = 0;
  // gate|up as one projection (column blocks of one [d, 2·ff] W_eff) and
  // one dX GEMM, when both are merged LoRA linears without bias
  bool fuse_gu = false;
  // fp16-W rank-r panel path with LoRA on all of q, k, v (gate and up): one
  // column-segmented launch for their forward, one K-segmented launch for
  // their dX (each projection keeps its own W), with the fused layouts below
  bool seg_qkv = false, seg_gu = false;
  // fused activation layouts: q|k|v outputs and their dY as column blocks of
  // one [M, nqkv] buffer, gate|up of one [M, 2·ff] (fuse_* or seg_*)
  bool lay_qkv = false, lay_gu = false;
  // operator-level split points: shape of the forward whose activations are
  // kept (0 = none) and whether its logits buffer now holds dlogits
  int api_nseq = 0, api_S = 0;
  bool api_dlogits = false;
  // dlogits formed beside the logits by mft_model_ce(backward = 2) for the
  // pending forward (upstream factor alt_up), adopted by its backward = 1
  // call: the two buffers trade places
  float* logits_alt = nullptr;
  void* logits_alt_mem = nullptr;  // the allocation (either buffer may be the one in use)
  bool alt_ready = false;
  float alt_up = 0.f;
  int64_t last_rows = 0;  // token rows of the last forward (activation accessor)
  // captured train-step graph
  hipStream_t cap_stream = nullptr;
  bool stream_registered = false;  // m->stream is in the sync check's stream list
  hipEvent_t ev_in = nullptr, ev_out = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  bool capturing = false;
  std::vector<TimedLaunch> graph_timed;  // event pairs recorded by the graph
  std::vector<hipEvent_t> gev_pool;
  struct {
    const void *ids, *mask, *labels;
    int n_micro, seqs, S;
    float upstream;
    bool timing, training;
  } graph_key{};
  // timing
  bool timing = false;
  std::vector<TimedLaunch> launches;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_next = 0;
  double t_ms[CLS_MAX] = {0}, t_work[CLS_MAX] = {0};
  int64_t t_n[CLS_MAX] = {0};
};

namespace {

const char* kGpt2Lin[4] = {"attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"};
const char* kHfLin[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                         "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                         "mlp.down_proj"};

int add_param(mft_model_s* m, const std::string& name, int64_t d0, int64_t d1, bool trainable,
              bool f16, InitKind init) {
  Param p;
  p.name = name;
  p.ndim = d1 > 0 ? 2 : 1;
  p.dims[0] = d0;
  p.dims[1] = d1 > 0 ? d1 : 0;
  p.numel = d0 * (d1 > 0 ? d1 : 1);
  p.trainable = trainable;
  p.f16 = f16;
  p.init = init;
  m->P.push_back(p);
  return (int)m->P.size() - 1;
}

void add_linear(mft_model_s* m, Linear& l, const std::string& pfx, const char* nm, int K, int N,
                bool bias, bool lora) {
  l.K = K;
  l.N = N;
  l.W = add_param(m, pfx + "." + nm + ".weight", K, N, false, m->c.w_fp16 != 0, INIT_NORMAL);
  m->P[l.W].streamable = true;
  if (bias) l.b = add_param(m, pfx + "." + nm + ".bias", N, 0, false, false, INIT_NORMAL);
  if (lora && m->c.lora_r > 0) {
    l.A = add_param(m, pfx + "." + nm + ".lora_A", m->c.lora_r, K, true, false, INIT_LORA_A);
    l.B = add_param(m, pfx + "." + nm + ".lora_B", N, m->c.lora_r, true, false, INIT_LORA_B);
  }
}

void build_params(mft_model_s* m) {
  const mft_model_cfg& c = m->c;
  const int d = c.d, hd = c.head_dim, H = c.n_head, Hk = c.n_kv_head;
  const bool f16 = c.w_fp16 != 0;
  m->L.resize(c.n_layer);
  if (c.arch == MFT_ARCH_GPT2) {
    m->wte = add_param(m, "wte", c.vocab, d, false, f16, INIT_NORMAL);
    m->P[m->wte].streamable = true;
    m->wpe = add_param(m, "wpe", c.max_pos, d, false, false, INIT_NORMAL);
    for (int i = 0; i < c.n_layer; ++i) {
      Layer& L = m->L[i];
      const std::string pfx = "h." + std::to_string(i);
      L.n1w = add_param(m, pfx + ".ln_1.weight", d, 0, false, false, INIT_ONE);
      L.n1b = add_param(m, pfx + ".ln_1.bias", d, 0, false, false, INIT_ZERO);
      add_linear(m, L.lin[G_ATTN], pfx, kGpt2Lin[0], d, 3 * d, true, c.lora_mask & 1);
      add_linear(m, L.lin[G_PROJ], pfx, kGpt2Lin[1], d, d, true, c.lora_mask & 2);
      L.n2w = add_param(m, pfx + ".ln_2.weight", d, 0, false, false, INIT_ONE);
      L.n2b = add_param(m, pfx + ".ln_2.bias", d, 0, false, false, INIT_ZERO);
      add_linear(m, L.lin[G_FC], pfx, kGpt2Lin[2], d, c.d_ff, true, c.lora_mask & 4);
      add_linear(m, L.lin[G_FC2], pfx, kGpt2Lin[3], c.d_ff, d, true, c.lora_mask & 8);
    }
    m->nfw = add_param(m, "ln_f.weight", d, 0, false, false, INIT_ONE);
    m->nfb = add_param(m, "ln_f.bias", d, 0, false, false, INIT_ZERO);
    return;
  }
  const bool qwen = c.arch == MFT_ARCH_QWEN2;
  const InitKind norm_init = qwen ? INIT_ONE : INIT_ZERO;
  m->wte = add_param(m, "embed_tokens.weight", c.vocab, d, false, f16, INIT_NORMAL);
  m->P[m->wte].streamable = true;
  for (int i = 0; i < c.n_layer; ++i) {
    Layer& L = m->L[i];
    const std::string pfx = "layers." + std::to_string(i);
    L.n1w = add_param(m, pfx + ".input_layernorm.weight", d, 0, false, false, norm_init);
    const int outs[7] = {H * hd, Hk * hd, Hk * hd, d, c.d_ff, c.d_ff, d};
    const int ins[7] = {d, d, d, H * hd, d, d, c.d_ff};
    for (int t = 0; t < 4; ++t) add_linear(m, L.lin[t], pfx, kHfLin[t], ins[t], outs[t], false, (c.lora_mask >> t) & 1);
    // Qwen2's q/k/v biases are placed back to back in the frozen arena, so a
    // fused q|k|v GEMM can take them as one bias vector.
    if (qwen)
      for (int t = 0; t < 3; ++t)
        L.lin[t].b = add_param(m, pfx + "." + kHfLin[t] + ".bias", outs[t], 0, false, false, INIT_NORMAL);
    if (!qwen) {
      L.qn = add_param(m, pfx + ".self_attn.q_norm.weight", hd, 0, false, false, INIT_ZERO);
      L.kn = add_param(m, pfx + ".self_attn.k_norm.weight", hd, 0, false, false, INIT_ZERO);
      L.pan = add_param(m, pfx + ".post_attention_layernorm.weight", d, 0, false, false, INIT_ZERO);
      L.n2w = add_param(m, pfx + ".pre_feedforward_layernorm.weight", d, 0, false, false, INIT_ZERO);
      L.pfn = add_param(m, pfx + ".post_feedforward_layernorm.weight", d, 0, false, false, INIT_ZERO);
    } else {
      L.n2w = add_param(m, pfx + ".post_attention_layernorm.weight", d, 0, false, false, INIT_ONE);
    }
    for (int t = 4; t < 7; ++t)
      add_linear(m, L.lin[t], pfx, kHfLin[t], ins[t], outs[t], false, (c.lora_mask >> t) & 1);
  }
  m->nfw = add_param(m, "norm.weight", d, 0, false, false, norm_init);
}

void assign_dropout_streams(mft_model_s* m) {
  for (size_t li = 0; li < m->L.size(); ++li)
    for (int t = 0; t < T_MAX; ++t) m->L[li].lin[t].lid = (int)li * 8 + t;
}

size_t shard_round(size_t b) { return (b + 255) & ~size_t(255); }

void alloc_params(mft_model_s* m) {
  size_t fb = 0, hb = 0, largest = 0;
  int64_t ln = 0;
  ShardStore& sh = m->sh;
  const bool sharded = m->c.shard_budget > 0;
  for (size_t i = 0; i < m->P.size(); ++i) {
    Param& p = m->P[i];
    const size_t bytes = (size_t)p.numel * (p.f16 ? 2 : 4);
    if (p.trainable) {
      p.offset = (size_t)ln;
      ln += (p.numel + 63) / 64 * 64;
    } else if (sharded && p.streamable) {
      p.offset = hb;
      hb += shard_round(bytes);
      largest = std::max(largest, shard_round(bytes));
      p.shard = (int)sh.ents.size();
      ShardStore::Entry e;
      e.param = (int)i;
      e.bytes = bytes;
      sh.ents.push_back(e);
    } else {
      p.offset = fb;
      fb += shard_round(bytes);
    }
  }
  if (sharded) {
    const int64_t budget = m->c.shard_budget & ~int64_t(255);
    if (budget < (int64_t)largest)
      throw Error(MFT_EINVAL, "shard_budget (" + std::to_string(m->c.shard_budget) +
                                  " bytes) is below the largest streamed tensor (" + std::to_string(largest) +
                                  " bytes)");
    sh.budget = budget;
    if (hipHostMalloc(reinterpret_cast<void**>(&sh.host), hb ? hb : 256, hipHostMallocDefault) != hipSuccess)
      throw Error(MFT_ENOMEM, "shard store host memory (" + std::to_string(hb) + " bytes)");
    std::memset(sh.host, 0, hb ? hb : 256);
    if (hipMalloc(reinterpret_cast<void**>(&sh.pool), (size_t)budget) != hipSuccess)
      throw Error(MFT_ENOMEM, "shard store pool (" + std::to_string(budget) + " bytes)");
    sh.free_blocks[0] = budget;
    MFT_HIP(hipStreamCreateWithFlags(&sh.copy, hipStreamNonBlocking));
    register_stream(sh.copy);
    for (auto& e : sh.ents) {
      MFT_HIP(hipEventCreateWithFlags(&e.ready, hipEventDisableTiming));
      MFT_HIP(hipEventCreateWithFlags(&e.used, hipEventDisableTiming));
    }
  }
  m->frozen_bytes = fb;
  if (hipMalloc(&m->frozen, fb ? fb : 256) != hipSuccess)
    throw Error(MFT_ENOMEM, "frozen parameter arena (" + std::to_string(fb) + " bytes)");
  m->lora_n = ln;
  const size_t lb = (size_t)(ln ? ln : 64) * sizeof(float);
  float* arr[4];
  for (int i = 0; i < 4; ++i) {
    if (hipMalloc(reinterpret_cast<void**>(&arr[i]), lb) != hipSuccess)
      throw Error(MFT_ENOMEM, "LoRA arena");
    MFT_HIP(hipMemset(arr[i], 0, lb));
  }
  m->lora_p = arr[0];
  m->lora_g = arr[1];
  m->lora_m = arr[2];
  m->lora_v = arr[3];
  MFT_HIP(hipMemset(m->frozen, 0, fb ? fb : 256));
  for (auto& p : m->P) {
    if (p.trainable) {
      p.data = m->lora_p + p.offset;
      p.grad = m->lora_g + p.offset;
    } else if (p.shard >= 0) {
      p.data = sh.host + p.offset;
    } else {
      p.data = static_cast<char*>(m->frozen) + p.offset;
    }
  }
}

// ---- shard store --------------------------------------------------------------
int64_t shard_alloc(ShardStore& sh, size_t need) {
  for (auto it = sh.free_blocks.begin(); it != sh.free_blocks.end(); ++it) {
    if ((size_t)it->second >= need) {
      const int64_t off = it->first, rest = it->second - (int64_t)need;
      sh.free_blocks.erase(it);
      if (rest > 0) sh.free_blocks[off + (int64_t)need] = rest;
      return off;
    }
  }
  return -1;
}

void shard_free(ShardStore& sh, int64_t off, int64_t bytes) {
  auto it = sh.free_blocks.emplace(off, bytes).first;
  auto nx = std::next(it);
  if (nx != sh.free_blocks.end() && it->first + it->second == nx->first) {
    it->second += nx->second;
    sh.free_blocks.erase(nx);
  }
  if (it != sh.free_blocks.begin()) {
    auto pv = std::prev(it);
    if (pv->first + pv->second == it->first) {
      pv->second += it->second;
      sh.free_blocks.erase(it);
    }
  }
}

// Uses until entry j is next needed, counted from use position pos of the
// current pass, read off the previous pass's order (a step repeats its use
// order): positions pos.. of this pass, then the next pass from its start;
// a large value when the previous pass never used it.
int64_t shard_next_use(const ShardStore& sh, int j, size_t pos) {
  const size_t n = sh.prev.size();
  for (size_t q = pos; q < n; ++q)
    if (sh.prev[q] == j) return (int64_t)(q - pos);
  for (size_t q = 0; q < std::min(pos, n); ++q)
    if (sh.prev[q] == j) return (int64_t)(n - pos + q);
  return INT64_MAX / 2;
}

// Makes entry i resident: evicts entries no launch holds until a first-fit
// block is free — the one needed furthest ahead in the step's use order
// (Belady's rule over the previous pass's order; least recently used while
// there is no previous pass) — then copies the tensor on the copy stream,
// behind the last uses of every evicted block.  When nothing more can be
// evicted, a prefetch returns false (the use will load it); a use throws.
// Tuning hook: MFT_SHARD_LRU=1 evicts least recently used entries always.
bool shard_load(mft_model_s* m, int i, bool prefetch = false) {
  static const bool lru_only = [] {
    const char* e = getenv("MFT_SHARD_LRU");
    return e && atoi(e) != 0;
  }();
  ShardStore& sh = m->sh;
  const size_t need = shard_round(sh.ents[i].bytes);
  const size_t pos = sh.seq.size();  // this pass's position of the use being served
  int64_t off;
  while ((off = shard_alloc(sh, need)) < 0) {
    int v = -1;
    int64_t v_next = -1;
    for (int j = 0; j < (int)sh.ents.size(); ++j) {
      const ShardStore::Entry& c = sh.ents[j];
      if (j == i || c.off < 0 || c.held) continue;
      const int64_t nx = lru_only || sh.prev.empty() ? 0 : shard_next_use(sh, j, pos);
      if (v < 0 || nx > v_next || (nx == v_next && c.last < sh.ents[v].last)) {
        v = j;
        v_next = nx;
      }
    }
    if (v < 0) {
      if (prefetch) return false;
      throw Error(MFT_EINVAL, "shard budget too small for the tensors one launch uses");
    }
    ShardStore::Entry& ev = sh.ents[v];
    if (ev.used_valid) MFT_HIP(hipStreamWaitEvent(sh.copy, ev.used, 0));
    shard_free(sh, ev.off, (int64_t)shard_round(ev.bytes));
    ev.off = -1;
  }
  ShardStore::Entry& e = sh.ents[i];
  e.off = off;
  MFT_HIP(hipMemcpyAsync(sh.pool + off, sh.host + m->P[e.param].offset, e.bytes, hipMemcpyHostToDevice, sh.copy));
  MFT_HIP(hipEventRecord(e.ready, sh.copy));
  e.ready_valid = true;
  ++sh.loads;
  return true;
}

// Device address of frozen parameter p for the next launch on the model's
// stream (the shard store's pool copy when p is streamed); release() follows
// the launch.
struct WeightUse {
  mft_model_s* m;
  int p;
  const void* ptr;
  WeightUse(mft_model_s* mm, int pi) : m(mm), p(pi) {
    const int i = m->P[p].shard;
    if (i < 0) {
      ptr = m->P[p].data;
      return;
    }
    ShardStore& sh = m->sh;
    if (sh.deferred_code) {  // a prefetch issued after an earlier use failed
      const int code = sh.deferred_code;
      sh.deferred_code = 0;
      throw Error(code, "shard store prefetch failed: " + sh.deferred);
    }
    ShardStore::Entry& e = sh.ents[i];
    e.held = true;
    e.last = ++sh.clock;
    if (e.off < 0) shard_load(m, i);
    else ++sh.hits;
    if (e.ready_valid) MFT_HIP(hipStreamWaitEvent(m->stream, e.ready, 0));
    sh.seq.push_back(i);
    ptr = sh.pool + e.off;
  }
  ~WeightUse() {
    const int i = m->P[p].shard;
    if (i < 0) return;
    ShardStore& sh = m->sh;
    ShardStore::Entry& e = sh.ents[i];
    e.held = false;
    if (hipEventRecord(e.used, m->stream) != hipSuccess) return;
    e.used_valid = true;
    // prefetch the tensor that followed this use in the previous pass
    const size_t pos = sh.seq.size();
    if (pos < sh.prev.size()) {
      ShardStore::Entry& n = sh.ents[sh.prev[pos]];
      if (n.off < 0 && !n.held) {
        n.last = ++sh.clock;
        // A budget that cannot hold it now makes the prefetch a no-op; any
        // other failure (a HIP copy, event or wait error) is kept and thrown
        // by the next use, since a destructor cannot throw.
        try {
          (void)shard_load(m, sh.prev[pos], true);
        } catch (const Error& err) {
          sh.deferred_code = err.code;
          sh.deferred = err.what();
        } catch (const std::exception& err) {
          sh.deferred_code = MFT_EHIP;
          sh.deferred = err.what();
        }
      }
    }
  }
};

// A new pass (forward, then its backward) starts a new use order.
void shard_begin(mft_model_s* m) {
  ShardStore& sh = m->sh;
  if (!sh.copy || sh.seq.empty()) return;
  sh.prev.swap(sh.seq);
  sh.seq.clear();
}

// Drops every pool copy (host copies rewritten, or the pool reused as scratch).
void shard_reset(mft_model_s* m) {
  ShardStore& sh = m->sh;
  if (!sh.copy) return;
  MFT_HIP(hipStreamSynchronize(m->stream));
  MFT_HIP(hipStreamSynchronize(sh.copy));
  for (auto& e : sh.ents) {
    e.off = -1;
    e.held = e.used_valid = e.ready_valid = false;
  }
  sh.free_blocks.clear();
  sh.free_blocks[0] = sh.budget;
  sh.seq.clear();
  sh.prev.clear();
}

bool layer_local(const mft_model_cfg& c, int i) {
  return c.arch == MFT_ARCH_GEMMA3 && c.sliding_pattern > 0 && ((i + 1) % c.sliding_pattern) != 0;
}
float attn_scale(const mft_model_cfg& c) {
  return c.attn_scale > 0.f ? c.attn_scale : 1.f / std::sqrt((float)c.head_dim);
}

// The batched rank-r kernels (merged-weight and rank-r panel paths) take
// r ∈ {4, 8, 16, 32} and LoRA linears with K and N multiples of 4.
bool lora_batched(const mft_model_s* m) {
  const int r = m->c.lora_r;
  if (r != 4 && r != 8 && r != 16 && r != 32) return false;
  // dropout masks the LoRA branch's input only, which a merged W_eff cannot express
  if (m->c.lora_dropout > 0.f) return false;
  bool any = false;
  for (const auto& L : m->L)
    for (const auto& l : L.lin) {
      if (l.A < 0) continue;
      if (l.N % 4 || l.K % 4) return false;
      any = true;
    }
  return any;
}

// The merged-weight path serves fp32 W; LoRA linears over fp16-stored W take
// the rank-r panel path, so W stays 2 bytes per element.  Tuning hook:
// MFT_LORA_MERGE=0 puts fp32 models on the panel path too, =2 merges fp16 W
// into an fp32 W_eff as well.
bool lora_merge(const mft_model_s* m) {
  static const int hook = [] {
    const char* e = getenv("MFT_LORA_MERGE");
    return e ? atoi(e) : 1;
  }();
  if (!hook || !lora_batched(m)) return false;
  if (m->c.shard_budget > 0) return false;  // streamed W: no whole-model merge
  if (hook == 2) return true;
  for (const auto& L : m->L)
    for (const auto& l : L.lin)
      if (l.A >= 0 && m->P[l.W].f16) return false;
  return true;
}

// q, k and v fuse into one projection when all three are merged LoRA
// linears and (Qwen2) their biases sit back to back.
bool qkv_fusable(const mft_model_s* m) {
  if (m->c.arch == MFT_ARCH_GPT2 || !lora_merge(m)) return false;
  for (const auto& L : m->L) {
    for (int t = 0; t < 3; ++t)
      if (L.lin[t].A < 0) return false;
    if (L.lin[0].b >= 0) {
      const char* b0 = static_cast<const char*>(m->P[L.lin[0].b].data);
      if (L.lin[1].b < 0 || L.lin[2].b < 0 ||
          static_cast<const char*>(m->P[L.lin[1].b].data) != b0 + 4 * (size_t)L.lin[0].N ||
          static_cast<const char*>(m->P[L.lin[2].b].data) != b0 + 4 * (size_t)(L.lin[0].N + L.lin[1].N))
        return false;
    }
  }
  return true;
}

// gate and up fuse into one projection when both are merged LoRA linears
// without bias (their W_eff become column blocks of one array).
bool gu_fusable(const mft_model_s* m) {
  if (m->c.arch == MFT_ARCH_GPT2 || !lora_merge(m)) return false;
  for (const auto& L : m->L) {
    const Linear &g = L.lin[T_GATE], &u = L.lin[T_UP];
    if (g.A < 0 || u.A < 0 || g.b >= 0 || u.b >= 0 || g.K != u.K || g.N != u.N) return false;
  }
  return true;
}

// The rank-r panel path's segmented launches (gemm_h_segments forward,
// gemm_h_ksegments dX) for linears t0 .. t0+n-1 of every layer: each a LoRA
// linear over fp16 W resident in HBM (no shard store), no bias, one input
// width, output widths in 64-column tiles, and n·r ≤ 32 for the dX's rank
// panels.  Tuning hook: MFT_GROUP_FWD=0 keeps one launch per projection.
bool segment_fusable(const mft_model_s* m, int t0, int n) {
  static const bool on = [] {
    const char* e = getenv("MFT_GROUP_FWD");
    return !e || atoi(e) != 0;
  }();
  const mft_model_cfg& c = m->c;
  if (!on || c.arch == MFT_ARCH_GPT2 || !lora_batched(m) || lora_merge(m) || c.shard_budget > 0 ||
      n * c.lora_r > 32)
    return false;
  for (const auto& L : m->L)
    for (int t = t0; t < t0 + n; ++t) {
      const Linear& l = L.lin[t];
      if (l.A < 0 || l.b >= 0 || !m->P[l.W].f16 || l.K != L.lin[t0].K || l.N % 64 != 0 || l.K % 32 != 0)
        return false;
    }
  return true;
}

void alloc_acts(mft_model_s* m) {
  const mft_model_cfg& c = m->c;
  m->fuse_qkv = qkv_fusable(m);
  m->fuse_gu = gu_fusable(m);
  m->nqkv = c.n_head * c.head_dim + 2 * c.n_kv_head * c.head_dim;
  m->seg_qkv = segment_fusable(m, T_Q, 3);
  m->seg_gu = segment_fusable(m, T_GATE, 2);
  m->lay_qkv = m->fuse_qkv || m->seg_qkv;
  m->lay_gu = m->fuse_gu || m->seg_gu;
  const int64_t M = m->max_tokens;
  const int64_t d = c.d, H = c.n_head, Hk = c.n_kv_head, hd = c.head_dim, ff = c.d_ff, r = c.lora_r;
  const bool gpt2 = c.arch == MFT_ARCH_GPT2, gemma = c.arch == MFT_ARCH_GEMMA3;
  // size estimate (floats) — computed by a dry run of the same carve-up
  auto carve = [&](Bump& b) {
    m->A.assign(c.n_layer, Acts{});
    for (int l = 0; l < c.n_layer; ++l) {
      Acts& a = m->A[l];
      std::memset(&a, 0, sizeof(a));
      a.x = b.f(M * d);
      a.n1 = b.f(M * d);
      a.rstd1 = b.f(M);
      if (gpt2) {
        a.mean1 = b.f(M);
        a.q = b.f(M * 3 * d);
        a.k = a.q + d;
        a.v = a.q + 2 * d;
        a.qs = a.ks = a.vs = 3 * d;
      } else if (m->lay_qkv) {
        // one [M, nqkv] projection output: q|k|v (Qwen2), qraw|kraw|v (Gemma3)
        const int64_t nq = H * hd, nk = Hk * hd, nt = m->nqkv;
        a.qkv = b.f(M * nt);
        a.dyqkv = b.f(M * nt);
        if (gemma) {
          a.qraw = a.qkv;
          a.kraw = a.qkv + nq;
          a.q = b.f(M * nq);
          a.k = b.f(M * nk);
          a.qs = nq;
          a.ks = nk;
          a.qrs = b.f(M * H);
          a.krs = b.f(M * Hk);
        } else {
          a.q = a.qkv;
          a.k = a.qkv + nq;
          a.qs = a.ks = nt;
        }
        a.v = a.qkv + nq + nk;
        a.vs = nt;
      } else {
        a.q = b.f(M * H * hd);
        a.k = b.f(M * Hk * hd);
        a.v = b.f(M * Hk * hd);
        a.qs = H * hd;
        a.ks = a.vs = Hk * hd;
        if (gemma) {
          a.qraw = b.f(M * H * hd);
          a.kraw = b.f(M * Hk * hd);
          a.qrs = b.f(M * H);
          a.krs = b.f(M * Hk);
        }
      }
      Layer& L = m->L[l];
      const bool keep_dy = lora_batched(m);
      for (int t = 0; t < T_MAX; ++t)
        if (L.lin[t].A >= 0) {
          if (c.lora_dropout > 0.f) L.lin[t].xd = b.f(M * L.lin[t].K);
          a.xa[t] = b.f(M * r);
          a.U[t] = b.f(M * r);
          if (m->lay_qkv && t < 3) {  // views of the fused gradient
            a.DY[t] = a.dyqkv + (t == 0 ? 0 : H * hd + (t - 1) * Hk * hd);
            a.dy_ld[t] = m->nqkv;
          } else if (m->lay_gu && (t == T_GATE || t == T_UP)) {
            if (t == T_GATE) a.dygu = b.f(M * 2 * ff);
            a.DY[t] = a.dygu + (t == T_GATE ? 0 : ff);
            a.dy_ld[t] = 2 * ff;
          } else if (keep_dy) {
            a.DY[t] = b.f(M * L.lin[t].N);
            a.dy_ld[t] = L.lin[t].N;
          }
        }
      a.att = b.f(M * H * hd);
      a.lse = b.f(M * H);
      a.o = b.f(M * d);
      if (gemma) a.ors = b.f(M);
      a.hmid = b.f(M * d);
      a.n2 = b.f(M * d);
      a.rstd2 = b.f(M);
      if (gpt2) a.mean2 = b.f(M);
      if (m->lay_gu) {
        a.gu = b.f(M * 2 * ff);
        a.gate = a.gu;
        a.up = a.gu + ff;
      } else {
        a.gate = b.f(M * ff);
        if (!gpt2) a.up = b.f(M * ff);
      }
      a.act = b.f(M * ff);
      a.mo = b.f(M * d);
      if (gemma) a.mrs = b.f(M);
    }
    m->h_final = b.f(M * d);
    m->hf = b.f(M * d);
    m->frstd = b.f(M);
    m->fmean = b.f(M);
    m->ldv = (c.vocab + 3) / 4 * 4;
    m->logits = b.f(M * m->ldv);
    if (c.vocab > 13 * 4096 && gemm_wide_plan((int)M, (int)c.vocab)) {
      m->stats_ld = cdiv(c.vocab, 64);
      m->row_stats = reinterpret_cast<float2*>(b.f(2 * M * m->stats_ld));
    }
    m->dh = b.f(M * d);
    m->dh2 = b.f(M * d);
    m->dtmp = b.f(M * d);
    m->dn = b.f(M * d);
    m->datt = b.f(M * H * hd);
    m->dq = b.f(M * H * hd);
    m->dk = b.f(M * Hk * hd);
    m->dv = b.f(M * Hk * hd);
    m->dtq = b.f(M * H * hd);
    m->dtk = b.f(M * Hk * hd);
    if (gpt2) m->dqkv = b.f(M * 3 * d);
    m->dact = b.f(M * ff);
    m->dgate = b.f(M * ff);
    m->dup = b.f(M * ff);
    m->row_nll = b.f(M);
    if (!gpt2) {
      m->rope_tab[0] = reinterpret_cast<float2*>(b.f(M * hd));  // M positions × hd/2 pairs
      if (gemma) m->rope_tab[1] = reinterpret_cast<float2*>(b.f(M * hd));
    }
    const int64_t wide = std::max<int64_t>({d, ff, H * hd, 3 * d});
    const int64_t wsf = std::max<int64_t>(
        M * std::max<int64_t>(r, 1) + 16 * std::max<int64_t>(r, 1) * wide + 8 * M * wide,
        (int64_t)attn_scratch_bound_floats(M, (int)H, (int)hd));
    m->ws.ptr = b.f(wsf);
    m->ws.bytes = (size_t)wsf * sizeof(float);
  };
  Bump dry;
  dry.base = nullptr;
  dry.cap = SIZE_MAX / 2;
  carve(dry);
  const size_t need = dry.used;
  if (hipMalloc(&m->act_mem, need) != hipSuccess)
    throw Error(MFT_ENOMEM, "activation arena (" + std::to_string(need) + " bytes)");
  m->act.base = static_cast<char*>(m->act_mem);
  m->act.cap = need;
  m->act.used = 0;
  carve(m->act);
  // logits padding columns are never written and must stay finite (they are
  // read, times zero rows of E, by the LM-head backward's vector loads).
  MFT_HIP(hipMemset(m->logits, 0, sizeof(float) * (size_t)M * m->ldv));
  if (m->rope_tab[0]) rope_table(m->stream, c.rope_theta, (int)hd, (int)M, m->rope_tab[0]);
  if (m->rope_tab[1]) rope_table(m->stream, c.rope_local_theta, (int)hd, (int)M, m->rope_tab[1]);
  MFT_HIP(hipStreamSynchronize(m->stream));
  void* sc = nullptr;
  MFT_HIP(hipMalloc(&sc, 4096 + kOptBlocks * sizeof(double)));
  MFT_HIP(hipMemset(sc, 0, 4096 + kOptBlocks * sizeof(double)));
  m->d_loss = reinterpret_cast<double*>(sc);                               // 64 doubles
  m->d_cnt = reinterpret_cast<int64_t*>(static_cast<char*>(sc) + 512);     // 64 int64
  m->d_tmpcnt = reinterpret_cast<int64_t*>(static_cast<char*>(sc) + 1024);
  m->d_sumsq = reinterpret_cast<double*>(static_cast<char*>(sc) + 1280);
  m->d_clip = reinterpret_cast<float*>(static_cast<char*>(sc) + 1536);
  m->d_hp = reinterpret_cast<float*>(static_cast<char*>(sc) + 1792);
  m->d_t = reinterpret_cast<int*>(static_cast<char*>(sc) + 2048);
  m->d_err = reinterpret_cast<int*>(static_cast<char*>(sc) + 2304);
  m->d_drop_step = reinterpret_cast<int*>(static_cast<char*>(sc) + 2560);
  m->d_partials = reinterpret_cast<double*>(static_cast<char*>(sc) + 4096);
  MFT_HIP(hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking));
  register_stream(m->cap_stream);
  MFT_HIP(hipEventCreateWithFlags(&m->ev_in, hipEventDisableTiming));
  MFT_HIP(hipEventCreateWithFlags(&m->ev_out, hipEventDisableTiming));
}

// ---- merged LoRA: W_eff arena and job tables --------------------------------------
// Input x of LoRA linear t of layer li (its dY lives in A[li].DY[t]).
const float* lora_x(mft_model_s* m, int li, int t) {
  const Acts& a = m->A[li];
  if (m->c.arch == MFT_ARCH_GPT2) {
    const float* xs[4] = {a.n1, a.att, a.n2, a.act};
    return xs[t];
  }
  const float* xs[T_MAX] = {a.n1, a.n1, a.n1, a.att, a.n2, a.n2, a.act};
  return xs[t];
}

float lscale(const mft_model_s* m);

// Builds W_eff buffers and the device job tables once the activation arena
// exists (the tables hold activation and gradient pointers).  Leaves
// `merged` false when a shape does not fit the batched kernels (then every
// LoRA linear keeps its rank-r epilogue path).
void build_lora_tables(mft_model_s* m) {
  const mft_model_cfg& c = m->c;
  const int r = c.lora_r;
  if (!lora_batched(m)) return;
  const bool panel = !lora_merge(m);
  const bool gpt2 = c.arch == MFT_ARCH_GPT2;
  const int nt = gpt2 ? 4 : T_MAX;
  size_t weff_floats = 0;
  if (!panel)
  for (auto& L : m->L)
    for (int t = 0; t < nt; ++t) {
      const Linear& l = L.lin[t];
      if (l.A < 0) continue;
      if (m->fuse_qkv && t < 3) {
        if (t == 0) weff_floats += ((size_t)l.K * m->nqkv + 63) / 64 * 64;  // one [d, nqkv] block
        continue;
      }
      if (m->fuse_gu && (t == T_GATE || t == T_UP)) {
        if (t == T_GATE) weff_floats += ((size_t)l.K * 2 * l.N + 63) / 64 * 64;  // one [d, 2·ff] block
        continue;
      }
      weff_floats += ((size_t)l.K * l.N + 63) / 64 * 64;
    }
  if (!panel && hipMalloc(&m->weff_mem, weff_floats * sizeof(float)) != hipSuccess)
    throw Error(MFT_ENOMEM, "merged LoRA weights (" + std::to_string(weff_floats * 4) + " bytes)");
  const float s = lscale(m);
  std::vector<MergeJob> mj;
  std::vector<RankJob> rj;
  struct Pending {
    size_t off;
    int njobs, nproj, outer_blocks;
    double work;
    ProjJobs pj;
  };
  std::vector<Pending> pend;
  auto proj_job = [&](const float* X, int64_t ldx, int K, const float* Y, bool y_rk, float* out) {
    RankJob j{};
    j.kind = 0; j.K = K; j.y_rk = y_rk ? 1 : 0; j.X = X; j.ldx = ldx; j.Y = Y; j.out = out; j.scale = 1.f;
    return j;
  };
  auto outer_job = [&](const float* P, const float* X, int64_t ldx, int C, float* out, int64_t osj, int64_t osc) {
    RankJob j{};
    j.kind = 1; j.K = C; j.accumulate = 1; j.blocks = rank_outer_blocks(C); j.X = X; j.ldx = ldx; j.Y = P;
    j.out = out; j.osj = osj; j.osc = osc; j.scale = s;
    return j;
  };
  // Appends one batch (projections first, then outer products) and returns
  // its index.
  auto add_batch = [&](std::vector<RankJob> proj, std::vector<RankJob> outer) {
    if (proj.empty() && outer.empty()) return -1;
    Pending p{rj.size(), (int)(proj.size() + outer.size()), (int)proj.size(), 0, 0.0, ProjJobs{}};
    // a few projections of one Y layout and nothing else: also kept by value
    if (outer.empty() && proj.size() <= (size_t)kMaxProjJobs) {
      bool same = true;
      for (auto& j : proj) same = same && j.y_rk == proj[0].y_rk;
      if (same) {
        for (auto& j : proj) p.pj.j[p.pj.n++] = ProjJob{j.X, j.ldx, j.Y, j.K, j.y_rk, j.out, j.inv_s};
      }
    }
    // timing work in HBM bytes per token row: a projection reads a K-wide
    // row and writes r values; an outer product reads a C-wide row and r values
    for (auto& j : proj) {
      p.work += 4.0 * (j.K + r);
      rj.push_back(j);
    }
    for (auto& j : outer) {
      j.block0 = p.outer_blocks;
      p.outer_blocks += j.blocks;
      p.work += 4.0 * (j.K + r);
      rj.push_back(j);
    }
    pend.push_back(p);
    return (int)pend.size() - 1;
  };
  std::vector<RankJob> xa_jobs, u_jobs, db_jobs, da_jobs;
  size_t woff = 0;
  int tiles = 0;
  // input / gradient groups of the panel path: GPT-2's four linears each
  // alone; q|k|v (input n1), o, gate|up (input n2), down
  auto group = [&](int t) { return gpt2 ? t : (t < 3 ? 0 : t == T_O ? 1 : t < T_DOWN ? 2 : 3); };
  for (int li = 0; li < c.n_layer; ++li) {
    Layer& L = m->L[li];
    Acts& a = m->A[li];
    if (panel) {
      for (int g = 0; g < 4; ++g) {
        std::vector<RankJob> gx, gu;
        int first = -1;
        for (int t = 0; t < nt; ++t) {
          Linear& l = L.lin[t];
          if (l.A < 0 || group(t) != g) continue;
          if (first < 0) first = t;
          const int64_t dld = a.dy_ld[t];
          // with fp16 W: the group's first projection also writes the row
          // scales of the shared input, every dY projection those of its dY
          float* slot_f = m->rscale ? m->rscale + (int64_t)first * m->max_tokens : nullptr;
          float* slot_b = m->rscale ? m->rscale + (int64_t)t * m->max_tokens : nullptr;
          RankJob jx = proj_job(lora_x(m, li, t), l.K, l.K, static_cast<const float*>(m->P[l.A].data), true,
                                a.xa[t]);
          if (t == first) jx.inv_s = slot_f;
          gx.push_back(jx);
          RankJob ju = proj_job(a.DY[t], dld, l.N, static_cast<const float*>(m->P[l.B].data), false, a.U[t]);
          ju.inv_s = slot_b;
          gu.push_back(ju);
          l.rs_fwd = slot_f;
          l.rs_bwd = slot_b;
          db_jobs.push_back(outer_job(a.xa[t], a.DY[t], dld, l.N, m->P[l.B].grad, 1, r));
          da_jobs.push_back(outer_job(a.U[t], lora_x(m, li, t), l.K, l.K, m->P[l.A].grad, l.K, 1));
        }
        if (first < 0) continue;
        for (int t = 0; t < nt; ++t)
          if (L.lin[t].A >= 0) L.lin[t].u = a.U[t];
        L.lin[first].xa_batch = add_batch(gx, {});
        L.lin[first].u_batch = add_batch(gu, {});
      }
      continue;
    }
    for (int t = 0; t < nt; ++t) {
      Linear& l = L.lin[t];
      if (l.A < 0) continue;
      if (m->fuse_qkv && t < 3) {  // column block t of the layer's [d, nqkv] W_eff
        if (t == 0) {
          l.weff = static_cast<float*>(m->weff_mem) + woff;
          woff += ((size_t)l.K * m->nqkv + 63) / 64 * 64;
        } else {
          l.weff = L.lin[t - 1].weff + L.lin[t - 1].N;
        }
        l.weff_ld = m->nqkv;
      } else if (m->fuse_gu && (t == T_GATE || t == T_UP)) {  // column block of the layer's [d, 2·ff] W_eff
        if (t == T_GATE) {
          l.weff = static_cast<float*>(m->weff_mem) + woff;
          woff += ((size_t)l.K * 2 * l.N + 63) / 64 * 64;
        } else {
          l.weff = L.lin[T_GATE].weff + L.lin[T_GATE].N;
        }
        l.weff_ld = 2 * l.N;
      } else {
        l.weff = static_cast<float*>(m->weff_mem) + woff;
        woff += ((size_t)l.K * l.N + 63) / 64 * 64;
        l.weff_ld = l.N;
      }
      MergeJob g{};
      g.W = m->P[l.W].data; g.A = static_cast<const float*>(m->P[l.A].data);
      g.B = static_cast<const float*>(m->P[l.B].data); g.out = l.weff; g.K = l.K; g.N = l.N;
      g.ldo = l.weff_ld;
      g.f16 = m->P[l.W].f16 ? 1 : 0; g.tile0 = tiles;
      tiles += (int)merge_tiles(l.K, l.N);
      mj.push_back(g);
      const float* x = lora_x(m, li, t);
      const float* dy = a.DY[t];
      // xa = x·Aᵀ; U = dY·B; dB += s·dYᵀ·xa (out(j,n) = dB[n][j]); dA += s·Uᵀ·x
      const int64_t dld = a.dy_ld[t];
      xa_jobs.push_back(proj_job(x, l.K, l.K, static_cast<const float*>(m->P[l.A].data), true, a.xa[t]));
      u_jobs.push_back(proj_job(dy, dld, l.N, static_cast<const float*>(m->P[l.B].data), false, a.U[t]));
      db_jobs.push_back(outer_job(a.xa[t], dy, dld, l.N, m->P[l.B].grad, 1, r));
      da_jobs.push_back(outer_job(a.U[t], x, l.K, l.K, m->P[l.A].grad, l.K, 1));
    }
  }
  if (panel) {
    m->db_batch = add_batch({}, db_jobs);
  } else {
    m->xa_batch = add_batch(xa_jobs, {});
    m->udb_batch = add_batch(u_jobs, db_jobs);
  }
  m->da_batch = add_batch({}, da_jobs);
  const size_t mbytes = (mj.size() * sizeof(MergeJob) + 255) & ~size_t(255);
  const size_t bytes = mbytes + rj.size() * sizeof(RankJob);
  if (hipMalloc(&m->tables, bytes) != hipSuccess) throw Error(MFT_ENOMEM, "LoRA job tables");
  MFT_HIP(hipMemcpy(m->tables, mj.data(), mj.size() * sizeof(MergeJob), hipMemcpyHostToDevice));
  const RankJob* d_rank = reinterpret_cast<const RankJob*>(static_cast<char*>(m->tables) + mbytes);
  MFT_HIP(hipMemcpy(const_cast<RankJob*>(d_rank), rj.data(), rj.size() * sizeof(RankJob), hipMemcpyHostToDevice));
  m->d_merge = static_cast<const MergeJob*>(m->tables);
  m->n_merge = (int)mj.size();
  m->merge_tiles_total = tiles;
  for (auto& p : pend) m->batches.push_back({d_rank + p.off, p.njobs, p.nproj, p.outer_blocks, p.work, p.pj});
  m->merged = !panel;
  m->panel = panel;
}

// Row-scale slots for the fp16 matrix-core GEMMs (models with fp16-stored W).
void alloc_row_scales(mft_model_s* m) {
  bool any_f16 = false;
  for (const Param& p : m->P) any_f16 = any_f16 || p.f16;
  if (any_f16 && hipMalloc(&m->rscale, (size_t)(T_MAX + 2) * m->max_tokens * sizeof(float)) != hipSuccess)
    throw Error(MFT_ENOMEM, "row scales");
  if (m->rscale) m->dl_rscale = m->rscale + (int64_t)(T_MAX + 1) * m->max_tokens;
}

// ---- timing helpers -------------------------------------------------------------
hipEvent_t next_event(mft_model_s* m) {
  if (m->capturing) {  // events owned by the captured graph
    hipEvent_t e;
    MFT_HIP(hipEventCreate(&e));
    m->gev_pool.push_back(e);
    return e;
  }
  if (m->ev_next == m->ev_pool.size()) {
    hipEvent_t e;
    MFT_HIP(hipEventCreate(&e));
    m->ev_pool.push_back(e);
  }
  return m->ev_pool[m->ev_next++];
}

struct Timed {
  mft_model_s* m;
  KernelEvents ev;
  int cls;
  double work;
  Timed(mft_model_s* mm, int c, double w) : m(mm), cls(c), work(w) {
    if (m->timing) {
      ev.start = next_event(m);
      ev.stop = next_event(m);
    }
  }
  // Events for a GEMM launch: the main kernel and its split-K reduction.
  const KernelEvents* events() {
    if (!m->timing) return nullptr;
    ev.tail_start = next_event(m);
    ev.tail_stop = next_event(m);
    return &ev;
  }
  void begin() {
    if (m->timing) MFT_HIP(hipEventRecord(ev.start, m->stream));
  }
  void end() {
    if (m->timing) MFT_HIP(hipEventRecord(ev.stop, m->stream));
  }
  ~Timed() {
    if (!m->timing) return;
    TimedLaunch t{cls, work, ev.start, ev.stop};
    if (ev.tail_used) {
      t.c = ev.tail_start;
      t.d = ev.tail_stop;
    }
    if (m->capturing) m->graph_timed.push_back(t);
    else m->launches.push_back(t);
  }
};

void collect_timing(mft_model_s* m) {
  if (m->launches.empty()) return;
  MFT_HIP(hipStreamSynchronize(m->stream));
  for (auto& t : m->launches) {
    float ms = 0.f, ms2 = 0.f;
    MFT_HIP(hipEventElapsedTime(&ms, t.a, t.b));
    if (t.c) MFT_HIP(hipEventElapsedTime(&ms2, t.c, t.d));
    m->t_ms[t.cls] += ms + ms2;
    m->t_work[t.cls] += t.work;
    m->t_n[t.cls] += 1;
  }
  m->launches.clear();
  m->ev_next = 0;
}

// ---- building blocks ---------------------------------------------------------------
float lscale(const mft_model_s* m) { return m->c.lora_alpha / (float)m->c.lora_r; }

DropStream drop_stream(const mft_model_s* m) {
  return DropStream{m->c.lora_dropout, m->c.dropout_seed, m->d_drop_step, m->drop_n_fwd, m->drop_rows};
}

void run_batch(mft_model_s* m, int idx, int64_t M);

// ---- alignment-dump debug mode ------------------------------------------------
bool keeps(const mft_model_s* m, int li) { return li >= 0 && li < 64 && ((m->retain >> li) & 1); }

// Device buffer of the retained (layer, name) activation or gradient,
// rows × cols floats (grown on demand; debug mode only, never captured).
float* kept_buf(mft_model_s* m, bool grad, int layer, const char* name, int64_t rows, int64_t cols) {
  auto& k = (grad ? m->kept_grad : m->kept_act)[{layer, name}];
  const size_t need = (size_t)(rows * cols) * sizeof(float);
  if (k.cap < need) {
    if (k.p) MFT_HIP(hipFree(k.p));
    k.p = nullptr;
    k.cap = 0;
    if (hipMalloc(&k.p, need) != hipSuccess) throw Error(MFT_ENOMEM, "retained debug tensor");
    k.cap = need;
  }
  k.rows = rows;
  k.cols = cols;
  return k.p;
}

void keep_copy(mft_model_s* m, bool grad, int layer, const char* name, const float* src, int64_t rows, int64_t cols,
               int64_t ld) {
  float* d = kept_buf(m, grad, layer, name, rows, cols);
  MFT_HIP(hipMemcpy2DAsync(d, cols * sizeof(float), src, ld * sizeof(float), cols * sizeof(float), rows,
                           hipMemcpyDeviceToDevice, m->stream));
}

// q and k rows before RoPE (after Gemma3's q/k norms) of layer li, from the
// rows after it: RoPE⁻¹ of a copy (activations: of a.q/a.k; gradients: of dq/dk).
void keep_pre_rope(mft_model_s* m, bool grad, int li, const float* q, int64_t q_ld, const float* k, int64_t k_ld,
                   int64_t M, int S) {
  const mft_model_cfg& c = m->c;
  const int64_t qw = (int64_t)c.n_head * c.head_dim, kw = (int64_t)c.n_kv_head * c.head_dim;
  keep_copy(m, grad, li, "q_normed", q, M, qw, q_ld);
  keep_copy(m, grad, li, "k_normed", k, M, kw, k_ld);
  HeadRows hq, hk;
  hq.H = c.n_head;
  hk.H = c.n_kv_head;
  hq.in = hq.out = kept_buf(m, grad, li, "q_normed", M, qw);
  hk.in = hk.out = kept_buf(m, grad, li, "k_normed", M, kw);
  hq.in_ld = hq.out_ld = qw;
  hk.in_ld = hk.out_ld = kw;
  qk_rope_bwd(m->stream, hq, hk, M, S, c.head_dim, m->rope_tab[layer_local(c, li) ? 1 : 0], (int)m->max_tokens);
}

// Scores and probabilities of layer li (forward), or their gradients from
// dO = datt (backward), as dense [B, Hq, S, S] tensors.
void keep_attention(mft_model_s* m, const Acts& a, int li, const float* mask, int nseq, int S, const float* datt) {
  const mft_model_cfg& c = m->c;
  DebugAttn g;
  g.q = a.q; g.k = a.k; g.v = a.v; g.o = a.att; g.lse = a.lse; g.kpad = mask;
  g.q_rs = a.qs; g.k_rs = a.ks; g.v_rs = a.vs; g.o_rs = (int64_t)c.n_head * c.head_dim;
  g.B = nseq; g.Hq = c.n_head; g.Hkv = c.n_kv_head; g.S = S; g.hd = c.head_dim;
  g.causal = 1;
  g.window = layer_local(c, li) ? c.sliding_window : 0;
  g.scale = attn_scale(c);
  const int64_t rows = (int64_t)nseq * c.n_head * S;
  if (datt) {
    g.dout = datt;
    g.do_rs = (int64_t)c.n_head * c.head_dim;
    g.dprobs = kept_buf(m, true, li, "probs", rows, S);
    g.dscores = kept_buf(m, true, li, "scores", rows, S);
  } else {
    g.scores = kept_buf(m, false, li, "scores", rows, S);
    g.probs = kept_buf(m, false, li, "probs", rows, S);
  }
  debug_attn(m->stream, g);
}

// Whether C = x·op(W) runs on the fp16 matrix cores (lin_gemm).
// C = x·op(W) (+ epilogue) for a linear's frozen W.  fp16-stored W runs on
// the fp16 matrix cores with x's row scales from inv_s (written by the
// batched rank-r launch that read x) or, when null, from a row_scales launch
// timed with the linear class.  Tuning hook: MFT_GEMM_F16=0 keeps fp16 W on
// the fp32 kernels (widened in the tile load).
bool f16_path(const mft_model_s* m, const Param& W, const float* x, int64_t ldx, const void* wptr, int64_t ldw,
              bool b_nk, int N, int K, int r) {
  static const int f16_mode = [] {
    const char* e = getenv("MFT_GEMM_F16");
    return e ? atoi(e) : 1;
  }();
  return W.f16 && f16_mode && m->rscale && gemm_h_ok(N, K, b_nk, r) && ldx % 4 == 0 && ldx >= K &&
         ((uintptr_t)x & 15) == 0 && ldw % 8 == 0 && ((uintptr_t)wptr & 15) == 0;
}

void lin_gemm(mft_model_s* m, const float* x, int64_t ldx, const Param& W, const void* wptr, int64_t ldw, bool b_nk,
              float* C, int64_t ldc, int64_t M, int N, int K, const GemmEpilogue& ep, Scratch ws,
              const KernelEvents* ev, const float* inv_s, int cls = CLS_LINEAR) {
  if (f16_path(m, W, x, ldx, wptr, ldw, b_nk, N, K, ep.r)) {
    if (!inv_s) {
      float* slot = m->rscale + (int64_t)T_MAX * m->max_tokens;
      Timed ts(m, cls, 0.0);
      ts.begin();
      row_scales(m->stream, x, ldx, (int)M, K, slot);
      ts.end();
      inv_s = slot;
    }
    gemm_h(m->stream, x, ldx, inv_s, static_cast<const uint16_t*>(wptr), ldw, b_nk, C, ldc, (int)M, N, K, ep, ws, ev);
    return;
  }
  gemm(m->stream, x, ldx, wptr, ldw, b_nk, W.f16, C, ldc, (int)M, N, K, ep, ws, ev);
}

// y = x·W (+ LoRA) + bias (+ resid); with gelu_out, y keeps the
// pre-activation and gelu_out receives GELU(y) (GPT-2 c_fc).
void lin_fwd(mft_model_s* m, const Linear& l, const float* x, int64_t M, float* y, float* xa,
             const float* resid, float* gelu_out = nullptr, const RowNorm* norm = nullptr) {
  const Param& W = m->P[l.W];
  const WeightUse wu(m, l.W);
  const bool lora = l.A >= 0;
  const int r = lora ? m->c.lora_r : 0;
  GemmEpilogue ep;
  ep.bias = l.b >= 0 ? static_cast<const float*>(m->P[l.b].data) : nullptr;
  ep.resid = resid;
  ep.gelu_out = gelu_out;
  ep.norm = norm;
  if (lora && m->merged) {  // y = x·W_eff (+ bias, residual)
    Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K);
    gemm(m->stream, x, l.K, l.weff, l.weff_ld, false, false, y, l.N, (int)M, l.N, l.K, ep, m->ws, t.events());
    return;
  }
  if (lora && m->panel) {  // y = x·W + s·xa·Bᵀ, xa from the group's batched launch
    run_batch(m, l.xa_batch, M);
    ep.P = xa;
    ep.Q = static_cast<const float*>(m->P[l.B].data);
    ep.r = r;
    ep.qsn = r;
    ep.qsj = 1;
    ep.lscale = lscale(m);
    Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K + 2.0 * M * l.N * r);
    lin_gemm(m, x, l.K, W, wu.ptr, l.N, false, y, l.N, M, l.N, l.K, ep, m->ws, t.events(), l.rs_fwd);
    return;
  }
  if (lora) {
    // training forward with LoRA dropout: the branch reads xd = x∘mask
    const float* xin = x;
    if (m->fwd_dropout) {
      dropout_apply(m->stream, x, l.K, M, l.K, drop_stream(m), l.lid, l.xd);
      xin = l.xd;
    }
    Timed tr(m, CLS_RANK, 4.0 * M * (l.K + r));  // bytes: read x, write xa
    tr.begin();
    rank_proj(m->stream, xin, l.K, static_cast<const float*>(m->P[l.A].data), 1, l.K, (int)M, l.K, r, xa);
    tr.end();
    ep.P = xa;
    ep.Q = static_cast<const float*>(m->P[l.B].data);
    ep.r = r;
    ep.qsn = r;
    ep.qsj = 1;
    ep.lscale = lscale(m);
  }
  Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K + 2.0 * M * l.N * r);
  lin_gemm(m, x, l.K, W, wu.ptr, l.N, false, y, l.N, M, l.N, l.K, ep, m->ws, t.events(), nullptr);
}

// Rank-r panel path: the projections ts[0..nt) of one shared input x (q|k|v,
// gate|up) as one column-segmented fp16 launch, after the group's batched
// x·Aᵀ projections (which also write x's row scales).  False, with nothing
// launched, when a member does not qualify (no LoRA, a bias, a streamed
// weight, a shape the fp16 kernel or a 64-wide tile does not take).
bool lin_fwd_group(mft_model_s* m, const Layer& L, const int* ts, int nt, const float* x, int64_t M,
                   float* const* ys, int64_t ldy, const Acts& a) {
  if (!m->panel || nt < 2 || nt > 3) return false;
  const Linear& l0 = L.lin[ts[0]];
  const int K = l0.K, r = m->c.lora_r;
  GemmHSegmentArg seg[3];
  double work = 0.0;
  for (int i = 0; i < nt; ++i) {
    const Linear& l = L.lin[ts[i]];
    const Param& W = m->P[l.W];
    if (l.A < 0 || l.b >= 0 || l.K != K || l.N % 64 != 0 || W.shard >= 0 || l.rs_fwd != l0.rs_fwd || !l.rs_fwd ||
        !f16_path(m, W, x, K, W.data, l.N, false, l.N, K, r))
      return false;
    seg[i] = GemmHSegmentArg{static_cast<const uint16_t*>(W.data), l.N, l.N, ys[i], ldy > 0 ? ldy : l.N,
                             a.xa[ts[i]], static_cast<const float*>(m->P[l.B].data)};
    work += 2.0 * M * l.N * K + 2.0 * M * l.N * r;
  }
  run_batch(m, l0.xa_batch, M);
  GemmEpilogue ep;
  ep.r = r;
  ep.qsn = r;
  ep.qsj = 1;
  ep.lscale = lscale(m);
  Timed t(m, CLS_LINEAR, work);
  MFT_CHECK_ARG(gemm_h_segments(m->stream, x, K, l0.rs_fwd, false, seg, nt, (int)M, K, ep, t.events()),
                "segmented projection launch");
  return true;
}

// Rank-r panel path: dX of the projections ts[0..nt) of one input, whose dY
// are column blocks of dy (pitch ldy), as one K-segmented fp16 launch after
// the group's batched U = dY·B projections (which write each dY block's row
// scales); dx null: the projections only (their dA still needs U).
void lin_bwd_group(mft_model_s* m, const Layer& L, const int* ts, int nt, const float* dy, int64_t ldy, int64_t M,
                   float* dx, const GemmEpilogue& ep_in) {
  const Linear& l0 = L.lin[ts[0]];
  run_batch(m, l0.u_batch, M);
  if (!dx) return;
  const int r = m->c.lora_r;
  GemmHKSegmentArg seg[3];
  double work = 0.0;
  for (int i = 0; i < nt; ++i) {
    const Linear& l = L.lin[ts[i]];
    seg[i] = GemmHKSegmentArg{static_cast<const uint16_t*>(m->P[l.W].data), l.N, l.N, l.rs_bwd, l.u,
                              static_cast<const float*>(m->P[l.A].data)};
    work += 2.0 * M * l.N * l.K + 2.0 * M * l.K * r;
  }
  GemmEpilogue ep = ep_in;
  ep.r = r;
  ep.qsn = 1;
  ep.qsj = l0.K;
  ep.lscale = lscale(m);
  Timed t(m, CLS_LINEAR, work);
  gemm_h_ksegments(m->stream, dy, ldy, seg, nt, dx, l0.K, (int)M, l0.K, ep, m->ws, t.events());
}

// dx = dy·Wᵀ (+ LoRA) (+ beta·dx); with gelu_grad_of = the pre-activation
// that fed a GELU into this layer, dx is the gradient of that pre-activation
// instead; norm: the backward of the norm that produced x, applied to dx.
void lin_bwd(mft_model_s* m, const Linear& l, const float* dy, const float* x, const float* xa,
             int64_t M, float* dx, const float* gelu_grad_of = nullptr, const RowNorm* norm = nullptr,
             float beta = 0.f) {
  const Param& W = m->P[l.W];
  const WeightUse wu(m, l.W);
  const bool lora = l.A >= 0;
  if (lora && m->merged) {  // dX = dY·W_effᵀ; dA/dB come from the batched launches
    if (dx) {
      GemmEpilogue ep;
      ep.gelu_grad_of = gelu_grad_of;
      ep.norm = norm;
      ep.beta = beta;
      Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K);
      gemm(m->stream, dy, l.N, l.weff, l.weff_ld, true, false, dx, l.K, (int)M, l.K, l.N, ep, m->ws, t.events());
    }
    return;
  }
  const int r = lora ? m->c.lora_r : 0;
  if (lora && m->panel) {  // dX = dY·Wᵀ + s·U·A, U from the group's batched launch; dA, dB at the end
    run_batch(m, l.u_batch, M);
    if (dx) {
      GemmEpilogue ep;
      ep.gelu_grad_of = gelu_grad_of;
      ep.norm = norm;
      ep.beta = beta;
      ep.P = l.u;
      ep.Q = static_cast<const float*>(m->P[l.A].data);
      ep.r = r;
      ep.qsn = 1;
      ep.qsj = l.K;
      ep.lscale = lscale(m);
      Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K + 2.0 * M * l.K * r);
      lin_gemm(m, dy, l.N, W, wu.ptr, l.N, true, dx, l.K, M, l.K, l.N, ep, m->ws, t.events(), l.rs_bwd);
    }
    return;
  }
  float* U = m->ws.ptr;
  Scratch rest = m->ws.offset((size_t)(M * (r > 0 ? r : 1)));
  if (lora) {
    Timed tr(m, CLS_RANK, 4.0 * M * (l.N + r));  // bytes: read dy, write U
    tr.begin();
    rank_proj(m->stream, dy, l.N, static_cast<const float*>(m->P[l.B].data), r, 1, (int)M, l.N, r, U);
    tr.end();
  }
  if (lora && m->fwd_dropout) {
    // dX = dY·Wᵀ + s·(U·A)∘mask: the masked rank-r term is added after the
    // GEMM, then the fused epilogue steps the plain path takes (GELU', the
    // norm backward) run on the complete gradient; dA reads xd = x∘mask.
    if (dx) {
      GemmEpilogue ep;
      ep.beta = beta;
      Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K);
      gemm(m->stream, dy, l.N, wu.ptr, l.N, true, W.f16, dx, l.K, (int)M, l.K, l.N, ep, rest, t.events());
      dropout_dx(m->stream, dx, M, l.K, U, static_cast<const float*>(m->P[l.A].data), r, lscale(m),
                 drop_stream(m), l.lid);
      if (gelu_grad_of) gelu_grad_scale(m->stream, dx, gelu_grad_of, M * l.K);
      if (norm && norm->kind != NORM_NONE) row_norm(m->stream, dx, M, l.K, *norm);
    }
    Timed tr(m, CLS_RANK, 4.0 * M * (l.K + l.N + 2 * r));
    tr.begin();
    rank_outer_pair(m->stream, (int)M, r, lscale(m), true, U, l.xd, l.K, l.K, m->P[l.A].grad, l.K, 1, xa, dy,
                    l.N, l.N, m->P[l.B].grad, 1, r);
    tr.end();
    return;
  }
  if (dx) {
    GemmEpilogue ep;
    ep.gelu_grad_of = gelu_grad_of;
    ep.norm = norm;
    ep.beta = beta;
    if (lora) {
      ep.P = U;
      ep.Q = static_cast<const float*>(m->P[l.A].data);
      ep.r = r;
      ep.qsn = 1;
      ep.qsj = l.K;
      ep.lscale = lscale(m);
    }
    Timed t(m, CLS_LINEAR, 2.0 * M * l.N * l.K + 2.0 * M * l.K * r);
    gemm(m->stream, dy, l.N, wu.ptr, l.N, true, W.f16, dx, l.K, (int)M, l.K, l.N, ep, rest, t.events());
  }
  if (lora) {
    Timed tr(m, CLS_RANK, 4.0 * M * (l.K + l.N + 2 * r));  // bytes: read x, dy, U, xa
    tr.begin();
    // dA += s·Uᵀ·x and dB += s·dyᵀ·xa in one launch
    rank_outer_pair(m->stream, (int)M, r, lscale(m), true, U, x, l.K, l.K, m->P[l.A].grad, l.K, 1, xa, dy,
                    l.N, l.N, m->P[l.B].grad, 1, r);
    tr.end();
  }
}

// One table-driven launch of batched rank-r work (see build_lora_tables).
// A batch of at most three projections (the rank-r panel path's per-layer
// groups) runs as one by-value launch, a workgroup per row and job; larger
// batches and outer products read their job table.  Tuning hook:
// MFT_PROJ_JOBS=0 keeps every batch on the table kernel.
void run_batch(mft_model_s* m, int idx, int64_t M) {
  if (idx < 0) return;
  static const bool by_value = [] {
    const char* e = getenv("MFT_PROJ_JOBS");
    return !e || atoi(e) != 0;
  }();
  const mft_model_s::Batch& b = m->batches[idx];
  Timed t(m, CLS_RANK, b.work_per_row * M);
  t.begin();
  if (by_value && b.pj.n > 0) rank_proj_jobs(m->stream, b.pj, (int)M, m->c.lora_r);
  else rank_batch(m->stream, b.jobs, b.njobs, b.nproj, b.outer_blocks, (int)M, m->c.lora_r);
  t.end();
}

// W_eff = W + s·Aᵀ·Bᵀ for every LoRA linear (one launch).
void merge_lora(mft_model_s* m) {
  if (!m->merged) return;
  double work = 0.0;  // HBM bytes: read W (fp32 or fp16), write W_eff
  for (auto& L : m->L)
    for (auto& l : L.lin)
      if (l.weff) work += (double)l.K * l.N * ((m->P[l.W].f16 ? 2 : 4) + 4);
  Timed t(m, CLS_RANK, work);
  t.begin();
  lora_merge(m->stream, m->d_merge, m->n_merge, m->merge_tiles_total, m->c.lora_r, lscale(m));
  t.end();
}

template <typename T>
const T* pd(const mft_model_s* m, int i) {
  return i < 0 ? nullptr : static_cast<const T*>(m->P[i].data);
}

void attention_fwd(mft_model_s* m, Acts& a, int li, const float* mask, int nseq, int S) {
  const mft_model_cfg& c = m->c;
  AttnArgs g{a.q, a.k, a.v, a.qs, a.ks, a.vs, nseq, c.n_head, c.n_kv_head, S, c.head_dim,
             attn_scale(c), 1, layer_local(c, li) ? c.sliding_window : 0, mask};
  const double work = 2.0 * 2.0 * nseq * c.n_head * (double)S * S * c.head_dim * 0.5;
  Timed t(m, CLS_ATTN, work);
  t.begin();
  attn_fwd(m->stream, g, a.att, (int64_t)c.n_head * c.head_dim, a.lse, m->ws);
  t.end();
}

// n_fwd: the micro-batch forwards this launch stands for (nseq/n_fwd
// sequences each); with LoRA dropout each draws its own masks.
void forward(mft_model_s* m, const int32_t* ids, const float* mask, int nseq, int S, bool train, int n_fwd) {
  const mft_model_cfg& c = m->c;
  for (auto& kv : m->kept_grad) kv.second.rows = 0;  // retained gradients belong to one step
  m->dl_rs_fresh = false;                              // new logits: no dlogits scales yet
  m->alt_ready = false;
  m->fwd_dropout = train && c.lora_dropout > 0.f && c.lora_r > 0 && c.lora_mask != 0;
  m->drop_n_fwd = n_fwd;
  m->drop_rows = (int64_t)(nseq / n_fwd) * S;
  if (m->fwd_dropout) dropout_step(m->stream, m->d_drop_step, n_fwd);  // these forwards' mask streams
  const int64_t M = (int64_t)nseq * S;
  const int d = c.d, H = c.n_head, Hk = c.n_kv_head, hd = c.head_dim;
  const bool gpt2 = c.arch == MFT_ARCH_GPT2, gemma = c.arch == MFT_ARCH_GEMMA3;
  const hipStream_t s = m->stream;
  const Param& E = m->P[m->wte];
  m->last_rows = M;
  shard_begin(m);
  merge_lora(m);  // A, B (or W) may have changed since the last forward
  // Input norm of layer li (li == n_layer: the final norm).  GPT-2 and Qwen2
  // run it inside the GEMM that produced its input (the previous layer's
  // residual-fused down projection); Gemma3's post-norms sit in between.
  auto norm1 = [&](int li) {
    const bool fin = li == c.n_layer;
    RowNorm nm;
    nm.kind = gpt2 ? NORM_LN_FWD : NORM_RMS_FWD;
    nm.w = pd<float>(m, fin ? m->nfw : m->L[li].n1w);
    nm.b = gpt2 ? pd<float>(m, fin ? m->nfb : m->L[li].n1b) : nullptr;
    nm.eps = c.norm_eps;
    nm.unit_offset = gemma ? 1 : 0;
    nm.y = fin ? m->hf : m->A[li].n1;
    nm.mean = gpt2 ? (fin ? m->fmean : m->A[li].mean1) : nullptr;
    nm.rstd = fin ? m->frstd : m->A[li].rstd1;
    return nm;
  };
  // Gemma3's sandwich after a sublayer: y = resid + RMSNorm_w(C) (rstd kept),
  // then the norm `next` of y (pre-FFN norm, next input norm or final norm).
  auto sandwich = [&](int w, const float* resid, float* y, float* rstd, const RowNorm& next) {
    RowNorm nm;
    nm.kind = NORM_RMS_RES_RMS;
    nm.w = pd<float>(m, w);
    nm.eps = c.norm_eps;
    nm.unit_offset = 1;
    nm.resid = resid;
    nm.y = y;
    nm.rstd = rstd;
    nm.w2 = next.w;
    nm.y2 = next.y;
    nm.rstd2 = next.rstd;
    return nm;
  };
  auto norm2 = [&](int li) {  // the pre-MLP norm of layer li
    RowNorm nm;
    Acts& a = m->A[li];
    nm.kind = gpt2 ? NORM_LN_FWD : NORM_RMS_FWD;
    nm.w = pd<float>(m, m->L[li].n2w);
    nm.b = gpt2 ? pd<float>(m, m->L[li].n2b) : nullptr;
    nm.eps = c.norm_eps;
    nm.unit_offset = gemma ? 1 : 0;
    nm.y = a.n2;
    nm.mean = gpt2 ? a.mean2 : nullptr;
    nm.rstd = a.rstd2;
    return nm;
  };
  // The embedding gather and layer 0's input norm run as one launch, which
  // also clears the step's loss and count slots when a step begins.
  bool first_norm = false;
  {
    const WeightUse we(m, m->wte);
    const float* wpe = gpt2 ? pd<float>(m, m->wpe) : nullptr;
    const float scale = gemma ? std::sqrt((float)d) : 1.f;
    void* zero = m->zero_pending ? static_cast<void*>(m->d_loss) : nullptr;
    first_norm = embed_norm(s, ids, M, S, we.ptr, c.vocab, E.f16, wpe, d, scale, m->A[0].x, m->d_err, norm1(0),
                            zero, kStatWords);
    if (!first_norm) {
      if (zero) fill_const(s, static_cast<float*>(zero), 2 * kStatWords, 0.f);
      embed(s, ids, M, S, we.ptr, c.vocab, E.f16, wpe, d, scale, m->A[0].x, m->d_err);
    }
    m->zero_pending = false;
  }
  for (int li = 0; li < c.n_layer; ++li) {
    const Layer& L = m->L[li];
    Acts& a = m->A[li];
    float* hout = li + 1 < c.n_layer ? m->A[li + 1].x : m->h_final;
    if (li == 0 && !first_norm) row_norm(s, a.x, M, d, norm1(li));
    const RowNorm n2 = norm2(li), nx = norm1(li + 1);
    if (gpt2) {
      lin_fwd(m, L.lin[G_ATTN], a.n1, M, a.q, a.xa[G_ATTN], nullptr);
      attention_fwd(m, a, li, mask, nseq, S);
      lin_fwd(m, L.lin[G_PROJ], a.att, M, a.hmid, a.xa[G_PROJ], a.x, nullptr, &n2);  // residual + LN fused
      lin_fwd(m, L.lin[G_FC], a.n2, M, a.gate, a.xa[G_FC], nullptr, a.act);         // GELU fused
      lin_fwd(m, L.lin[G_FC2], a.act, M, hout, a.xa[G_FC2], a.hmid, nullptr, &nx);   // residual + LN fused
      continue;
    }
    if (m->fuse_qkv) {  // q|k|v = n1·W_eff[d, nqkv] (+ the back-to-back biases) in one GEMM
      const int nt = m->nqkv;
      GemmEpilogue ep;
      ep.bias = pd<float>(m, L.lin[T_Q].b);
      Timed t(m, CLS_LINEAR, 2.0 * M * nt * d);
      gemm(s, a.n1, d, L.lin[T_Q].weff, nt, false, false, a.qkv, nt, (int)M, nt, d, ep, m->ws, t.events());
    } else {
      static const int qkv[3] = {T_Q, T_K, T_V};
      float* const ys[3] = {gemma ? a.qraw : a.q, gemma ? a.kraw : a.k, a.v};
      const bool grouped = lin_fwd_group(m, L, qkv, 3, a.n1, M, ys, m->lay_qkv ? m->nqkv : 0, a);
      MFT_CHECK_ARG(grouped || !m->seg_qkv, "segmented q|k|v projection did not qualify");
      if (!grouped) {
        lin_fwd(m, L.lin[T_Q], a.n1, M, ys[0], a.xa[T_Q], nullptr);
        lin_fwd(m, L.lin[T_K], a.n1, M, ys[1], a.xa[T_K], nullptr);
        lin_fwd(m, L.lin[T_V], a.n1, M, ys[2], a.xa[T_V], nullptr);
      }
    }
    {
      // Gemma3's per-head q/k RMSNorms and RoPE (in place for Qwen2), q and
      // k rows in one launch
      const int64_t raw_ld = m->lay_qkv ? m->nqkv : 0;
      HeadRows hq, hk;
      hq.H = (int)H;
      hk.H = (int)Hk;
      if (gemma) {
        hq.in = a.qraw; hq.in_ld = raw_ld ? raw_ld : H * hd; hq.w = pd<float>(m, L.qn); hq.rstd = a.qrs;
        hk.in = a.kraw; hk.in_ld = raw_ld ? raw_ld : Hk * hd; hk.w = pd<float>(m, L.kn); hk.rstd = a.krs;
      } else {
        hq.in = a.q; hq.in_ld = a.qs;
        hk.in = a.k; hk.in_ld = a.ks;
      }
      hq.out = a.q; hq.out_ld = a.qs;
      hk.out = a.k; hk.out_ld = a.ks;
      qk_rope_fwd(s, hq, hk, M, S, hd, c.norm_eps, m->rope_tab[layer_local(c, li) ? 1 : 0], (int)m->max_tokens);
    }
    attention_fwd(m, a, li, mask, nseq, S);
    if (gemma && keeps(m, li)) {  // alignment-dump debug mode
      keep_pre_rope(m, false, li, a.q, a.qs, a.k, a.ks, M, S);
      keep_attention(m, a, li, mask, nseq, S, nullptr);
    }
    if (gemma) {  // post-attention norm, residual add and pre-FFN norm in the o projection's epilogue
      const RowNorm sw = sandwich(L.pan, a.x, a.hmid, a.ors, norm2(li));
      lin_fwd(m, L.lin[T_O], a.att, M, a.o, a.xa[T_O], nullptr, nullptr, &sw);
    } else {
      lin_fwd(m, L.lin[T_O], a.att, M, a.hmid, a.xa[T_O], a.x, nullptr, &n2);  // residual + norm fused
    }
    if (m->fuse_gu) {  // gate|up = n2·W_eff[d, 2·ff] in one GEMM
      const int n2f = 2 * c.d_ff;
      Timed t(m, CLS_LINEAR, 2.0 * M * n2f * d);
      gemm(s, a.n2, d, L.lin[T_GATE].weff, n2f, false, false, a.gu, n2f, (int)M, n2f, d, GemmEpilogue(), m->ws,
           t.events());
      glu_fwd_rows(s, a.gate, a.up, M, c.d_ff, n2f, gemma ? 0 : 1, a.act);
    } else {
      static const int gu[2] = {T_GATE, T_UP};
      float* const ys[2] = {a.gate, a.up};
      const bool grouped = lin_fwd_group(m, L, gu, 2, a.n2, M, ys, m->lay_gu ? 2 * c.d_ff : 0, a);
      MFT_CHECK_ARG(grouped || !m->seg_gu, "segmented gate|up projection did not qualify");
      if (!grouped) {
        lin_fwd(m, L.lin[T_GATE], a.n2, M, a.gate, a.xa[T_GATE], nullptr);
        lin_fwd(m, L.lin[T_UP], a.n2, M, a.up, a.xa[T_UP], nullptr);
      }
      if (m->lay_gu) glu_fwd_rows(s, a.gate, a.up, M, c.d_ff, 2 * c.d_ff, gemma ? 0 : 1, a.act);
      else glu_fwd(s, a.gate, a.up, M * c.d_ff, gemma ? 0 : 1, a.act);
    }
    if (gemma && keeps(m, li))  // GELU(gate) alone (alignment-dump debug mode)
      debug_gelu(s, a.gate, m->lay_gu ? 2 * c.d_ff : c.d_ff, kept_buf(m, false, li, "gate_act", M, c.d_ff), c.d_ff,
                 M, c.d_ff);
    if (gemma) {  // post-FFN norm, residual add and the next input norm in the down projection's epilogue
      const RowNorm sw = sandwich(L.pfn, a.hmid, hout, a.mrs, norm1(li + 1));
      lin_fwd(m, L.lin[T_DOWN], a.act, M, a.mo, a.xa[T_DOWN], nullptr, nullptr, &sw);
    } else {
      lin_fwd(m, L.lin[T_DOWN], a.act, M, hout, a.xa[T_DOWN], a.hmid, nullptr, &nx);  // residual + norm fused
    }
  }
  // LM head: logits = hf · Eᵀ, E [V, d] is the [N, K] operand.
  const WeightUse wh(m, m->wte);
  Timed t(m, CLS_LMHEAD, 2.0 * M * c.vocab * d);
  GemmEpilogue head;
  head.site = 1;
  // fp16 E: the fp16 matrix cores (any tile plan there emits the row statistics)
  const bool h16 = f16_path(m, E, m->hf, d, wh.ptr, d, true, (int)c.vocab, d, 0);
  m->stats_fresh = m->row_stats && (h16 || gemm_wide_plan((int)M, (int)c.vocab));
  if (m->stats_fresh) {
    head.stats = m->row_stats;
    head.stats_ld = m->stats_ld;
  }
  lin_gemm(m, m->hf, d, E, wh.ptr, d, true, m->logits, m->ldv, M, (int)c.vocab, d, head, m->ws, t.events(), nullptr,
           CLS_LMHEAD);
}

void cross_entropy(mft_model_s* m, const int32_t* labels, int n_micro, int seqs, int S,
                   float upstream, bool backward) {
  const mft_model_cfg& c = m->c;
  if (m->n_micro_pending + n_micro > 64) throw Error(MFT_EINVAL, "more than 64 micro-batches pending");
  for (int i = 0; i < n_micro; ++i) {
    const int64_t row0 = (int64_t)i * seqs * S;
    float* lg = m->logits + row0 * m->ldv;
    Timed t(m, CLS_CE, 8.0 * (double)seqs * S * c.vocab);
    t.begin();
    ce_fwd_bwd(m->stream, lg, labels + row0, seqs, S, c.vocab, m->ldv, -100, upstream, 0,
               m->d_loss + m->n_micro_pending, m->d_cnt + m->n_micro_pending, backward ? lg : nullptr,
               m->row_nll + row0, m->d_tmpcnt, m->d_err + 1,
               m->stats_fresh ? m->row_stats + row0 * m->stats_ld : nullptr, m->stats_ld,
               backward && m->dl_rscale ? m->dl_rscale + row0 : nullptr);
    t.end();
    if (backward && m->dl_rscale) m->dl_rs_fresh = true;
    m->n_micro_pending++;
  }
}

void backward(mft_model_s* m, const float* mask, int nseq, int S) {
  const mft_model_cfg& c = m->c;
  const int64_t M = (int64_t)nseq * S;
  const int d = c.d, H = c.n_head, Hk = c.n_kv_head, hd = c.head_dim;
  const bool gpt2 = c.arch == MFT_ARCH_GPT2, gemma = c.arch == MFT_ARCH_GEMMA3;
  const hipStream_t s = m->stream;
  const Param& E = m->P[m->wte];
  // Where dY of linear t of layer li goes: its own kept buffer for a LoRA
  // linear on the merged path, else the shared temporary `fb`.
  auto dyb = [&](int li, int t, float* fb) -> float* {
    return (m->merged || m->panel) && m->L[li].lin[t].A >= 0 ? m->A[li].DY[t] : fb;
  };
  // Residual-stream gradient entering layer li's MLP block (GPT-2 / Qwen2: the
  // dY of c_fc2 / down_proj) and its attention block (dY of c_proj / o_proj).
  // Norm backward passes write them out of place: dres_out = dres_in + ∂norm.
  auto res_in = [&](int li) { return gemma ? m->dh : dyb(li, gpt2 ? G_FC2 : T_DOWN, m->dh); };
  auto res_mid = [&](int li) { return gemma ? m->dh2 : dyb(li, gpt2 ? G_PROJ : T_O, m->dh2); };
  run_batch(m, m->xa_batch, M);  // xa = x·Aᵀ of every LoRA linear
  const int top = c.n_layer - 1;
  // Backward of a norm (ln: LayerNorm, else RMSNorm) over input rows x, run
  // in the epilogue of the GEMM producing its output gradient: y = resid + ∂x.
  auto norm_bwd = [&](const float* x, int w, float* mean, float* rstd, float* y, const float* resid) {
    RowNorm nm;
    nm.kind = gpt2 ? NORM_LN_BWD : NORM_RMS_BWD;
    nm.x = x;
    nm.w = pd<float>(m, w);
    nm.mean = mean;
    nm.rstd = rstd;
    nm.unit_offset = gemma ? 1 : 0;
    nm.y = y;
    nm.resid = resid;
    nm.skip_c = true;
    return nm;
  };
  // Gemma3: extend a norm backward with that of the post-norm whose output
  // fed it through the residual stream: layer li's post-attention norm
  // (attn) or post-FFN norm; its input gradient is the o or down projection's dY.
  auto post_bwd = [&](RowNorm nm, int li, bool attn) {
    const Acts& pa = m->A[li];
    nm.kind = NORM_RMS_BWD_POST;
    nm.x2 = attn ? pa.o : pa.mo;
    nm.w2 = pd<float>(m, attn ? m->L[li].pan : m->L[li].pfn);
    nm.rstd2 = attn ? pa.ors : pa.mrs;
    nm.y2 = dyb(li, attn ? T_O : T_DOWN, m->dtmp);
    return nm;
  };
  {
    // dhf = dlogits · E, E [V, d] is the [K, N] operand; the final norm's
    // backward runs in its epilogue.
    Timed t(m, CLS_LMHEAD, 2.0 * M * c.vocab * d);
    RowNorm nf = norm_bwd(m->h_final, m->nfw, gpt2 ? m->fmean : nullptr, m->frstd, res_in(top), nullptr);
    if (gemma) nf = post_bwd(nf, top, false);  // + the top layer's post-FFN norm backward
    GemmEpilogue head;
    head.site = 1;
    head.norm = &nf;
    const WeightUse wh(m, m->wte);
    lin_gemm(m, m->logits, m->ldv, E, wh.ptr, d, false, m->dn, d, M, d, (int)c.vocab, head, m->ws, t.events(),
             m->dl_rs_fresh ? m->dl_rscale : nullptr, CLS_LMHEAD);
    m->dl_rs_fresh = false;
  }
  const int64_t nf = M * c.d_ff;
  for (int li = top; li >= 0; --li) {
    const Layer& L = m->L[li];
    Acts& a = m->A[li];
    float* rin = res_in(li);
    float* rmid = res_mid(li);
    // alignment-dump debug mode (Gemma3): this layer's activation gradients
    // are kept, including its input's (formed at layer 0 too), and the fused
    // norm backwards also store the GEMM output they consume (d(norm output))
    const bool kp = gemma && keeps(m, li);
    const int64_t qw = (int64_t)H * hd, kw = (int64_t)Hk * hd, ffw = c.d_ff;
    const bool need_dx = li > 0 || kp;
    RowNorm nb2 = norm_bwd(a.hmid, L.n2w, gpt2 ? a.mean2 : nullptr, a.rstd2, rmid, rin);
    float* rnext = need_dx ? res_in(li - 1) : nullptr;
    RowNorm nb1 = norm_bwd(a.x, L.n1w, gpt2 ? a.mean1 : nullptr, a.rstd1, rnext, rmid);
    if (gemma) {
      nb2 = post_bwd(nb2, li, true);                            // + this layer's post-attention norm backward
      if (li > 0) nb1 = post_bwd(nb1, li - 1, false);           // + the next lower layer's post-FFN norm backward
    }
    if (kp) {
      nb1.skip_c = nb2.skip_c = false;
      keep_copy(m, true, li, "out", rin, M, d, d);
      keep_copy(m, true, li, "down_proj", dyb(li, T_DOWN, m->dtmp), M, d, d);
    }
    // ---- MLP block ----
    if (gpt2) {
      float* dgate = dyb(li, G_FC, m->dgate);
      lin_bwd(m, L.lin[G_FC2], rin, a.act, a.xa[G_FC2], M, dgate, a.gate);  // GELU' fused
      lin_bwd(m, L.lin[G_FC], dgate, a.n2, a.xa[G_FC], M, m->dn, nullptr, &nb2);  // LN backward fused
    } else {
      // Gemma3: the post-FFN norm's backward ran with the norm backward that
      // produced rin (the layer above's, or the LM head's final norm)
      const float* dmo = gemma ? dyb(li, T_DOWN, m->dtmp) : rin;
      lin_bwd(m, L.lin[T_DOWN], dmo, a.act, a.xa[T_DOWN], M, m->dact);
      if (kp) {
        keep_copy(m, true, li, "act", m->dact, M, ffw, ffw);
        debug_mul(s, m->dact, ffw, a.up, m->lay_gu ? 2 * ffw : ffw, kept_buf(m, true, li, "gate_act", M, ffw), ffw,
                  M, ffw);  // d(GELU(gate)) = d(act)∘up
      }
      if (m->lay_gu) {
        // dgate|dup in the fused [M, 2·ff] gradient, then one GEMM gives
        // dn = dgu·W_eff[d, 2·ff]ᵀ (panel path: over the two W as K segments)
        // with the pre-FFN norm's backward fused
        const int n2f = 2 * c.d_ff;
        glu_bwd_rows(s, m->dact, a.gate, a.up, M, c.d_ff, n2f, gemma ? 0 : 1, a.DY[T_GATE], a.DY[T_UP]);
        if (kp) {
          keep_copy(m, true, li, "gate", a.DY[T_GATE], M, ffw, n2f);
          keep_copy(m, true, li, "up", a.DY[T_UP], M, ffw, n2f);
        }
        GemmEpilogue ep;
        ep.norm = &nb2;
        if (m->fuse_gu) {
          Timed t(m, CLS_LINEAR, 2.0 * M * n2f * d);
          gemm(s, a.dygu, n2f, L.lin[T_GATE].weff, n2f, true, false, m->dn, d, (int)M, d, n2f, ep, m->ws,
               t.events());
        } else {
          static const int gu[2] = {T_GATE, T_UP};
          lin_bwd_group(m, L, gu, 2, a.dygu, n2f, M, m->dn, ep);
        }
      } else {
        float* dgate = dyb(li, T_GATE, m->dgate);
        float* dup = dyb(li, T_UP, m->dup);
        glu_bwd(s, m->dact, a.gate, a.up, nf, gemma ? 0 : 1, dgate, dup);
        if (kp) {
          keep_copy(m, true, li, "gate", dgate, M, ffw, ffw);
          keep_copy(m, true, li, "up", dup, M, ffw, ffw);
        }
        lin_bwd(m, L.lin[T_GATE], dgate, a.n2, a.xa[T_GATE], M, m->dn);
        lin_bwd(m, L.lin[T_UP], dup, a.n2, a.xa[T_UP], M, m->dn, nullptr, &nb2, 1.f);  // dn += ...; norm fused
      }
    }
    if (kp) {
      keep_copy(m, true, li, "norm2", m->dn, M, d, d);
      keep_copy(m, true, li, "mid", rmid, M, d, d);
    }
    // ---- attention block ----
    // Gemma3: the post-attention norm's backward ran with the pre-FFN norm's
    const float* dox = gemma ? dyb(li, T_O, m->dtmp) : rmid;
    if (kp) keep_copy(m, true, li, "o_proj", dox, M, d, d);
    lin_bwd(m, gpt2 ? L.lin[G_PROJ] : L.lin[T_O], dox, a.att, a.xa[gpt2 ? G_PROJ : T_O], M, m->datt);
    if (kp) {
      keep_copy(m, true, li, "attn", m->datt, M, qw, qw);
      keep_attention(m, a, li, mask, nseq, S, m->datt);
    }
    AttnArgs g{a.q, a.k, a.v, a.qs, a.ks, a.vs, nseq, H, Hk, S, hd, attn_scale(c), 1,
               layer_local(c, li) ? c.sliding_window : 0, mask};
    // algorithmic: dV, dP, dQ, dK (the recomputed scores are not counted), causal half
    const double awork = 2.0 * 4.0 * nseq * H * (double)S * S * hd * 0.5;
    if (gpt2) {
      float* dqkv = dyb(li, G_ATTN, m->dqkv);
      {
        Timed t(m, CLS_ATTN, awork);
        t.begin();
        attn_bwd(s, g, a.att, (int64_t)H * hd, m->datt, (int64_t)H * hd, a.lse, dqkv, 3 * d, dqkv + d, 3 * d,
                 dqkv + 2 * d, 3 * d, m->ws);
        t.end();
      }
      lin_bwd(m, L.lin[G_ATTN], dqkv, a.n1, a.xa[G_ATTN], M, need_dx ? m->dn : nullptr, nullptr,
              need_dx ? &nb1 : nullptr);  // LN backward fused
      continue;
    }
    if (m->lay_qkv) {
      // dq|dk|dv land in the fused [M, nqkv] gradient (Gemma3: dq, dk first
      // through RoPE's inverse and the q/k norms' backward), then one GEMM
      // gives dn = dqkv·W_eff[d, nqkv]ᵀ (panel path: over the three W as K
      // segments) with the input norm's backward fused.
      const int64_t nt = m->nqkv;
      float* dq = gemma ? m->dq : a.DY[T_Q];
      float* dk = gemma ? m->dk : a.DY[T_K];
      const int64_t qld = gemma ? (int64_t)H * hd : nt, kld = gemma ? (int64_t)Hk * hd : nt;
      {
        Timed t(m, CLS_ATTN, awork);
        t.begin();
        attn_bwd(s, g, a.att, (int64_t)H * hd, m->datt, (int64_t)H * hd, a.lse, dq, qld, dk, kld, a.DY[T_V], nt,
                 m->ws);
        t.end();
      }
      if (kp) {
        keep_copy(m, true, li, "q", dq, M, qw, qld);
        keep_copy(m, true, li, "k", dk, M, kw, kld);
        keep_copy(m, true, li, "v", a.DY[T_V], M, kw, nt);
        keep_pre_rope(m, true, li, dq, qld, dk, kld, M, S);
      }
      {
        // RoPE's inverse (in place for Qwen2), then Gemma3's q/k norm
        // backward into the fused gradient; q and k rows in one launch
        HeadRows hq, hk;
        hq.H = (int)H;
        hk.H = (int)Hk;
        hq.in = dq; hq.in_ld = qld;
        hk.in = dk; hk.in_ld = kld;
        if (gemma) {
          hq.out = a.DY[T_Q]; hq.out_ld = nt; hq.w = pd<float>(m, L.qn); hq.rstd = a.qrs; hq.x = a.qraw; hq.x_ld = nt;
          hk.out = a.DY[T_K]; hk.out_ld = nt; hk.w = pd<float>(m, L.kn); hk.rstd = a.krs; hk.x = a.kraw; hk.x_ld = nt;
        } else {
          hq.out = dq; hq.out_ld = qld;
          hk.out = dk; hk.out_ld = kld;
        }
        qk_rope_bwd(s, hq, hk, M, S, hd, m->rope_tab[layer_local(c, li) ? 1 : 0], (int)m->max_tokens);
      }
      if (kp) {
        keep_copy(m, true, li, "q_proj", a.DY[T_Q], M, qw, nt);
        keep_copy(m, true, li, "k_proj", a.DY[T_K], M, kw, nt);
      }
      if (m->seg_qkv) {
        GemmEpilogue ep;
        ep.norm = &nb1;
        static const int qkv[3] = {T_Q, T_K, T_V};
        lin_bwd_group(m, L, qkv, 3, a.dyqkv, nt, M, need_dx ? m->dn : nullptr, ep);
      } else if (need_dx) {
        GemmEpilogue ep;
        ep.norm = &nb1;
        Timed t(m, CLS_LINEAR, 2.0 * M * nt * d);
        gemm(s, a.dyqkv, nt, L.lin[T_Q].weff, nt, true, false, m->dn, d, (int)M, d, (int)nt, ep, m->ws,
             t.events());
      }
      if (kp) {
        keep_copy(m, true, li, "norm1", m->dn, M, d, d);
        keep_copy(m, true, li, "x", rnext, M, d, d);
        if (li == 0) keep_copy(m, true, -1, "embed", rnext, M, d, d);
      }
      continue;
    }
    // q/k dY: after RoPE's inverse (Qwen2) or after the q/k norms' backward (Gemma3)
    float* dq = gemma ? m->dq : dyb(li, T_Q, m->dq);
    float* dk = gemma ? m->dk : dyb(li, T_K, m->dk);
    float* dv = dyb(li, T_V, m->dv);
    {
      Timed t(m, CLS_ATTN, awork);
      t.begin();
      attn_bwd(s, g, a.att, (int64_t)H * hd, m->datt, (int64_t)H * hd, a.lse, dq, (int64_t)H * hd, dk,
               (int64_t)Hk * hd, dv, (int64_t)Hk * hd, m->ws);
      t.end();
    }
    if (kp) {
      keep_copy(m, true, li, "q", dq, M, qw, qw);
      keep_copy(m, true, li, "k", dk, M, kw, kw);
      keep_copy(m, true, li, "v", dv, M, kw, kw);
      keep_pre_rope(m, true, li, dq, qw, dk, kw, M, S);
    }
    const float* dqx = dq;
    const float* dkx = dk;
    {
      // RoPE's inverse (in place for Qwen2), then Gemma3's q/k norm
      // backward; q and k rows in one launch
      HeadRows hq, hk;
      hq.H = (int)H;
      hk.H = (int)Hk;
      hq.in = dq; hq.in_ld = (int64_t)H * hd;
      hk.in = dk; hk.in_ld = (int64_t)Hk * hd;
      hq.out = dq; hq.out_ld = hq.in_ld;
      hk.out = dk; hk.out_ld = hk.in_ld;
      if (gemma) {
        float* tq = dyb(li, T_Q, m->dtq);
        float* tk = dyb(li, T_K, m->dtk);
        hq.out = tq; hq.w = pd<float>(m, L.qn); hq.rstd = a.qrs; hq.x = a.qraw; hq.x_ld = hq.in_ld;
        hk.out = tk; hk.w = pd<float>(m, L.kn); hk.rstd = a.krs; hk.x = a.kraw; hk.x_ld = hk.in_ld;
        dqx = tq;
        dkx = tk;
      }
      qk_rope_bwd(s, hq, hk, M, S, hd, m->rope_tab[layer_local(c, li) ? 1 : 0], (int)m->max_tokens);
    }
    // dn = dq·Wqᵀ + dk·Wkᵀ + dv·Wvᵀ accumulated in the GEMM epilogues, the
    // input norm's backward fused into the last one.
    if (kp) {
      keep_copy(m, true, li, "q_proj", dqx, M, qw, qw);
      keep_copy(m, true, li, "k_proj", dkx, M, kw, kw);
    }
    float* dn = need_dx ? m->dn : nullptr;
    lin_bwd(m, L.lin[T_Q], dqx, a.n1, a.xa[T_Q], M, dn);
    lin_bwd(m, L.lin[T_K], dkx, a.n1, a.xa[T_K], M, dn, nullptr, nullptr, 1.f);
    lin_bwd(m, L.lin[T_V], dv, a.n1, a.xa[T_V], M, dn, nullptr, need_dx ? &nb1 : nullptr, 1.f);
    if (kp) {
      keep_copy(m, true, li, "norm1", m->dn, M, d, d);
      keep_copy(m, true, li, "x", rnext, M, d, d);
      if (li == 0) keep_copy(m, true, -1, "embed", rnext, M, d, d);
    }
  }
  run_batch(m, m->udb_batch, M);  // merged: U = dY·B and dB += s·dYᵀ·xa of every LoRA linear
  run_batch(m, m->db_batch, M);   // panel: dB += s·dYᵀ·xa of every LoRA linear
  run_batch(m, m->da_batch, M);   // dA += s·Uᵀ·x of every LoRA linear
}

// Hyper-parameters reach the device as kernel arguments: of the optimizer's
// first launch in an eager step, of a one-block kernel launched ahead of a
// captured step graph's replay — no host buffer is read by the device.
void upload_hparams(mft_model_s* m, float lr, float b1, float b2, float eps, float wd, float clip) {
  set_hparams(m->stream, m->d_hp, lr, b1, b2, eps, wd, clip, m->d_sumsq, m->d_t);
}

// clip_and_get_grad_norm + Adam::step + zero_grad on the flat LoRA arrays
// in two launches.  With hp (an eager step) the first launch also writes the
// hyper-parameters and advances d_t; without (a captured graph, or after an
// explicit upload_hparams) it reads d_hp / d_t only.
void opt_device(mft_model_s* m, const HpArgs* hp = nullptr) {
  const hipStream_t s = m->stream;
  opt_partials(s, m->lora_g, m->lora_n, m->d_partials, hp, m->d_hp, m->d_t);
  adam_partials(s, m->lora_p, m->lora_g, m->lora_m, m->lora_v, m->lora_n, m->d_hp, m->d_t, m->d_partials, m->d_clip,
                true);
}

// The 64 per-micro loss sums (doubles) and the 64 counts (int64) that follow
// them are cleared by the step's first launch (the forward's embedding).
void zero_stats(mft_model_s* m, int n_micro) {
  (void)n_micro;
  m->zero_pending = true;
}

void drop_graph(mft_model_s* m) {
  if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
  m->graph_exec = nullptr;
  for (auto e : m->gev_pool) (void)hipEventDestroy(e);
  m->gev_pool.clear();
  m->graph_timed.clear();
}

void forward(mft_model_s* m, const int32_t* ids, const float* mask, int nseq, int S, bool train, int n_fwd);
void cross_entropy(mft_model_s* m, const int32_t* labels, int n_micro, int seqs, int S, float upstream,
                   bool backward);
void backward(mft_model_s* m, const float* mask, int nseq, int S);

// Capture one whole training step (stats reset, fwd, CE, bwd, clip, Adam) on
// the model's private stream into an executable graph.
void capture_step(mft_model_s* m, const int32_t* ids, const float* mask, const int32_t* labels, int n_micro,
                  int seqs, int S, float upstream) {
  MFT_HIP(hipStreamSynchronize(m->stream));
  MFT_HIP(hipStreamSynchronize(m->cap_stream));
  drop_graph(m);
  const hipStream_t saved = m->stream;
  m->stream = m->cap_stream;
  m->capturing = true;
  hipGraph_t g = nullptr;
  try {
    MFT_HIP(hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeThreadLocal));
    zero_stats(m, n_micro);
    m->n_micro_pending = 0;
    forward(m, ids, mask, n_micro * seqs, S, m->training, n_micro);
    cross_entropy(m, labels, n_micro, seqs, S, upstream, true);
    backward(m, mask, n_micro * seqs, S);
    opt_device(m);
    MFT_HIP(hipStreamEndCapture(m->cap_stream, &g));
    MFT_HIP(hipGraphInstantiate(&m->graph_exec, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
  } catch (...) {
    hipGraph_t junk = nullptr;
    (void)hipStreamEndCapture(m->cap_stream, &junk);
    if (junk) (void)hipGraphDestroy(junk);
    if (g) (void)hipGraphDestroy(g);
    m->stream = saved;
    m->capturing = false;
    drop_graph(m);
    throw;
  }
  m->stream = saved;
  m->capturing = false;
  m->graph_key.ids = ids;
  m->graph_key.mask = mask;
  m->graph_key.labels = labels;
  m->graph_key.n_micro = n_micro;
  m->graph_key.seqs = seqs;
  m->graph_key.S = S;
  m->graph_key.upstream = upstream;
  m->graph_key.timing = m->timing;
  m->graph_key.training = m->training;
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return MFT_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return MFT_EHIP;
  }
}

void check_cfg(const mft_model_cfg& c) {
  MFT_CHECK_ARG(c.arch >= 0 && c.arch <= 2, "unknown arch");
  MFT_CHECK_ARG(c.n_layer > 0 && c.d > 0 && c.n_head > 0 && c.n_kv_head > 0 && c.head_dim > 0 && c.d_ff > 0 &&
                    c.vocab > 0,
                "bad model dims");
  MFT_CHECK_ARG(c.n_head % c.n_kv_head == 0, "n_head must be a multiple of n_kv_head");
  MFT_CHECK_ARG(c.arch != MFT_ARCH_GPT2 || c.n_head * c.head_dim == c.d, "GPT-2 needs n_head*head_dim == d");
  MFT_CHECK_ARG(c.arch != MFT_ARCH_GPT2 || c.n_head == c.n_kv_head, "GPT-2 has no GQA");
  MFT_CHECK_ARG(c.lora_r == 0 || c.lora_r == 4 || c.lora_r == 8 || c.lora_r == 16 || c.lora_r == 32,
                "lora_r must be 0, 4, 8, 16 or 32");
  MFT_CHECK_ARG(c.d % 4 == 0 && c.d_ff % 4 == 0 && c.head_dim % 4 == 0, "dims must be multiples of 4");
  MFT_CHECK_ARG(c.lora_dropout >= 0.f && c.lora_dropout < 1.f, "lora_dropout must lie in [0, 1)");
}

}  // namespace

extern "C" {

int mft_model_create(mft_model* out, const mft_model_cfg* cfg, int64_t max_tokens, void* stream) {
  return guarded([&] {
    if (!out || !cfg) throw Error(MFT_EINVAL, "null argument");
    check_cfg(*cfg);
    if (max_tokens <= 0) throw Error(MFT_EINVAL, "max_tokens must be positive");
    auto* m = new mft_model_s();
    try {
      m->c = *cfg;
      m->stream = reinterpret_cast<hipStream_t>(stream);
      register_stream(m->stream);
      m->stream_registered = true;
      m->max_tokens = max_tokens;
      build_params(m);
      assign_dropout_streams(m);
      alloc_params(m);
      alloc_acts(m);
      alloc_row_scales(m);
      build_lora_tables(m);
    } catch (...) {
      mft_model_destroy(m);
      throw;
    }
    *out = m;
  });
}

int mft_model_destroy(mft_model m) {
  return guarded([&] {
    if (!m) return;
    (void)hipStreamSynchronize(m->stream);
    if (m->cap_stream) (void)hipStreamSynchronize(m->cap_stream);
    drop_graph(m);
    if (m->stream_registered) unregister_stream(m->stream);
    if (m->cap_stream) {
      unregister_stream(m->cap_stream);
      (void)hipStreamDestroy(m->cap_stream);
    }
    if (m->ev_in) (void)hipEventDestroy(m->ev_in);
    if (m->ev_out) (void)hipEventDestroy(m->ev_out);
    for (auto e : m->ev_pool) (void)hipEventDestroy(e);
    for (auto* km : {&m->kept_act, &m->kept_grad})
      for (auto& kv : *km)
        if (kv.second.p) (void)hipFree(kv.second.p);
    void* bufs[] = {m->frozen, m->lora_p, m->lora_g, m->lora_m, m->lora_v, m->act_mem, (void*)m->d_loss,
                    m->weff_mem, m->tables, m->rscale, m->logits_alt_mem};
    for (void* b : bufs)
      if (b) (void)hipFree(b);
    ShardStore& sh = m->sh;
    if (sh.copy) (void)hipStreamSynchronize(sh.copy);
    for (auto& e : sh.ents) {
      if (e.ready) (void)hipEventDestroy(e.ready);
      if (e.used) (void)hipEventDestroy(e.used);
    }
    if (sh.copy) {
      unregister_stream(sh.copy);
      (void)hipStreamDestroy(sh.copy);
    }
    if (sh.pool) (void)hipFree(sh.pool);
    if (sh.host) (void)hipHostFree(sh.host);
    delete m;
  });
}

int mft_model_shard_stats(mft_model m, int64_t* loads, int64_t* hits, int64_t* budget) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    if (loads) *loads = m->sh.loads;
    if (hits) *hits = m->sh.hits;
    if (budget) *budget = m->sh.budget;
  });
}

int mft_model_shard_reset(mft_model m) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    shard_reset(m);
  });
}

int mft_model_num_params(mft_model m) { return m ? (int)m->P.size() : 0; }

int mft_model_set_training(mft_model m, int training) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    m->training = training != 0;
  });
}

int mft_model_param_info(mft_model m, int i, const char** name, int* ndim, int64_t* dims, int* trainable,
                         int* is_f16, void** data, float** grad) {
  return guarded([&] {
    if (!m || i < 0 || i >= (int)m->P.size()) throw Error(MFT_EINVAL, "param index out of range");
    const Param& p = m->P[i];
    if (name) *name = p.name.c_str();
    if (ndim) *ndim = p.ndim;
    if (dims) {
      dims[0] = p.dims[0];
      dims[1] = p.dims[1];
    }
    if (trainable) *trainable = p.trainable;
    if (is_f16) *is_f16 = p.f16;
    if (data) *data = p.data;
    if (grad) *grad = p.grad;
  });
}

int mft_model_init_params(mft_model m, uint64_t seed, float std, float a_std, float b_std) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    shard_reset(m);  // streamed tensors are generated in the pool, then copied to the host store
    for (size_t i = 0; i < m->P.size(); ++i) {
      Param& p = m->P[i];
      const uint64_t ps = seed * 0x100000001b3ull + i * 0x9e3779b97f4a7c15ull;
      void* dst = p.shard >= 0 ? static_cast<void*>(m->sh.pool) : p.data;
      switch (p.init) {
        case INIT_NORMAL:
          if (p.f16) fill_normal_f16(m->stream, static_cast<uint16_t*>(dst), p.numel, ps, std);
          else fill_normal(m->stream, static_cast<float*>(dst), p.numel, ps, std, 0.f);
          if (p.shard >= 0)
            MFT_HIP(hipMemcpyAsync(p.data, dst, (size_t)p.numel * (p.f16 ? 2 : 4), hipMemcpyDeviceToHost, m->stream));
          break;
        case INIT_ONE: fill_const(m->stream, static_cast<float*>(p.data), p.numel, 1.f); break;
        case INIT_ZERO: fill_const(m->stream, static_cast<float*>(p.data), p.numel, 0.f); break;
        case INIT_LORA_A: fill_normal(m->stream, static_cast<float*>(p.data), p.numel, ps, a_std, 0.f); break;
        case INIT_LORA_B: fill_normal(m->stream, static_cast<float*>(p.data), p.numel, ps, b_std, 0.f); break;
      }
    }
    MFT_HIP(hipStreamSynchronize(m->stream));
  });
}

int mft_model_fwd_bwd(mft_model m, const int32_t* ids, const float* mask, const int32_t* labels, int n_micro,
                      int seqs_per_micro, int S, float upstream) {
  return guarded([&] {
    if (!m || !ids || !labels) throw Error(MFT_EINVAL, "null argument");
    const int nseq = n_micro * seqs_per_micro;
    if (n_micro <= 0 || seqs_per_micro <= 0 || S <= 0) throw Error(MFT_EINVAL, "empty batch");
    if ((int64_t)nseq * S > m->max_tokens) throw Error(MFT_EINVAL, "batch exceeds max_tokens");
    if (m->c.arch == MFT_ARCH_GPT2 && S > m->c.max_pos) throw Error(MFT_EINVAL, "seq_len exceeds n_positions");
    forward(m, ids, mask, nseq, S, m->training, n_micro);
    cross_entropy(m, labels, n_micro, seqs_per_micro, S, upstream, true);
    backward(m, mask, nseq, S);
  });
}

int mft_model_forward(mft_model m, const int32_t* ids, const float* mask, const int32_t* labels, int n_micro,
                      int seqs_per_micro, int S, float* logits) {
  return guarded([&] {
    if (!m || !ids) throw Error(MFT_EINVAL, "null argument");
    const int nseq = n_micro * seqs_per_micro;
    if ((int64_t)nseq * S > m->max_tokens) throw Error(MFT_EINVAL, "batch exceeds max_tokens");
    forward(m, ids, mask, nseq, S, false, 1);
    if (logits)
      MFT_HIP(hipMemcpy2DAsync(logits, sizeof(float) * m->c.vocab, m->logits, sizeof(float) * m->ldv,
                               sizeof(float) * m->c.vocab, (size_t)nseq * S, hipMemcpyDeviceToDevice,
                               m->stream));
    if (labels) cross_entropy(m, labels, n_micro, seqs_per_micro, S, 1.f, false);
  });
}

int mft_model_forward_train(mft_model m, const int32_t* ids, const float* mask, int nseq, int S) {
  return guarded([&] {
    if (!m || !ids) throw Error(MFT_EINVAL, "null argument");
    if (nseq <= 0 || S <= 0) throw Error(MFT_EINVAL, "empty batch");
    if ((int64_t)nseq * S > m->max_tokens) throw Error(MFT_EINVAL, "batch exceeds max_tokens");
    if (m->c.arch == MFT_ARCH_GPT2 && S > m->c.max_pos) throw Error(MFT_EINVAL, "seq_len exceeds n_positions");
    forward(m, ids, mask, nseq, S, m->training, 1);
    m->api_nseq = nseq;
    m->api_S = S;
    m->api_dlogits = false;
  });
}

int mft_model_logits(mft_model m, float** logits, int64_t* ld) {
  return guarded([&] {
    if (!m || !logits || !ld) throw Error(MFT_EINVAL, "null argument");
    *logits = m->logits;
    *ld = m->ldv;
  });
}

int mft_model_ce(mft_model m, const int32_t* labels, int nseq, int S, int ignore_index, float upstream,
                 int64_t norm_count, int backward, double* loss_sum, int64_t* n_valid) {
  return guarded([&] {
    if (!m || !labels) throw Error(MFT_EINVAL, "null argument");
    if (nseq != m->api_nseq || S != m->api_S || nseq <= 0)
      throw Error(MFT_EINVAL, "mft_model_ce: no forward of this shape is pending");
    if (m->api_dlogits) throw Error(MFT_EINVAL, "mft_model_ce: the logits were already turned into dlogits");
    if (backward == 2) {  // the loss, and the dlogits beside the logits
      if (!m->logits_alt) {
        const size_t bytes = sizeof(float) * (size_t)m->max_tokens * m->ldv;
        if (hipMalloc(&m->logits_alt_mem, bytes) != hipSuccess)
          throw Error(MFT_ENOMEM, "second logits buffer (" + std::to_string(bytes) + " bytes)");
        m->logits_alt = static_cast<float*>(m->logits_alt_mem);
        // its padding columns must stay finite, as the logits buffer's
        MFT_HIP(hipMemsetAsync(m->logits_alt, 0, bytes, m->stream));
      }
      ce_fwd_bwd(m->stream, m->logits, labels, nseq, S, m->c.vocab, m->ldv, ignore_index, upstream, norm_count,
                 loss_sum, n_valid, m->logits_alt, m->row_nll, m->d_tmpcnt, m->d_err + 1, nullptr, 0, m->dl_rscale);
      m->alt_ready = true;
      m->alt_up = upstream;
      return;
    }
    if (backward && m->alt_ready && m->alt_up == upstream && !loss_sum && !n_valid) {
      // adopt the dlogits formed with the loss: no second pass over the logits
      std::swap(m->logits, m->logits_alt);
      drop_graph(m);  // a captured step holds the other buffer's address
      m->alt_ready = false;
      m->api_dlogits = true;
      m->dl_rs_fresh = m->dl_rscale != nullptr;
      return;
    }
    ce_fwd_bwd(m->stream, m->logits, labels, nseq, S, m->c.vocab, m->ldv, ignore_index, upstream, norm_count,
               loss_sum, n_valid, backward ? m->logits : nullptr, m->row_nll, m->d_tmpcnt, m->d_err + 1, nullptr, 0,
               backward && m->dl_rscale ? m->dl_rscale : nullptr);
    if (backward) {
      m->api_dlogits = true;
      m->alt_ready = false;
      m->dl_rs_fresh = m->dl_rscale != nullptr;
    }
  });
}

int mft_model_backward(mft_model m, const float* mask, int nseq, int S) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    if (nseq != m->api_nseq || S != m->api_S || nseq <= 0 || !m->api_dlogits)
      throw Error(MFT_EINVAL, "mft_model_backward: needs mft_model_forward_train and mft_model_ce(backward) first");
    backward(m, mask, nseq, S);
    m->api_nseq = m->api_S = 0;
    m->api_dlogits = false;
  });
}

int mft_model_opt_step(mft_model m, float lr, float b1, float b2, float eps, float wd, float clip) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    const HpArgs hp{lr, b1, b2, eps, wd, clip};
    opt_device(m, &hp);
    m->adam_t++;
  });
}

int mft_model_train_step(mft_model m, const int32_t* ids, const float* mask, const int32_t* labels,
                         int n_micro, int seqs_per_micro, int S, float upstream, float lr, float b1,
                         float b2, float eps, float wd, float clip, int use_graph) {
  // no captured graph for a streamed (sharded) model, whose pool addresses
  // change from step to step, or in sync-check mode, whose device waits
  // cannot be captured
  if (m && (m->sh.budget > 0 || g_sync_check)) use_graph = 0;
  return guarded([&] {
    if (!m || !ids || !labels) throw Error(MFT_EINVAL, "null argument");
    const int nseq = n_micro * seqs_per_micro;
    if (n_micro <= 0 || seqs_per_micro <= 0 || S <= 0) throw Error(MFT_EINVAL, "empty batch");
    if ((int64_t)nseq * S > m->max_tokens) throw Error(MFT_EINVAL, "batch exceeds max_tokens");
    if (m->c.arch == MFT_ARCH_GPT2 && S > m->c.max_pos) throw Error(MFT_EINVAL, "seq_len exceeds n_positions");
    if (!use_graph) {
      zero_stats(m, n_micro);
      m->n_micro_pending = 0;
      forward(m, ids, mask, nseq, S, m->training, n_micro);
      cross_entropy(m, labels, n_micro, seqs_per_micro, S, upstream, true);
      backward(m, mask, nseq, S);
      const HpArgs hp{lr, b1, b2, eps, wd, clip};
      opt_device(m, &hp);
      m->adam_t++;
      return;
    }
    const bool same = m->graph_exec && m->graph_key.ids == ids && m->graph_key.mask == mask &&
                      m->graph_key.labels == labels && m->graph_key.n_micro == n_micro &&
                      m->graph_key.seqs == seqs_per_micro && m->graph_key.S == S &&
                      m->graph_key.upstream == upstream && m->graph_key.timing == m->timing &&
                      m->graph_key.training == m->training;
    if (!same) capture_step(m, ids, mask, labels, n_micro, seqs_per_micro, S, upstream);
    upload_hparams(m, lr, b1, b2, eps, wd, clip);
    MFT_HIP(hipEventRecord(m->ev_in, m->stream));
    MFT_HIP(hipStreamWaitEvent(m->cap_stream, m->ev_in, 0));
    MFT_HIP(hipGraphLaunch(m->graph_exec, m->cap_stream));
    MFT_HIP(hipEventRecord(m->ev_out, m->cap_stream));
    MFT_HIP(hipStreamWaitEvent(m->stream, m->ev_out, 0));
    m->n_micro_pending = n_micro;
    m->adam_t++;
    if (m->timing) {
      // The graph re-records the same events on every replay: read them now.
      MFT_HIP(hipStreamSynchronize(m->cap_stream));
      for (auto& t : m->graph_timed) {
        float ms = 0.f, ms2 = 0.f;
        MFT_HIP(hipEventElapsedTime(&ms, t.a, t.b));
        if (t.c) MFT_HIP(hipEventElapsedTime(&ms2, t.c, t.d));
        m->t_ms[t.cls] += ms + ms2;
        m->t_work[t.cls] += t.work;
        m->t_n[t.cls] += 1;
      }
    }
  });
}

int mft_model_read_stats(mft_model m, float* mean_loss, int64_t* n_valid, float* grad_norm) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    MFT_HIP(hipStreamSynchronize(m->stream));
    double ls[64];
    int64_t cn[64];
    float cl[2];
    const int n = m->n_micro_pending;
    if (n > 0) {
      MFT_HIP(hipMemcpy(ls, m->d_loss, sizeof(double) * n, hipMemcpyDeviceToHost));
      MFT_HIP(hipMemcpy(cn, m->d_cnt, sizeof(int64_t) * n, hipMemcpyDeviceToHost));
    }
    MFT_HIP(hipMemcpy(cl, m->d_clip, sizeof(cl), hipMemcpyDeviceToHost));
    int err[2] = {0, 0};
    MFT_HIP(hipMemcpy(err, m->d_err, sizeof(err), hipMemcpyDeviceToHost));
    double acc = 0.0;
    int64_t tot = 0;
    for (int i = 0; i < n; ++i) {
      acc += cn[i] > 0 ? ls[i] / (double)cn[i] : 0.0;
      tot += cn[i];
    }
    if (mean_loss) *mean_loss = n > 0 ? (float)(acc / n) : 0.f;
    if (n_valid) *n_valid = tot;
    if (grad_norm) *grad_norm = cl[1];
    MFT_HIP(hipMemset(m->d_loss, 0, 1024));
    m->n_micro_pending = 0;
    if (err[0] || err[1]) {
      MFT_HIP(hipMemset(m->d_err, 0, sizeof(err)));
      throw Error(MFT_EINVAL, std::string("mft_model_read_stats: since the last call ") +
                                  (err[0] ? "a token id was outside [0, vocab) (its embedding row was zeroed)" : "") +
                                  (err[0] && err[1] ? "; " : "") +
                                  (err[1] ? "a label outside [0, vocab) other than ignore_index was treated as ignored"
                                          : ""));
    }
  });
}

int mft_model_activation(mft_model m, int layer, const char* name, const float** ptr, int64_t* rows,
                         int64_t* cols, int64_t* ld) {
  return guarded([&] {
    if (!m || !name || !ptr) throw Error(MFT_EINVAL, "null argument");
    if (m->last_rows == 0) throw Error(MFT_EINVAL, "mft_model_activation: no forward has run");
    const mft_model_cfg& c = m->c;
    const std::string n = name;
    const int64_t d = c.d, hq = (int64_t)c.n_head * c.head_dim, hk = (int64_t)c.n_kv_head * c.head_dim;
    const bool gpt2 = c.arch == MFT_ARCH_GPT2, gemma = c.arch == MFT_ARCH_GEMMA3;
    const float* p = nullptr;
    int64_t w = 0, pitch = 0;
    auto set = [&](const float* q, int64_t width, int64_t l) {
      p = q;
      w = width;
      pitch = l;
    };
    if (layer < 0) {
      if (n == "embed") set(m->A[0].x, d, d);
      else if (n == "final_norm") set(m->hf, d, d);
    } else {
      if (layer >= c.n_layer) throw Error(MFT_EINVAL, "mft_model_activation: layer out of range");
      const Acts& a = m->A[layer];
      if (n == "x") set(a.x, d, d);
      else if (n == "norm1") set(a.n1, d, d);
      else if (n == "q") set(a.q, hq, a.qs);
      else if (n == "k") set(a.k, hk, a.ks);
      else if (n == "v") set(a.v, hk, a.vs);
      else if (n == "q_proj" && gemma) set(a.qraw, hq, m->lay_qkv ? m->nqkv : hq);
      else if (n == "k_proj" && gemma) set(a.kraw, hk, m->lay_qkv ? m->nqkv : hk);
      else if (n == "attn") set(a.att, hq, hq);
      else if (n == "o_proj" && gemma) set(a.o, d, d);
      else if (n == "mid") set(a.hmid, d, d);
      else if (n == "norm2") set(a.n2, d, d);
      else if (n == "gate") set(a.gate, c.d_ff, m->lay_gu ? 2 * c.d_ff : c.d_ff);
      else if (n == "up" && !gpt2) set(a.up, c.d_ff, m->lay_gu ? 2 * c.d_ff : c.d_ff);
      else if (n == "act") set(a.act, c.d_ff, c.d_ff);
      else if (n == "down_proj" && gemma) set(a.mo, d, d);
      else if (n == "out") set(layer + 1 < c.n_layer ? m->A[layer + 1].x : m->h_final, d, d);
    }
    if (!p) {  // the alignment-dump debug mode's extra activations
      auto it = m->kept_act.find({layer, n});
      if (it != m->kept_act.end() && it->second.p) {
        *ptr = it->second.p;
        if (rows) *rows = it->second.rows;
        if (cols) *cols = it->second.cols;
        if (ld) *ld = it->second.cols;
        return;
      }
    }
    if (!p) throw Error(MFT_EINVAL, "mft_model_activation: this model keeps no activation '" + n + "'");
    *ptr = p;
    if (rows) *rows = m->last_rows;
    if (cols) *cols = w;
    if (ld) *ld = pitch;
  });
}

int mft_model_set_retain(mft_model m, uint64_t layer_mask) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    if (layer_mask && m->c.arch != MFT_ARCH_GEMMA3)
      throw Error(MFT_EINVAL, "mft_model_set_retain: the alignment dump's retention serves Gemma3 models");
    if (m->capturing) throw Error(MFT_EINVAL, "mft_model_set_retain: not while a step graph is being captured");
    m->retain = layer_mask;
  });
}

int mft_model_activation_grad(mft_model m, int layer, const char* name, const float** ptr, int64_t* rows,
                              int64_t* cols, int64_t* ld) {
  return guarded([&] {
    if (!m || !name || !ptr) throw Error(MFT_EINVAL, "null argument");
    auto it = m->kept_grad.find({layer, name});
    if (it == m->kept_grad.end() || !it->second.p || it->second.rows == 0)
      throw Error(MFT_EINVAL, std::string("mft_model_activation_grad: no retained gradient '") + name + "'");
    *ptr = it->second.p;
    if (rows) *rows = it->second.rows;
    if (cols) *cols = it->second.cols;
    if (ld) *ld = it->second.cols;
  });
}

int mft_model_set_timing(mft_model m, int enable) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    if (!enable) collect_timing(m);
    m->timing = enable != 0;
  });
}

int mft_model_timing(mft_model m, int cls, double* ms, double* work, int64_t* launches) {
  return guarded([&] {
    if (!m || cls < 0 || cls >= CLS_MAX) throw Error(MFT_EINVAL, "bad class");
    collect_timing(m);
    if (ms) *ms = m->t_ms[cls];
    if (work) *work = m->t_work[cls];
    if (launches) *launches = m->t_n[cls];
  });
}

int mft_model_reset_timing(mft_model m) {
  return guarded([&] {
    if (!m) throw Error(MFT_EINVAL, "null model");
    collect_timing(m);
    for (int i = 0; i < CLS_MAX; ++i) {
      m->t_ms[i] = m->t_work[i] = 0;
      m->t_n[i] = 0;
    }
  });
}

}  // extern "C"
