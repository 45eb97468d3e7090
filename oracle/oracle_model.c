/*
 * oracle_model.c — CPU restatement of the three LoRA training graphs
 * (GPT-2, Qwen2, Gemma3) and of one optimizer step.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Step order follows gpt2_small_lora_finetune/src/main.cpp:456-505:
 *   for each micro-batch: forward (:473) → lm_cross_entropy (:475) →
 *   mul(loss, 1/accum)->backward() (:481-485); then clip_and_get_grad_norm
 *   (:490, body :384-409) → Adam step (:497-502) → zero_grad (:503-505).
 * Graph semantics:
 *   GPT-2   embed wte+wpe → L×{LN → c_attn(LoRA) → causal MHA → c_proj(LoRA)
 *           → +res → LN → c_fc → GELU(tanh) → c_proj → +res} → LN_f → h·wteᵀ
 *           (main.cpp:204 tie_weights; main.cpp:271-272 LoRA targets).
 *   Qwen2   embed → L×{RMSNorm → q,k,v(+bias) → RoPE(θ) → GQA attn → o → +res
 *           → RMSNorm → down(silu(gate)·up) → +res} → RMSNorm → tied head
 *           (qwen_lora_finetune/src/wikitext_main.cpp:63-79; HF Qwen2).
 *   Gemma3  embed·√d → L×{RMSNorm(1+w) → q,k,v → per-head QK-RMSNorm → RoPE
 *           (local/global θ) → GQA attn (scale query_pre_attn_scalar^-½) → o →
 *           post-attn norm → +res → pre-ff norm → down(gelu(gate)·up) →
 *           post-ff norm → +res} → norm → tied head
 *           (op order = debug names gemma_3_270m_lora_finetune/src/main.cpp:562-596,
 *           scale :605; HF Gemma3 for the norm forms).
 * Frozen weights get no gradient; the backward stops below layer 0's first
 * trainable input (nothing under it is trainable).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
  char name[96];
  int ndim;
  int64_t dims[2];
  int64_t numel;
  int trainable, is_f16;
  void* data;
  float* grad;
  float *m, *v;
} oparam;

enum { T_Q = 0, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_MAX };
enum { G_ATTN = 0, G_PROJ, G_FC, G_FC2 };

typedef struct {
  int W, b, A, B; /* param indices, -1 if absent */
  int K, N;
  int lid;        /* dropout stream id: layer·8 + target */
} olinear;

typedef struct {
  /* norms */
  int n1w, n1b, n2w, n2b, qn, kn, pan, pfn; /* pan/pfn: Gemma post norms */
  olinear lin[T_MAX];
  int nlin;
} olayer;

struct orc_model {
  orc_model_cfg c;
  oparam* p;
  int np, cap;
  int wte, wpe, nfw, nfb;
  olayer* L;
  int t; /* Adam step count */
  uint32_t drop_step; /* training forwards run (LoRA dropout stream) */
  int training;       /* the current forward drops LoRA inputs */
  /* activation cache for the current micro-batch */
  int B, S;
  float** act;
  int nact;
  /* retained intermediates (orc_model_set_retain) */
  uint64_t retain;
  struct kept {
    int layer, grad;
    char name[16];
    float* data;
    int64_t n;
  } * kept;
  int nkept;
};

static void* xmalloc(size_t n) {
  void* p = calloc(1, n ? n : 1);
  if (!p) { fprintf(stderr, "oracle: out of memory (%zu)\n", n); abort(); }
  return p;
}

static int add_param(orc_model* m, const char* name, int64_t d0, int64_t d1,
                     int trainable, int f16) {
  if (m->np == m->cap) {
    m->cap = m->cap ? m->cap * 2 : 64;
    m->p = (oparam*)realloc(m->p, sizeof(oparam) * (size_t)m->cap);
  }
  oparam* p = &m->p[m->np];
  memset(p, 0, sizeof(*p));
  snprintf(p->name, sizeof(p->name), "%s", name);
  p->ndim = d1 > 0 ? 2 : 1;
  p->dims[0] = d0;
  p->dims[1] = d1 > 0 ? d1 : 0;
  p->numel = d0 * (d1 > 0 ? d1 : 1);
  p->trainable = trainable;
  p->is_f16 = f16;
  p->data = xmalloc((size_t)p->numel * (f16 ? 2 : 4));
  if (trainable) {
    p->grad = (float*)xmalloc((size_t)p->numel * 4);
    p->m = (float*)xmalloc((size_t)p->numel * 4);
    p->v = (float*)xmalloc((size_t)p->numel * 4);
  }
  return m->np++;
}

static const char* gpt2_lin_names[4] = {"attn.c_attn", "attn.c_proj", "mlp.c_fc",
                                        "mlp.c_proj"};
static const char* hf_lin_names[7] = {"self_attn.q_proj", "self_attn.k_proj",
                                      "self_attn.v_proj", "self_attn.o_proj",
                                      "mlp.gate_proj",    "mlp.up_proj",
                                      "mlp.down_proj"};

static void add_linear(orc_model* m, olinear* l, const char* pfx,
                       const char* nm, int K, int N, int bias, int lora) {
  char buf[128];
  const orc_model_cfg* c = &m->c;
  l->K = K;
  l->N = N;
  snprintf(buf, sizeof buf, "%s.%s.weight", pfx, nm);
  l->W = add_param(m, buf, K, N, 0, c->w_fp16);
  l->b = -1;
  if (bias) {
    snprintf(buf, sizeof buf, "%s.%s.bias", pfx, nm);
    l->b = add_param(m, buf, N, 0, 0, 0);
  }
  l->A = l->B = -1;
  if (lora && c->lora_r > 0) {
    snprintf(buf, sizeof buf, "%s.%s.lora_A", pfx, nm);
    l->A = add_param(m, buf, c->lora_r, K, 1, 0);
    snprintf(buf, sizeof buf, "%s.%s.lora_B", pfx, nm);
    l->B = add_param(m, buf, N, c->lora_r, 1, 0);
  }
}

orc_model* orc_model_create(const orc_model_cfg* cfg) {
  orc_model* m = (orc_model*)xmalloc(sizeof(orc_model));
  m->c = *cfg;
  const orc_model_cfg* c = &m->c;
  const int d = c->d, hd = c->head_dim, H = c->n_head, Hk = c->n_kv_head;
  char pfx[64], buf[128];
  m->L = (olayer*)xmalloc(sizeof(olayer) * (size_t)c->n_layer);
  if (c->arch == ORC_GPT2) {
    m->wte = add_param(m, "wte", c->vocab, d, 0, c->w_fp16);
    m->wpe = add_param(m, "wpe", c->max_pos, d, 0, 0);
    for (int i = 0; i < c->n_layer; ++i) {
      olayer* L = &m->L[i];
      snprintf(pfx, sizeof pfx, "h.%d", i);
      snprintf(buf, sizeof buf, "%s.ln_1.weight", pfx); L->n1w = add_param(m, buf, d, 0, 0, 0);
      snprintf(buf, sizeof buf, "%s.ln_1.bias", pfx);   L->n1b = add_param(m, buf, d, 0, 0, 0);
      add_linear(m, &L->lin[G_ATTN], pfx, gpt2_lin_names[0], d, 3 * d, 1, c->lora_mask & 1);
      add_linear(m, &L->lin[G_PROJ], pfx, gpt2_lin_names[1], d, d, 1, c->lora_mask & 2);
      snprintf(buf, sizeof buf, "%s.ln_2.weight", pfx); L->n2w = add_param(m, buf, d, 0, 0, 0);
      snprintf(buf, sizeof buf, "%s.ln_2.bias", pfx);   L->n2b = add_param(m, buf, d, 0, 0, 0);
      add_linear(m, &L->lin[G_FC], pfx, gpt2_lin_names[2], d, c->d_ff, 1, c->lora_mask & 4);
      add_linear(m, &L->lin[G_FC2], pfx, gpt2_lin_names[3], c->d_ff, d, 1, c->lora_mask & 8);
      L->nlin = 4;
    }
    m->nfw = add_param(m, "ln_f.weight", d, 0, 0, 0);
    m->nfb = add_param(m, "ln_f.bias", d, 0, 0, 0);
  } else {
    const int qwen = c->arch == ORC_QWEN2;
    m->wte = add_param(m, "embed_tokens.weight", c->vocab, d, 0, c->w_fp16);
    m->wpe = -1;
    for (int i = 0; i < c->n_layer; ++i) {
      olayer* L = &m->L[i];
      snprintf(pfx, sizeof pfx, "layers.%d", i);
      snprintf(buf, sizeof buf, "%s.input_layernorm.weight", pfx);
      L->n1w = add_param(m, buf, d, 0, 0, 0);
      L->n1b = -1;
      const int outs[7] = {H * hd, Hk * hd, Hk * hd, d, c->d_ff, c->d_ff, d};
      const int ins[7] = {d, d, d, H * hd, d, d, c->d_ff};
      for (int t = 0; t < 4; ++t)
        add_linear(m, &L->lin[t], pfx, hf_lin_names[t], ins[t], outs[t],
                   qwen && t < 3, (c->lora_mask >> t) & 1);
      L->qn = L->kn = L->pan = L->pfn = -1;
      if (!qwen) {
        snprintf(buf, sizeof buf, "%s.self_attn.q_norm.weight", pfx); L->qn = add_param(m, buf, hd, 0, 0, 0);
        snprintf(buf, sizeof buf, "%s.self_attn.k_norm.weight", pfx); L->kn = add_param(m, buf, hd, 0, 0, 0);
        snprintf(buf, sizeof buf, "%s.post_attention_layernorm.weight", pfx); L->pan = add_param(m, buf, d, 0, 0, 0);
        snprintf(buf, sizeof buf, "%s.pre_feedforward_layernorm.weight", pfx); L->n2w = add_param(m, buf, d, 0, 0, 0);
        snprintf(buf, sizeof buf, "%s.post_feedforward_layernorm.weight", pfx); L->pfn = add_param(m, buf, d, 0, 0, 0);
      } else {
        snprintf(buf, sizeof buf, "%s.post_attention_layernorm.weight", pfx); L->n2w = add_param(m, buf, d, 0, 0, 0);
      }
      L->n2b = -1;
      for (int t = 4; t < 7; ++t)
        add_linear(m, &L->lin[t], pfx, hf_lin_names[t], ins[t], outs[t], 0,
                   (c->lora_mask >> t) & 1);
      L->nlin = 7;
    }
    m->nfw = add_param(m, "norm.weight", d, 0, 0, 0);
    m->nfb = -1;
  }
  for (int li = 0; li < c->n_layer; ++li)
    for (int t = 0; t < T_MAX; ++t) m->L[li].lin[t].lid = li * 8 + t;
  return m;
}

static void free_acts(orc_model* m) {
  for (int i = 0; i < m->nact; ++i) free(m->act[i]);
  free(m->act);
  m->act = NULL;
  m->nact = 0;
}

static void clear_kept(orc_model* m) {
  for (int i = 0; i < m->nkept; ++i) free(m->kept[i].data);
  free(m->kept);
  m->kept = NULL;
  m->nkept = 0;
}

void orc_model_set_retain(orc_model* m, uint64_t layer_mask) { m->retain = layer_mask; }

const float* orc_model_retained(const orc_model* m, int layer, const char* name, int grad, int64_t* n) {
  for (int i = 0; i < m->nkept; ++i)
    if (m->kept[i].layer == layer && m->kept[i].grad == grad && !strcmp(m->kept[i].name, name)) {
      if (n) *n = m->kept[i].n;
      return m->kept[i].data;
    }
  if (n) *n = 0;
  return NULL;
}

static int keeps(const orc_model* m, int layer) {
  return layer >= 0 && layer < 64 && ((m->retain >> layer) & 1);
}

/* Copies rows x cols of src (rows ld apart) as retained (layer, name, grad). */
static void keep(orc_model* m, int layer, const char* name, int grad, const float* src, int64_t rows,
                 int64_t cols, int64_t ld) {
  float* d = (float*)xmalloc(sizeof(float) * (size_t)(rows * cols));
  for (int64_t r = 0; r < rows; ++r) memcpy(d + r * cols, src + r * ld, sizeof(float) * (size_t)cols);
  m->kept = (struct kept*)realloc(m->kept, sizeof(struct kept) * (size_t)(m->nkept + 1));
  struct kept* k = &m->kept[m->nkept++];
  k->layer = layer;
  k->grad = grad;
  snprintf(k->name, sizeof(k->name), "%s", name);
  k->data = d;
  k->n = rows * cols;
}

void orc_model_destroy(orc_model* m) {
  if (!m) return;
  clear_kept(m);
  for (int i = 0; i < m->np; ++i) {
    free(m->p[i].data); free(m->p[i].grad); free(m->p[i].m); free(m->p[i].v);
  }
  free(m->p);
  free(m->L);
  free_acts(m);
  free(m);
}

int orc_model_num_params(const orc_model* m) { return m->np; }

int64_t orc_model_param_info(const orc_model* m, int i, const char** name,
                             int* ndim, int64_t* dims, int* trainable,
                             int* is_f16) {
  const oparam* p = &m->p[i];
  if (name) *name = p->name;
  if (ndim) *ndim = p->ndim;
  if (dims) { dims[0] = p->dims[0]; dims[1] = p->dims[1]; }
  if (trainable) *trainable = p->trainable;
  if (is_f16) *is_f16 = p->is_f16;
  return p->numel;
}
void* orc_model_param_data(orc_model* m, int i) { return m->p[i].data; }
float* orc_model_param_grad(orc_model* m, int i) { return m->p[i].grad; }

/* ---- helpers ------------------------------------------------------------ */
static float* P(orc_model* m, int i) { return i < 0 ? NULL : (float*)m->p[i].data; }

static float* F(orc_model* m, int64_t n) { /* cached activation buffer */
  m->act = (float**)realloc(m->act, sizeof(float*) * (size_t)(m->nact + 1));
  float* b = (float*)xmalloc((size_t)n * 4);
  m->act[m->nact++] = b;
  return b;
}

/* fp32 view of a frozen weight (dequantised copy when stored as fp16) */
static const float* wview(orc_model* m, int i, float** tmp) {
  oparam* p = &m->p[i];
  *tmp = NULL;
  if (!p->is_f16) return (const float*)p->data;
  *tmp = (float*)xmalloc((size_t)p->numel * 4);
  orc_f16_to_f32((const uint16_t*)p->data, *tmp, p->numel);
  return *tmp;
}

static float lscale(const orc_model* m) { return m->c.lora_alpha / (float)m->c.lora_r; }

static int dropout_active(const orc_model* m, const olinear* l) {
  return l->A >= 0 && m->training && m->c.lora_dropout > 0.0f;
}

/* y = x·W + b + s·(xd·Aᵀ)·Bᵀ, xd = x (or x∘mask with LoRA dropout in a
 * training forward: PEFT's lora_B(lora_A(dropout(x)))·s).  xa = xd·Aᵀ and
 * xd are kept for the backward. */
static void lin_fwd(orc_model* m, const olinear* l, const float* x, int64_t M,
                    float* y, float** xa_out, float** xd_out) {
  float* tmp;
  const float* W = wview(m, l->W, &tmp);
  const int r = m->c.lora_r;
  float* xa = NULL;
  *xd_out = NULL;
  if (l->A >= 0) xa = F(m, M * r);
  if (!dropout_active(m, l)) {
    orc_lora_linear_fwd(x, M, l->K, W, l->N, P(m, l->b), P(m, l->A), P(m, l->B),
                        l->A >= 0 ? r : 0, lscale(m), y, xa);
  } else {
    const int64_t K = l->K, N = l->N;
    float* xd = F(m, M * K);
    orc_dropout_mask(m->c.dropout_seed, m->drop_step, (uint32_t)l->lid, M * K, m->c.lora_dropout, xd);
    for (int64_t i = 0; i < M * K; ++i) xd[i] *= x[i];
    orc_lora_linear_fwd(x, M, K, W, N, P(m, l->b), NULL, NULL, 0, 0.0f, y, NULL);
    const float* A = P(m, l->A);
    const float* Bm = P(m, l->B);
    const float s = lscale(m);
#pragma omp parallel for
    for (int64_t i = 0; i < M; ++i) {
      for (int j = 0; j < r; ++j) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += (double)xd[i * K + k] * A[(int64_t)j * K + k];
        xa[i * r + j] = (float)acc;
      }
      for (int64_t n = 0; n < N; ++n) {
        double t = 0.0;
        for (int j = 0; j < r; ++j) t += (double)xa[i * r + j] * Bm[n * r + j];
        y[i * N + n] += (float)(s * t);
      }
    }
    *xd_out = xd;
  }
  free(tmp);
  *xa_out = xa;
}

/* dX = dY·Wᵀ + s·(dY·B·A)∘mask; dA += s·(dY·B)ᵀ·xd; dB += s·dYᵀ·xa (no
 * mask: xd = x without dropout). */
static void lin_bwd(orc_model* m, const olinear* l, const float* dy,
                    const float* x, const float* xa, const float* xd, int64_t M, float* dx) {
  float* tmp;
  const float* W = wview(m, l->W, &tmp);
  int r = l->A >= 0 ? m->c.lora_r : 0;
  if (!xd) {
    orc_lora_linear_bwd(dy, x, W, P(m, l->A), P(m, l->B), xa, M, l->K, l->N, r,
                        lscale(m), dx, l->A >= 0 ? m->p[l->A].grad : NULL,
                        l->B >= 0 ? m->p[l->B].grad : NULL, 1);
  } else {
    const int64_t K = l->K, N = l->N;
    const float s = lscale(m);
    const float* A = P(m, l->A);
    const float* Bm = P(m, l->B);
    float* dA = m->p[l->A].grad;
    float* dB = m->p[l->B].grad;
    if (dx) orc_lora_linear_bwd(dy, x, W, NULL, NULL, NULL, M, K, N, 0, 0.0f, dx, NULL, NULL, 1);
    float* U = (float*)xmalloc(sizeof(float) * (size_t)(M * r));
    float* mask = (float*)xmalloc(sizeof(float) * (size_t)(M * K));
    orc_dropout_mask(m->c.dropout_seed, m->drop_step, (uint32_t)l->lid, M * K, m->c.lora_dropout, mask);
#pragma omp parallel for
    for (int64_t i = 0; i < M; ++i)
      for (int j = 0; j < r; ++j) {
        double acc = 0.0;
        for (int64_t n = 0; n < N; ++n) acc += (double)dy[i * N + n] * Bm[n * r + j];
        U[i * r + j] = (float)acc;
      }
    if (dx) {
#pragma omp parallel for
      for (int64_t i = 0; i < M; ++i)
        for (int64_t k = 0; k < K; ++k) {
          double t = 0.0;
          for (int j = 0; j < r; ++j) t += (double)U[i * r + j] * A[(int64_t)j * K + k];
          dx[i * K + k] += (float)(s * t * mask[i * K + k]);
        }
    }
#pragma omp parallel for
    for (int j = 0; j < r; ++j)
      for (int64_t k = 0; k < K; ++k) {
        double t = 0.0;
        for (int64_t i = 0; i < M; ++i) t += (double)U[i * r + j] * xd[i * K + k];
        dA[(int64_t)j * K + k] += (float)(s * t);
      }
#pragma omp parallel for
    for (int64_t n = 0; n < N; ++n)
      for (int j = 0; j < r; ++j) {
        double t = 0.0;
        for (int64_t i = 0; i < M; ++i) t += (double)dy[i * N + n] * xa[i * r + j];
        dB[n * r + j] += (float)(s * t);
      }
    free(U);
    free(mask);
  }
  free(tmp);
}

static void add_into(float* a, const float* b, int64_t n) {
#pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) a[i] += b[i];
}

typedef struct {
  float *x, *n1, *mean1, *rstd1;
  float *q, *k, *v;       /* attention inputs (after norm/rope) */
  float *qraw, *kraw;     /* Gemma: pre-QK-norm projections */
  float *qrs, *krs;       /* Gemma: per (token,head) rstd */
  int64_t qs, ks, vs;     /* row strides of q/k/v */
  float *xa[T_MAX];
  float *xd[T_MAX];       /* LoRA inputs after dropout (training forwards) */
  float *att, *lse;
  float *o, *ors;         /* Gemma: o_proj output before post-attn norm */
  float *hmid;
  float *n2, *mean2, *rstd2;
  float *gate, *up, *act;
  float *mo, *mrs;        /* Gemma: mlp output before post-ff norm */
} lcache;

static int layer_is_local(const orc_model_cfg* c, int i) {
  return c->arch == ORC_GEMMA3 && c->sliding_pattern > 0 &&
         ((i + 1) % c->sliding_pattern) != 0;
}

static float attn_scale(const orc_model_cfg* c) {
  return c->attn_scale > 0.0f ? c->attn_scale : 1.0f / sqrtf((float)c->head_dim);
}

/* Forward of the whole graph for one micro-batch.  Returns final hidden
 * (after the final norm) and fills caches; logits written to `logits`. */
static void forward_all(orc_model* m, const int32_t* ids, const float* mask,
                        int B, int S, lcache* cache, float** hf_out,
                        float** hlast_out, float** fmean, float** frstd,
                        float* logits) {
  const orc_model_cfg* c = &m->c;
  const int64_t M = (int64_t)B * S;
  const int d = c->d, H = c->n_head, Hk = c->n_kv_head, hd = c->head_dim;
  const int gpt2 = c->arch == ORC_GPT2, gemma = c->arch == ORC_GEMMA3;
  float* h = F(m, M * d);
  {
    const oparam* e = &m->p[m->wte];
    float sc = gemma ? (float)sqrt((double)d) : 1.0f;
    orc_embed(ids, M, S, e->is_f16 ? NULL : (const float*)e->data,
              e->is_f16 ? (const uint16_t*)e->data : NULL,
              gpt2 ? P(m, m->wpe) : NULL, d, sc, h);
  }
  if (m->retain) {
    clear_kept(m);
    if (keeps(m, 0)) keep(m, -1, "embed", 0, h, M, d, d);
  }
  for (int li = 0; li < c->n_layer; ++li) {
    olayer* L = &m->L[li];
    lcache* C = &cache[li];
    const int kp = keeps(m, li);
    memset(C, 0, sizeof(*C));
    C->x = h;
    C->n1 = F(m, M * d);
    C->rstd1 = F(m, M);
    if (gpt2) {
      C->mean1 = F(m, M);
      orc_layernorm_fwd(h, P(m, L->n1w), P(m, L->n1b), M, d, c->norm_eps, C->n1, C->mean1, C->rstd1);
      float* qkv = F(m, M * 3 * d);
      lin_fwd(m, &L->lin[G_ATTN], C->n1, M, qkv, &C->xa[G_ATTN], &C->xd[G_ATTN]);
      C->q = qkv; C->k = qkv + d; C->v = qkv + 2 * d;
      C->qs = C->ks = C->vs = 3 * d;
    } else {
      orc_rmsnorm_fwd(h, P(m, L->n1w), M, d, c->norm_eps, gemma, C->n1, C->rstd1);
      C->q = F(m, M * H * hd); C->k = F(m, M * Hk * hd); C->v = F(m, M * Hk * hd);
      C->qs = (int64_t)H * hd; C->ks = C->vs = (int64_t)Hk * hd;
      lin_fwd(m, &L->lin[T_Q], C->n1, M, C->q, &C->xa[T_Q], &C->xd[T_Q]);
      lin_fwd(m, &L->lin[T_K], C->n1, M, C->k, &C->xa[T_K], &C->xd[T_K]);
      lin_fwd(m, &L->lin[T_V], C->n1, M, C->v, &C->xa[T_V], &C->xd[T_V]);
      if (gemma) { /* QK RMSNorm over head_dim, (1+w) form */
        C->qraw = F(m, M * H * hd); C->kraw = F(m, M * Hk * hd);
        memcpy(C->qraw, C->q, sizeof(float) * (size_t)(M * H * hd));
        memcpy(C->kraw, C->k, sizeof(float) * (size_t)(M * Hk * hd));
        C->qrs = F(m, M * H); C->krs = F(m, M * Hk);
        orc_rmsnorm_fwd(C->qraw, P(m, L->qn), M * H, hd, c->norm_eps, 1, C->q, C->qrs);
        orc_rmsnorm_fwd(C->kraw, P(m, L->kn), M * Hk, hd, c->norm_eps, 1, C->k, C->krs);
        if (kp) {
          keep(m, li, "q_normed", 0, C->q, M, (int64_t)H * hd, (int64_t)H * hd);
          keep(m, li, "k_normed", 0, C->k, M, (int64_t)Hk * hd, (int64_t)Hk * hd);
        }
      }
      double th = layer_is_local(c, li) ? c->rope_local_theta : c->rope_theta;
      orc_rope(C->q, C->qs, B, S, H, hd, th, 0);
      orc_rope(C->k, C->ks, B, S, Hk, hd, th, 0);
    }
    C->att = F(m, M * H * hd);
    C->lse = F(m, (int64_t)B * H * S);
    int win = layer_is_local(c, li) ? c->sliding_window : 0;
    orc_attn_fwd(C->q, C->qs, C->k, C->ks, C->v, C->vs, B, H, Hk, S, hd,
                 attn_scale(c), 1, win, mask, C->att, (int64_t)H * hd, C->lse);
    if (kp) {
      const int64_t ns = (int64_t)B * H * S * S;
      float* sc = (float*)xmalloc(sizeof(float) * (size_t)ns);
      float* pr = (float*)xmalloc(sizeof(float) * (size_t)ns);
      orc_attn_probs(C->q, C->qs, C->k, C->ks, C->v, C->vs, NULL, 0, B, H, Hk, S, hd, attn_scale(c), 1, win,
                     mask, sc, pr, NULL, NULL);
      keep(m, li, "scores", 0, sc, 1, ns, ns);
      keep(m, li, "probs", 0, pr, 1, ns, ns);
      free(sc);
      free(pr);
    }
    float* hmid = F(m, M * d);
    const olinear* lo = gpt2 ? &L->lin[G_PROJ] : &L->lin[T_O];
    C->o = F(m, M * d);
    lin_fwd(m, lo, C->att, M, C->o, gpt2 ? &C->xa[G_PROJ] : &C->xa[T_O], gpt2 ? &C->xd[G_PROJ] : &C->xd[T_O]);
    if (gemma) {
      C->ors = F(m, M);
      float* on = F(m, M * d);
      orc_rmsnorm_fwd(C->o, P(m, L->pan), M, d, c->norm_eps, 1, on, C->ors);
      for (int64_t i = 0; i < M * d; ++i) hmid[i] = h[i] + on[i];
    } else {
      for (int64_t i = 0; i < M * d; ++i) hmid[i] = h[i] + C->o[i];
    }
    C->hmid = hmid;
    C->n2 = F(m, M * d);
    C->rstd2 = F(m, M);
    if (gpt2) {
      C->mean2 = F(m, M);
      orc_layernorm_fwd(hmid, P(m, L->n2w), P(m, L->n2b), M, d, c->norm_eps, C->n2, C->mean2, C->rstd2);
    } else {
      orc_rmsnorm_fwd(hmid, P(m, L->n2w), M, d, c->norm_eps, gemma, C->n2, C->rstd2);
    }
    const int64_t nf = M * c->d_ff;
    C->gate = F(m, nf);
    C->act = F(m, nf);
    float* hout = F(m, M * d);
    C->mo = F(m, M * d);
    if (gpt2) {
      lin_fwd(m, &L->lin[G_FC], C->n2, M, C->gate, &C->xa[G_FC], &C->xd[G_FC]);
      orc_glu_fwd(C->gate, NULL, nf, 0, C->act);
      lin_fwd(m, &L->lin[G_FC2], C->act, M, C->mo, &C->xa[G_FC2], &C->xd[G_FC2]);
    } else {
      C->up = F(m, nf);
      lin_fwd(m, &L->lin[T_GATE], C->n2, M, C->gate, &C->xa[T_GATE], &C->xd[T_GATE]);
      lin_fwd(m, &L->lin[T_UP], C->n2, M, C->up, &C->xa[T_UP], &C->xd[T_UP]);
      orc_glu_fwd(C->gate, C->up, nf, gemma ? 0 : 1, C->act);
      lin_fwd(m, &L->lin[T_DOWN], C->act, M, C->mo, &C->xa[T_DOWN], &C->xd[T_DOWN]);
    }
    if (gemma) {
      C->mrs = F(m, M);
      float* mn = F(m, M * d);
      orc_rmsnorm_fwd(C->mo, P(m, L->pfn), M, d, c->norm_eps, 1, mn, C->mrs);
      for (int64_t i = 0; i < M * d; ++i) hout[i] = hmid[i] + mn[i];
    } else {
      for (int64_t i = 0; i < M * d; ++i) hout[i] = hmid[i] + C->mo[i];
    }
    if (kp) {
      const int64_t qw = (int64_t)H * hd, kw = (int64_t)Hk * hd, ff = c->d_ff;
      keep(m, li, "x", 0, C->x, M, d, d);
      keep(m, li, "norm1", 0, C->n1, M, d, d);
      if (!gpt2) {
        keep(m, li, "q_proj", 0, gemma ? C->qraw : C->q, M, qw, qw);
        keep(m, li, "k_proj", 0, gemma ? C->kraw : C->k, M, kw, kw);
      }
      keep(m, li, "q", 0, C->q, M, qw, C->qs);
      keep(m, li, "k", 0, C->k, M, kw, C->ks);
      keep(m, li, "v", 0, C->v, M, kw, C->vs);
      keep(m, li, "attn", 0, C->att, M, qw, qw);
      keep(m, li, "o_proj", 0, C->o, M, d, d);
      keep(m, li, "mid", 0, C->hmid, M, d, d);
      keep(m, li, "norm2", 0, C->n2, M, d, d);
      keep(m, li, "gate", 0, C->gate, M, ff, ff);
      if (C->up) keep(m, li, "up", 0, C->up, M, ff, ff);
      keep(m, li, "act", 0, C->act, M, ff, ff);
      keep(m, li, "down_proj", 0, C->mo, M, d, d);
      keep(m, li, "out", 0, hout, M, d, d);
      if (C->up) {  /* the activation of gate alone */
        float* ga = (float*)xmalloc(sizeof(float) * (size_t)(M * ff));
        orc_glu_fwd(C->gate, NULL, M * ff, gemma ? 0 : 1, ga);
        keep(m, li, "gate_act", 0, ga, M, ff, ff);
        free(ga);
      }
    }
    h = hout;
  }
  float* hf = F(m, M * d);
  *frstd = F(m, M);
  *fmean = NULL;
  if (gpt2) {
    *fmean = F(m, M);
    orc_layernorm_fwd(h, P(m, m->nfw), P(m, m->nfb), M, d, c->norm_eps, hf, *fmean, *frstd);
  } else {
    orc_rmsnorm_fwd(h, P(m, m->nfw), M, d, c->norm_eps, gemma, hf, *frstd);
  }
  if (logits) {
    float* tmp;
    const float* E = wview(m, m->wte, &tmp);
    orc_sgemm(0, 1, M, c->vocab, d, 1.0f, hf, d, E, d, 0.0f, logits, c->vocab);
    free(tmp);
  }
  *hf_out = hf;
  *hlast_out = h;
}

float orc_model_forward(orc_model* m, const int32_t* ids, const float* mask,
                        const int32_t* labels, int B, int S, float* logits) {
  const int64_t M = (int64_t)B * S;
  lcache* cache = (lcache*)xmalloc(sizeof(lcache) * (size_t)m->c.n_layer);
  float *hf, *hl, *fm, *fr;
  float* lg = logits ? logits : (float*)xmalloc((size_t)(M * m->c.vocab) * 4);
  m->training = 0;  /* evaluation: no dropout */
  forward_all(m, ids, mask, B, S, cache, &hf, &hl, &fm, &fr, lg);
  double ls = 0.0;
  int64_t n = orc_ce_fwd_bwd(lg, labels, B, S, m->c.vocab, -100, 1.0f, 0, &ls, NULL, NULL);
  if (!logits) free(lg);
  free(cache);
  free_acts(m);
  return n > 0 ? (float)(ls / (double)n) : 0.0f;
}

float orc_model_fwd_bwd(orc_model* m, const int32_t* ids, const float* mask,
                        const int32_t* labels, int B, int S, float upstream) {
  const orc_model_cfg* c = &m->c;
  const int64_t M = (int64_t)B * S;
  const int d = c->d, H = c->n_head, Hk = c->n_kv_head, hd = c->head_dim;
  const int gpt2 = c->arch == ORC_GPT2, gemma = c->arch == ORC_GEMMA3;
  lcache* cache = (lcache*)xmalloc(sizeof(lcache) * (size_t)c->n_layer);
  float *hf, *hl, *fm, *fr;
  float* logits = (float*)xmalloc((size_t)(M * c->vocab) * 4);
  /* a training forward: the LoRA dropout stream advances */
  m->training = 1;
  if (c->lora_dropout > 0.0f) m->drop_step++;
  forward_all(m, ids, mask, B, S, cache, &hf, &hl, &fm, &fr, logits);
  double ls = 0.0;
  int64_t n = orc_ce_fwd_bwd(logits, labels, B, S, c->vocab, -100, upstream, 0,
                             &ls, logits /* dlogits in place */, NULL);
  float loss = n > 0 ? (float)(ls / (double)n) : 0.0f;
  /* LM head backward: dhf = dlogits·E (tied, frozen) */
  float* dhf = F(m, M * d);
  {
    float* tmp;
    const float* E = wview(m, m->wte, &tmp);
    orc_sgemm(0, 0, M, d, c->vocab, 1.0f, logits, c->vocab, E, d, 0.0f, dhf, d);
    free(tmp);
  }
  free(logits);
  float* dh = F(m, M * d);
  if (gpt2)
    orc_layernorm_bwd(dhf, hl, P(m, m->nfw), fm, fr, M, d, dh, 0);
  else
    orc_rmsnorm_bwd(dhf, hl, P(m, m->nfw), fr, M, d, gemma, dh, 0);

  const int64_t nf = M * c->d_ff;
  float* dact = F(m, nf);
  float* dgate = F(m, nf);
  float* dup = F(m, nf);
  float* dn = F(m, M * d);
  float* dtmp = F(m, M * d);
  float* datt = F(m, M * H * hd);
  float* dq = F(m, M * H * hd);
  float* dk = F(m, M * Hk * hd);
  float* dv = F(m, M * Hk * hd);
  float* dqkv = gpt2 ? F(m, M * 3 * d) : NULL;
  float* dn1 = F(m, M * d);

  for (int li = c->n_layer - 1; li >= 0; --li) {
    olayer* L = &m->L[li];
    lcache* C = &cache[li];
    const int kp = keeps(m, li);
    const int64_t qw = (int64_t)H * hd, kw = (int64_t)Hk * hd, ff = c->d_ff;
    if (kp) keep(m, li, "out", 1, dh, M, d, d);
    /* ---- MLP block: hout = hmid + [postnorm](mlp(n2)) ---- */
    const float* dmo = dh;
    if (gemma) {
      orc_rmsnorm_bwd(dh, C->mo, P(m, L->pfn), C->mrs, M, d, 1, dtmp, 0);
      dmo = dtmp;
    }
    if (kp) keep(m, li, "down_proj", 1, dmo, M, d, d);
    if (gpt2) {
      lin_bwd(m, &L->lin[G_FC2], dmo, C->act, C->xa[G_FC2], C->xd[G_FC2], M, dact);
      orc_glu_bwd(dact, C->gate, NULL, nf, 0, dgate, NULL);
      lin_bwd(m, &L->lin[G_FC], dgate, C->n2, C->xa[G_FC], C->xd[G_FC], M, dn);
      orc_layernorm_bwd(dn, C->hmid, P(m, L->n2w), C->mean2, C->rstd2, M, d, dh, 1);
    } else {
      lin_bwd(m, &L->lin[T_DOWN], dmo, C->act, C->xa[T_DOWN], C->xd[T_DOWN], M, dact);
      orc_glu_bwd(dact, C->gate, C->up, nf, gemma ? 0 : 1, dgate, dup);
      if (kp) {
        keep(m, li, "act", 1, dact, M, ff, ff);
        keep(m, li, "gate", 1, dgate, M, ff, ff);
        keep(m, li, "up", 1, dup, M, ff, ff);
        float* dga = (float*)xmalloc(sizeof(float) * (size_t)nf);  /* d(gate_act) = dact∘up */
        for (int64_t i = 0; i < nf; ++i) dga[i] = dact[i] * C->up[i];
        keep(m, li, "gate_act", 1, dga, M, ff, ff);
        free(dga);
      }
      lin_bwd(m, &L->lin[T_GATE], dgate, C->n2, C->xa[T_GATE], C->xd[T_GATE], M, dn);
      lin_bwd(m, &L->lin[T_UP], dup, C->n2, C->xa[T_UP], C->xd[T_UP], M, dtmp);
      add_into(dn, dtmp, M * d);
      if (kp) keep(m, li, "norm2", 1, dn, M, d, d);
      orc_rmsnorm_bwd(dn, C->hmid, P(m, L->n2w), C->rstd2, M, d, gemma, dh, 1);
    }
    if (kp) keep(m, li, "mid", 1, dh, M, d, d);
    /* dh now holds d(hmid).  ---- attention block ---- */
    const float* dox = dh;
    if (gemma) {
      orc_rmsnorm_bwd(dh, C->o, P(m, L->pan), C->ors, M, d, 1, dtmp, 0);
      dox = dtmp;
    }
    lin_bwd(m, gpt2 ? &L->lin[G_PROJ] : &L->lin[T_O], dox, C->att,
            C->xa[gpt2 ? G_PROJ : T_O], C->xd[gpt2 ? G_PROJ : T_O], M, datt);
    int win = layer_is_local(c, li) ? c->sliding_window : 0;
    /* nothing trainable below layer 0 (its input gradient only when retained) */
    const int need_dx = li > 0 || kp;
    if (kp) {
      keep(m, li, "o_proj", 1, dox, M, d, d);
      keep(m, li, "attn", 1, datt, M, qw, qw);
      const int64_t ns = (int64_t)B * H * S * S;
      float* dpr = (float*)xmalloc(sizeof(float) * (size_t)ns);
      float* dsc = (float*)xmalloc(sizeof(float) * (size_t)ns);
      orc_attn_probs(C->q, C->qs, C->k, C->ks, C->v, C->vs, datt, qw, B, H, Hk, S, hd, attn_scale(c), 1, win,
                     mask, NULL, NULL, dpr, dsc);
      keep(m, li, "probs", 1, dpr, 1, ns, ns);
      keep(m, li, "scores", 1, dsc, 1, ns, ns);
      free(dpr);
      free(dsc);
    }
    if (gpt2) {
      orc_attn_bwd(C->q, C->qs, C->k, C->ks, C->v, C->vs, C->att, (int64_t)H * hd,
                   datt, (int64_t)H * hd, C->lse, B, H, Hk, S, hd, attn_scale(c), 1,
                   win, mask, dqkv, 3 * d, dqkv + d, 3 * d, dqkv + 2 * d, 3 * d);
      lin_bwd(m, &L->lin[G_ATTN], dqkv, C->n1, C->xa[G_ATTN], C->xd[G_ATTN], M, need_dx ? dn1 : NULL);
      if (need_dx)
        orc_layernorm_bwd(dn1, C->x, P(m, L->n1w), C->mean1, C->rstd1, M, d, dh, 1);
    } else {
      orc_attn_bwd(C->q, C->qs, C->k, C->ks, C->v, C->vs, C->att, (int64_t)H * hd,
                   datt, (int64_t)H * hd, C->lse, B, H, Hk, S, hd, attn_scale(c), 1,
                   win, mask, dq, (int64_t)H * hd, dk, (int64_t)Hk * hd, dv,
                   (int64_t)Hk * hd);
      if (kp) {
        keep(m, li, "q", 1, dq, M, qw, qw);
        keep(m, li, "k", 1, dk, M, kw, kw);
        keep(m, li, "v", 1, dv, M, kw, kw);
      }
      double th = layer_is_local(c, li) ? c->rope_local_theta : c->rope_theta;
      orc_rope(dq, (int64_t)H * hd, B, S, H, hd, th, 1);
      orc_rope(dk, (int64_t)Hk * hd, B, S, Hk, hd, th, 1);
      if (kp && gemma) {
        keep(m, li, "q_normed", 1, dq, M, qw, qw);
        keep(m, li, "k_normed", 1, dk, M, kw, kw);
      }
      if (gemma) {
        float* t1 = F(m, M * H * hd);
        float* t2 = F(m, M * Hk * hd);
        orc_rmsnorm_bwd(dq, C->qraw, P(m, L->qn), C->qrs, M * H, hd, 1, t1, 0);
        orc_rmsnorm_bwd(dk, C->kraw, P(m, L->kn), C->krs, M * Hk, hd, 1, t2, 0);
        memcpy(dq, t1, sizeof(float) * (size_t)(M * H * hd));
        memcpy(dk, t2, sizeof(float) * (size_t)(M * Hk * hd));
      }
      if (kp) {
        keep(m, li, "q_proj", 1, dq, M, qw, qw);
        keep(m, li, "k_proj", 1, dk, M, kw, kw);
      }
      lin_bwd(m, &L->lin[T_Q], dq, C->n1, C->xa[T_Q], C->xd[T_Q], M, need_dx ? dn1 : NULL);
      lin_bwd(m, &L->lin[T_K], dk, C->n1, C->xa[T_K], C->xd[T_K], M, need_dx ? dtmp : NULL);
      if (need_dx) add_into(dn1, dtmp, M * d);
      lin_bwd(m, &L->lin[T_V], dv, C->n1, C->xa[T_V], C->xd[T_V], M, need_dx ? dtmp : NULL);
      if (need_dx) {
        add_into(dn1, dtmp, M * d);
        if (kp) keep(m, li, "norm1", 1, dn1, M, d, d);
        orc_rmsnorm_bwd(dn1, C->x, P(m, L->n1w), C->rstd1, M, d, gemma, dh, 1);
        if (kp) {
          keep(m, li, "x", 1, dh, M, d, d);
          if (li == 0) keep(m, -1, "embed", 1, dh, M, d, d);
        }
      }
    }
  }
  free(cache);
  free_acts(m);
  return loss;
}

float orc_model_opt_step(orc_model* m, float lr, float b1, float b2, float eps,
                         float wd, float clip) {
  double ss = 0.0;
  for (int i = 0; i < m->np; ++i)
    if (m->p[i].trainable) ss += orc_sumsq(m->p[i].grad, m->p[i].numel);
  float norm;
  float sc = orc_clip_scale(ss, clip, &norm);
  m->t++;
  for (int i = 0; i < m->np; ++i) {
    oparam* p = &m->p[i];
    if (!p->trainable) continue;
    if (sc != 1.0f)
      for (int64_t j = 0; j < p->numel; ++j) p->grad[j] *= sc;
    orc_adam_step((float*)p->data, p->grad, p->m, p->v, p->numel, lr, b1, b2, eps, wd, m->t);
    memset(p->grad, 0, sizeof(float) * (size_t)p->numel);
  }
  return norm;
}
