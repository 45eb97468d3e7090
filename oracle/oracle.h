/*
 * oracle.h — CPU restatement of MobileFineTuner's LoRA training hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * step engine, bench.py's GPU leg) links, loads or calls this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker / the timed CPU port.
 *
 * The reference's own `operators/finetune_ops` library is not part of the
 * published tree (every driver pulls it from ../operators, e.g.
 * gpt2_small_lora_finetune/CMakeLists.txt:9-10), so each function restates
 * the semantics that the drivers and their PyTorch mirrors fix; each cites
 * the reference lines it follows.  Where those lines leave a choice open the
 * comment says which choice is taken.
 *
 * Parity pins (tests/test_oracle_*.py): every function here is checked
 * against an independent formulation (fp64 torch autograd of the forward
 * definition, central finite differences, closed forms, exhaustive fp16
 * enumeration, HF transformers model classes for the model graphs).
 *
 * Layout conventions (all row-major, fp32 unless noted):
 *   linear weight W   [K, N]   (in, out)   gpt2_small_lora_finetune/src/main.cpp:211-214
 *   LoRA A            [r, K],  LoRA B [N, r]  (PEFT layout, README.md:282,296)
 *   activations       [M, C]   with M = B*S tokens, token-major
 *   q/k/v             token-major [B, S, H, hd] with an explicit row stride
 *                     (elements between consecutive tokens)
 *   lse               [B, H, S]
 */
#ifndef MFT_ORACLE_H
#define MFT_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- BLAS plumbing (used by the CPU-baseline timing) ------------------- */
/* use_blas=0 → built-in loops with fp64 accumulation (parity default);
 * use_blas=1 → dlopen'd cblas_sgemm (MKL, then OpenBLAS), the analogue of the
 * reference's -DUSE_BLAS=ON build (README.md:64,68-73). */
int         orc_set_blas(int use_blas);
const char* orc_blas_backend(void);
void        orc_set_threads(int n);
int         orc_get_threads(void);
/* C[M,N] = alpha*op(A)*op(B) + beta*C; op(A) is [M,K], op(B) is [K,N]. */
void orc_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K,
               float alpha, const float* A, int64_t lda, const float* B,
               int64_t ldb, float beta, float* C, int64_t ldc);

/* ---- a1/a2 LoRA linear ------------------------------------------------- */
void orc_lora_linear_fwd(const float* x, int64_t M, int64_t K, const float* W,
                         int64_t N, const float* bias, const float* A,
                         const float* B, int r, float scale, float* y,
                         float* xa);
void orc_lora_linear_bwd(const float* dy, const float* x, const float* W,
                         const float* A, const float* B, const float* xa,
                         int64_t M, int64_t K, int64_t N, int r, float scale,
                         float* dx, float* dA, float* dB, int accumulate);

/* ---- a7 fp16 storage --------------------------------------------------- */
void  orc_f16_to_f32(const uint16_t* src, float* dst, int64_t n);
void  orc_f32_to_f16(const float* src, uint16_t* dst, int64_t n); /* RNE */
float orc_half_bits_to_float(uint16_t h);
uint16_t orc_float_to_half_bits(float f);

/* ---- a3/a4 attention --------------------------------------------------- */
void orc_attn_fwd(const float* q, int64_t q_rs, const float* k, int64_t k_rs,
                  const float* v, int64_t v_rs, int B, int Hq, int Hkv, int S,
                  int hd, float scale, int causal, int window,
                  const float* kpad, float* o, int64_t o_rs, float* lse);
void orc_attn_bwd(const float* q, int64_t q_rs, const float* k, int64_t k_rs,
                  const float* v, int64_t v_rs, const float* o, int64_t o_rs,
                  const float* dout, int64_t do_rs, const float* lse, int B,
                  int Hq, int Hkv, int S, int hd, float scale, int causal,
                  int window, const float* kpad, float* dq, int64_t dq_rs, float* dk,
                  int64_t dk_rs, float* dv, int64_t dv_rs);

/* ---- a5/a6 shifted LM cross-entropy ------------------------------------ */
/* Returns number of valid targets; loss_sum (fp64) = Σ NLL over them.
 * dlogits (nullable, may alias logits) = (softmax-onehot)*upstream/n_valid,
 * where n_valid is `norm_count` when >0, else the count found here.
 * row_nll (nullable) [B*S]: NLL per row, 0 for ignored/last rows. */
int64_t orc_ce_fwd_bwd(const float* logits, const int32_t* labels, int B,
                       int S, int64_t V, int ignore_index, float upstream,
                       int64_t norm_count, double* loss_sum, float* dlogits,
                       float* row_nll);

/* ---- a8/a9 optimizer + clip ------------------------------------------- */
void   orc_adam_step(float* p, const float* g, float* m, float* v, int64_t n,
                     float lr, float b1, float b2, float eps, float wd, int t);
double orc_sumsq(const float* g, int64_t n);
float  orc_clip_scale(double sumsq, float max_norm, float* norm_out);

/* ---- a10 support ops --------------------------------------------------- */
void orc_layernorm_fwd(const float* x, const float* g, const float* b,
                       int64_t M, int64_t C, float eps, float* y, float* mean,
                       float* rstd);
void orc_layernorm_bwd(const float* dy, const float* x, const float* g,
                       const float* mean, const float* rstd, int64_t M,
                       int64_t C, float* dx, int accumulate);
/* unit_offset=1 → Gemma3 form x*rstd*(1+w); 0 → Qwen2/Llama form x*rstd*w */
void orc_rmsnorm_fwd(const float* x, const float* w, int64_t M, int64_t C,
                     float eps, int unit_offset, float* y, float* rstd);
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* w,
                     const float* rstd, int64_t M, int64_t C, int unit_offset,
                     float* dx, int accumulate);
float orc_gelu_tanh(float x);
float orc_gelu_tanh_grad(float x);
float orc_silu(float x);
float orc_silu_grad(float x);
/* act: 0 = gelu_tanh, 1 = silu.  out = act(gate)*up (GeGLU / SwiGLU); when
 * up == NULL, out = act(gate) (GPT-2 MLP). */
void orc_glu_fwd(const float* gate, const float* up, int64_t n, int act,
                 float* out);
void orc_glu_bwd(const float* dout, const float* gate, const float* up,
                 int64_t n, int act, float* dgate, float* dup);
/* HF rotate_half RoPE over [B,S,H,hd] (row stride rs), position = s. */
void orc_rope(float* x, int64_t rs, int B, int S, int H, int hd, double theta,
              int inverse);
void orc_embed(const int32_t* ids, int64_t M, int S, const float* wte,
               const uint16_t* wte_f16, const float* wpe, int64_t C,
               float scale, float* h);

/* ---- LoRA dropout mask ----------------------------------------------------
 * PEFT's lora_dropout on the LoRA branch input: xd = x∘keep/(1−p).  keep of
 * element idx (= row·K + column) of LoRA linear `lid` (= layer·8 + target)
 * in the `step`-th training forward: the top 24 bits of
 * mix64(mix64(seed ^ step<<20 ^ lid) + idx) are ≥ ⌊p·2^24⌋, where mix64 is
 * the splitmix64 output function (Steele, Lea, Flood 2014; constants of
 * Vigna's reference).  The reference's own RNG is not in the published tree;
 * this counter-based form lets the backward regenerate the forward's mask.
 * mask[i] = 1/(1−p) where kept, 0 elsewhere. */
void orc_dropout_mask(uint64_t seed, uint32_t step, uint32_t lid, int64_t n,
                      float p, float* mask);

/* ---- model-level step (GPT-2 / Qwen2 / Gemma3 LoRA) --------------------- */
enum { ORC_GPT2 = 0, ORC_QWEN2 = 1, ORC_GEMMA3 = 2 };
typedef struct {
  int arch, n_layer, d, n_head, n_kv_head, head_dim, d_ff, max_pos;
  int64_t vocab;
  int lora_r;
  float lora_alpha;
  int lora_mask;   /* bit i → target i in the arch's target list */
  float norm_eps;
  double rope_theta, rope_local_theta;
  int sliding_pattern; /* Gemma3: every n-th layer global; 0 = all global */
  int sliding_window;  /* Gemma3 local layers: key window; 0 = none */
  float attn_scale;    /* 0 → 1/sqrt(head_dim) */
  int w_fp16;          /* frozen linear + embedding weights stored fp16 */
  float lora_dropout;  /* LoRA input dropout in training forwards (0 = off) */
  uint64_t dropout_seed;
} orc_model_cfg;

/* Scores / probabilities of one attention and their gradients in closed
 * form, [B, Hq, S, S] each (NULL outputs skipped; dout NULL: no gradients). */
void orc_attn_probs(const float* q, int64_t q_rs, const float* k, int64_t k_rs,
                    const float* v, int64_t v_rs, const float* dout, int64_t do_rs,
                    int B, int Hq, int Hkv, int S, int hd, float scale, int causal,
                    int window, const float* kpad, float* scores, float* probs,
                    float* dprobs, float* dscores);
typedef struct orc_model orc_model;
orc_model* orc_model_create(const orc_model_cfg* cfg);
void       orc_model_destroy(orc_model* m);
int        orc_model_num_params(const orc_model* m);
/* name/shape/trainable of param i; returns numel.  dims has room for 2. */
int64_t    orc_model_param_info(const orc_model* m, int i, const char** name,
                                int* ndim, int64_t* dims, int* trainable,
                                int* is_f16);
void*      orc_model_param_data(orc_model* m, int i);
float*     orc_model_param_grad(orc_model* m, int i);
/* One micro-batch forward + CE + backward; grads accumulate.  Returns the
 * micro-batch mean loss.  upstream = 1/accum (loss scaling, main.cpp:480-485).
 * A training forward: with lora_dropout > 0 it advances the dropout step and
 * drops LoRA inputs (orc_dropout_mask); orc_model_forward never does. */
float orc_model_fwd_bwd(orc_model* m, const int32_t* ids, const float* mask,
                        const int32_t* labels, int B, int S, float upstream);
/* Forward only; writes logits [B*S, V] when logits != NULL; returns loss. */
float orc_model_forward(orc_model* m, const int32_t* ids, const float* mask,
                        const int32_t* labels, int B, int S, float* logits);
/* Retained intermediates (the Gemma driver's alignment dump,
 * gemma_3_270m_lora_finetune/src/main.cpp:547-657): with bit l of layer_mask
 * set, later forwards keep layer l's activations and backwards its
 * activation gradients, until the next forward.  Names per layer: "x",
 * "norm1", "q_proj", "k_proj", "v", "q_normed", "k_normed" (after the q/k
 * norms, before RoPE), "q", "k" (after RoPE), "attn", "o_proj", "mid",
 * "norm2", "gate", "up", "gate_act", "act", "down_proj", "out" — token-major
 * [B·S, width] — and "scores", "probs" [B, Hq, S, S]; layer −1: "embed".
 * orc_model_retained returns the kept buffer (NULL if absent) and its size. */
void orc_model_set_retain(orc_model* m, uint64_t layer_mask);
const float* orc_model_retained(const orc_model* m, int layer, const char* name, int grad, int64_t* n);
/* clip + Adam on the LoRA params, then zero grads (main.cpp:489-505). */
float orc_model_opt_step(orc_model* m, float lr, float b1, float b2, float eps,
                         float wd, float clip);

#ifdef __cplusplus
}
#endif
#endif
