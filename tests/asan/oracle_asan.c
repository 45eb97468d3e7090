/* Runs every CPU-oracle entry point once on small ragged shapes, built with
 * AddressSanitizer + UndefinedBehaviorSanitizer (tests/test_oracle_asan.py).
 * Buffers are allocated at their exact sizes, so any read or write past a
 * tensor the oracle is handed is reported.  Exit status 0 = clean. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/oracle.h"

static uint64_t rs = 88172645463325252ull;
static float rnd(void) {
  rs ^= rs << 13;
  rs ^= rs >> 7;
  rs ^= rs << 17;
  return (float)((rs >> 40) & 0xFFFFFF) / 16777216.0f - 0.5f;
}
static float* vec(int64_t n) {
  float* p = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  for (int64_t i = 0; i < n; ++i) p[i] = rnd();
  return p;
}
static float* zeros(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

static int finite_all(const float* p, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (!isfinite(p[i])) return 0;
  return 1;
}
#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                               \
    }                                                         \
  } while (0)

static int ops(void) {
  orc_set_blas(0);
  /* LoRA linear, ragged M, K, N, r */
  const int64_t M = 7, K = 13, N = 11;
  const int r = 3;
  float *x = vec(M * K), *W = vec(K * N), *bias = vec(N), *A = vec(r * K), *B = vec(N * r);
  float *y = zeros(M * N), *xa = zeros(M * r), *dy = vec(M * N), *dx = zeros(M * K), *dA = zeros(r * K),
        *dB = zeros(N * r);
  orc_lora_linear_fwd(x, M, K, W, N, bias, A, B, r, 2.f, y, xa);
  orc_lora_linear_bwd(dy, x, W, A, B, xa, M, K, N, r, 2.f, dx, dA, dB, 1);
  CHECK(finite_all(y, M * N) && finite_all(dx, M * K) && finite_all(dA, r * K) && finite_all(dB, N * r));
  free(x); free(W); free(bias); free(A); free(B); free(y); free(xa); free(dy); free(dx); free(dA); free(dB);

  /* attention: GQA, causal + window + key padding, padded row strides */
  const int Bb = 2, Hq = 4, Hkv = 2, S = 9, hd = 8;
  const int64_t qrs = Hq * hd + 3, krs = Hkv * hd + 1, vrs = Hkv * hd + 2, ors = Hq * hd + 5;
  float *q = vec(Bb * S * qrs), *k = vec(Bb * S * krs), *v = vec(Bb * S * vrs), *o = zeros(Bb * S * ors),
        *lse = zeros(Bb * Hq * S), *dout = vec(Bb * S * ors), *dq = zeros(Bb * S * qrs), *dk = zeros(Bb * S * krs),
        *dv = zeros(Bb * S * vrs), *kpad = zeros(Bb * S);
  for (int i = 0; i < Bb * S; ++i) kpad[i] = (i % S) < S - 2 ? 1.f : 0.f;
  orc_attn_fwd(q, qrs, k, krs, v, vrs, Bb, Hq, Hkv, S, hd, 0.35f, 1, 4, kpad, o, ors, lse);
  orc_attn_bwd(q, qrs, k, krs, v, vrs, o, ors, dout, ors, lse, Bb, Hq, Hkv, S, hd, 0.35f, 1, 4, kpad, dq, qrs, dk,
               krs, dv, vrs);
  CHECK(finite_all(dq, Bb * S * qrs) && finite_all(dk, Bb * S * krs) && finite_all(dv, Bb * S * vrs));
  free(q); free(k); free(v); free(o); free(lse); free(dout); free(dq); free(dk); free(dv); free(kpad);

  /* shifted CE: odd vocabulary, ignore_index, an out-of-range label */
  const int CB = 2, CS = 5;
  const int64_t V = 37;
  float* logits = vec(CB * CS * V);
  float* row_nll = zeros(CB * CS);
  int32_t labels[10] = {1, 5, -100, 36, 2, 0, 40, 7, 3, 9};
  double loss = 0.0;
  const int64_t nv = orc_ce_fwd_bwd(logits, labels, CB, CS, V, -100, 1.f, 0, &loss, logits, row_nll);
  CHECK(nv > 0 && isfinite(loss) && finite_all(logits, CB * CS * V));
  free(logits); free(row_nll);

  /* optimizer */
  const int64_t n = 29;
  float *p = vec(n), *g = vec(n), *m = zeros(n), *vv = zeros(n);
  const double ss = orc_sumsq(g, n);
  float norm = 0.f;
  const float sc = orc_clip_scale(ss, 0.1f, &norm);
  CHECK(sc > 0.f && sc <= 1.f);
  for (int t = 1; t <= 3; ++t) orc_adam_step(p, g, m, vv, n, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, t);
  CHECK(finite_all(p, n));
  free(p); free(g); free(m); free(vv);

  /* norms, GLU, RoPE, embedding, fp16, dropout */
  const int64_t NM = 5, NC = 12;
  float *nx = vec(NM * NC), *ng = vec(NC), *nb = vec(NC), *ny = zeros(NM * NC), *mean = zeros(NM), *rstd = zeros(NM),
        *ndy = vec(NM * NC), *ndx = zeros(NM * NC);
  orc_layernorm_fwd(nx, ng, nb, NM, NC, 1e-5f, ny, mean, rstd);
  orc_layernorm_bwd(ndy, nx, ng, mean, rstd, NM, NC, ndx, 0);
  orc_rmsnorm_fwd(nx, ng, NM, NC, 1e-6f, 1, ny, rstd);
  orc_rmsnorm_bwd(ndy, nx, ng, rstd, NM, NC, 1, ndx, 1);
  CHECK(finite_all(ndx, NM * NC));
  float *gate = vec(NM * NC), *up = vec(NM * NC), *go = zeros(NM * NC), *dgate = zeros(NM * NC), *dup = zeros(NM * NC);
  for (int act = 0; act < 2; ++act) {
    orc_glu_fwd(gate, up, NM * NC, act, go);
    orc_glu_bwd(ndy, gate, up, NM * NC, act, dgate, dup);
  }
  orc_glu_fwd(gate, NULL, NM * NC, 0, go);
  float* rx = vec(2 * 3 * (2 * 8 + 5)); /* [B·S rows, stride 21] */
  orc_rope(rx, 2 * 8 + 5, 2, 3, 2, 8, 10000.0, 0);
  orc_rope(rx, 2 * 8 + 5, 2, 3, 2, 8, 10000.0, 1);
  int32_t ids[6] = {0, 4, 2, 9, 1, 3};
  float *wte = vec(10 * NC), *wpe = vec(3 * NC), *h = zeros(6 * NC);
  orc_embed(ids, 6, 3, wte, NULL, wpe, NC, 1.f, h);
  uint16_t* hb = (uint16_t*)malloc(10 * NC * sizeof(uint16_t));
  orc_f32_to_f16(wte, hb, 10 * NC);
  orc_f16_to_f32(hb, wte, 10 * NC);
  orc_embed(ids, 6, 3, NULL, hb, NULL, NC, 2.f, h);
  CHECK(finite_all(h, 6 * NC));
  float* mask = zeros(101);
  orc_dropout_mask(7, 3, 9, 101, 0.25f, mask);
  free(nx); free(ng); free(nb); free(ny); free(mean); free(rstd); free(ndy); free(ndx); free(gate); free(up);
  free(go); free(dgate); free(dup); free(rx); free(wte); free(wpe); free(h); free(hb); free(mask);
  return 0;
}

/* One model step per architecture with every parameter randomised. */
static int model(int arch) {
  orc_model_cfg c;
  memset(&c, 0, sizeof c);
  c.arch = arch;
  c.n_layer = 2;
  c.d = 32;
  c.n_head = 4;
  c.n_kv_head = arch == ORC_GPT2 ? 4 : 2;
  c.head_dim = 8;
  c.d_ff = 48;
  c.max_pos = 16;
  c.vocab = 53;
  c.lora_r = 4;
  c.lora_alpha = 8.f;
  c.lora_mask = arch == ORC_GPT2 ? 0xF : 0x7F;
  c.norm_eps = 1e-5f;
  c.rope_theta = 10000.0;
  c.rope_local_theta = 10000.0;
  c.sliding_pattern = arch == ORC_GEMMA3 ? 2 : 0;
  c.sliding_window = arch == ORC_GEMMA3 ? 5 : 0;
  c.w_fp16 = arch == ORC_GEMMA3;
  c.lora_dropout = 0.1f;
  c.dropout_seed = 11;
  orc_model* m = orc_model_create(&c);
  CHECK(m != NULL);
  for (int i = 0; i < orc_model_num_params(m); ++i) {
    const char* name;
    int ndim, tr, f16;
    int64_t dims[2];
    const int64_t cnt = orc_model_param_info(m, i, &name, &ndim, dims, &tr, &f16);
    void* d = orc_model_param_data(m, i);
    for (int64_t j = 0; j < cnt; ++j) {
      const float val = 0.1f * rnd();
      if (f16) ((uint16_t*)d)[j] = orc_float_to_half_bits(val);
      else ((float*)d)[j] = val;
    }
  }
  const int B = 2, S = 7;
  int32_t ids[14], labels[14];
  float mask[14];
  for (int i = 0; i < B * S; ++i) {
    ids[i] = (int32_t)((i * 17 + 3) % c.vocab);
    labels[i] = i == 4 ? -100 : ids[i];
    mask[i] = i % S == S - 1 ? 0.f : 1.f;
  }
  const float l0 = orc_model_fwd_bwd(m, ids, mask, labels, B, S, 0.5f);
  const float l1 = orc_model_fwd_bwd(m, ids, NULL, labels, B, S, 0.5f);
  orc_model_opt_step(m, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.f, 1.f);
  float* logits = zeros((int64_t)B * S * c.vocab);
  const float l2 = orc_model_forward(m, ids, NULL, labels, B, S, logits);
  CHECK(isfinite(l0) && isfinite(l1) && isfinite(l2) && finite_all(logits, (int64_t)B * S * c.vocab));
  free(logits);
  orc_model_destroy(m);
  return 0;
}

int main(void) {
  if (ops()) return 1;
  for (int arch = 0; arch < 3; ++arch)
    if (model(arch)) return 1;
  printf("oracle under ASan/UBSan: clean\n");
  return 0;
}
