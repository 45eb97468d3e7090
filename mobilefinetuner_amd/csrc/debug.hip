// debug.hip — kernels of the alignment-dump debug mode only (the retained
// intermediates of gemma_3_270m_lora_finetune/src/main.cpp:547-657), never
// on the training path: dense attention scores / probabilities and their
// gradients for the layers being dumped, an elementwise product and a GELU.
// Plain one-thread-per-element code: the debug mode runs once on one batch.
#include <cfloat>

#include "common.h"

namespace mft {
namespace {

// Thread (row, j), row = (b·Hq + h)·S + i: scores = scale·q_i·k_j
// (−FLT_MAX where masked: causal, window, key padding), probs = exp(scores −
// lse) from the forward's log-sum-exp (0 where masked), and with dout:
// dprobs = dO_i·v_j, dscores = probs·(dprobs − Σ_d dO_i·O_i).
__global__ __launch_bounds__(256) void dbg_attn_kernel(DebugAttn a) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int64_t row = blockIdx.y;
  if (j >= a.S) return;
  const int i = (int)(row % a.S);
  const int h = (int)((row / a.S) % a.Hq);
  const int b = (int)(row / ((int64_t)a.S * a.Hq));
  const int kh = h / (a.Hq / a.Hkv);
  const float* qi = a.q + ((int64_t)b * a.S + i) * a.q_rs + (int64_t)h * a.hd;
  const float* kj = a.k + ((int64_t)b * a.S + j) * a.k_rs + (int64_t)kh * a.hd;
  bool ok = (!a.causal || j <= i) && (a.window <= 0 || i - j < a.window);
  if (a.kpad) ok = ok && a.kpad[(int64_t)b * a.S + j] > 0.5f;
  const float lse = a.lse[row];
  ok = ok && lse > -INFINITY;
  float s = 0.f;
  for (int d = 0; d < a.hd; ++d) s = fmaf(qi[d], kj[d], s);
  s *= a.scale;
  const float p = ok ? expf(s - lse) : 0.f;
  const int64_t at = row * a.S + j;
  if (a.scores) a.scores[at] = ok ? s : -FLT_MAX;
  if (a.probs) a.probs[at] = p;
  if (!a.dout) return;
  const float* gi = a.dout + ((int64_t)b * a.S + i) * a.do_rs + (int64_t)h * a.hd;
  const float* oi = a.o + ((int64_t)b * a.S + i) * a.o_rs + (int64_t)h * a.hd;
  const float* vj = a.v + ((int64_t)b * a.S + j) * a.v_rs + (int64_t)kh * a.hd;
  float dp = 0.f, delta = 0.f;
  for (int d = 0; d < a.hd; ++d) {
    dp = fmaf(gi[d], vj[d], dp);
    delta = fmaf(gi[d], oi[d], delta);
  }
  if (a.dprobs) a.dprobs[at] = dp;
  if (a.dscores) a.dscores[at] = p * (dp - delta);
}

__global__ __launch_bounds__(256) void dbg_mul_kernel(const float* a, int64_t lda, const float* b, int64_t ldb,
                                                      float* out, int64_t ldo, int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / cols, c = e % cols;
    out[r * ldo + c] = a[r * lda + c] * b[r * ldb + c];
  }
}

__global__ __launch_bounds__(256) void dbg_gelu_kernel(const float* x, int64_t ldx, float* out, int64_t ldo,
                                                       int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / cols, c = e % cols;
    out[r * ldo + c] = gelu_tanh(x[r * ldx + c]);
  }
}

unsigned grid_of(int64_t n) { return (unsigned)std::min<int64_t>(cdiv(n, 256), 8192); }

}  // namespace

void debug_attn(hipStream_t s, const DebugAttn& a) {
  MFT_CHECK_ARG(a.q && a.k && a.lse && a.S > 0 && a.Hq > 0 && a.Hkv > 0 && a.Hq % a.Hkv == 0, "debug_attn");
  MFT_CHECK_ARG(!a.dout || (a.v && a.o), "debug_attn: gradients need v and o");
  hipLaunchKernelGGL(dbg_attn_kernel, dim3((unsigned)cdiv(a.S, 256), (unsigned)((int64_t)a.B * a.Hq * a.S)),
                     dim3(256), 0, s, a);
  MFT_LAUNCH_CHECK();
}

void debug_mul(hipStream_t s, const float* a, int64_t lda, const float* b, int64_t ldb, float* out, int64_t ldo,
               int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(dbg_mul_kernel, dim3(grid_of(rows * cols)), dim3(256), 0, s, a, lda, b, ldb, out, ldo, rows,
                     cols);
  MFT_LAUNCH_CHECK();
}

void debug_gelu(hipStream_t s, const float* x, int64_t ldx, float* out, int64_t ldo, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(dbg_gelu_kernel, dim3(grid_of(rows * cols)), dim3(256), 0, s, x, ldx, out, ldo, rows, cols);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
