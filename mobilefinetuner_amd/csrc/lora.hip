// lora.hip — LoRA-linear forward/backward composed from the GEMM and the
// rank-r kernels.
//
// Forward:  xa = x·Aᵀ (skinny, one pass over x), then one GEMM
//           y = x·W + bias + scale·xa·Bᵀ (+ resid) with the rank-r term and
//           the residual applied in the GEMM epilogue — no extra pass over y.
// Backward: U = dy·B (skinny), dx = dy·Wᵀ + scale·U·A in one GEMM (rank-r
//           term in the epilogue), dA (+)= scale·Uᵀ·x and dB (+)= scale·dyᵀ·xa
//           as split-M reductions with a fixed summation order
//           (deterministic, no atomics).
#include <algorithm>

#include "common.h"

namespace mft {

size_t lora_bwd_scratch_floats(int64_t M, int64_t K, int64_t N, int r) {
  const int64_t c = K > N ? K : N;
  return (size_t)(M * r + 16 * r * c);
}

void lora_linear_fwd(hipStream_t s, const float* x, int64_t M, int64_t K,
                     const void* W, bool w_f16, int64_t N, const float* bias,
                     const float* A, const float* B, int r, float scale,
                     float* y, float* xa, const float* resid, Scratch ws,
                     const KernelEvents* ev) {
  MFT_CHECK_ARG(x && W && y, "null tensor");
  GemmEpilogue ep;
  ep.bias = bias;
  ep.resid = resid;
  if (A && B && r > 0) {
    MFT_CHECK_ARG(xa != nullptr, "xa buffer required when LoRA is active");
    rank_proj(s, x, K, A, /*ysk=*/1, /*ysj=*/K, (int)M, (int)K, r, xa);
    ep.P = xa;
    ep.Q = B;
    ep.r = r;
    ep.qsn = r;
    ep.qsj = 1;
    ep.lscale = scale;
  }
  if (!(w_f16 && gemm_f16w(s, x, K, W, N, /*b_nk=*/false, y, N, (int)M, (int)N, (int)K, ep, ws, ev)))
    gemm(s, x, K, W, N, /*b_nk=*/false, w_f16, y, N, (int)M, (int)N, (int)K, ep, ws, ev);
}

void lora_linear_bwd(hipStream_t s, const float* dy, const float* x,
                     const void* W, bool w_f16, const float* A, const float* B,
                     const float* xa, int64_t M, int64_t K, int64_t N, int r,
                     float scale, float* dx, float* dA, float* dB,
                     bool accumulate, bool dx_accumulate, Scratch ws,
                     const KernelEvents* ev) {
  MFT_CHECK_ARG(dy && W, "null tensor");
  const bool lora = A && B && r > 0;
  float* U = nullptr;
  Scratch rest = ws;
  if (lora) {
    MFT_CHECK_ARG(x && xa, "x and xa required for LoRA grads");
    MFT_CHECK_ARG(ws.ptr && ws.bytes >= (size_t)(M * r) * sizeof(float), "scratch too small for U");
    U = ws.ptr;
    rest = ws.offset((size_t)(M * r));
    rank_proj(s, dy, N, B, /*ysk=*/r, /*ysj=*/1, (int)M, (int)N, r, U);
  }
  if (dx) {
    GemmEpilogue ep;
    ep.beta = dx_accumulate ? 1.f : 0.f;
    if (lora) {
      ep.P = U;
      ep.Q = A;  // Q(n=k, j) = A[j, k]
      ep.r = r;
      ep.qsn = 1;
      ep.qsj = K;
      ep.lscale = scale;
    }
    // dx[M,K] = dy[M,N] · Wᵀ: W [K,N] is the [N_out=K, K_red=N] operand.
    if (!(w_f16 && gemm_f16w(s, dy, N, W, N, /*b_nk=*/true, dx, K, (int)M, (int)K, (int)N, ep, rest, ev)))
      gemm(s, dy, N, W, N, /*b_nk=*/true, w_f16, dx, K, (int)M, (int)K, (int)N, ep, rest, ev);
  }
  if (lora) {
    // dA(j,k) = s·Σ_m U[m,j]·x[m,k] → dA[j*K + k];  dB(n,j) = s·Σ_m xa[m,j]·dy[m,n] → dB[n*r + j]
    if (dA && dB)
      rank_outer_pair(s, (int)M, r, scale, accumulate, U, x, K, (int)K, dA, K, 1, xa, dy, N, (int)N, dB, 1, r);
    else if (dA)
      rank_outer(s, U, x, K, (int)M, (int)K, r, scale, dA, /*osj=*/K, /*osc=*/1, accumulate, rest);
    else if (dB)
      rank_outer(s, xa, dy, N, (int)M, (int)N, r, scale, dB, /*osj=*/1, /*osc=*/r, accumulate, rest);
  }
}

// ---- LoRA dropout (PEFT's lora_dropout on the LoRA branch input) ------------
// keep(idx) of stream `lid` in training forward `step`: the top 24 bits of
// mix64(mix64(seed ^ step<<20 ^ lid) + idx) are >= threshold, with
// threshold = floor(p·2^24) and mix64 the splitmix64 output function;
// idx = row·K + column within one forward's [M, K] input.  A launch over
// n_fwd micro-batch forwards at once (rows_per_fwd rows each) gives forward
// j the step *step - n_fwd + 1 + j, as if each micro-batch ran its own
// forward.  The backward regenerates the forward's mask from the same
// counter (the step is a device scalar, so a captured graph advances it on
// every replay).
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct DropArgs {
  uint32_t thr;
  float inv;
  uint64_t seed;
  const int* step;
  int n_fwd;
  int64_t rows_per_fwd;
  int lid;
};

DropArgs drop_args(const DropStream& d, int lid) {
  MFT_CHECK_ARG(d.p > 0.f && d.p < 1.f, "dropout probability must lie in (0, 1)");
  MFT_CHECK_ARG(d.n_fwd > 0 && d.rows_per_fwd > 0, "empty dropout stream");
  return DropArgs{dropout_threshold(d.p), 1.f / (1.f - d.p), d.seed, d.step, d.n_fwd, d.rows_per_fwd, lid};
}

// keep decision of row m, column k of a [M, K] input
__device__ __forceinline__ bool drop_keep(const DropArgs& a, int step0, int64_t m, int64_t k, int64_t K) {
  const int64_t j = m / a.rows_per_fwd;
  const uint32_t step = (uint32_t)(step0 - a.n_fwd + 1 + (int)j);
  const uint64_t key = mix64(a.seed ^ ((uint64_t)step << 20) ^ (uint64_t)(uint32_t)a.lid);
  const uint64_t idx = (uint64_t)((m - j * a.rows_per_fwd) * K + k);
  return (uint32_t)(mix64(key + idx) >> 40) >= a.thr;
}

__global__ void dropout_step_kernel(int* step, int n) {
  if (threadIdx.x == 0) *step += n;
}

__global__ void dropout_apply_kernel(const float* __restrict__ x, int64_t ldx, int64_t M, int64_t K, DropArgs a,
                                     float* __restrict__ xd) {
  const int step0 = *a.step;
  const int64_t n = M * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / K, k = i % K;
    xd[i] = drop_keep(a, step0, m, k, K) ? x[m * ldx + k] * a.inv : 0.f;
  }
}

// dx[m,k] += scale·mask(m,k)·Σ_j U[m,j]·A[j,k]
__global__ void dropout_dx_kernel(float* __restrict__ dx, int64_t M, int64_t K, const float* __restrict__ U,
                                  const float* __restrict__ A, int r, float scale, DropArgs a) {
  const int step0 = *a.step;
  const int64_t n = M * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / K, k = i % K;
    if (!drop_keep(a, step0, m, k, K)) continue;
    float t = 0.f;
    for (int j = 0; j < r; ++j) t = fmaf(U[m * r + j], A[(int64_t)j * K + k], t);
    dx[i] += scale * a.inv * t;
  }
}

__global__ void gelu_grad_scale_kernel(float* __restrict__ x, const float* __restrict__ pre, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    x[i] *= gelu_tanh_grad(pre[i]);
}

unsigned elem_grid(int64_t n) { return (unsigned)std::min<int64_t>(cdiv(n, 256), 8192); }

}  // namespace

uint32_t dropout_threshold(float p) { return (uint32_t)((double)p * 16777216.0); }

void dropout_step(hipStream_t s, int* step, int n) {
  hipLaunchKernelGGL(dropout_step_kernel, dim3(1), dim3(64), 0, s, step, n);
  MFT_LAUNCH_CHECK();
}

void dropout_apply(hipStream_t s, const float* x, int64_t ldx, int64_t M, int64_t K, const DropStream& d, int lid,
                   float* xd) {
  const DropArgs a = drop_args(d, lid);
  hipLaunchKernelGGL(dropout_apply_kernel, dim3(elem_grid(M * K)), dim3(256), 0, s, x, ldx, M, K, a, xd);
  MFT_LAUNCH_CHECK();
}

void dropout_dx(hipStream_t s, float* dx, int64_t M, int64_t K, const float* U, const float* A, int r, float scale,
                const DropStream& d, int lid) {
  const DropArgs a = drop_args(d, lid);
  hipLaunchKernelGGL(dropout_dx_kernel, dim3(elem_grid(M * K)), dim3(256), 0, s, dx, M, K, U, A, r, scale, a);
  MFT_LAUNCH_CHECK();
}

void gelu_grad_scale(hipStream_t s, float* x, const float* pre, int64_t n) {
  hipLaunchKernelGGL(gelu_grad_scale_kernel, dim3(elem_grid(n)), dim3(256), 0, s, x, pre, n);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
