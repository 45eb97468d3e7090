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

}  // namespace mft
