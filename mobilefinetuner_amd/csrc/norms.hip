// norms.hip — LayerNorm / RMSNorm forward and backward with the row held in
// registers: one wave64 per row, each lane loads NV 128-bit chunks up front
// (all loads in flight at once), reduces with shuffles and writes once.
// HBM traffic is the algorithmic minimum (fwd: read x, write y; bwd: read
// dy and x, write/accumulate dx).  Rows wider than 2048, C % 4 != 0 or
// unaligned rows go to the row-loop kernels in elementwise.hip.
// The same row code also finishes split-K GEMM outputs (splitk_norm_vec):
// the norm whose input is a linear layer's output then runs inside that
// GEMM's reduction pass.
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace mft {
namespace {

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int NV>
__device__ __forceinline__ void load_row(const float* __restrict__ base, int C4, int lane,
                                         floatx4 (&v)[NV]) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = lane + 64 * i;
    v[i] = q < C4 ? reinterpret_cast<const floatx4*>(base)[q] : floatx4{0.f, 0.f, 0.f, 0.f};
  }
}

// ---- the four norms on a row held in registers (lane owns chunks lane+64i) --
template <int NV>
__device__ __forceinline__ void ln_fwd_row(const floatx4 (&v)[NV], int C, int lane, const float* __restrict__ g,
                                           const float* __restrict__ b, float eps, float* __restrict__ yrow,
                                           float* mean, float* rstd) {
  const int C4 = C / 4;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  const float mu = wsum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (lane + 64 * i >= C4) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = v[i][e] - mu;
      q = fmaf(d, d, q);
    }
  }
  const float rs = rsqrtf(wsum(q) / (float)C + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    const floatx4 gv = reinterpret_cast<const floatx4*>(g)[qi];
    const floatx4 bv = reinterpret_cast<const floatx4*>(b)[qi];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf((v[i][e] - mu) * rs, gv[e], bv[e]);
    reinterpret_cast<floatx4*>(yrow)[qi] = o;
  }
  if (lane == 0) {
    if (mean) *mean = mu;
    if (rstd) *rstd = rs;
  }
}

// gv: dy row (overwritten); xrow: the norm's input row.
template <int NV>
__device__ __forceinline__ void ln_bwd_row(floatx4 (&gv)[NV], const float* __restrict__ xrow, int C, int lane,
                                           const float* __restrict__ g, float mu, float rs, float* dxrow,
                                           const float* residrow) {
  const int C4 = C / 4;
  floatx4 xv[NV];
  load_row<NV>(xrow, C4, lane, xv);
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    const floatx4 gg = reinterpret_cast<const floatx4*>(g)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[i][e] = (xv[i][e] - mu) * rs;   // x̂
      gv[i][e] = gv[i][e] * gg[e];       // dx̂
      s1 += gv[i][e];
      s2 = fmaf(gv[i][e], xv[i][e], s2);
    }
  }
  s1 = wsum(s1) / (float)C;
  s2 = wsum(s2) / (float)C;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    floatx4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = rs * (gv[i][e] - s1 - xv[i][e] * s2);
    if (residrow) {
      const floatx4 old = reinterpret_cast<const floatx4*>(residrow)[qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += old[e];
    }
    reinterpret_cast<floatx4*>(dxrow)[qi] = r;
  }
}

template <int NV>
__device__ __forceinline__ void rms_fwd_row(const floatx4 (&v)[NV], int C, int lane, const float* __restrict__ w,
                                            float eps, int unit_offset, float* __restrict__ yrow, float* rstd) {
  const int C4 = C / 4;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) s = fmaf(v[i][e], v[i][e], s);
  const float rs = rsqrtf(wsum(s) / (float)C + eps);
  const float off = unit_offset ? 1.f : 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(w)[qi];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[i][e] * rs * (off + wv[e]);
    reinterpret_cast<floatx4*>(yrow)[qi] = o;
  }
  if (lane == 0 && rstd) *rstd = rs;
}

template <int NV>
__device__ __forceinline__ void rms_bwd_row(floatx4 (&gv)[NV], const float* __restrict__ xrow, int C, int lane,
                                            const float* __restrict__ w, float rs, int unit_offset, float* dxrow,
                                            const float* residrow) {
  const int C4 = C / 4;
  floatx4 xv[NV];
  load_row<NV>(xrow, C4, lane, xv);
  const float off = unit_offset ? 1.f : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(w)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gv[i][e] *= off + wv[e];          // dy·w'
      xv[i][e] *= rs;                   // x̂
      s = fmaf(gv[i][e], xv[i][e], s);
    }
  }
  s = wsum(s) / (float)C;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    floatx4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = rs * (gv[i][e] - xv[i][e] * s);
    if (residrow) {
      const floatx4 old = reinterpret_cast<const floatx4*>(residrow)[qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += old[e];
    }
    reinterpret_cast<floatx4*>(dxrow)[qi] = r;
  }
}

// ---- standalone launches: one wave per row, four rows per workgroup ----------
template <int NV>
__global__ __launch_bounds__(256) void ln_fwd_vec(const float* __restrict__ x,
                                                  const float* __restrict__ g,
                                                  const float* __restrict__ b, int64_t M, int C,
                                                  float eps, float* __restrict__ y,
                                                  float* __restrict__ mean,
                                                  float* __restrict__ rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  floatx4 v[NV];
  load_row<NV>(x + row * C, C / 4, lane, v);
  ln_fwd_row<NV>(v, C, lane, g, b, eps, y + row * C, mean ? mean + row : nullptr, rstd ? rstd + row : nullptr);
}

template <int NV>
__global__ __launch_bounds__(256) void ln_bwd_vec(const float* __restrict__ dy,
                                                  const float* __restrict__ x,
                                                  const float* __restrict__ g,
                                                  const float* __restrict__ mean,
                                                  const float* __restrict__ rstd, int64_t M, int C,
                                                  float* dx, const float* resid) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  floatx4 gv[NV];
  load_row<NV>(dy + row * C, C / 4, lane, gv);
  ln_bwd_row<NV>(gv, x + row * C, C, lane, g, mean[row], rstd[row], dx + row * C,
                 resid ? resid + row * C : nullptr);
}

template <int NV>
__global__ __launch_bounds__(256) void rms_fwd_vec(const float* __restrict__ x,
                                                   const float* __restrict__ w, int64_t M, int C,
                                                   float eps, int unit_offset,
                                                   float* __restrict__ y,
                                                   float* __restrict__ rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  floatx4 v[NV];
  load_row<NV>(x + row * C, C / 4, lane, v);
  rms_fwd_row<NV>(v, C, lane, w, eps, unit_offset, y + row * C, rstd ? rstd + row : nullptr);
}

template <int NV>
__global__ __launch_bounds__(256) void rms_bwd_vec(const float* __restrict__ dy,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ rstd, int64_t M,
                                                   int C, int unit_offset, float* dx,
                                                   const float* resid) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  floatx4 gv[NV];
  load_row<NV>(dy + row * C, C / 4, lane, gv);
  rms_bwd_row<NV>(gv, x + row * C, C, lane, w, rstd[row], unit_offset, dx + row * C,
                  resid ? resid + row * C : nullptr);
}

// ---- split-K reduction + GEMM epilogue + norm ---------------------------------
// Each wave finishes one row of C: the partials are summed in split order and
// the epilogue (bias, residual, beta·C, GELU') applied exactly as the plain
// reduction does, C is stored (unless skip_c) and the row goes straight into
// the norm, so the norm's input is never re-read from memory and the norm
// costs no launch of its own.
template <int NV, int KIND>
__global__ __launch_bounds__(256) void splitk_norm_vec(const float* __restrict__ partial, int splits, int64_t M,
                                                       int C, float* Cout, GemmEpilogue ep, RowNorm nm) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const int C4 = C / 4;
  const int64_t plane = M * C;
  floatx4 v[NV];
  load_row<NV>(partial + row * C, C4, lane, v);
  for (int z = 1; z < splits; ++z) {
    floatx4 t[NV];
    load_row<NV>(partial + z * plane + row * C, C4, lane, t);
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += t[i];
  }
  const int64_t r4 = row * C4;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = lane + 64 * i;
    if (qi >= C4) continue;
    if (ep.bias) v[i] += reinterpret_cast<const floatx4*>(ep.bias)[qi];
    if (ep.resid) v[i] += reinterpret_cast<const floatx4*>(ep.resid)[r4 + qi];
    if (ep.beta != 0.f) {
      const floatx4 old = reinterpret_cast<const floatx4*>(Cout)[r4 + qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[i][e] = fmaf(ep.beta, old[e], v[i][e]);
    }
    if (ep.gelu_grad_of) {
      const floatx4 pre = reinterpret_cast<const floatx4*>(ep.gelu_grad_of)[r4 + qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[i][e] *= gelu_tanh_grad(pre[e]);
    }
    if (!nm.skip_c) reinterpret_cast<floatx4*>(Cout)[r4 + qi] = v[i];
    if (ep.gelu_out) {
      floatx4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = gelu_tanh(v[i][e]);
      reinterpret_cast<floatx4*>(ep.gelu_out)[r4 + qi] = a;
    }
  }
  if constexpr (KIND == NORM_LN_FWD) {
    ln_fwd_row<NV>(v, C, lane, nm.w, nm.b, nm.eps, nm.y + row * C, nm.mean ? nm.mean + row : nullptr,
                   nm.rstd ? nm.rstd + row : nullptr);
  } else if constexpr (KIND == NORM_RMS_FWD) {
    rms_fwd_row<NV>(v, C, lane, nm.w, nm.eps, nm.unit_offset, nm.y + row * C, nm.rstd ? nm.rstd + row : nullptr);
  } else if constexpr (KIND == NORM_LN_BWD) {
    ln_bwd_row<NV>(v, nm.x + row * C, C, lane, nm.w, nm.mean[row], nm.rstd[row], nm.y + row * C,
                   nm.resid ? nm.resid + row * C : nullptr);
  } else {
    rms_bwd_row<NV>(v, nm.x + row * C, C, lane, nm.w, nm.rstd[row], nm.unit_offset, nm.y + row * C,
                    nm.resid ? nm.resid + row * C : nullptr);
  }
}

bool vec_ok(int64_t C, std::initializer_list<const void*> ptrs) {
  if (C % 4 != 0 || C > 2048) return false;
  for (const void* p : ptrs)
    if (p && ((uintptr_t)p & 15)) return false;
  return true;
}

#define MFT_NV_DISPATCH(NVVAL, KERNEL, ...)                                              \
  switch (NVVAL) {                                                                       \
    case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;                           \
    case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;                           \
    case 3: hipLaunchKernelGGL(KERNEL<3>, __VA_ARGS__); break;                           \
    case 4: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;                           \
    case 5: hipLaunchKernelGGL(KERNEL<5>, __VA_ARGS__); break;                           \
    case 6: hipLaunchKernelGGL(KERNEL<6>, __VA_ARGS__); break;                           \
    case 7: hipLaunchKernelGGL(KERNEL<7>, __VA_ARGS__); break;                           \
    default: hipLaunchKernelGGL(KERNEL<8>, __VA_ARGS__); break;                          \
  }

}  // namespace

void layernorm_fwd(hipStream_t s, const float* x, const float* g, const float* b, int64_t M,
                   int64_t C, float eps, float* y, float* mean, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {x, g, b, y})) return layernorm_fwd_rowloop(s, x, g, b, M, C, eps, y, mean, rstd);
  const int nv = (int)cdiv(C, 256);
  MFT_NV_DISPATCH(nv, ln_fwd_vec, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s, x, g, b, M, (int)C, eps,
                  y, mean, rstd);
  MFT_LAUNCH_CHECK();
}

void layernorm_bwd(hipStream_t s, const float* dy, const float* x, const float* g,
                   const float* mean, const float* rstd, int64_t M, int64_t C, float* dx,
                   const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {dy, x, g, dx, resid}))
    return layernorm_bwd_rowloop(s, dy, x, g, mean, rstd, M, C, dx, resid);
  const int nv = (int)cdiv(C, 256);
  MFT_NV_DISPATCH(nv, ln_bwd_vec, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s, dy, x, g, mean, rstd, M,
                  (int)C, dx, resid);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_fwd(hipStream_t s, const float* x, const float* w, int64_t M, int64_t C, float eps,
                 bool unit_offset, float* y, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {x, w, y})) return rmsnorm_fwd_rowloop(s, x, w, M, C, eps, unit_offset, y, rstd);
  const int nv = (int)cdiv(C, 256);
  MFT_NV_DISPATCH(nv, rms_fwd_vec, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s, x, w, M, (int)C, eps,
                  unit_offset ? 1 : 0, y, rstd);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_bwd(hipStream_t s, const float* dy, const float* x, const float* w, const float* rstd,
                 int64_t M, int64_t C, bool unit_offset, float* dx, const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {dy, x, w, dx, resid}))
    return rmsnorm_bwd_rowloop(s, dy, x, w, rstd, M, C, unit_offset, dx, resid);
  const int nv = (int)cdiv(C, 256);
  MFT_NV_DISPATCH(nv, rms_bwd_vec, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s, dy, x, w, rstd, M,
                  (int)C, unit_offset ? 1 : 0, dx, resid);
  MFT_LAUNCH_CHECK();
}

void row_norm(hipStream_t s, const float* c, int64_t M, int64_t C, const RowNorm& nm) {
  switch (nm.kind) {
    case NORM_LN_FWD: return layernorm_fwd(s, c, nm.w, nm.b, M, C, nm.eps, nm.y, nm.mean, nm.rstd);
    case NORM_RMS_FWD: return rmsnorm_fwd(s, c, nm.w, M, C, nm.eps, nm.unit_offset != 0, nm.y, nm.rstd);
    case NORM_LN_BWD: return layernorm_bwd(s, c, nm.x, nm.w, nm.mean, nm.rstd, M, C, nm.y, nm.resid);
    case NORM_RMS_BWD: return rmsnorm_bwd(s, c, nm.x, nm.w, nm.rstd, M, C, nm.unit_offset != 0, nm.y, nm.resid);
    default: MFT_CHECK_ARG(false, "unknown norm kind");
  }
}

template <int KIND>
void splitk_norm_launch(hipStream_t s, int nv, const float* partial, int splits, int M, int N, float* C,
                        const GemmEpilogue& ep, const RowNorm& nm) {
  const dim3 grid((unsigned)cdiv(M, 4)), block(256);
  switch (nv) {
    case 1: hipLaunchKernelGGL((splitk_norm_vec<1, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 2: hipLaunchKernelGGL((splitk_norm_vec<2, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 3: hipLaunchKernelGGL((splitk_norm_vec<3, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 4: hipLaunchKernelGGL((splitk_norm_vec<4, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 5: hipLaunchKernelGGL((splitk_norm_vec<5, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 6: hipLaunchKernelGGL((splitk_norm_vec<6, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    case 7: hipLaunchKernelGGL((splitk_norm_vec<7, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
    default: hipLaunchKernelGGL((splitk_norm_vec<8, KIND>), grid, block, 0, s, partial, splits, M, N, C, ep, nm); break;
  }
  MFT_LAUNCH_CHECK();
}

bool splitk_norm(hipStream_t s, const float* partial, int splits, int M, int N, float* C, int64_t ldc,
                 const GemmEpilogue& ep, const RowNorm& nm) {
  if (ldc != N || splits < 1 || M <= 0) return false;
  if (!vec_ok(N, {partial, C, ep.bias, ep.resid, ep.gelu_out, ep.gelu_grad_of, nm.w, nm.b, nm.y, nm.x, nm.resid}))
    return false;
  const int nv = (int)cdiv(N, 256);
  switch (nm.kind) {
    case NORM_LN_FWD: splitk_norm_launch<NORM_LN_FWD>(s, nv, partial, splits, M, N, C, ep, nm); return true;
    case NORM_RMS_FWD: splitk_norm_launch<NORM_RMS_FWD>(s, nv, partial, splits, M, N, C, ep, nm); return true;
    case NORM_LN_BWD: splitk_norm_launch<NORM_LN_BWD>(s, nv, partial, splits, M, N, C, ep, nm); return true;
    case NORM_RMS_BWD: splitk_norm_launch<NORM_RMS_BWD>(s, nv, partial, splits, M, N, C, ep, nm); return true;
    default: return false;
  }
}

}  // namespace mft
