// norms.hip — LayerNorm / RMSNorm forward and backward with the row held in
// registers: one wave64 per row, each lane loads NV 128-bit chunks up front
// (all loads in flight at once), reduces with shuffles and writes once.
// HBM traffic is the algorithmic minimum (fwd: read x, write y; bwd: read
// dy and x, write/accumulate dx).  Rows wider than 2048, C % 4 != 0 or
// unaligned rows go to the row-loop kernels in elementwise.hip.
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
  const int C4 = C / 4;
  floatx4 v[NV];
  load_row<NV>(x + row * C, C4, lane, v);
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
    reinterpret_cast<floatx4*>(y + row * C)[qi] = o;
  }
  if (lane == 0) {
    if (mean) mean[row] = mu;
    if (rstd) rstd[row] = rs;
  }
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
  const int C4 = C / 4;
  floatx4 xv[NV], gv[NV];
  load_row<NV>(x + row * C, C4, lane, xv);
  load_row<NV>(dy + row * C, C4, lane, gv);
  const float mu = mean[row], rs = rstd[row];
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
    floatx4* o = reinterpret_cast<floatx4*>(dx + row * C) + qi;
    floatx4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = rs * (gv[i][e] - s1 - xv[i][e] * s2);
    if (resid) {
      const floatx4 old = reinterpret_cast<const floatx4*>(resid + row * C)[qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += old[e];
    }
    *o = r;
  }
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
  const int C4 = C / 4;
  floatx4 v[NV];
  load_row<NV>(x + row * C, C4, lane, v);
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
    reinterpret_cast<floatx4*>(y + row * C)[qi] = o;
  }
  if (lane == 0 && rstd) rstd[row] = rs;
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
  const int C4 = C / 4;
  floatx4 xv[NV], gv[NV];
  load_row<NV>(x + row * C, C4, lane, xv);
  load_row<NV>(dy + row * C, C4, lane, gv);
  const float rs = rstd[row];
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
    floatx4* o = reinterpret_cast<floatx4*>(dx + row * C) + qi;
    floatx4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = rs * (gv[i][e] - xv[i][e] * s);
    if (resid) {
      const floatx4 old = reinterpret_cast<const floatx4*>(resid + row * C)[qi];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += old[e];
    }
    *o = r;
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

}  // namespace mft
