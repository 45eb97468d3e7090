// norms.hip — LayerNorm / RMSNorm forward and backward with the row held in
// registers.  A row is owned by a group of RW waves (RW = 4 for rows wider
// than 512 floats, so a 1024-wide row is one 128-bit chunk per thread of a
// 256-thread workgroup; 2 or 1 for narrow rows such as per-head q/k norms);
// every thread loads its NV chunks up front (all loads in flight at once),
// sums reduce with wave shuffles plus one LDS step across the group, and the
// row is written once.  HBM traffic is the algorithmic minimum (fwd: read
// x, write y; bwd: read dy and x, write/accumulate dx).  Rows wider than
// 4096, C % 4 != 0 or unaligned rows go to the row-loop kernels in
// elementwise.hip.
//
// The same row code also finishes split-K GEMM outputs (splitk_norm_vec):
// the norm whose input is a linear layer's output runs inside that GEMM's
// reduction pass, with every split's partial load issued before the first
// is used.
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace mft {
namespace {

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Thread placement: row group `grp` of the workgroup (4 / RW groups), lane
// `gl` ∈ [0, 64·RW) within it; chunk q = gl + 64·RW·i for i < NV.
template <int RW>
struct Place {
  int wave, grp, gl;
  __device__ __forceinline__ Place() {
    wave = (int)threadIdx.x >> 6;
    grp = wave / RW;
    gl = (wave % RW) * 64 + ((int)threadIdx.x & 63);
  }
};

// Σ over the row group of one or two per-thread values.  red: LDS slots
// [2][4] owned by this call site (distinct sites use distinct slots, so
// no barrier is needed before a slot is reused within the kernel).
template <int RW>
__device__ __forceinline__ void row_sum2(float& a, float& b, float (*red)[4], int wave) {
  a = wsum(a);
  b = wsum(b);
  if constexpr (RW > 1) {
    if ((threadIdx.x & 63) == 0) {
      red[0][wave] = a;
      red[1][wave] = b;
    }
    __syncthreads();
    const int g0 = wave & ~(RW - 1);
    a = red[0][g0];
    b = red[1][g0];
#pragma unroll
    for (int i = 1; i < RW; ++i) {
      a += red[0][g0 + i];
      b += red[1][g0 + i];
    }
  }
}
template <int RW>
__device__ __forceinline__ float row_sum(float a, float (*red)[4], int wave) {
  float b = 0.f;
  row_sum2<RW>(a, b, red, wave);
  return a;
}

template <int NV, int RW>
__device__ __forceinline__ void load_row(const float* __restrict__ base, int C4, int gl, floatx4 (&v)[NV]) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = gl + 64 * RW * i;
    v[i] = q < C4 ? reinterpret_cast<const floatx4*>(base)[q] : floatx4{0.f, 0.f, 0.f, 0.f};
  }
}

// ---- the four norms on a row held in registers ---------------------------
// `valid` is false for a row group past the last row (it still takes part
// in the group's barriers, reading a clamped row, and stores nothing).
template <int NV, int RW>
__device__ __forceinline__ void ln_fwd_row(const floatx4 (&v)[NV], int C, const Place<RW>& pl, bool valid,
                                           float (*red)[4], const float* __restrict__ g,
                                           const float* __restrict__ b, float eps, float* __restrict__ yrow,
                                           float* mean, float* rstd) {
  const int C4 = C / 4;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  const float mu = row_sum<RW>(s, red, pl.wave) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (pl.gl + 64 * RW * i >= C4) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = v[i][e] - mu;
      q = fmaf(d, d, q);
    }
  }
  const float rs = rsqrtf(row_sum<RW>(q, red + 2, pl.wave) / (float)C + eps);
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 gv = reinterpret_cast<const floatx4*>(g)[qi];
    const floatx4 bv = reinterpret_cast<const floatx4*>(b)[qi];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf((v[i][e] - mu) * rs, gv[e], bv[e]);
    reinterpret_cast<floatx4*>(yrow)[qi] = o;
  }
  if (pl.gl == 0) {
    if (mean) *mean = mu;
    if (rstd) *rstd = rs;
  }
}

// gv: dy row (overwritten); xv: the norm's input row (overwritten).
template <int NV, int RW>
__device__ __forceinline__ void ln_bwd_row(floatx4 (&gv)[NV], floatx4 (&xv)[NV], int C, const Place<RW>& pl,
                                           bool valid, float (*red)[4], const float* __restrict__ g, float mu,
                                           float rs, float* dxrow, const float* residrow) {
  const int C4 = C / 4;
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
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
  row_sum2<RW>(s1, s2, red, pl.wave);
  s1 /= (float)C;
  s2 /= (float)C;
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
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

template <int NV, int RW>
__device__ __forceinline__ void rms_fwd_row(const floatx4 (&v)[NV], int C, const Place<RW>& pl, bool valid,
                                            float (*red)[4], const float* __restrict__ w, float eps,
                                            int unit_offset, float* __restrict__ yrow, float* rstd) {
  const int C4 = C / 4;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) s = fmaf(v[i][e], v[i][e], s);
  const float rs = rsqrtf(row_sum<RW>(s, red, pl.wave) / (float)C + eps);
  if (!valid) return;
  const float off = unit_offset ? 1.f : 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(w)[qi];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[i][e] * rs * (off + wv[e]);
    reinterpret_cast<floatx4*>(yrow)[qi] = o;
  }
  if (pl.gl == 0 && rstd) *rstd = rs;
}

template <int NV, int RW>
__device__ __forceinline__ void rms_bwd_row(floatx4 (&gv)[NV], floatx4 (&xv)[NV], int C, const Place<RW>& pl,
                                            bool valid, float (*red)[4], const float* __restrict__ w, float rs,
                                            int unit_offset, float* dxrow, const float* residrow) {
  const int C4 = C / 4;
  const float off = unit_offset ? 1.f : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(w)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gv[i][e] *= off + wv[e];          // dy·w'
      xv[i][e] *= rs;                   // x̂
      s = fmaf(gv[i][e], xv[i][e], s);
    }
  }
  s = row_sum<RW>(s, red, pl.wave) / (float)C;
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
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

// Gemma3's sandwich: y = resid + v·rstd·(off + w), then y2 = y·rstd2·(off +
// w2), with the arithmetic of rms_fwd_row followed by an elementwise add and
// a second rms_fwd_row.
// xres: the row of nm.resid (loaded by the caller with the row itself).
template <int NV, int RW>
__device__ __forceinline__ void rms_res_rms_row(const floatx4 (&v)[NV], const floatx4 (&xres)[NV], int C,
                                                const Place<RW>& pl, bool valid, float (*red)[4], const RowNorm& nm,
                                                int64_t r) {
  const int C4 = C / 4;
  const float off = nm.unit_offset ? 1.f : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) s = fmaf(v[i][e], v[i][e], s);
  const float rs = rsqrtf(row_sum<RW>(s, red, pl.wave) / (float)C + nm.eps);
  floatx4 h[NV];
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    h[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(nm.w)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[i][e] = xres[i][e] + v[i][e] * rs * (off + wv[e]);
      s2 = fmaf(h[i][e], h[i][e], s2);
    }
  }
  const float rs2 = rsqrtf(row_sum<RW>(s2, red + 2, pl.wave) / (float)C + nm.eps);
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(nm.w2)[qi];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = h[i][e] * rs2 * (off + wv[e]);
    reinterpret_cast<floatx4*>(nm.y + r * C)[qi] = h[i];
    reinterpret_cast<floatx4*>(nm.y2 + r * C)[qi] = o;
  }
  if (pl.gl == 0) {
    if (nm.rstd) nm.rstd[r] = rs;
    if (nm.rstd2) nm.rstd2[r] = rs2;
  }
}

// Backward of an RMSNorm whose input came out of a post-norm: stage 1 is
// rms_bwd_row with the residual (y = resid + ∂x over rows x with w, rstd[r]);
// stage 2 is rms_bwd_row of y over the post-norm's input rows x2 (w2,
// rstd2[r], no residual) into y2.  gv: the incoming gradient; xv, x2v, rv:
// the rows of x, x2 and resid (all overwritten).
template <int NV, int RW>
__device__ __forceinline__ void rms_bwd_post_row(floatx4 (&gv)[NV], floatx4 (&xv)[NV], floatx4 (&x2v)[NV],
                                                 const floatx4 (&rv)[NV], int C, const Place<RW>& pl, bool valid,
                                                 float (*red)[4], const RowNorm& nm, int64_t r) {
  const int C4 = C / 4;
  const float off = nm.unit_offset ? 1.f : 0.f;
  const float rs = nm.rstd[r];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(nm.w)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gv[i][e] *= off + wv[e];
      xv[i][e] *= rs;
      s = fmaf(gv[i][e], xv[i][e], s);
    }
  }
  s = row_sum<RW>(s, red, pl.wave) / (float)C;
  const float rs2 = nm.rstd2[r];
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    const floatx4 w2 = reinterpret_cast<const floatx4*>(nm.w2)[qi];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float y = rs * (gv[i][e] - xv[i][e] * s);
      if (nm.resid) y += rv[i][e];
      gv[i][e] = y;  // stage 1's output, kept for the store
      xv[i][e] = y * (off + w2[e]);
      x2v[i][e] *= rs2;
      s2 = fmaf(xv[i][e], x2v[i][e], s2);
    }
  }
  s2 = row_sum<RW>(s2, red + 2, pl.wave) / (float)C;
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = rs2 * (xv[i][e] - x2v[i][e] * s2);
    reinterpret_cast<floatx4*>(nm.y + r * C)[qi] = gv[i];
    reinterpret_cast<floatx4*>(nm.y2 + r * C)[qi] = o;
  }
}

// ---- standalone launches: 4 / RW rows per 256-thread workgroup -------------
template <int NV, int RW>
__global__ __launch_bounds__(256) void ln_fwd_vec(const float* __restrict__ x, const float* __restrict__ g,
                                                  const float* __restrict__ b, int64_t M, int C, float eps,
                                                  float* __restrict__ y, float* __restrict__ mean,
                                                  float* __restrict__ rstd) {
  __shared__ float red[4][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 v[NV];
  load_row<NV, RW>(x + r * C, C / 4, pl.gl, v);
  ln_fwd_row<NV, RW>(v, C, pl, valid, red, g, b, eps, y + r * C, mean ? mean + r : nullptr,
                     rstd ? rstd + r : nullptr);
}

template <int NV, int RW>
__global__ __launch_bounds__(256) void ln_bwd_vec(const float* __restrict__ dy, const float* __restrict__ x,
                                                  const float* __restrict__ g, const float* __restrict__ mean,
                                                  const float* __restrict__ rstd, int64_t M, int C, float* dx,
                                                  const float* resid) {
  __shared__ float red[2][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 gv[NV], xv[NV];
  load_row<NV, RW>(dy + r * C, C / 4, pl.gl, gv);
  load_row<NV, RW>(x + r * C, C / 4, pl.gl, xv);
  ln_bwd_row<NV, RW>(gv, xv, C, pl, valid, red, g, mean[r], rstd[r], dx + r * C, resid ? resid + r * C : nullptr);
}

// Row r of a segmented operand starts at (r / seg)·ld + (r % seg)·C: seg
// rows of C per token, tokens ld apart (seg = 1, ld = C: plain rows).  Lets a
// per-head norm read or write head rows inside a fused q|k|v buffer.
__device__ __forceinline__ int64_t seg_off(int64_t r, int seg, int64_t ld, int C) {
  return (r / seg) * ld + (r % seg) * C;
}

template <int NV, int RW>
__global__ __launch_bounds__(256) void rms_fwd_vec(const float* __restrict__ x, const float* __restrict__ w,
                                                   int64_t M, int C, float eps, int unit_offset,
                                                   float* __restrict__ y, float* __restrict__ rstd, int seg,
                                                   int64_t x_ld, int64_t y_ld) {
  __shared__ float red[2][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 v[NV];
  load_row<NV, RW>(x + seg_off(r, seg, x_ld, C), C / 4, pl.gl, v);
  rms_fwd_row<NV, RW>(v, C, pl, valid, red, w, eps, unit_offset, y + seg_off(r, seg, y_ld, C),
                      rstd ? rstd + r : nullptr);
}

template <int NV, int RW>
__global__ __launch_bounds__(256) void rms_bwd_vec(const float* __restrict__ dy, const float* __restrict__ x,
                                                   const float* __restrict__ w, const float* __restrict__ rstd,
                                                   int64_t M, int C, int unit_offset, float* dx,
                                                   const float* resid, int seg, int64_t dy_ld, int64_t x_ld,
                                                   int64_t dx_ld) {
  __shared__ float red[2][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 gv[NV], xv[NV];
  load_row<NV, RW>(dy + seg_off(r, seg, dy_ld, C), C / 4, pl.gl, gv);
  load_row<NV, RW>(x + seg_off(r, seg, x_ld, C), C / 4, pl.gl, xv);
  const int64_t o = seg_off(r, seg, dx_ld, C);
  rms_bwd_row<NV, RW>(gv, xv, C, pl, valid, red, w, rstd[r], unit_offset, dx + o, resid ? resid + o : nullptr);
}

template <int NV, int RW>
__global__ __launch_bounds__(256) void rms_res_rms_vec(const float* __restrict__ x, int64_t M, int C, RowNorm nm) {
  __shared__ float red[4][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 v[NV], xres[NV];
  load_row<NV, RW>(nm.resid + r * C, C / 4, pl.gl, xres);
  load_row<NV, RW>(x + r * C, C / 4, pl.gl, v);
  rms_res_rms_row<NV, RW>(v, xres, C, pl, valid, red, nm, r);
}

template <int NV, int RW>
__global__ __launch_bounds__(256) void rms_bwd_post_vec(const float* __restrict__ dy, int64_t M, int C, RowNorm nm) {
  __shared__ float red[4][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  floatx4 gv[NV], xv[NV], x2v[NV], rv[NV];
  load_row<NV, RW>(nm.x + r * C, C / 4, pl.gl, xv);
  load_row<NV, RW>(nm.x2 + r * C, C / 4, pl.gl, x2v);
  if (nm.resid) load_row<NV, RW>(nm.resid + r * C, C / 4, pl.gl, rv);
  load_row<NV, RW>(dy + r * C, C / 4, pl.gl, gv);
  rms_bwd_post_row<NV, RW>(gv, xv, x2v, rv, C, pl, valid, red, nm, r);
}

// ---- q/k head rows: per-head RMSNorm + RoPE in one pass -------------------
// One wave per head row of hd = 64·E values, lane l holding values
// [l·E, l·E + E): the RoPE partner of value i < hd/2 is i + hd/2, held by
// lane l ^ 32 at the same slot, so the rotation is one lane exchange.  The
// angles come from the table (no transcendental per element).  Rows of q
// come first, then rows of k.
__global__ void rope_table_kernel(double theta, int hd, int npos, float2* __restrict__ tab) {
  const int half = hd / 2;
  const int64_t n = (int64_t)npos * half;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(idx % half), p = (int)(idx / half);
    const double inv = pow(theta, -2.0 * i / (double)hd);
    double sn, cs;
    sincos((double)p * inv, &sn, &cs);
    tab[idx] = make_float2((float)cs, (float)sn);
  }
}

template <int E>
struct HeadVec {
  float v[E];
};

template <int E>
__device__ __forceinline__ HeadVec<E> load_head(const float* p) {
  HeadVec<E> r;
  if constexpr (E == 4) {
    const floatx4 t = *reinterpret_cast<const floatx4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) r.v[e] = t[e];
  } else if constexpr (E == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r.v[0] = t.x;
    r.v[1] = t.y;
  } else {
    r.v[0] = *p;
  }
  return r;
}

template <int E>
__device__ __forceinline__ void store_head(float* p, const HeadVec<E>& r) {
  if constexpr (E == 4) {
    *reinterpret_cast<floatx4*>(p) = floatx4{r.v[0], r.v[1], r.v[2], r.v[3]};
  } else if constexpr (E == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(r.v[0], r.v[1]);
  } else {
    *p = r.v[0];
  }
}

// x rotated by the angle of (pos, slot): lanes < 32 hold the first half
// (x1), lanes ≥ 32 the second (x2); out1 = x1·c − x2·s, out2 = x2·c + x1·s
// (sign of s flipped for the inverse).
template <int E>
__device__ __forceinline__ void rotate(HeadVec<E>& r, const float2* __restrict__ trow, int lane, bool inverse) {
  const bool upper = lane >= 32;
  const int i0 = (lane & 31) * E;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float other = __shfl_xor(r.v[e], 32, 64);
    const float2 cs = trow[i0 + e];
    const float sn = inverse ? -cs.y : cs.y;
    const float x1 = upper ? other : r.v[e], x2 = upper ? r.v[e] : other;
    r.v[e] = upper ? x2 * cs.x + x1 * sn : x1 * cs.x - x2 * sn;
  }
}

template <int E, bool NORM>
__global__ __launch_bounds__(256) void qk_rope_fwd_kernel(HeadRows q, HeadRows k, int64_t M, int S, float eps,
                                                          const float2* __restrict__ tab) {
  constexpr int HD = 64 * E, HALF = HD / 2;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nq = M * q.H;
  if (row >= nq + M * k.H) return;  // whole wave
  const bool isq = row < nq;
  const HeadRows& hr = isq ? q : k;
  const int64_t r = isq ? row : row - nq;
  const int64_t t = r / hr.H;
  const int h = (int)(r % hr.H);
  HeadVec<E> v = load_head<E>(hr.in + t * hr.in_ld + (int64_t)h * HD + lane * E);
  if constexpr (NORM) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) s = fmaf(v.v[e], v.v[e], s);
    const float rs = rsqrtf(wsum(s) / (float)HD + eps);
#pragma unroll
    for (int e = 0; e < E; ++e) v.v[e] = v.v[e] * rs * (1.f + hr.w[lane * E + e]);
    if (lane == 0) hr.rstd[r] = rs;
  }
  rotate<E>(v, tab + (int64_t)(t % S) * HALF, lane, false);
  store_head<E>(hr.out + t * hr.out_ld + (int64_t)h * HD + lane * E, v);
}

template <int E, bool NORM>
__global__ __launch_bounds__(256) void qk_rope_bwd_kernel(HeadRows q, HeadRows k, int64_t M, int S,
                                                          const float2* __restrict__ tab) {
  constexpr int HD = 64 * E, HALF = HD / 2;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nq = M * q.H;
  if (row >= nq + M * k.H) return;  // whole wave
  const bool isq = row < nq;
  const HeadRows& hr = isq ? q : k;
  const int64_t r = isq ? row : row - nq;
  const int64_t t = r / hr.H;
  const int h = (int)(r % hr.H);
  HeadVec<E> g = load_head<E>(hr.in + t * hr.in_ld + (int64_t)h * HD + lane * E);
  rotate<E>(g, tab + (int64_t)(t % S) * HALF, lane, true);
  if constexpr (NORM) {
    const HeadVec<E> x = load_head<E>(hr.x + t * hr.x_ld + (int64_t)h * HD + lane * E);
    const float rs = hr.rstd[r];
    float xh[E];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      g.v[e] *= 1.f + hr.w[lane * E + e];  // dy·w'
      xh[e] = x.v[e] * rs;                 // x̂
      s = fmaf(g.v[e], xh[e], s);
    }
    s = wsum(s) / (float)HD;
#pragma unroll
    for (int e = 0; e < E; ++e) g.v[e] = rs * (g.v[e] - xh[e] * s);
  }
  store_head<E>(hr.out + t * hr.out_ld + (int64_t)h * HD + lane * E, g);
}

// ---- split-K reduction + GEMM epilogue + norm ------------------------------
// Each row group finishes one row of C: the partials are summed in split
// order and the epilogue (bias, residual, beta·C, GELU') applied exactly as
// the plain reduction does, C is stored (unless skip_c) and the row goes
// straight into the norm, so the norm's input is never re-read and the norm
// costs no launch of its own.  Partial loads are issued four splits at a
// time before any is added, and the norm's other row operands (residual,
// the input rows of a backward) are loaded first, so a row's loads overlap.
template <int NV, int RW, int KIND>
__global__ __launch_bounds__(256) void splitk_norm_vec(const float* __restrict__ partial, int splits, int64_t M,
                                                       int C, float* Cout, GemmEpilogue ep, RowNorm nm) {
  __shared__ float red[4][4];
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  const int C4 = C / 4;
  const int64_t plane = M * C;
  constexpr bool BWD = KIND == NORM_LN_BWD || KIND == NORM_RMS_BWD;
  floatx4 xv[NV], rv[NV];
  if constexpr (BWD) load_row<NV, RW>(nm.x + r * C, C4, pl.gl, xv);
  if constexpr (KIND == NORM_RMS_RES_RMS) load_row<NV, RW>(nm.resid + r * C, C4, pl.gl, xv);
  floatx4 x2v[KIND == NORM_RMS_BWD_POST ? NV : 1], nrv[KIND == NORM_RMS_BWD_POST ? NV : 1];
  if constexpr (KIND == NORM_RMS_BWD_POST) {
    load_row<NV, RW>(nm.x + r * C, C4, pl.gl, xv);
    load_row<NV, RW>(nm.x2 + r * C, C4, pl.gl, x2v);
    if (nm.resid) load_row<NV, RW>(nm.resid + r * C, C4, pl.gl, nrv);
  }
  if (ep.resid) load_row<NV, RW>(ep.resid + r * C, C4, pl.gl, rv);
  floatx4 v[NV];
  load_row<NV, RW>(partial + r * C, C4, pl.gl, v);
  for (int z0 = 1; z0 < splits; z0 += 4) {
    floatx4 t[4][NV];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (z0 + j < splits) load_row<NV, RW>(partial + (z0 + j) * plane + r * C, C4, pl.gl, t[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (z0 + j < splits) {
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] += t[j][i];
      }
  }
  const int64_t r4 = r * C4;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int qi = pl.gl + 64 * RW * i;
    if (qi >= C4) continue;
    if (ep.bias) v[i] += reinterpret_cast<const floatx4*>(ep.bias)[qi];
    if (ep.resid) v[i] += rv[i];
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
    if (!valid) continue;
    if (!nm.skip_c) reinterpret_cast<floatx4*>(Cout)[r4 + qi] = v[i];
    if (ep.gelu_out) {
      floatx4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = gelu_tanh(v[i][e]);
      reinterpret_cast<floatx4*>(ep.gelu_out)[r4 + qi] = a;
    }
  }
  if constexpr (KIND == NORM_LN_FWD) {
    ln_fwd_row<NV, RW>(v, C, pl, valid, red, nm.w, nm.b, nm.eps, nm.y + r * C, nm.mean ? nm.mean + r : nullptr,
                       nm.rstd ? nm.rstd + r : nullptr);
  } else if constexpr (KIND == NORM_RMS_FWD) {
    rms_fwd_row<NV, RW>(v, C, pl, valid, red, nm.w, nm.eps, nm.unit_offset, nm.y + r * C,
                        nm.rstd ? nm.rstd + r : nullptr);
  } else if constexpr (KIND == NORM_LN_BWD) {
    ln_bwd_row<NV, RW>(v, xv, C, pl, valid, red, nm.w, nm.mean[r], nm.rstd[r], nm.y + r * C,
                       nm.resid ? nm.resid + r * C : nullptr);
  } else if constexpr (KIND == NORM_RMS_RES_RMS) {
    rms_res_rms_row<NV, RW>(v, xv, C, pl, valid, red, nm, r);
  } else if constexpr (KIND == NORM_RMS_BWD_POST) {
    rms_bwd_post_row<NV, RW>(v, xv, x2v, nrv, C, pl, valid, red, nm, r);
  } else {
    rms_bwd_row<NV, RW>(v, xv, C, pl, valid, red, nm.w, nm.rstd[r], nm.unit_offset, nm.y + r * C,
                        nm.resid ? nm.resid + r * C : nullptr);
  }
}

bool vec_ok(int64_t C, std::initializer_list<const void*> ptrs) {
  if (C % 4 != 0 || C > 4096) return false;
  for (const void* p : ptrs)
    if (p && ((uintptr_t)p & 15)) return false;
  return true;
}

// Row-group shape for width C: RW waves per row, NV chunks per thread.
struct RowShape {
  int rw, nv;
};
RowShape row_shape(int64_t C) {
  const int64_t c4 = C / 4;
  const int rw = c4 > 128 ? 4 : (c4 > 64 ? 2 : 1);
  return {rw, (int)cdiv(c4, 64 * rw)};
}
dim3 row_grid(int64_t M, const RowShape& sh) { return dim3((unsigned)cdiv(M, 4 / sh.rw)); }

// Instantiated shapes: RW = 1 or 2 with NV = 1 (C ≤ 512), RW = 4 with
// NV = 1..4 (C ≤ 4096).
#define MFT_ROW_DISPATCH(SH, KERNEL, ...)                                    \
  do {                                                                       \
    if ((SH).rw == 1) hipLaunchKernelGGL((KERNEL<1, 1>), __VA_ARGS__);        \
    else if ((SH).rw == 2) hipLaunchKernelGGL((KERNEL<1, 2>), __VA_ARGS__);   \
    else if ((SH).nv == 1) hipLaunchKernelGGL((KERNEL<1, 4>), __VA_ARGS__);   \
    else if ((SH).nv == 2) hipLaunchKernelGGL((KERNEL<2, 4>), __VA_ARGS__);   \
    else if ((SH).nv == 3) hipLaunchKernelGGL((KERNEL<3, 4>), __VA_ARGS__);   \
    else hipLaunchKernelGGL((KERNEL<4, 4>), __VA_ARGS__);                     \
  } while (0)

// ---- embedding gather + the first layer's input norm ----------------------
// Row r: e = wte[ids[r]]·scale (+ wpe[r mod S]) is stored as the residual
// stream x (an id outside [0, V) stores a zero row and raises *bad), then
// normalised from registers into nm.y, exactly as embed() followed by
// row_norm().  Workgroup 0 also clears `zero` (nzero 8-byte words: the
// step's loss and count slots), so neither needs a launch of its own.
template <int NV, int RW, int KIND, bool F16>
__global__ __launch_bounds__(256) void embed_norm_vec(const int32_t* __restrict__ ids, int64_t M, int S,
                                                      const void* __restrict__ wte, int64_t V,
                                                      const float* __restrict__ wpe, int C, float scale,
                                                      float* __restrict__ x, int* bad, RowNorm nm,
                                                      unsigned long long* zero, int nzero) {
  __shared__ float red[4][4];
  if (zero && blockIdx.x == 0)
    for (int i = threadIdx.x; i < nzero; i += 256) zero[i] = 0ull;
  const Place<RW> pl;
  const int64_t row = (int64_t)blockIdx.x * (4 / RW) + pl.grp;
  const bool valid = row < M;
  const int64_t r = valid ? row : M - 1;
  const int64_t id = ids[r];
  const bool ok = id >= 0 && id < V;
  const int C4 = C / 4;
  const int64_t pos = r % S;
  floatx4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = pl.gl + 64 * RW * i;
    v[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (q >= C4 || !ok) continue;
    floatx4 e;
    if constexpr (F16) e = widen4(reinterpret_cast<const uint2*>(wte)[id * C4 + q]);
    else e = reinterpret_cast<const floatx4*>(wte)[id * C4 + q];
    const floatx4 p = wpe ? reinterpret_cast<const floatx4*>(wpe)[pos * C4 + q] : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float t = e[k] * scale;
      if (wpe) t += p[k];
      v[i][k] = t;
    }
  }
  if (valid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int q = pl.gl + 64 * RW * i;
      if (q < C4) reinterpret_cast<floatx4*>(x)[r * C4 + q] = v[i];
    }
    if (!ok && bad && pl.gl == 0) atomicOr(bad, 1);
  }
  if constexpr (KIND == NORM_LN_FWD)
    ln_fwd_row<NV, RW>(v, C, pl, valid, red, nm.w, nm.b, nm.eps, nm.y + r * C, nm.mean ? nm.mean + r : nullptr,
                       nm.rstd ? nm.rstd + r : nullptr);
  else
    rms_fwd_row<NV, RW>(v, C, pl, valid, red, nm.w, nm.eps, nm.unit_offset, nm.y + r * C,
                        nm.rstd ? nm.rstd + r : nullptr);
}

template <int KIND, bool F16>
void embed_norm_launch(hipStream_t s, const RowShape& sh, const int32_t* ids, int64_t M, int S, const void* wte,
                       int64_t V, const float* wpe, int C, float scale, float* x, int* bad, const RowNorm& nm,
                       unsigned long long* zero, int nzero) {
  const dim3 grid = row_grid(M, sh), block(256);
#define MFT_EMBED_NORM(NV, RW)                                                                                       \
  hipLaunchKernelGGL((embed_norm_vec<NV, RW, KIND, F16>), grid, block, 0, s, ids, M, S, wte, V, wpe, C, scale, x, bad, \
                     nm, zero, nzero)
  if (sh.rw == 1) MFT_EMBED_NORM(1, 1);
  else if (sh.rw == 2) MFT_EMBED_NORM(1, 2);
  else if (sh.nv == 1) MFT_EMBED_NORM(1, 4);
  else if (sh.nv == 2) MFT_EMBED_NORM(2, 4);
  else if (sh.nv == 3) MFT_EMBED_NORM(3, 4);
  else MFT_EMBED_NORM(4, 4);
#undef MFT_EMBED_NORM
  MFT_LAUNCH_CHECK();
}

template <int KIND>
void splitk_norm_launch(hipStream_t s, const RowShape& sh, const float* partial, int splits, int M, int N, float* C,
                        const GemmEpilogue& ep, const RowNorm& nm) {
  const dim3 grid = row_grid(M, sh), block(256);
  const int64_t m = M;
  if (sh.rw == 1) MFT_LAUNCH_TAIL((splitk_norm_vec<1, 1, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  else if (sh.rw == 2) MFT_LAUNCH_TAIL((splitk_norm_vec<1, 2, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  else if (sh.nv == 1) MFT_LAUNCH_TAIL((splitk_norm_vec<1, 4, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  else if (sh.nv == 2) MFT_LAUNCH_TAIL((splitk_norm_vec<2, 4, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  else if (sh.nv == 3) MFT_LAUNCH_TAIL((splitk_norm_vec<3, 4, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  else MFT_LAUNCH_TAIL((splitk_norm_vec<4, 4, KIND>), grid, block, 0, s, partial, splits, m, N, C, ep, nm);
  MFT_LAUNCH_CHECK();
}

}  // namespace

void layernorm_fwd(hipStream_t s, const float* x, const float* g, const float* b, int64_t M,
                   int64_t C, float eps, float* y, float* mean, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {x, g, b, y})) return layernorm_fwd_rowloop(s, x, g, b, M, C, eps, y, mean, rstd);
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, ln_fwd_vec, row_grid(M, sh), dim3(256), 0, s, x, g, b, M, (int)C, eps, y, mean, rstd);
  MFT_LAUNCH_CHECK();
}

void layernorm_bwd(hipStream_t s, const float* dy, const float* x, const float* g,
                   const float* mean, const float* rstd, int64_t M, int64_t C, float* dx,
                   const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {dy, x, g, dx, resid}))
    return layernorm_bwd_rowloop(s, dy, x, g, mean, rstd, M, C, dx, resid);
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, ln_bwd_vec, row_grid(M, sh), dim3(256), 0, s, dy, x, g, mean, rstd, M, (int)C, dx, resid);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_fwd(hipStream_t s, const float* x, const float* w, int64_t M, int64_t C, float eps,
                 bool unit_offset, float* y, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {x, w, y})) return rmsnorm_fwd_rowloop(s, x, w, M, C, eps, unit_offset, y, rstd);
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, rms_fwd_vec, row_grid(M, sh), dim3(256), 0, s, x, w, M, (int)C, eps, unit_offset ? 1 : 0,
                   y, rstd, 1, C, C);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_fwd_seg(hipStream_t s, const float* x, int64_t x_ld, const float* w, int64_t M, int64_t C, int seg,
                     float eps, bool unit_offset, float* y, int64_t y_ld, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0 && seg > 0 && M % seg == 0, "segmented norm: bad shape");
  MFT_CHECK_ARG(vec_ok(C, {x, w, y}) && x_ld % 4 == 0 && y_ld % 4 == 0 && x_ld >= seg * C && y_ld >= seg * C,
                "segmented norm: 16-byte aligned rows required");
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, rms_fwd_vec, row_grid(M, sh), dim3(256), 0, s, x, w, M, (int)C, eps, unit_offset ? 1 : 0,
                   y, rstd, seg, x_ld, y_ld);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_bwd(hipStream_t s, const float* dy, const float* x, const float* w, const float* rstd,
                 int64_t M, int64_t C, bool unit_offset, float* dx, const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  if (!vec_ok(C, {dy, x, w, dx, resid}))
    return rmsnorm_bwd_rowloop(s, dy, x, w, rstd, M, C, unit_offset, dx, resid);
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, rms_bwd_vec, row_grid(M, sh), dim3(256), 0, s, dy, x, w, rstd, M, (int)C,
                   unit_offset ? 1 : 0, dx, resid, 1, C, C, C);
  MFT_LAUNCH_CHECK();
}

void rmsnorm_bwd_seg(hipStream_t s, const float* dy, int64_t dy_ld, const float* x, int64_t x_ld, const float* w,
                     const float* rstd, int64_t M, int64_t C, int seg, bool unit_offset, float* dx, int64_t dx_ld) {
  MFT_CHECK_ARG(M > 0 && C > 0 && seg > 0 && M % seg == 0, "segmented norm: bad shape");
  MFT_CHECK_ARG(vec_ok(C, {dy, x, w, dx}) && dy_ld % 4 == 0 && x_ld % 4 == 0 && dx_ld % 4 == 0 &&
                    dy_ld >= seg * C && x_ld >= seg * C && dx_ld >= seg * C,
                "segmented norm: 16-byte aligned rows required");
  const RowShape sh = row_shape(C);
  MFT_ROW_DISPATCH(sh, rms_bwd_vec, row_grid(M, sh), dim3(256), 0, s, dy, x, w, rstd, M, (int)C,
                   unit_offset ? 1 : 0, dx, nullptr, seg, dy_ld, x_ld, dx_ld);
  MFT_LAUNCH_CHECK();
}

void row_norm(hipStream_t s, const float* c, int64_t M, int64_t C, const RowNorm& nm) {
  if (nm.kind == NORM_RMS_RES_RMS) {
    MFT_CHECK_ARG(M > 0 && C > 0 && nm.resid && nm.y && nm.y2 && nm.w && nm.w2, "sandwich norm: missing operand");
    if (vec_ok(C, {c, nm.w, nm.w2, nm.resid, nm.y, nm.y2})) {
      const RowShape sh = row_shape(C);
      MFT_ROW_DISPATCH(sh, rms_res_rms_vec, row_grid(M, sh), dim3(256), 0, s, c, M, (int)C, nm);
      MFT_LAUNCH_CHECK();
      return;
    }
    // row-loop fallback: the same three steps as separate launches
    rmsnorm_fwd(s, c, nm.w, M, C, nm.eps, nm.unit_offset != 0, nm.y, nm.rstd);
    add_inplace(s, nm.y, nm.resid, M * C);
    rmsnorm_fwd(s, nm.y, nm.w2, M, C, nm.eps, nm.unit_offset != 0, nm.y2, nm.rstd2);
    return;
  }
  if (nm.kind == NORM_RMS_BWD_POST) {
    MFT_CHECK_ARG(M > 0 && C > 0 && nm.x && nm.x2 && nm.y && nm.y2 && nm.w && nm.w2 && nm.rstd && nm.rstd2,
                  "post-norm backward: missing operand");
    if (vec_ok(C, {c, nm.x, nm.x2, nm.w, nm.w2, nm.resid, nm.y, nm.y2})) {
      const RowShape sh = row_shape(C);
      MFT_ROW_DISPATCH(sh, rms_bwd_post_vec, row_grid(M, sh), dim3(256), 0, s, c, M, (int)C, nm);
      MFT_LAUNCH_CHECK();
      return;
    }
    // row-loop fallback: the two backward passes as two launches
    rmsnorm_bwd(s, c, nm.x, nm.w, nm.rstd, M, C, nm.unit_offset != 0, nm.y, nm.resid);
    rmsnorm_bwd(s, nm.y, nm.x2, nm.w2, nm.rstd2, M, C, nm.unit_offset != 0, nm.y2, nullptr);
    return;
  }
  switch (nm.kind) {
    case NORM_LN_FWD: return layernorm_fwd(s, c, nm.w, nm.b, M, C, nm.eps, nm.y, nm.mean, nm.rstd);
    case NORM_RMS_FWD: return rmsnorm_fwd(s, c, nm.w, M, C, nm.eps, nm.unit_offset != 0, nm.y, nm.rstd);
    case NORM_LN_BWD: return layernorm_bwd(s, c, nm.x, nm.w, nm.mean, nm.rstd, M, C, nm.y, nm.resid);
    case NORM_RMS_BWD: return rmsnorm_bwd(s, c, nm.x, nm.w, nm.rstd, M, C, nm.unit_offset != 0, nm.y, nm.resid);
    default: MFT_CHECK_ARG(false, "unknown norm kind");
  }
}

void rope_table(hipStream_t s, double theta, int hd, int npos, float2* tab) {
  MFT_CHECK_ARG(hd % 2 == 0 && npos > 0 && tab, "rope table: bad shape");
  const int64_t n = (int64_t)npos * (hd / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 4096)), dim3(256), 0, s,
                     theta, hd, npos, tab);
  MFT_LAUNCH_CHECK();
}

namespace {
void check_heads(const HeadRows& r, int hd, bool fwd) {
  const int E = hd / 64;
  MFT_CHECK_ARG(r.H > 0 && r.in && r.out && r.in_ld >= (int64_t)r.H * hd && r.out_ld >= (int64_t)r.H * hd,
                "q/k head rows: bad shape");
  MFT_CHECK_ARG(r.in_ld % E == 0 && r.out_ld % E == 0 && ((uintptr_t)r.in % (4 * E)) == 0 &&
                    ((uintptr_t)r.out % (4 * E)) == 0,
                "q/k head rows: rows must be aligned to the lane vector");
  if (r.w) {
    MFT_CHECK_ARG(r.rstd != nullptr, "q/k head norm: rstd required");
    if (!fwd)
      MFT_CHECK_ARG(r.x && r.x_ld >= (int64_t)r.H * hd && r.x_ld % E == 0 && ((uintptr_t)r.x % (4 * E)) == 0,
                    "q/k head norm backward: saved input rows required");
  }
}
}  // namespace

#define MFT_QK_DISPATCH(KERNEL, NORM, ...)                                                                    \
  do {                                                                                                        \
    if (hd == 64) hipLaunchKernelGGL((KERNEL<1, NORM>), __VA_ARGS__);                                          \
    else if (hd == 128) hipLaunchKernelGGL((KERNEL<2, NORM>), __VA_ARGS__);                                    \
    else hipLaunchKernelGGL((KERNEL<4, NORM>), __VA_ARGS__);                                                   \
  } while (0)

void qk_rope_fwd(hipStream_t s, const HeadRows& q, const HeadRows& k, int64_t M, int S, int hd, float eps,
                 const float2* tab, int npos) {
  MFT_CHECK_ARG(hd == 64 || hd == 128 || hd == 256, "q/k head rows: head_dim must be 64, 128 or 256");
  MFT_CHECK_ARG(M > 0 && S > 0 && M % S == 0 && S <= npos && tab, "q/k head rows: positions past the RoPE table");
  MFT_CHECK_ARG((q.w == nullptr) == (k.w == nullptr), "q/k head rows: both or neither normalised");
  check_heads(q, hd, true);
  check_heads(k, hd, true);
  const int64_t rows = M * (q.H + k.H);
  const dim3 grid((unsigned)cdiv(rows, 4)), block(256);
  if (q.w) MFT_QK_DISPATCH(qk_rope_fwd_kernel, true, grid, block, 0, s, q, k, M, S, eps, tab);
  else MFT_QK_DISPATCH(qk_rope_fwd_kernel, false, grid, block, 0, s, q, k, M, S, eps, tab);
  MFT_LAUNCH_CHECK();
}

void qk_rope_bwd(hipStream_t s, const HeadRows& q, const HeadRows& k, int64_t M, int S, int hd, const float2* tab,
                 int npos) {
  MFT_CHECK_ARG(hd == 64 || hd == 128 || hd == 256, "q/k head rows: head_dim must be 64, 128 or 256");
  MFT_CHECK_ARG(M > 0 && S > 0 && M % S == 0 && S <= npos && tab, "q/k head rows: positions past the RoPE table");
  MFT_CHECK_ARG((q.w == nullptr) == (k.w == nullptr), "q/k head rows: both or neither normalised");
  check_heads(q, hd, false);
  check_heads(k, hd, false);
  const int64_t rows = M * (q.H + k.H);
  const dim3 grid((unsigned)cdiv(rows, 4)), block(256);
  if (q.w) MFT_QK_DISPATCH(qk_rope_bwd_kernel, true, grid, block, 0, s, q, k, M, S, tab);
  else MFT_QK_DISPATCH(qk_rope_bwd_kernel, false, grid, block, 0, s, q, k, M, S, tab);
  MFT_LAUNCH_CHECK();
}

bool embed_norm(hipStream_t s, const int32_t* ids, int64_t M, int S, const void* wte, int64_t V, bool w_f16,
                const float* wpe, int64_t C, float scale, float* x, int* bad, const RowNorm& nm, void* zero,
                int nzero) {
  if (M <= 0 || S <= 0 || V <= 0 || (nm.kind != NORM_LN_FWD && nm.kind != NORM_RMS_FWD)) return false;
  if (!vec_ok(C, {wpe, x, nm.w, nm.b, nm.y, w_f16 ? nullptr : wte}) || ((uintptr_t)wte & 7)) return false;
  const RowShape sh = row_shape(C);
  unsigned long long* z = static_cast<unsigned long long*>(zero);
  if (nm.kind == NORM_LN_FWD) {
    if (w_f16) embed_norm_launch<NORM_LN_FWD, true>(s, sh, ids, M, S, wte, V, wpe, (int)C, scale, x, bad, nm, z, nzero);
    else embed_norm_launch<NORM_LN_FWD, false>(s, sh, ids, M, S, wte, V, wpe, (int)C, scale, x, bad, nm, z, nzero);
  } else {
    if (w_f16) embed_norm_launch<NORM_RMS_FWD, true>(s, sh, ids, M, S, wte, V, wpe, (int)C, scale, x, bad, nm, z, nzero);
    else embed_norm_launch<NORM_RMS_FWD, false>(s, sh, ids, M, S, wte, V, wpe, (int)C, scale, x, bad, nm, z, nzero);
  }
  return true;
}

bool splitk_norm(hipStream_t s, const float* partial, int splits, int M, int N, float* C, int64_t ldc,
                 const GemmEpilogue& ep, const RowNorm& nm) {
  if (ldc != N || splits < 1 || M <= 0) return false;
  if (!vec_ok(N, {partial, C, ep.bias, ep.resid, ep.gelu_out, ep.gelu_grad_of, nm.w, nm.b, nm.y, nm.x, nm.resid,
                  nm.w2, nm.y2, nm.x2}))
    return false;
  const RowShape sh = row_shape(N);
  switch (nm.kind) {
    case NORM_LN_FWD: splitk_norm_launch<NORM_LN_FWD>(s, sh, partial, splits, M, N, C, ep, nm); return true;
    case NORM_RMS_FWD: splitk_norm_launch<NORM_RMS_FWD>(s, sh, partial, splits, M, N, C, ep, nm); return true;
    case NORM_LN_BWD: splitk_norm_launch<NORM_LN_BWD>(s, sh, partial, splits, M, N, C, ep, nm); return true;
    case NORM_RMS_BWD: splitk_norm_launch<NORM_RMS_BWD>(s, sh, partial, splits, M, N, C, ep, nm); return true;
    case NORM_RMS_RES_RMS:
      splitk_norm_launch<NORM_RMS_RES_RMS>(s, sh, partial, splits, M, N, C, ep, nm);
      return true;
    case NORM_RMS_BWD_POST:
      splitk_norm_launch<NORM_RMS_BWD_POST>(s, sh, partial, splits, M, N, C, ep, nm);
      return true;
    default: return false;
  }
}

}  // namespace mft
