// attention.hip — memory-efficient causal attention with GQA, forward and
// backward, for head_dim ∈ {64, 128, 256}.
//
// Forward: one workgroup per (query block, query head, batch).  Q, K, V
// blocks are staged in LDS; scores for a BQ×BKV tile are formed, the
// running row max / row sum are updated online (flash-style), and the
// output accumulator lives in registers.  The S×S probabilities are never
// written to HBM; lse [B,Hq,S] is kept for the backward.
// Backward: delta = rowsum(dO∘O); a key-block kernel recomputes P from lse
// and accumulates dK, dV for one KV head over every query head of its GQA
// group (no repeat_kv copy, no atomics); a query-block kernel recomputes P
// and dP and accumulates dQ.  All reductions have a fixed order.
#include "common.h"

namespace mft {
namespace {

struct AttnParams {
  const float *q, *k, *v, *o, *dout, *lse, *delta;
  int64_t q_rs, k_rs, v_rs, o_rs, do_rs;
  float *out, *lse_out, *dq, *dk, *dv;
  int64_t out_rs, dq_rs, dk_rs, dv_rs;
  int B, Hq, Hkv, S;
  float scale;
  int causal, window;
  const float* kpad;
};

__device__ __forceinline__ bool key_visible(const AttnParams& p, int b, int i, int j) {
  if (j >= p.S) return false;
  if (p.causal && j > i) return false;
  if (p.window > 0 && i - j >= p.window) return false;
  if (p.kpad && !(p.kpad[(int64_t)b * p.S + j] > 0.5f)) return false;
  return true;
}

// Range of key blocks that can be visible from query rows [q0, q1].
__device__ __forceinline__ void key_range(const AttnParams& p, int q0, int q1, int bkv,
                                          int& kb0, int& kb1) {
  int jmax = p.causal ? min(q1, p.S - 1) : p.S - 1;
  int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  kb0 = jmin / bkv;
  kb1 = jmax / bkv;  // inclusive
}

// TPR threads cooperate on one row; reduce among them.
template <int TPR>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = 1; off < TPR; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = 1; off < TPR; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ------------------------------------------------------------------------------
// Forward.  BQ query rows, BKV keys per tile, TPR = 256/BQ threads per row.
// Thread (row i, part t) owns output dims d = t + TPR*u.
// ------------------------------------------------------------------------------
template <int HD, int BQ, int BKV>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnParams p) {
  constexpr int TPR = 256 / BQ;
  constexpr int DPT = HD / TPR;
  constexpr int KP = HD + 1;     // LDS pitch for K (column reads by row)
  constexpr int PP = BKV + 1;
  extern __shared__ float smem[];
  float* Qs = smem;              // [BQ][KP]
  float* Ks = Qs + BQ * KP;      // [BKV][KP]
  float* Vs = Ks + BKV * KP;     // [BKV][HD]
  float* Ps = Vs + BKV * HD;     // [BQ][PP]

  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kh = h / (p.Hq / p.Hkv);
  const int q0 = qb * BQ;
  const int tid = threadIdx.x;
  const int ri = tid / TPR, part = tid % TPR;
  const int qi = q0 + ri;

  for (int e = tid; e < BQ * HD; e += 256) {
    const int r = e / HD, d = e % HD;
    const int gi = q0 + r;
    Qs[r * KP + d] = gi < p.S ? p.q[((int64_t)b * p.S + gi) * p.q_rs + (int64_t)h * HD + d] : 0.f;
  }
  float acc[DPT];
#pragma unroll
  for (int u = 0; u < DPT; ++u) acc[u] = 0.f;
  float mrow = -INFINITY, lrow = 0.f;

  int kb0, kb1;
  key_range(p, q0, min(q0 + BQ - 1, p.S - 1), BKV, kb0, kb1);
  for (int kb = kb0; kb <= kb1; ++kb) {
    const int j0 = kb * BKV;
    __syncthreads();  // previous tile fully consumed
    for (int e = tid; e < BKV * HD; e += 256) {
      const int r = e / HD, d = e % HD;
      const int gj = j0 + r;
      float kv = 0.f, vv = 0.f;
      if (gj < p.S) {
        kv = p.k[((int64_t)b * p.S + gj) * p.k_rs + (int64_t)kh * HD + d];
        vv = p.v[((int64_t)b * p.S + gj) * p.v_rs + (int64_t)kh * HD + d];
      }
      Ks[r * KP + d] = kv;
      Vs[r * HD + d] = vv;
    }
    __syncthreads();
    // scores for keys j = part, part+TPR, ...
    float bmax = -INFINITY;
    for (int jj = part; jj < BKV; jj += TPR) {
      float sc = -INFINITY;
      if (qi < p.S && key_visible(p, b, qi, j0 + jj)) {
        float s = 0.f;
#pragma unroll 8
        for (int d = 0; d < HD; ++d) s = fmaf(Qs[ri * KP + d], Ks[jj * KP + d], s);
        sc = s * p.scale;
      }
      Ps[ri * PP + jj] = sc;
      bmax = fmaxf(bmax, sc);
    }
    bmax = group_max<TPR>(bmax);
    const float mnew = fmaxf(mrow, bmax);
    float corr = 1.f, lsum = 0.f;
    if (mnew > -INFINITY) {
      corr = __expf(mrow - mnew);
      for (int jj = part; jj < BKV; jj += TPR) {
        const float sc = Ps[ri * PP + jj];
        const float e = sc > -INFINITY ? __expf(sc - mnew) : 0.f;
        Ps[ri * PP + jj] = e;
        lsum += e;
      }
    } else {
      for (int jj = part; jj < BKV; jj += TPR) Ps[ri * PP + jj] = 0.f;
    }
    lsum = group_sum<TPR>(lsum);
    lrow = lrow * corr + lsum;
    mrow = mnew;
    __syncthreads();  // P row written by all TPR threads of the row
#pragma unroll
    for (int u = 0; u < DPT; ++u) acc[u] *= corr;
    for (int jj = 0; jj < BKV; ++jj) {
      const float pv = Ps[ri * PP + jj];
#pragma unroll
      for (int u = 0; u < DPT; ++u) acc[u] = fmaf(pv, Vs[jj * HD + part + TPR * u], acc[u]);
    }
  }
  if (qi < p.S) {
    const float inv = lrow > 0.f ? 1.f / lrow : 0.f;
    float* orow = p.out + ((int64_t)b * p.S + qi) * p.out_rs + (int64_t)h * HD;
#pragma unroll
    for (int u = 0; u < DPT; ++u) orow[part + TPR * u] = acc[u] * inv;
    if (part == 0)
      p.lse_out[((int64_t)b * p.Hq + h) * p.S + qi] = lrow > 0.f ? mrow + logf(lrow) : -INFINITY;
  }
}

// delta[b,h,i] = Σ_d dO[i,d]·O[i,d]; one wave per row.
template <int HD>
__global__ __launch_bounds__(256) void attn_delta_kernel(AttnParams p, float* delta) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // over B*S*Hq
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)p.B * p.S * p.Hq;
  if (row >= total) return;
  const int h = (int)(row % p.Hq);
  const int64_t tok = row / p.Hq;
  const float* o = p.o + tok * p.o_rs + (int64_t)h * HD;
  const float* g = p.dout + tok * p.do_rs + (int64_t)h * HD;
  float s = 0.f;
  for (int d = lane; d < HD; d += 64) s = fmaf(o[d], g[d], s);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) {
    const int b = (int)(tok / p.S), i = (int)(tok % p.S);
    delta[((int64_t)b * p.Hq + h) * p.S + i] = s;
  }
}

// ------------------------------------------------------------------------------
// dK, dV: one workgroup per (key block, KV head, batch); loops over the query
// heads of the group and the query blocks that can see the key block.
// Thread (key row r, part t) owns dims d = t + TPR*u of dK and dV.
// ------------------------------------------------------------------------------
template <int HD, int BQ, int BKV>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnParams p) {
  constexpr int TPR = 256 / BKV;
  constexpr int DPT = HD / TPR;
  constexpr int KP = HD + 1;
  constexpr int PP = BKV + 1;
  extern __shared__ float smem[];
  float* Ks = smem;             // [BKV][KP]
  float* Vs = Ks + BKV * KP;    // [BKV][KP]
  float* Qs = Vs + BKV * KP;    // [BQ][KP]
  float* Gs = Qs + BQ * KP;     // [BQ][KP]   dO
  float* Ps = Gs + BQ * KP;     // [BQ][PP]   P
  float* Ds = Ps + BQ * PP;     // [BQ][PP]   dS
  float* Ls = Ds + BQ * PP;     // [BQ]       lse
  float* Es = Ls + BQ;          // [BQ]       delta

  const int kb = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int grp = p.Hq / p.Hkv;
  const int j0 = kb * BKV;
  const int tid = threadIdx.x;
  const int rj = tid / TPR, part = tid % TPR;

  for (int e = tid; e < BKV * HD; e += 256) {
    const int r = e / HD, d = e % HD;
    const int gj = j0 + r;
    float kv = 0.f, vv = 0.f;
    if (gj < p.S) {
      kv = p.k[((int64_t)b * p.S + gj) * p.k_rs + (int64_t)kh * HD + d];
      vv = p.v[((int64_t)b * p.S + gj) * p.v_rs + (int64_t)kh * HD + d];
    }
    Ks[r * KP + d] = kv;
    Vs[r * KP + d] = vv;
  }
  float dK[DPT], dV[DPT];
#pragma unroll
  for (int u = 0; u < DPT; ++u) dK[u] = dV[u] = 0.f;

  // query rows that can see keys [j0, j0+BKV-1]
  const int jl = min(j0 + BKV - 1, p.S - 1);
  const int qstart = p.causal ? j0 : 0;
  const int qend = p.window > 0 ? min(p.S - 1, jl + p.window - 1) : p.S - 1;
  const int qb0 = qstart / BQ, qb1 = qend / BQ;
  constexpr int NT = BQ * BKV / 256;  // score elements per thread

  for (int hh = 0; hh < grp; ++hh) {
    const int h = kh * grp + hh;
    for (int qb = qb0; qb <= qb1; ++qb) {
      const int q0 = qb * BQ;
      __syncthreads();
      for (int e = tid; e < BQ * HD; e += 256) {
        const int r = e / HD, d = e % HD;
        const int gi = q0 + r;
        float qv = 0.f, gv = 0.f;
        if (gi < p.S) {
          qv = p.q[((int64_t)b * p.S + gi) * p.q_rs + (int64_t)h * HD + d];
          gv = p.dout[((int64_t)b * p.S + gi) * p.do_rs + (int64_t)h * HD + d];
        }
        Qs[r * KP + d] = qv;
        Gs[r * KP + d] = gv;
      }
      for (int e = tid; e < BQ; e += 256) {
        const int gi = q0 + e;
        const int64_t li = ((int64_t)b * p.Hq + h) * p.S + gi;
        Ls[e] = gi < p.S ? p.lse[li] : -INFINITY;
        Es[e] = gi < p.S ? p.delta[li] : 0.f;
      }
      __syncthreads();
      // P and dS for the BQ×BKV tile; element (i, j) with j fastest.
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int e = tid + 256 * t;
        const int i = e / BKV, j = e % BKV;
        const int gi = q0 + i, gj = j0 + j;
        float pv = 0.f, ds = 0.f;
        if (gi < p.S && key_visible(p, b, gi, gj) && Ls[i] > -INFINITY) {
          float s = 0.f, dp = 0.f;
#pragma unroll 8
          for (int d = 0; d < HD; ++d) {
            s = fmaf(Qs[i * KP + d], Ks[j * KP + d], s);
            dp = fmaf(Gs[i * KP + d], Vs[j * KP + d], dp);
          }
          pv = __expf(s * p.scale - Ls[i]);
          ds = pv * (dp - Es[i]) * p.scale;
        }
        Ps[i * PP + j] = pv;
        Ds[i * PP + j] = ds;
      }
      __syncthreads();
      for (int i = 0; i < BQ; ++i) {
        const float pv = Ps[i * PP + rj];
        const float ds = Ds[i * PP + rj];
#pragma unroll
        for (int u = 0; u < DPT; ++u) {
          const int d = part + TPR * u;
          dV[u] = fmaf(pv, Gs[i * KP + d], dV[u]);
          dK[u] = fmaf(ds, Qs[i * KP + d], dK[u]);
        }
      }
    }
  }
  const int gj = j0 + rj;
  if (gj < p.S) {
    float* dkr = p.dk + ((int64_t)b * p.S + gj) * p.dk_rs + (int64_t)kh * HD;
    float* dvr = p.dv + ((int64_t)b * p.S + gj) * p.dv_rs + (int64_t)kh * HD;
#pragma unroll
    for (int u = 0; u < DPT; ++u) {
      dkr[part + TPR * u] = dK[u];
      dvr[part + TPR * u] = dV[u];
    }
  }
}

// ------------------------------------------------------------------------------
// dQ: one workgroup per (query block, query head, batch).
// ------------------------------------------------------------------------------
template <int HD, int BQ, int BKV>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnParams p) {
  constexpr int TPR = 256 / BQ;
  constexpr int DPT = HD / TPR;
  constexpr int KP = HD + 1;
  constexpr int PP = BKV + 1;
  extern __shared__ float smem[];
  float* Qs = smem;             // [BQ][KP]
  float* Gs = Qs + BQ * KP;     // [BQ][KP]
  float* Ks = Gs + BQ * KP;     // [BKV][KP]
  float* Vs = Ks + BKV * KP;    // [BKV][KP]
  float* Ds = Vs + BKV * KP;    // [BQ][PP]
  float* Ls = Ds + BQ * PP;
  float* Es = Ls + BQ;

  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kh = h / (p.Hq / p.Hkv);
  const int q0 = qb * BQ;
  const int tid = threadIdx.x;
  const int ri = tid / TPR, part = tid % TPR;
  for (int e = tid; e < BQ * HD; e += 256) {
    const int r = e / HD, d = e % HD;
    const int gi = q0 + r;
    float qv = 0.f, gv = 0.f;
    if (gi < p.S) {
      qv = p.q[((int64_t)b * p.S + gi) * p.q_rs + (int64_t)h * HD + d];
      gv = p.dout[((int64_t)b * p.S + gi) * p.do_rs + (int64_t)h * HD + d];
    }
    Qs[r * KP + d] = qv;
    Gs[r * KP + d] = gv;
  }
  for (int e = tid; e < BQ; e += 256) {
    const int gi = q0 + e;
    const int64_t li = ((int64_t)b * p.Hq + h) * p.S + gi;
    Ls[e] = gi < p.S ? p.lse[li] : -INFINITY;
    Es[e] = gi < p.S ? p.delta[li] : 0.f;
  }
  float dQ[DPT];
#pragma unroll
  for (int u = 0; u < DPT; ++u) dQ[u] = 0.f;
  int kb0, kb1;
  key_range(p, q0, min(q0 + BQ - 1, p.S - 1), BKV, kb0, kb1);
  constexpr int NT = BQ * BKV / 256;
  for (int kb = kb0; kb <= kb1; ++kb) {
    const int j0 = kb * BKV;
    __syncthreads();
    for (int e = tid; e < BKV * HD; e += 256) {
      const int r = e / HD, d = e % HD;
      const int gj = j0 + r;
      float kv = 0.f, vv = 0.f;
      if (gj < p.S) {
        kv = p.k[((int64_t)b * p.S + gj) * p.k_rs + (int64_t)kh * HD + d];
        vv = p.v[((int64_t)b * p.S + gj) * p.v_rs + (int64_t)kh * HD + d];
      }
      Ks[r * KP + d] = kv;
      Vs[r * KP + d] = vv;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int e = tid + 256 * t;
      const int i = e / BKV, j = e % BKV;
      const int gi = q0 + i, gj = j0 + j;
      float ds = 0.f;
      if (gi < p.S && key_visible(p, b, gi, gj) && Ls[i] > -INFINITY) {
        float s = 0.f, dp = 0.f;
#pragma unroll 8
        for (int d = 0; d < HD; ++d) {
          s = fmaf(Qs[i * KP + d], Ks[j * KP + d], s);
          dp = fmaf(Gs[i * KP + d], Vs[j * KP + d], dp);
        }
        const float pv = __expf(s * p.scale - Ls[i]);
        ds = pv * (dp - Es[i]) * p.scale;
      }
      Ds[i * PP + j] = ds;
    }
    __syncthreads();
    for (int j = 0; j < BKV; ++j) {
      const float ds = Ds[ri * PP + j];
#pragma unroll
      for (int u = 0; u < DPT; ++u) dQ[u] = fmaf(ds, Ks[j * KP + part + TPR * u], dQ[u]);
    }
  }
  const int gi = q0 + ri;
  if (gi < p.S) {
    float* dqr = p.dq + ((int64_t)b * p.S + gi) * p.dq_rs + (int64_t)h * HD;
#pragma unroll
    for (int u = 0; u < DPT; ++u) dqr[part + TPR * u] = dQ[u];
  }
}

template <int HD>
struct Tiles;
template <> struct Tiles<64>  { static constexpr int BQ = 64, BKV = 64; };
template <> struct Tiles<128> { static constexpr int BQ = 32, BKV = 32; };
template <> struct Tiles<256> { static constexpr int BQ = 32, BKV = 32; };

template <typename K>
void set_lds(K kernel, size_t bytes) {
  MFT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
}

template <int HD>
void fwd_impl(hipStream_t s, AttnParams& p) {
  constexpr int BQ = Tiles<HD>::BQ, BKV = Tiles<HD>::BKV;
  const size_t lds = sizeof(float) * (BQ * (HD + 1) + BKV * (HD + 1) + BKV * HD + BQ * (BKV + 1));
  auto kern = attn_fwd_kernel<HD, BQ, BKV>;
  set_lds(kern, lds);
  dim3 grid((unsigned)cdiv(p.S, BQ), p.Hq, p.B);
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, p);
  MFT_LAUNCH_CHECK();
}

template <int HD>
void bwd_impl(hipStream_t s, AttnParams& p, float* delta) {
  constexpr int BQ = Tiles<HD>::BQ, BKV = Tiles<HD>::BKV;
  const int64_t rows = (int64_t)p.B * p.S * p.Hq;
  hipLaunchKernelGGL(attn_delta_kernel<HD>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p, delta);
  MFT_LAUNCH_CHECK();
  p.delta = delta;
  {
    const size_t lds = sizeof(float) * (2 * BKV * (HD + 1) + 2 * BQ * (HD + 1) + 2 * BQ * (BKV + 1) + 2 * BQ);
    auto kern = attn_bwd_dkdv_kernel<HD, BQ, BKV>;
    set_lds(kern, lds);
    dim3 grid((unsigned)cdiv(p.S, BKV), p.Hkv, p.B);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, p);
    MFT_LAUNCH_CHECK();
  }
  {
    const size_t lds = sizeof(float) * (2 * BQ * (HD + 1) + 2 * BKV * (HD + 1) + BQ * (BKV + 1) + 2 * BQ);
    auto kern = attn_bwd_dq_kernel<HD, BQ, BKV>;
    set_lds(kern, lds);
    dim3 grid((unsigned)cdiv(p.S, BQ), p.Hq, p.B);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, p);
    MFT_LAUNCH_CHECK();
  }
}

AttnParams make_params(const AttnArgs& a) {
  MFT_CHECK_ARG(a.B > 0 && a.S > 0 && a.Hq > 0 && a.Hkv > 0, "empty attention");
  MFT_CHECK_ARG(a.Hq % a.Hkv == 0, "Hq must be a multiple of Hkv");
  MFT_CHECK_ARG(a.hd == 64 || a.hd == 128 || a.hd == 256, "head_dim must be 64, 128 or 256");
  AttnParams p{};
  p.q = a.q; p.k = a.k; p.v = a.v;
  p.q_rs = a.q_rs; p.k_rs = a.k_rs; p.v_rs = a.v_rs;
  p.B = a.B; p.Hq = a.Hq; p.Hkv = a.Hkv; p.S = a.S;
  p.scale = a.scale;
  p.causal = a.causal;
  p.window = a.window;
  p.kpad = a.kpad;
  return p;
}

}  // namespace

void attn_fwd(hipStream_t s, const AttnArgs& a, float* o, int64_t o_rs,
              float* lse) {
  AttnParams p = make_params(a);
  MFT_CHECK_ARG(o && lse, "null output");
  p.out = o;
  p.out_rs = o_rs;
  p.lse_out = lse;
  switch (a.hd) {
    case 64: fwd_impl<64>(s, p); break;
    case 128: fwd_impl<128>(s, p); break;
    default: fwd_impl<256>(s, p); break;
  }
}

void attn_bwd(hipStream_t s, const AttnArgs& a, const float* o, int64_t o_rs,
              const float* dout, int64_t do_rs, const float* lse, float* dq,
              int64_t dq_rs, float* dk, int64_t dk_rs, float* dv,
              int64_t dv_rs, float* delta_scratch) {
  AttnParams p = make_params(a);
  MFT_CHECK_ARG(o && dout && lse && dq && dk && dv && delta_scratch, "null tensor");
  p.o = o; p.o_rs = o_rs;
  p.dout = dout; p.do_rs = do_rs;
  p.lse = lse;
  p.dq = dq; p.dq_rs = dq_rs;
  p.dk = dk; p.dk_rs = dk_rs;
  p.dv = dv; p.dv_rs = dv_rs;
  switch (a.hd) {
    case 64: bwd_impl<64>(s, p, delta_scratch); break;
    case 128: bwd_impl<128>(s, p, delta_scratch); break;
    default: bwd_impl<256>(s, p, delta_scratch); break;
  }
}

}  // namespace mft
