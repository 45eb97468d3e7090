// attention_mfma.hip — causal GQA attention on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32), forward and backward, head_dim ∈ {64,128,256}.
//
// Lane layout of one 16×16×4 MFMA (lane l, i = l%16, g = l/16):
//   A[row i][k g], B[k g][col i], D[row 4g+v][col i] (v = 0..3).
// Inside each 16-wide slice of the reduction dimension, lane (i,g) supplies
// elements 4g..4g+3 over four consecutive MFMAs (the same permutation for A
// and B), so every operand fetch is one 128-bit read.
//
// Forward (per wave: 16 queries; per workgroup: 16·NW queries).  Scores are
// formed transposed, Sᵀ = K·Qᵀ, so a lane owns one query (column i) and four
// keys (rows 4g+v): the row max / row sum of the online softmax reduce over
// the lane's own values plus two cross-lane xor-shuffles, and the
// probabilities are already in the B-operand layout of Oᵀ += Vᵀ·Pᵀ — P never
// leaves registers.  Q stays in registers; K/V blocks are staged in LDS
// (pitch hd+4: conflict-free 128-bit and 32-bit reads).
//
// Backward: delta = rowsum(dO∘O) (one pass), then
//   dK/dV kernel — per wave 16 keys of one QUERY head; S and dP formed with
//     keys as columns so Pᵀ and dSᵀ feed dV += Pᵀ·dO and dK += dSᵀ·Q from
//     registers.  With GQA groups > 1 each query head writes a partial and a
//     small pass sums the group in head order (no repeat_kv copy, no atomics,
//     deterministic);
//   dQ kernel — per wave 16 queries; Sᵀ, dPᵀ transposed as in the forward so
//     dS feeds dQ += dS·K from registers.
// P is recomputed from the saved lse in both backward kernels.
#include <cstdlib>

#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace mft {
namespace {

struct AttnP {
  const float *q, *k, *v, *o, *dout, *lse, *delta;
  int64_t q_rs, k_rs, v_rs, o_rs, do_rs;
  float *out, *lse_out, *dq, *dk, *dv, *delta_out;
  float *pdk, *pdv;  // per-query-head dK/dV partials [B,S,Hq,hd] (GQA groups > 1)
  int64_t out_rs, dq_rs, dk_rs, dv_rs;
  int B, Hq, Hkv, S;
  float scale;
  int causal, window;
  const float* kpad;
};

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bool visible(const AttnP& p, int i, int j, const float* kp) {
  if (j >= p.S || i >= p.S) return false;
  if (p.causal && j > i) return false;
  if (p.window > 0 && i - j >= p.window) return false;
  if (kp && !(kp[j] > 0.5f)) return false;
  return true;
}

// Stage rows [r0, r0+ROWS) of two token-major [.., S, H, HD] tensors (head
// h) into LDS with pitch HD+4; rows past S are zero.  Branch-free: row
// indices are clamped into the tensor and the values selected to zero, and
// each thread issues a batch of CH loads per tensor before any LDS store, so
// a block's loads are in flight together instead of one latency per element.
template <int HD, int NT, int ROWS>
__device__ __forceinline__ void stage_pair(float* lds1, const float* src1, int64_t rs1, float* lds2,
                                           const float* src2, int64_t rs2, int b, int S, int h1, int h2,
                                           int r0, int tid) {
  constexpr int P = HD + 4;
  constexpr int TOTAL = ROWS * (HD / 4);
  static_assert(TOTAL % NT == 0, "staging shape");
  constexpr int ITEMS = TOTAL / NT;
  constexpr int CH = ITEMS < 512 / HD ? ITEMS : 512 / HD;
  static_assert(ITEMS % CH == 0, "staging batch");
#pragma unroll
  for (int base = 0; base < ITEMS; base += CH) {
    floatx4 v1[CH], v2[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int f = tid + NT * (base + c);
      const int r = f / (HD / 4), c4 = f % (HD / 4);
      const int gr = min(r0 + r, S - 1);
      const int64_t row = (int64_t)b * S + gr;
      v1[c] = *reinterpret_cast<const floatx4*>(src1 + row * rs1 + (int64_t)h1 * HD + 4 * c4);
      v2[c] = *reinterpret_cast<const floatx4*>(src2 + row * rs2 + (int64_t)h2 * HD + 4 * c4);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int f = tid + NT * (base + c);
      const int r = f / (HD / 4), c4 = f % (HD / 4);
      const bool ok = r0 + r < S;
      const floatx4 z = floatx4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<floatx4*>(lds1 + r * P + 4 * c4) = ok ? v1[c] : z;
      *reinterpret_cast<floatx4*>(lds2 + r * P + 4 * c4) = ok ? v2[c] : z;
    }
  }
}

// ------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------
template <int HD, int NW, int BKV>
__global__ __launch_bounds__(64 * NW) void attn_fwd_mfma(AttnP p) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;
  constexpr int NC = HD / 16;   // 16-wide slices of head_dim
  constexpr int KT = BKV / 16;  // key tiles per block
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ks = smem;            // [BKV][P]
  float* Vs = Ks + BKV * P;    // [BKV][P]
  float* Kp = Vs + BKV * P;    // [BKV] key-padding flags

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // 1-D grid, heaviest causal query blocks (the last ones) first.
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int nqb = (p.S + 16 * NW - 1) / (16 * NW);
  const int kh = h / (p.Hq / p.Hkv);
  const int q0 = (nqb - 1 - (int)blockIdx.x / (p.Hq * p.B)) * 16 * NW;
  const int qbase = q0 + 16 * w;
  const int qi = qbase + li;  // this lane's query
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;

  floatx4 qreg[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    qreg[c] = qi < p.S ? *reinterpret_cast<const floatx4*>(p.q + ((int64_t)b * p.S + qi) * p.q_rs +
                                                          (int64_t)h * HD + 16 * c + 4 * lg)
                       : floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;

  const int qlast_wg = min(q0 + 16 * NW - 1, p.S - 1);
  const int jmax = p.causal ? qlast_wg : p.S - 1;
  const int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  const int wave_qlast = min(qbase + 15, p.S - 1);
  for (int j0 = (jmin / BKV) * BKV; j0 <= jmax; j0 += BKV) {
    __syncthreads();
    stage_pair<HD, NT, BKV>(Ks, p.k, p.k_rs, Vs, p.v, p.v_rs, b, p.S, kh, kh, j0, tid);
    if (kpb)
      for (int j = tid; j < BKV; j += NT) Kp[j] = j0 + j < p.S ? kpb[j0 + j] : 0.f;
    __syncthreads();
    if (qbase > p.S - 1) continue;
    // skip tiles this wave cannot see
    floatx4 sacc[KT];
    bool tile_live[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int jt0 = j0 + 16 * kt;
      bool live = jt0 < p.S && !(p.causal && jt0 > wave_qlast);
      if (p.window > 0 && wave_qlast - (jt0 + 15) >= p.window + 15) live = false;
      tile_live[kt] = live;
      sacc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (!live) continue;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 kv = *reinterpret_cast<const floatx4*>(&Ks[(16 * kt + li) * P + 16 * c + 4 * lg]);
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[kt] = mfma4(kv[t], qreg[c][t], sacc[kt]);
      }
    }
    // lane holds S[q = qi][key = j0 + 16kt + 4lg + v]
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = j0 + 16 * kt + 4 * lg + v;
        const bool ok = tile_live[kt] && visible(p, qi, j, kpb ? Kp - j0 : nullptr);
        const float sv = ok ? sacc[kt][v] * p.scale : -INFINITY;
        sacc[kt][v] = sv;
        mloc = fmaxf(mloc, sv);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mnew = fmaxf(mrow, mloc);
    float corr = 1.f, lsum = 0.f;
    if (mnew > -INFINITY) {
      corr = __expf(mrow - mnew);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = sacc[kt][v] > -INFINITY ? __expf(sacc[kt][v] - mnew) : 0.f;
          sacc[kt][v] = e;
          lsum += e;
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) sacc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    lrow = lrow * corr + lsum;
    mrow = mnew;
#pragma unroll
    for (int c = 0; c < NC; ++c) oacc[c] *= corr;
    // Oᵀ[d][q] += Vᵀ[d][key] · Pᵀ[key][q]
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      if (!tile_live[kt]) continue;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          oacc[c] = mfma4(Vs[(16 * kt + 4 * lg + t) * P + 16 * c + li], sacc[kt][t], oacc[c]);
    }
  }
  // lane holds Oᵀ[d = 16c + 4lg + v][q = qi]; transpose through LDS for
  // coalesced row stores.
  __syncthreads();
  float* Os = smem;  // [16*NW][P]
  const float inv = lrow > 0.f ? 1.f / lrow : 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) Os[(16 * w + li) * P + 16 * c + 4 * lg + v] = oacc[c][v] * inv;
  if (lg == 0 && qi < p.S)
    p.lse_out[((int64_t)b * p.Hq + h) * p.S + qi] = lrow > 0.f ? mrow + __logf(lrow) : -INFINITY;
  __syncthreads();
  for (int f = tid; f < 16 * NW * (HD / 4); f += NT) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gq = q0 + r;
    if (gq < p.S)
      *reinterpret_cast<floatx4*>(p.out + ((int64_t)b * p.S + gq) * p.out_rs + (int64_t)h * HD + 4 * c4) =
          *reinterpret_cast<const floatx4*>(&Os[r * P + 4 * c4]);
  }
}

// delta[b,h,i] = Σ_d dO[i,d]·O[i,d]; one wave per row.
template <int HD>
__global__ __launch_bounds__(256) void attn_delta_mfma_kernel(AttnP p) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)p.B * p.S * p.Hq) return;
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
    p.delta_out[((int64_t)b * p.Hq + h) * p.S + i] = s;
  }
}

// ------------------------------------------------------------------------------
// dK, dV: workgroup = 16·NW keys of one KV head; wave = 16 keys.
// ------------------------------------------------------------------------------
template <int HD, int NW, int BQ>
__global__ __launch_bounds__(64 * NW) void attn_bwd_dkdv_mfma(AttnP p) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;
  constexpr int NC = HD / 16;
  constexpr int QT = BQ / 16;
  constexpr int BKEYS = 16 * NW;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ks = smem;               // [BKEYS][P]
  float* Vs = Ks + BKEYS * P;     // [BKEYS][P]
  float* Qs = Vs + BKEYS * P;     // [BQ][P]
  float* Gs = Qs + BQ * P;        // [BQ][P]  dO
  float* Ls = Gs + BQ * P;        // [BQ] lse
  float* Es = Ls + BQ;            // [BQ] delta
  float* Kp = Es + BQ;            // [BKEYS]

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // One workgroup per (key block, QUERY head): a GQA group's query heads
  // run in parallel and their dK/dV contributions are summed afterwards by
  // attn_group_sum_kernel in head order.
  // 1-D grid, heaviest causal key blocks (the first ones) first.
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int grp = p.Hq / p.Hkv;
  const int kh = h / grp;
  const int k0 = ((int)blockIdx.x / (p.Hq * p.B)) * BKEYS;
  const int kbase = k0 + 16 * w;
  const int kj = kbase + li;  // this lane's key (as S column)
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;

  stage_pair<HD, NT, BKEYS>(Ks, p.k, p.k_rs, Vs, p.v, p.v_rs, b, p.S, kh, kh, k0, tid);
  if (kpb)
    for (int j = tid; j < BKEYS; j += NT) Kp[j] = k0 + j < p.S ? kpb[k0 + j] : 0.f;

  floatx4 dkacc[NC], dvacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dkacc[c] = dvacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int klast = min(k0 + BKEYS - 1, p.S - 1);
  const int qstart = p.causal ? k0 : 0;
  const int qend = p.window > 0 ? min(p.S - 1, klast + p.window - 1) : p.S - 1;
  {
    for (int qb0 = (qstart / BQ) * BQ; qb0 <= qend; qb0 += BQ) {
      __syncthreads();
      stage_pair<HD, NT, BQ>(Qs, p.q, p.q_rs, Gs, p.dout, p.do_rs, b, p.S, h, h, qb0, tid);
      for (int e = tid; e < BQ; e += NT) {
        const int gi = qb0 + e;
        const int64_t l = ((int64_t)b * p.Hq + h) * p.S + gi;
        Ls[e] = gi < p.S ? p.lse[l] : -INFINITY;
        Es[e] = gi < p.S ? p.delta[l] : 0.f;
      }
      __syncthreads();
      if (kbase > p.S - 1) continue;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int qt0 = qb0 + 16 * qt;
        if (qt0 > p.S - 1) continue;
        if (p.causal && qt0 + 15 < kbase) continue;
        if (p.window > 0 && qt0 - (kbase + 15) >= p.window) continue;
        // S[q][key] and dP[q][key]: D[row q = 4lg+v][col key = li]
        floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const floatx4 qa = *reinterpret_cast<const floatx4*>(&Qs[(16 * qt + li) * P + 16 * c + 4 * lg]);
          const floatx4 ga = *reinterpret_cast<const floatx4*>(&Gs[(16 * qt + li) * P + 16 * c + 4 * lg]);
          const floatx4 kb = *reinterpret_cast<const floatx4*>(&Ks[(16 * w + li) * P + 16 * c + 4 * lg]);
          const floatx4 vb = *reinterpret_cast<const floatx4*>(&Vs[(16 * w + li) * P + 16 * c + 4 * lg]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            s4 = mfma4(qa[t], kb[t], s4);
            dp4 = mfma4(ga[t], vb[t], dp4);
          }
        }
        floatx4 pv, ds;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int qr = 16 * qt + 4 * lg + v;
          const int gi = qb0 + qr;
          const float lse = Ls[qr];
          float pp = 0.f, d = 0.f;
          if (lse > -INFINITY && visible(p, gi, kj, kpb ? Kp - k0 : nullptr)) {
            pp = __expf(s4[v] * p.scale - lse);
            d = pp * (dp4[v] - Es[qr]) * p.scale;
          }
          pv[v] = pp;
          ds[v] = d;
        }
        // dV[key][d] += Σ_q P[q][key] dO[q][d];  dK[key][d] += Σ_q dS[q][key] Q[q][d]
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int qr = 16 * qt + 4 * lg + t;
            dvacc[c] = mfma4(pv[t], Gs[qr * P + 16 * c + li], dvacc[c]);
            dkacc[c] = mfma4(ds[t], Qs[qr * P + 16 * c + li], dkacc[c]);
          }
      }
    }
  }
  // lane holds [key = kbase + 4lg + v][d = 16c + li]; a group of one query
  // head writes dK/dV directly, larger groups write per-head partials.
  const bool direct = grp == 1;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gk = kbase + 4 * lg + v;
    if (gk >= p.S) continue;
    const int64_t tok = (int64_t)b * p.S + gk;
    float* dkr = direct ? p.dk + tok * p.dk_rs + (int64_t)kh * HD : p.pdk + (tok * p.Hq + h) * HD;
    float* dvr = direct ? p.dv + tok * p.dv_rs + (int64_t)kh * HD : p.pdv + (tok * p.Hq + h) * HD;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      dkr[16 * c + li] = dkacc[c][v];
      dvr[16 * c + li] = dvacc[c][v];
    }
  }
}

// dK/dV[b,s,kh,:] = Σ_{j<grp} partial[b,s,kh·grp+j,:], in j order.
template <int HD>
__global__ __launch_bounds__(256) void attn_group_sum_kernel(AttnP p) {
  const int grp = p.Hq / p.Hkv;
  const int64_t total = (int64_t)p.B * p.S * p.Hkv * (HD / 4);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c4 = (int)(i % (HD / 4));
    const int64_t r = i / (HD / 4);
    const int kh = (int)(r % p.Hkv);
    const int64_t tok = r / p.Hkv;
    floatx4 sk = floatx4{0.f, 0.f, 0.f, 0.f}, sv = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < grp; ++j) {
      const int64_t off = (tok * p.Hq + kh * grp + j) * HD + 4 * c4;
      sk += *reinterpret_cast<const floatx4*>(p.pdk + off);
      sv += *reinterpret_cast<const floatx4*>(p.pdv + off);
    }
    float* dk = p.dk + tok * p.dk_rs + (int64_t)kh * HD + 4 * c4;
    float* dv = p.dv + tok * p.dv_rs + (int64_t)kh * HD + 4 * c4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dk[e] = sk[e];
      dv[e] = sv[e];
    }
  }
}

// ------------------------------------------------------------------------------
// dQ: workgroup = 16·NW queries of one head; wave = 16 queries.
// ------------------------------------------------------------------------------
template <int HD, int NW, int BKV>
__global__ __launch_bounds__(64 * NW) void attn_bwd_dq_mfma(AttnP p) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;
  constexpr int NC = HD / 16;
  constexpr int KT = BKV / 16;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ks = smem;            // [BKV][P]
  float* Vs = Ks + BKV * P;    // [BKV][P]
  float* Kp = Vs + BKV * P;    // [BKV]

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int nqb = (p.S + 16 * NW - 1) / (16 * NW);
  const int kh = h / (p.Hq / p.Hkv);
  const int q0 = (nqb - 1 - (int)blockIdx.x / (p.Hq * p.B)) * 16 * NW;
  const int qbase = q0 + 16 * w;
  const int qi = qbase + li;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;

  floatx4 qreg[NC], greg[NC], dqacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t off = (int64_t)h * HD + 16 * c + 4 * lg;
    const bool ok = qi < p.S;
    qreg[c] = ok ? *reinterpret_cast<const floatx4*>(p.q + ((int64_t)b * p.S + qi) * p.q_rs + off)
                 : floatx4{0.f, 0.f, 0.f, 0.f};
    greg[c] = ok ? *reinterpret_cast<const floatx4*>(p.dout + ((int64_t)b * p.S + qi) * p.do_rs + off)
                 : floatx4{0.f, 0.f, 0.f, 0.f};
    dqacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float lse = -INFINITY, dlt = 0.f;
  if (qi < p.S) {
    const int64_t l = ((int64_t)b * p.Hq + h) * p.S + qi;
    lse = p.lse[l];
    dlt = p.delta[l];
  }
  const int qlast_wg = min(q0 + 16 * NW - 1, p.S - 1);
  const int jmax = p.causal ? qlast_wg : p.S - 1;
  const int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  const int wave_qlast = min(qbase + 15, p.S - 1);
  for (int j0 = (jmin / BKV) * BKV; j0 <= jmax; j0 += BKV) {
    __syncthreads();
    stage_pair<HD, NT, BKV>(Ks, p.k, p.k_rs, Vs, p.v, p.v_rs, b, p.S, kh, kh, j0, tid);
    if (kpb)
      for (int j = tid; j < BKV; j += NT) Kp[j] = j0 + j < p.S ? kpb[j0 + j] : 0.f;
    __syncthreads();
    if (qbase > p.S - 1) continue;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int jt0 = j0 + 16 * kt;
      if (jt0 >= p.S || (p.causal && jt0 > wave_qlast)) continue;
      if (p.window > 0 && wave_qlast - (jt0 + 15) >= p.window + 15) continue;
      // Sᵀ and dPᵀ: D[row key = 4lg+v][col q = li]
      floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 ka = *reinterpret_cast<const floatx4*>(&Ks[(16 * kt + li) * P + 16 * c + 4 * lg]);
        const floatx4 va = *reinterpret_cast<const floatx4*>(&Vs[(16 * kt + li) * P + 16 * c + 4 * lg]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          s4 = mfma4(ka[t], qreg[c][t], s4);
          dp4 = mfma4(va[t], greg[c][t], dp4);
        }
      }
      floatx4 ds;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = jt0 + 4 * lg + v;
        float d = 0.f;
        if (lse > -INFINITY && visible(p, qi, j, kpb ? Kp - j0 : nullptr)) {
          const float pp = __expf(s4[v] * p.scale - lse);
          d = pp * (dp4[v] - dlt) * p.scale;
        }
        ds[v] = d;
      }
      // dQ[q][d] += Σ_key dS[q][key] K[key][d]: A = dS (row q = li, k = key 4lg+t)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          dqacc[c] = mfma4(ds[t], Ks[(16 * kt + 4 * lg + t) * P + 16 * c + li], dqacc[c]);
    }
  }
  // lane holds dQ[q = qbase + 4lg + v][d = 16c + li]
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gq = qbase + 4 * lg + v;
    if (gq >= p.S) continue;
    float* r = p.dq + ((int64_t)b * p.S + gq) * p.dq_rs + (int64_t)h * HD;
#pragma unroll
    for (int c = 0; c < NC; ++c) r[16 * c + li] = dqacc[c][v];
  }
}

template <typename K>
void set_lds(K kernel, size_t bytes) {
  MFT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
}

// Tile configuration per head_dim (LDS ≤ 160 KiB per workgroup).
template <int HD> struct Cfg;
template <> struct Cfg<64>  { static constexpr int FBKV = 64, BQ = 64, DQBKV = 64; };
template <> struct Cfg<128> { static constexpr int FBKV = 32, BQ = 32, DQBKV = 32; };
template <> struct Cfg<256> { static constexpr int FBKV = 32, BQ = 16, DQBKV = 32; };

template <int HD, int NW>
void fwd_launch(hipStream_t s, AttnP& p) {
  constexpr int BKV = Cfg<HD>::FBKV;
  constexpr int P = HD + 4;
  const size_t lds = sizeof(float) * std::max<size_t>(2 * BKV * P + BKV, 16 * NW * P);
  auto kern = attn_fwd_mfma<HD, NW, BKV>;
  set_lds(kern, lds);
  dim3 grid((unsigned)(cdiv(p.S, 16 * NW) * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
}

template <int HD, int NW>
void dkdv_launch(hipStream_t s, AttnP& p) {
  constexpr int P = HD + 4;
  constexpr int BQ = Cfg<HD>::BQ;
  const size_t lds = sizeof(float) * (2 * 16 * NW * P + 2 * BQ * P + 2 * BQ + 16 * NW);
  auto kern = attn_bwd_dkdv_mfma<HD, NW, BQ>;
  set_lds(kern, lds);
  dim3 grid((unsigned)(cdiv(p.S, 16 * NW) * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
}

template <int HD, int NW>
void dq_launch(hipStream_t s, AttnP& p) {
  constexpr int P = HD + 4;
  constexpr int BKV = Cfg<HD>::DQBKV;
  const size_t lds = sizeof(float) * (2 * BKV * P + BKV);
  auto kern = attn_bwd_dq_mfma<HD, NW, BKV>;
  set_lds(kern, lds);
  dim3 grid((unsigned)(cdiv(p.S, 16 * NW) * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
}

// Waves per workgroup (16 queries or keys each): four (two at head_dim 256,
// for LDS) — the waves of a workgroup share every staged K/V (or Q/dO)
// block, and with the heavy-first 1-D grid this measured fastest at
// S = 128–1024 on MI355X.
int pick_nw(const AttnArgs& a) {
  // Tuning hook: MFT_ATTN_NW = 1, 2 or 4 waves per workgroup (4 not at hd 256).
  static const char* forced = getenv("MFT_ATTN_NW");
  if (forced) {
    const int nw = atoi(forced);
    if (nw == 1 || nw == 2 || (nw == 4 && a.hd != 256)) return nw;
  }
  return a.hd == 256 ? 2 : 4;
}

template <int HD>
void bwd_launch(hipStream_t s, AttnP& p, int nw) {
  if (nw == 4) { dkdv_launch<HD, 4>(s, p); dq_launch<HD, 4>(s, p); }
  else if (nw == 2) { dkdv_launch<HD, 2>(s, p); dq_launch<HD, 2>(s, p); }
  else { dkdv_launch<HD, 1>(s, p); dq_launch<HD, 1>(s, p); }
  if (p.Hq != p.Hkv) {
    const int64_t total = (int64_t)p.B * p.S * p.Hkv * (HD / 4);
    hipLaunchKernelGGL(attn_group_sum_kernel<HD>, dim3((unsigned)std::min<int64_t>(cdiv(total, 256), 4096)),
                       dim3(256), 0, s, p);
    MFT_LAUNCH_CHECK();
  }
}

AttnP make(const AttnArgs& a) {
  MFT_CHECK_ARG(a.B > 0 && a.S > 0 && a.Hq > 0 && a.Hkv > 0, "empty attention");
  MFT_CHECK_ARG(a.Hq % a.Hkv == 0, "Hq must be a multiple of Hkv");
  MFT_CHECK_ARG(a.hd == 64 || a.hd == 128 || a.hd == 256, "head_dim must be 64, 128 or 256");
  MFT_CHECK_ARG(a.q_rs % 4 == 0 && a.k_rs % 4 == 0 && a.v_rs % 4 == 0, "row strides must be multiples of 4");
  MFT_CHECK_ARG(((uintptr_t)a.q & 15) == 0 && ((uintptr_t)a.k & 15) == 0 && ((uintptr_t)a.v & 15) == 0,
                "q/k/v must be 16-byte aligned");
  AttnP p{};
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

void attn_fwd(hipStream_t s, const AttnArgs& a, float* o, int64_t o_rs, float* lse) {
  AttnP p = make(a);
  MFT_CHECK_ARG(o && lse, "null output");
  MFT_CHECK_ARG(o_rs % 4 == 0 && ((uintptr_t)o & 15) == 0, "o must be 16-byte aligned rows");
  p.out = o;
  p.out_rs = o_rs;
  p.lse_out = lse;
  switch (pick_nw(a)) {
    case 4: a.hd == 64 ? fwd_launch<64, 4>(s, p) : fwd_launch<128, 4>(s, p); break;
    case 2:
      a.hd == 64 ? fwd_launch<64, 2>(s, p) : a.hd == 128 ? fwd_launch<128, 2>(s, p) : fwd_launch<256, 2>(s, p);
      break;
    default:
      a.hd == 64 ? fwd_launch<64, 1>(s, p) : a.hd == 128 ? fwd_launch<128, 1>(s, p) : fwd_launch<256, 1>(s, p);
      break;
  }
}

void attn_bwd(hipStream_t s, const AttnArgs& a, const float* o, int64_t o_rs, const float* dout,
              int64_t do_rs, const float* lse, float* dq, int64_t dq_rs, float* dk, int64_t dk_rs,
              float* dv, int64_t dv_rs, Scratch ws) {
  AttnP p = make(a);
  MFT_CHECK_ARG(o && dout && lse && dq && dk && dv, "null tensor");
  MFT_CHECK_ARG(ws.ptr && ws.bytes >= attn_bwd_scratch_floats(a) * sizeof(float),
                "attention backward scratch too small");
  MFT_CHECK_ARG(do_rs % 4 == 0 && ((uintptr_t)dout & 15) == 0, "dout must be 16-byte aligned rows");
  p.o = o; p.o_rs = o_rs;
  p.dout = dout; p.do_rs = do_rs;
  p.lse = lse;
  p.dq = dq; p.dq_rs = dq_rs;
  p.dk = dk; p.dk_rs = dk_rs;
  p.dv = dv; p.dv_rs = dv_rs;
  const int64_t rows = (int64_t)a.B * a.S * a.Hq;
  p.delta_out = ws.ptr;
  p.delta = ws.ptr;
  if (a.Hq != a.Hkv) {
    // partial rows padded to a 16-byte boundary after delta
    float* part = ws.ptr + (rows + 3) / 4 * 4;
    p.pdk = part;
    p.pdv = part + rows * a.hd;
  }
  switch (a.hd) {
    case 64: hipLaunchKernelGGL(attn_delta_mfma_kernel<64>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL(attn_delta_mfma_kernel<128>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(attn_delta_mfma_kernel<256>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
  }
  MFT_LAUNCH_CHECK();
  const int nw = pick_nw(a);
  switch (a.hd) {
    case 64: bwd_launch<64>(s, p, nw); break;
    case 128: bwd_launch<128>(s, p, nw); break;
    default: bwd_launch<256>(s, p, nw); break;
  }
}

size_t attn_bwd_scratch_floats(const AttnArgs& a) {
  const size_t rows = (size_t)a.B * a.S * a.Hq;
  size_t n = (rows + 3) / 4 * 4;
  if (a.Hq != a.Hkv) n += 2 * rows * (size_t)a.hd;
  return n;
}

}  // namespace mft
