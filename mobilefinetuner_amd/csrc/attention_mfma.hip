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
  // key-split forward: chunks of ck keys per workgroup, partial O (relative
  // to the chunk's running max) and (max, sum) pairs per chunk
  int nch, ck;
  float* opart;   // [B, Hq, nch, S, HD]
  float2* mlpart; // [B, Hq, nch, S]
  // split backward: dK/dV over query chunks of cq queries (nqc of them),
  // dQ over key chunks of ckq keys (nkc); partial rows [chunk][B·S][Hq][HD]
  int nqc, cq, nkc, ckq;
  float* pdq;
};

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}


// Stage rows [r0, r0+ROWS) of two token-major [.., S, H, HD] tensors (head
// h1 / h2) into LDS; rows past S are zero.  Each tensor is stored row-major
// (dst[r][d], pitch HD+4: conflict-free 128-bit row reads), transposed
// (dst[d][r], pitch ROWS+4: one 128-bit read returns four consecutive rows
// of one column, the operand order of a product that reduces over rows), or
// both.  Row-major-only items give a wave whole rows; a tensor with a
// transposed copy gives 16 consecutive lanes 16 consecutive rows of one
// 4-column group, so the wave's scalar transposed stores land in 64 distinct
// banks and its 128-bit row stores in distinct bank groups.  Branch-free:
// row indices are clamped into the tensor and the values selected to zero,
// and each thread issues a batch of CH loads per tensor before any LDS store.
struct StageDst {
  float* row;  // [ROWS][HD+4] or unused
  float* trn;  // [HD][ROWS+4] or unused
};

template <int HD, int ROWS, bool T>
__device__ __forceinline__ void stage_item(int f, int& r, int& c4) {
  if constexpr (T) {
    r = ((f >> 4) / (HD / 4)) * 16 + (f & 15);
    c4 = (f >> 4) % (HD / 4);
  } else {
    r = f / (HD / 4);
    c4 = f % (HD / 4);
  }
}

template <int HD, int ROWS, bool R, bool T>
__device__ __forceinline__ void stage_store(const StageDst& d, int r, int c4, bool ok, const floatx4& v) {
  const floatx4 x = ok ? v : floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (R) *reinterpret_cast<floatx4*>(d.row + r * (HD + 4) + 4 * c4) = x;
  if constexpr (T) {
    constexpr int PT = ROWS + 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) d.trn[(4 * c4 + e) * PT + r] = x[e];
  }
}

template <int HD, int NT, int ROWS, bool R1, bool T1, bool R2, bool T2>
__device__ __forceinline__ void stage_pair(StageDst d1, const float* src1, int64_t rs1, StageDst d2,
                                           const float* src2, int64_t rs2, int b, int S, int h1, int h2,
                                           int r0, int tid) {
  static_assert(!(T1 || T2) || ROWS % 16 == 0, "transposed staging takes 16-row groups");
  constexpr int TOTAL = ROWS * (HD / 4);
  static_assert(TOTAL % NT == 0, "staging shape");
  constexpr int ITEMS = TOTAL / NT;
  constexpr int CH = ITEMS < 512 / HD ? ITEMS : 512 / HD;
  static_assert(ITEMS % CH == 0, "staging batch");
  // both tensors through buffer resources at the sequence's first row
  const __amdgpu_buffer_rsrc_t rs_1 = buf_rsrc(src1 + (int64_t)b * S * rs1 + (int64_t)h1 * HD);
  const __amdgpu_buffer_rsrc_t rs_2 = buf_rsrc(src2 + (int64_t)b * S * rs2 + (int64_t)h2 * HD);
#pragma unroll
  for (int base = 0; base < ITEMS; base += CH) {
    floatx4 v1[CH], v2[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int f = tid + NT * (base + c);
      int r, c4;
      stage_item<HD, ROWS, T1>(f, r, c4);
      v1[c] = buf_load4(rs_1, (uint32_t)(((int64_t)min(r0 + r, S - 1) * rs1 + 4 * c4) * 4), 0);
      stage_item<HD, ROWS, T2>(f, r, c4);
      v2[c] = buf_load4(rs_2, (uint32_t)(((int64_t)min(r0 + r, S - 1) * rs2 + 4 * c4) * 4), 0);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int f = tid + NT * (base + c);
      int r, c4;
      stage_item<HD, ROWS, T1>(f, r, c4);
      stage_store<HD, ROWS, R1, T1>(d1, r, c4, r0 + r < S, v1[c]);
      stage_item<HD, ROWS, T2>(f, r, c4);
      stage_store<HD, ROWS, R2, T2>(d2, r, c4, r0 + r < S, v2[c]);
    }
  }
}

// Most key chunks one forward query block is split into.
constexpr int kMaxChunks = 8;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x combined with the value held by lane l^16 (l^32): the gfx950 permlane
// swaps exchange rows between two registers in the VALU (no LDS round trip);
// with both operands = x, the two results hold this lane's and the partner
// lane's value, in an order that depends on the lane — so only commutative
// combinations are taken, and every lane of a pair gets the same bits.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------
template <int HD, int NW, int BKV, bool SPLIT>
__global__ __launch_bounds__(64 * NW) void attn_fwd_mfma(AttnP p) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;     // K row pitch
  constexpr int PV = BKV + 4;   // Vᵀ pitch
  constexpr int NC = HD / 16;   // 16-wide slices of head_dim
  constexpr int KT = BKV / 16;  // key tiles per block
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Ks = smem;            // [BKV][P]
  float* Vt = Ks + BKV * P;    // [HD][PV]  (V transposed)
  float* Kp = Vt + HD * PV;    // [BKV] key-padding flags

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int li = lane & 15, lg = lane >> 4;
  // 1-D grid, heaviest causal query blocks (the last ones) first; with a
  // key split, item t = blockIdx / (Hq·B) is (query block, key chunk)
  // = (nqb-1 - t % nqb, t / nqb).
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int nqb = (p.S + 16 * NW - 1) / (16 * NW);
  const int kh = h / (p.Hq / p.Hkv);
  const int item = (int)blockIdx.x / (p.Hq * p.B);
  const int q0 = (nqb - 1 - (SPLIT ? item % nqb : item)) * 16 * NW;
  const int chunk = SPLIT ? item / nqb : 0;
  const int qbase = q0 + 16 * w;
  const int qi = qbase + li;  // this lane's query
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;

  const int qlast_wg = min(q0 + 16 * NW - 1, p.S - 1);
  int jmax = p.causal ? qlast_wg : p.S - 1;
  int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  if constexpr (SPLIT) {
    // this workgroup's chunk of the block's key range; empty chunks exit
    jmin = max(jmin, chunk * p.ck);
    jmax = min(jmax, chunk * p.ck + p.ck - 1);
    if (jmin > jmax) return;
  }

  // Q carries scale·log2(e), so scores come out in base-2 units and the
  // softmax exponentials are single v_exp_f32.
  const float qscale = p.scale * kLog2e;
  floatx4 qreg[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    qreg[c] = qi < p.S ? *reinterpret_cast<const floatx4*>(p.q + ((int64_t)b * p.S + qi) * p.q_rs +
                                                          (int64_t)h * HD + 16 * c + 4 * lg) * qscale
                       : floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;
  // keys visible to this lane's query: [jlo, jhi]
  const int jhi = qi < p.S ? (p.causal ? qi : p.S - 1) : -1;
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;

  for (int j0 = (jmin / BKV) * BKV; j0 <= jmax; j0 += BKV) {
    __syncthreads();
    stage_pair<HD, NT, BKV, true, false, false, true>({Ks, nullptr}, p.k, p.k_rs, {nullptr, Vt}, p.v, p.v_rs, b, p.S,
                                                      kh, kh, j0, tid);
    for (int j = tid; j < BKV; j += NT) Kp[j] = j0 + j < p.S && (!kpb || kpb[j0 + j] > 0.5f) ? 1.f : 0.f;
    __syncthreads();
    if (qbase > p.S - 1) continue;
    // Every tile of the block is computed (straight-line code the scheduler
    // can interleave); tiles the wave cannot see are masked like any hidden
    // key.  A block every key of which is visible to all 16 queries skips
    // the per-element mask.
    const bool full = !kpb && j0 + BKV <= p.S && qbase + 15 < p.S && (!p.causal || j0 + BKV - 1 <= qbase) &&
                      (p.window <= 0 || qbase + 15 - j0 < p.window);
    floatx4 sacc[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      sacc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 kv = *reinterpret_cast<const floatx4*>(&Ks[(16 * kt + li) * P + 16 * c + 4 * lg]);
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[kt] = mfma4(kv[t], qreg[c][t], sacc[kt]);
      }
    }
    // lane holds S[q = qi][key = j0 + 16kt + 4lg + v] (base-2 units)
    if (!full) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const floatx4 kp4 = *reinterpret_cast<const floatx4*>(&Kp[16 * kt + 4 * lg]);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int j = j0 + 16 * kt + 4 * lg + v;
          const bool ok = (j >= jlo) & (j <= jhi) & (kp4[v] > 0.5f);
          sacc[kt][v] = ok ? sacc[kt][v] : -INFINITY;
        }
      }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v) mloc = fmaxf(mloc, sacc[kt][v]);
    mloc = max_xor32(max_xor16(mloc));
    const float mnew = fmaxf(mrow, mloc);
    // With nothing visible yet every score is -inf: referencing 0 keeps the
    // exponentials at exactly 0 instead of NaN.
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float corr = fast_exp2(mrow - mref);
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float e = fast_exp2(sacc[kt][v] - mref);
        sacc[kt][v] = e;
        lsum += e;
      }
    lsum = add_xor32(add_xor16(lsum));
    lrow = lrow * corr + lsum;
    mrow = mnew;
#pragma unroll
    for (int c = 0; c < NC; ++c) oacc[c] *= corr;
    // Oᵀ[d][q] += Vᵀ[d][key] · Pᵀ[key][q]; lane (i, g) reads Vᵀ[16c+i][16kt+4g .. +3]
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 va = *reinterpret_cast<const floatx4*>(&Vt[(16 * c + li) * PV + 16 * kt + 4 * lg]);
#pragma unroll
        for (int t = 0; t < 4; ++t) oacc[c] = mfma4(va[t], sacc[kt][t], oacc[c]);
      }
    }
  }
  // lane holds Oᵀ[d = 16c + 4lg + v][q = qi]; transpose through LDS for
  // coalesced row stores.  A key chunk stores O unnormalised with its
  // (max, sum) pair for attn_combine_kernel.
  __syncthreads();
  float* Os = smem;  // [16*NW][P]
  const float inv = SPLIT ? 1.f : lrow > 0.f ? 1.f / lrow : 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) Os[(16 * w + li) * P + 16 * c + 4 * lg + v] = oacc[c][v] * inv;
  const int64_t prow = (((int64_t)b * p.Hq + h) * p.nch + chunk) * p.S;  // partial rows of this chunk
  if (lg == 0 && qi < p.S) {
    if constexpr (SPLIT)
      p.mlpart[prow + qi] = make_float2(mrow, lrow);
    else  // lse in natural-log units: (m₂ + log₂ l)·ln 2
      p.lse_out[((int64_t)b * p.Hq + h) * p.S + qi] =
          lrow > 0.f ? (mrow + __builtin_amdgcn_logf(lrow)) * kLn2 : -INFINITY;
  }
  __syncthreads();
  for (int f = tid; f < 16 * NW * (HD / 4); f += NT) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gq = q0 + r;
    if (gq >= p.S) continue;
    float* dst = SPLIT ? p.opart + (prow + gq) * HD + 4 * c4
                       : p.out + ((int64_t)b * p.S + gq) * p.out_rs + (int64_t)h * HD + 4 * c4;
    *reinterpret_cast<floatx4*>(dst) = *reinterpret_cast<const floatx4*>(&Os[r * P + 4 * c4]);
  }
}

// Merges the key chunks of the split forward: for each query row,
// M = max_c m_c, L = Σ_c l_c·2^(m_c−M), O = Σ_c O_c·2^(m_c−M) / L and
// lse = (M + log₂ L)·ln 2, over the chunks its query block was given
// (same range test as the forward), in chunk order.  Thread = 4 columns of
// one (b, h, q) row.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnP p, int qblock) {
  const int64_t total = (int64_t)p.B * p.Hq * p.S * (HD / 4);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c4 = (int)(i % (HD / 4));
  const int64_t row = i / (HD / 4);  // (b·Hq + h)·S + q
  const int q = (int)(row % p.S);
  const int64_t bh = row / p.S;
  const int h = (int)(bh % p.Hq), b = (int)(bh / p.Hq);
  const int q0 = (q / qblock) * qblock;
  const int qlast = min(q0 + qblock - 1, p.S - 1);
  const int jmax = p.causal ? qlast : p.S - 1;
  const int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  const int c0 = jmin / p.ck, c1 = jmax / p.ck;
  const int64_t base = bh * p.nch * p.S + q;  // + c·S
  // all loads of the row issued together (chunks past c1 read as empty)
  float2 ml[kMaxChunks];
  floatx4 op[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const bool ok = c0 + i <= c1;
    const int64_t r = base + (int64_t)min(c0 + i, c1) * p.S;
    const float2 m2 = p.mlpart[r];
    const floatx4 o4 = *reinterpret_cast<const floatx4*>(p.opart + r * HD + 4 * c4);
    ml[i] = ok ? m2 : make_float2(-INFINITY, 0.f);
    op[i] = ok ? o4 : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) M = fmaxf(M, ml[i].x);
  const float Mref = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  floatx4 o = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const float wgt = fast_exp2(ml[i].x - Mref);  // 0 for a chunk with nothing visible
    L += ml[i].y * wgt;
    o += op[i] * wgt;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  *reinterpret_cast<floatx4*>(p.out + ((int64_t)b * p.S + q) * p.out_rs + (int64_t)h * HD + 4 * c4) = o * inv;
  if (c4 == 0) p.lse_out[row] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
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
// dK, dV: workgroup = 16·NW keys of one query head; wave = 16 keys.
// ------------------------------------------------------------------------------
template <int HD, int NW, int BQ, bool SPLIT>
__device__ __forceinline__ void attn_bwd_dkdv_role(const AttnP& p, int bid, float* smem) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;
  constexpr int PQ = BQ + 4;
  constexpr int NC = HD / 16;
  constexpr int QT = BQ / 16;
  constexpr int BKEYS = 16 * NW;
  // head_dim ≤ 128: each wave keeps its 16 keys' K/V rows in registers and
  // Q / dO also get a transposed LDS copy, so every MFMA operand is one
  // 128-bit read.  head_dim 256 (register and LDS budget): K/V rows stay in
  // LDS and the dV/dK operands are read by column.
  constexpr bool WIDE = HD > 128;
  float* Qs = smem;                              // [BQ][P]
  float* Gs = Qs + BQ * P;                       // [BQ][P]  dO
  float* Qt = Gs + BQ * P;                       // [HD][PQ] (not WIDE)
  float* Gt = Qt + (WIDE ? 0 : HD * PQ);         // [HD][PQ] (not WIDE)
  float* Ks = Gt + (WIDE ? 0 : HD * PQ);         // [BKEYS][P] (WIDE)
  float* Vs = Ks + (WIDE ? BKEYS * P : 0);       // [BKEYS][P] (WIDE)
  float* Ls = Vs + (WIDE ? BKEYS * P : 0);       // [BQ] lse·log2(e)
  float* Es = Ls + BQ;                           // [BQ] delta

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int li = lane & 15, lg = lane >> 4;
  // One workgroup per (key block, QUERY head[, query chunk]): a GQA
  // group's query heads (and a split's query chunks) run in parallel and
  // their dK/dV contributions are summed afterwards by attn_partial_sum_kernel
  // in (chunk, head) order.
  // 1-D grid, heaviest causal key blocks (the first ones) first; with a
  // query split, item t = bid / (Hq·B) is (key block, query chunk)
  // = (t % nkb, t / nkb).
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int grp = p.Hq / p.Hkv;
  const int kh = h / grp;
  const int nkb = (p.S + BKEYS - 1) / BKEYS;
  const int item = (int)bid / (p.Hq * p.B);
  const int k0 = (SPLIT ? item % nkb : item) * BKEYS;
  const int qc = SPLIT ? item / nkb : 0;
  const int kbase = k0 + 16 * w;
  const int kj = kbase + li;  // this lane's key (as S column)
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  // queries that see this lane's key: [qlo, qhi]
  const bool kvalid = kj < p.S && (!kpb || kpb[min(kj, p.S - 1)] > 0.5f);
  const int qlo = p.causal ? kj : 0;
  const int qhi = !kvalid ? -1 : p.window > 0 ? min(p.S - 1, kj + p.window - 1) : p.S - 1;

  // Scores in base-2 units: the K operand (registers) carries scale·log2(e);
  // the LDS copy of the WIDE form is scaled at use.
  const float qk2 = p.scale * kLog2e;
  const float sc = WIDE ? qk2 : 1.f;
  floatx4 kreg[WIDE ? 1 : NC], vreg[WIDE ? 1 : NC];
  if constexpr (WIDE) {
    stage_pair<HD, NT, BKEYS, true, false, true, false>({Ks, nullptr}, p.k, p.k_rs, {Vs, nullptr}, p.v,
                                                        p.v_rs, b, p.S, kh, kh, k0, tid);
  } else {
    const int64_t row = (int64_t)b * p.S + min(kj, p.S - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t off = (int64_t)kh * HD + 16 * c + 4 * lg;
      kreg[c] = *reinterpret_cast<const floatx4*>(p.k + row * p.k_rs + off) * qk2;
      vreg[c] = *reinterpret_cast<const floatx4*>(p.v + row * p.v_rs + off);
    }
  }

  floatx4 dkacc[NC], dvacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dkacc[c] = dvacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int klast = min(k0 + BKEYS - 1, p.S - 1);
  int qstart = p.causal ? k0 : 0;
  int qend = p.window > 0 ? min(p.S - 1, klast + p.window - 1) : p.S - 1;
  if constexpr (SPLIT) {
    // this workgroup's chunk of the block's query range; empty chunks exit
    // (whole workgroup, before any barrier)
    qstart = max(qstart, qc * p.cq);
    qend = min(qend, qc * p.cq + p.cq - 1);
    if (qstart > qend) return;
  }
  for (int qb0 = (qstart / BQ) * BQ; qb0 <= qend; qb0 += BQ) {
    __syncthreads();
    if constexpr (WIDE)
      stage_pair<HD, NT, BQ, true, false, true, false>({Qs, nullptr}, p.q, p.q_rs, {Gs, nullptr}, p.dout,
                                                       p.do_rs, b, p.S, h, h, qb0, tid);
    else
      stage_pair<HD, NT, BQ, true, true, true, true>({Qs, Qt}, p.q, p.q_rs, {Gs, Gt}, p.dout, p.do_rs, b,
                                                     p.S, h, h, qb0, tid);
    for (int e = tid; e < BQ; e += NT) {
      const int gi = qb0 + e;
      const int64_t l = ((int64_t)b * p.Hq + h) * p.S + gi;
      Ls[e] = gi < p.S ? p.lse[l] * kLog2e : 0.f;
      Es[e] = gi < p.S ? p.delta[l] : 0.f;
    }
    __syncthreads();
    if (kbase > p.S - 1) continue;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qt0 = qb0 + 16 * qt;
      // Tiles without a visible pair are computed and masked (straight-line
      // loop body); every query of a full tile sees every key of the wave.
      const bool full = !kpb && qt0 + 15 < p.S && kbase + 15 < p.S && (!p.causal || qt0 >= kbase + 15) &&
                        (p.window <= 0 || qt0 + 15 - kbase < p.window);
      // S[q][key] and dP[q][key]: D[row q = 4lg+v][col key = li]
      floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const floatx4 qa = *reinterpret_cast<const floatx4*>(&Qs[(16 * qt + li) * P + 16 * c + 4 * lg]);
        const floatx4 ga = *reinterpret_cast<const floatx4*>(&Gs[(16 * qt + li) * P + 16 * c + 4 * lg]);
        floatx4 kb, vb;
        if constexpr (WIDE) {
          kb = *reinterpret_cast<const floatx4*>(&Ks[(16 * w + li) * P + 16 * c + 4 * lg]);
          vb = *reinterpret_cast<const floatx4*>(&Vs[(16 * w + li) * P + 16 * c + 4 * lg]);
        } else {
          kb = kreg[c];
          vb = vreg[c];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          s4 = mfma4(qa[t], kb[t], s4);
          dp4 = mfma4(ga[t], vb[t], dp4);
        }
      }
      // P = 2^(S₂ − lse₂); dS/scale = P∘(dP − delta) (scale applied at the end)
      const floatx4 l4 = *reinterpret_cast<const floatx4*>(&Ls[16 * qt + 4 * lg]);
      const floatx4 e4 = *reinterpret_cast<const floatx4*>(&Es[16 * qt + 4 * lg]);
      floatx4 pv, ds;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int gi = qt0 + 4 * lg + v;
        // the mask selects the exponent, so a hidden entry is exactly 0
        const bool ok = full | ((gi >= qlo) & (gi <= qhi));
        const float pp = fast_exp2(ok ? fmaf(s4[v], sc, -l4[v]) : -INFINITY);
        pv[v] = pp;
        ds[v] = pp * (dp4[v] - e4[v]);
      }
      // dV[key][d] += Σ_q P[q][key] dO[q][d];  dK[key][d] += Σ_q dS[q][key] Q[q][d]
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (WIDE) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int qr = 16 * qt + 4 * lg + t;
            dvacc[c] = mfma4(pv[t], Gs[qr * P + 16 * c + li], dvacc[c]);
            dkacc[c] = mfma4(ds[t], Qs[qr * P + 16 * c + li], dkacc[c]);
          }
        } else {
          const floatx4 gt = *reinterpret_cast<const floatx4*>(&Gt[(16 * c + li) * PQ + 16 * qt + 4 * lg]);
          const floatx4 qtv = *reinterpret_cast<const floatx4*>(&Qt[(16 * c + li) * PQ + 16 * qt + 4 * lg]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            dvacc[c] = mfma4(pv[t], gt[t], dvacc[c]);
            dkacc[c] = mfma4(ds[t], qtv[t], dkacc[c]);
          }
        }
      }
    }
  }
  // lane holds [key = kbase + 4lg + v][d = 16c + li]; a group of one query
  // head without a query split writes dK/dV directly, otherwise each
  // (chunk, head) writes a partial row.
  const bool direct = grp == 1 && !SPLIT;
  const int64_t prow0 = (int64_t)qc * p.B * p.S;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gk = kbase + 4 * lg + v;
    if (gk >= p.S) continue;
    const int64_t tok = (int64_t)b * p.S + gk;
    float* dkr = direct ? p.dk + tok * p.dk_rs + (int64_t)kh * HD : p.pdk + ((prow0 + tok) * p.Hq + h) * HD;
    float* dvr = direct ? p.dv + tok * p.dv_rs + (int64_t)kh * HD : p.pdv + ((prow0 + tok) * p.Hq + h) * HD;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      dkr[16 * c + li] = dkacc[c][v] * p.scale;
      dvr[16 * c + li] = dvacc[c][v];
    }
  }
}

// dK/dV[b,s,kh,:] = Σ_{c} Σ_{j<grp} partial[c][b,s,kh·grp+j,:], in (c, j)
// order over the query chunks c the key's block was given (same range test
// as the dK/dV kernel; c = 0 only without a split).
// Workgroup blk of nblk (256 threads) takes a grid-stride share.
template <int HD>
__device__ __forceinline__ void partial_sum_role(const AttnP& p, int bkeys, int blk, int nblk) {
  const int grp = p.Hq / p.Hkv;
  const int64_t BS = (int64_t)p.B * p.S;
  const int64_t total = BS * p.Hkv * (HD / 4);
  for (int64_t i = (int64_t)blk * 256 + threadIdx.x; i < total; i += (int64_t)nblk * 256) {
    const int c4 = (int)(i % (HD / 4));
    const int64_t r = i / (HD / 4);
    const int kh = (int)(r % p.Hkv);
    const int64_t tok = r / p.Hkv;
    int c0 = 0, c1 = 0;
    if (p.nqc > 1) {
      const int k0 = ((int)(tok % p.S) / bkeys) * bkeys;
      const int klast = min(k0 + bkeys - 1, p.S - 1);
      const int qstart = p.causal ? k0 : 0;
      const int qend = p.window > 0 ? min(p.S - 1, klast + p.window - 1) : p.S - 1;
      c0 = qstart / p.cq;
      c1 = qend / p.cq;
    }
    // loads in batches of 4 partial rows (rows past the last read as zero
    // and are not added), summed in (c, j) order
    floatx4 sk = floatx4{0.f, 0.f, 0.f, 0.f}, sv = floatx4{0.f, 0.f, 0.f, 0.f};
    const int n = (c1 - c0 + 1) * grp;
    for (int t0 = 0; t0 < n; t0 += 4) {
      floatx4 bk[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = min(t0 + u, n - 1);
        const int c = c0 + t / grp, j = t % grp;
        const int64_t off = (((int64_t)c * BS + tok) * p.Hq + kh * grp + j) * HD + 4 * c4;
        bk[u] = *reinterpret_cast<const floatx4*>(p.pdk + off);
        bv[u] = *reinterpret_cast<const floatx4*>(p.pdv + off);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (t0 + u < n) {
          sk += bk[u];
          sv += bv[u];
        }
    }
    *reinterpret_cast<floatx4*>(p.dk + tok * p.dk_rs + (int64_t)kh * HD + 4 * c4) = sk;
    *reinterpret_cast<floatx4*>(p.dv + tok * p.dv_rs + (int64_t)kh * HD + 4 * c4) = sv;
  }
}
template <int HD>
__global__ __launch_bounds__(256) void attn_partial_sum_kernel(AttnP p, int bkeys) {
  partial_sum_role<HD>(p, bkeys, blockIdx.x, gridDim.x);
}

// dQ[b,s,h,:] = scale · Σ_c partial[c][b,s,h,:] over the key chunks c the
// query's block was given (same range test as the dQ kernel), in c order.
// Workgroup blk (256 threads) takes 256 consecutive float4 columns.
template <int HD>
__device__ __forceinline__ void dq_sum_role(const AttnP& p, int qblock, int blk) {
  const int64_t BS = (int64_t)p.B * p.S;
  const int64_t total = BS * p.Hq * (HD / 4);
  const int64_t i = (int64_t)blk * 256 + threadIdx.x;
  if (i >= total) return;
  const int c4 = (int)(i % (HD / 4));
  const int64_t r = i / (HD / 4);  // tok·Hq + h
  const int h = (int)(r % p.Hq);
  const int64_t tok = r / p.Hq;
  const int q0 = ((int)(tok % p.S) / qblock) * qblock;
  const int qlast = min(q0 + qblock - 1, p.S - 1);
  const int jmax = p.causal ? qlast : p.S - 1;
  const int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c = jmin / p.ckq; c <= jmax / p.ckq; ++c)
    s += *reinterpret_cast<const floatx4*>(p.pdq + (((int64_t)c * BS + tok) * p.Hq + h) * HD + 4 * c4);
  *reinterpret_cast<floatx4*>(p.dq + tok * p.dq_rs + (int64_t)h * HD + 4 * c4) = s * p.scale;
}
template <int HD>
__global__ __launch_bounds__(256) void attn_dq_sum_kernel(AttnP p, int qblock) {
  dq_sum_role<HD>(p, qblock, blockIdx.x);
}
// Both sums of a chunked backward in one launch: workgroups [0, nkv) sum
// the dK/dV partials, the rest the dQ partials (independent outputs).
template <int HD>
__global__ __launch_bounds__(256) void attn_sums_kernel(AttnP p, int bkeys, int qblock, int nkv) {
  if ((int)blockIdx.x < nkv) partial_sum_role<HD>(p, bkeys, blockIdx.x, nkv);
  else dq_sum_role<HD>(p, qblock, (int)blockIdx.x - nkv);
}

// ------------------------------------------------------------------------------
// dQ: workgroup = 16·NW queries of one head; wave = 16 queries.
// ------------------------------------------------------------------------------
template <int HD, int NW, int BKV, bool SPLIT>
__device__ __forceinline__ void attn_bwd_dq_role(const AttnP& p, int bid, float* smem) {
  constexpr int NT = 64 * NW;
  constexpr int P = HD + 4;
  constexpr int PK = BKV + 4;
  constexpr int NC = HD / 16;
  constexpr int KT = BKV / 16;
  // head_dim ≤ 128 also keeps a transposed copy of K for the dQ operand
  // (one 128-bit read instead of four column reads); 256 reads by column.
  constexpr bool WIDE = HD > 128;
  float* Ks = smem;                          // [BKV][P]
  float* Vs = Ks + BKV * P;                  // [BKV][P]
  float* Kt = Vs + BKV * P;                  // [HD][PK] (not WIDE)
  float* Kp = Kt + (WIDE ? 0 : HD * PK);     // [BKV] visible-key flags

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int li = lane & 15, lg = lane >> 4;
  // 1-D grid, heaviest causal query blocks first; with a key split, item
  // t = bid / (Hq·B) is (query block, key chunk) = (nqb-1 - t % nqb, t / nqb).
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int nqb = (p.S + 16 * NW - 1) / (16 * NW);
  const int kh = h / (p.Hq / p.Hkv);
  const int item = (int)bid / (p.Hq * p.B);
  const int q0 = (nqb - 1 - (SPLIT ? item % nqb : item)) * 16 * NW;
  const int kc = SPLIT ? item / nqb : 0;
  const int qbase = q0 + 16 * w;
  const int qi = qbase + li;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;

  const int qlast_wg = min(q0 + 16 * NW - 1, p.S - 1);
  int jmax = p.causal ? qlast_wg : p.S - 1;
  int jmin = p.window > 0 ? max(0, q0 - p.window + 1) : 0;
  if constexpr (SPLIT) {
    // this workgroup's chunk of the block's key range; empty chunks exit
    jmin = max(jmin, kc * p.ckq);
    jmax = min(jmax, kc * p.ckq + p.ckq - 1);
    if (jmin > jmax) return;
  }

  // Q carries scale·log2(e): scores in base-2 units against lse·log2(e).
  const float qscale = p.scale * kLog2e;
  floatx4 qreg[NC], greg[NC], dqacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t off = (int64_t)h * HD + 16 * c + 4 * lg;
    const bool ok = qi < p.S;
    qreg[c] = ok ? *reinterpret_cast<const floatx4*>(p.q + ((int64_t)b * p.S + qi) * p.q_rs + off) * qscale
                 : floatx4{0.f, 0.f, 0.f, 0.f};
    greg[c] = ok ? *reinterpret_cast<const floatx4*>(p.dout + ((int64_t)b * p.S + qi) * p.do_rs + off)
                 : floatx4{0.f, 0.f, 0.f, 0.f};
    dqacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float lse2 = 0.f, dlt = 0.f;
  if (qi < p.S) {
    const int64_t l = ((int64_t)b * p.Hq + h) * p.S + qi;
    lse2 = p.lse[l] * kLog2e;
    dlt = p.delta[l];
  }
  // keys visible to this lane's query: [jlo, jhi]
  const int jhi = qi < p.S ? (p.causal ? qi : p.S - 1) : -1;
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;
  for (int j0 = (jmin / BKV) * BKV; j0 <= jmax; j0 += BKV) {
    __syncthreads();
    if constexpr (WIDE)
      stage_pair<HD, NT, BKV, true, false, true, false>({Ks, nullptr}, p.k, p.k_rs, {Vs, nullptr}, p.v,
                                                        p.v_rs, b, p.S, kh, kh, j0, tid);
    else
      stage_pair<HD, NT, BKV, true, true, true, false>({Ks, Kt}, p.k, p.k_rs, {Vs, nullptr}, p.v, p.v_rs, b,
                                                       p.S, kh, kh, j0, tid);
    for (int j = tid; j < BKV; j += NT) Kp[j] = j0 + j < p.S && (!kpb || kpb[j0 + j] > 0.5f) ? 1.f : 0.f;
    __syncthreads();
    if (qbase > p.S - 1) continue;
    const bool full = !kpb && j0 + BKV <= p.S && qbase + 15 < p.S && (!p.causal || j0 + BKV - 1 <= qbase) &&
                      (p.window <= 0 || qbase + 15 - j0 < p.window);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int jt0 = j0 + 16 * kt;
      // tiles without a visible pair are computed and masked (straight-line
      // loop body)
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
      // dS/scale = P∘(dP − delta), P = 2^(S₂ − lse₂) (scale applied at the end)
      const floatx4 kp4 = *reinterpret_cast<const floatx4*>(&Kp[16 * kt + 4 * lg]);
      floatx4 ds;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = jt0 + 4 * lg + v;
        // the mask selects the exponent, so a hidden entry is exactly 0
        const bool ok = full | ((j >= jlo) & (j <= jhi) & (kp4[v] > 0.5f));
        const float pp = fast_exp2(ok ? s4[v] - lse2 : -INFINITY);
        ds[v] = pp * (dp4[v] - dlt);
      }
      // dQ[q][d] += Σ_key dS[q][key] K[key][d]: A = dS (row q = li, k = key 4lg+t)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (WIDE) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            dqacc[c] = mfma4(ds[t], Ks[(16 * kt + 4 * lg + t) * P + 16 * c + li], dqacc[c]);
        } else {
          const floatx4 kb = *reinterpret_cast<const floatx4*>(&Kt[(16 * c + li) * PK + 16 * kt + 4 * lg]);
#pragma unroll
          for (int t = 0; t < 4; ++t) dqacc[c] = mfma4(ds[t], kb[t], dqacc[c]);
        }
      }
    }
  }
  // lane holds dQ[q = qbase + 4lg + v][d = 16c + li]; a key chunk writes an
  // unscaled partial row for attn_dq_sum_kernel
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gq = qbase + 4 * lg + v;
    if (gq >= p.S) continue;
    const int64_t tok = (int64_t)b * p.S + gq;
    float* r = SPLIT ? p.pdq + (((int64_t)kc * p.B * p.S + tok) * p.Hq + h) * HD
                     : p.dq + tok * p.dq_rs + (int64_t)h * HD;
    const float sc = SPLIT ? 1.f : p.scale;
#pragma unroll
    for (int c = 0; c < NC; ++c) r[16 * c + li] = dqacc[c][v] * sc;
  }
}

// The backward's two main products in one launch: blocks [0, n_dkdv) run the
// dK/dV role (one per key block, query head and query chunk), the rest the
// dQ role (one per query block, head and key chunk).  The roles are
// independent given delta, so they fill the GPU together instead of as two
// half-empty launches at short sequence lengths.
template <int HD, int NW, int BQ, int BKV, bool SQ, bool SK>
__global__ __launch_bounds__(64 * NW) void attn_bwd_mfma(AttnP p, int n_dkdv) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int bid = (int)blockIdx.x;
  if (bid < n_dkdv) attn_bwd_dkdv_role<HD, NW, BQ, SQ>(p, bid, smem);
  else attn_bwd_dq_role<HD, NW, BKV, SK>(p, bid - n_dkdv, smem);
}

// ------------------------------------------------------------------------------
// Short sequences: a workgroup per 16-row tile, its inner loop split over
// the waves.
// ------------------------------------------------------------------------------
// At S ≤ 256 the blocked kernels above leave each workgroup one or two
// blocks of serial work on one wave per SIMD, so every block pays its load
// latency in full.  Here a workgroup owns one 16-query tile (forward, dQ)
// or one 16-key tile (dK/dV) of one head; its NW waves take the tile's
// visible inner tiles (16 keys, or 16 queries) round-robin, each reading its
// operands straight from global memory (L2) into MFMA operand registers,
// and the waves' partial results are merged through LDS in wave order
// (deterministic).  Operand layouts per lane (i = lane % 16, g = lane / 16):
// a 128-bit read Rows[i][16c + 4g .. +3] for an operand indexed (row i,
// reduction d), four 32-bit reads Rows[4g + t][16c + i] for an operand
// indexed (reduction row, column d).  The backward forms delta =
// rowsum(dO∘O) from O and dO rows it loads anyway (no separate pass).

// Forward: Sᵀ = K·Qᵀ (lane: query i, keys 4g+v of the tile), online softmax
// per query, O += P·V with P from registers (A operand) and V as four
// column reads; O partial [query 4g+v][d 16c+i] and (max, sum) per query to
// LDS, merged over the waves.
template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void attn_fwd_short(AttnP p) {
  constexpr int NC = HD / 16;
  constexpr int PO = HD + 4;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Os = smem;              // [NW][16][PO]
  float* Ms = Os + NW * 16 * PO;  // [NW][16]
  float* Ls = Ms + NW * 16;       // [NW][16]
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int nqt = (p.S + 15) / 16;
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int qt = nqt - 1 - (int)blockIdx.x / (p.Hq * p.B);  // heaviest (last) tiles first
  const int q0 = 16 * qt;
  const int kh = h / (p.Hq / p.Hkv);
  const int qi = q0 + li;
  const bool qok = qi < p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const int64_t tok0 = (int64_t)b * p.S;
  const int qlast = min(q0 + 15, p.S - 1);
  const int kt_hi = (p.causal ? qlast : p.S - 1) / 16;
  const int kt_lo = p.window > 0 ? max(0, q0 - p.window + 1) / 16 : 0;
  const int jhi = qok ? (p.causal ? qi : p.S - 1) : -1;  // keys visible to query qi
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;

  const float qscale = p.scale * kLog2e;  // scores in base-2 units
  floatx4 qreg[NC], oacc[NC];
  {
    const float* qr = p.q + (tok0 + min(qi, p.S - 1)) * p.q_rs + (int64_t)h * HD + 4 * lg;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(qr + 16 * c);
      qreg[c] = qok ? x * qscale : floatx4{0.f, 0.f, 0.f, 0.f};
      oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  float mrow = -INFINITY, lrow = 0.f;
  // K and V of this sequence and KV head through buffer resources (32-bit
  // per-lane offsets; a sequence's rows span well under 4 GiB)
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(p.k + tok0 * p.k_rs + (int64_t)kh * HD);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(p.v + tok0 * p.v_rs + (int64_t)kh * HD);
  auto load = [&](int kt, floatx4 (&kr)[NC], float (&vr)[NC][4]) {
    const uint32_t ko = (uint32_t)(((int64_t)min(16 * kt + li, p.S - 1) * p.k_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) kr[c] = buf_load4(rk, ko + 64u * c, 0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t vo = (uint32_t)(((int64_t)min(16 * kt + 4 * lg + t, p.S - 1) * p.v_rs + li) * 4);
#pragma unroll
      for (int c = 0; c < NC; ++c) vr[c][t] = buf_load1(rv, vo + 64u * c, 0);
    }
  };
  floatx4 kc[NC];
  float vc[NC][4];
  int kt = kt_lo + w;
  if (kt <= kt_hi) load(kt, kc, vc);
  for (; kt <= kt_hi; kt += NW) {
    floatx4 kn[NC];
    float vn[NC][4];
    const bool more = kt + NW <= kt_hi;
    if (more) load(kt + NW, kn, vn);
    floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) s = mfma4(kc[c][t], qreg[c][t], s);
    // lane holds S[query qi][key j0 + v]
    const int j0 = 16 * kt + 4 * lg;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = j0 + v;
      bool ok = (j >= jlo) & (j <= jhi) & (j < p.S);
      if (kpb) ok = ok & (kpb[min(j, p.S - 1)] > 0.5f);
      s[v] = ok ? s[v] : -INFINITY;
    }
    float mloc = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mloc = max_xor32(max_xor16(mloc));
    const float mnew = fmaxf(mrow, mloc);
    const float mref = mnew == -INFINITY ? 0.f : mnew;  // nothing visible yet: exact zeros, no NaN
    const float corr = fast_exp2(mrow - mref);
    floatx4 pr;
#pragma unroll
    for (int v = 0; v < 4; ++v) pr[v] = fast_exp2(s[v] - mref);
    const float lsum = add_xor32(add_xor16((pr[0] + pr[1]) + (pr[2] + pr[3])));
    lrow = lrow * corr + lsum;
    mrow = mnew;
    // O rows are queries 4g+v: their rescale factors live in lanes 4g+v
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float cv = __shfl(corr, 4 * lg + v, 64);
#pragma unroll
      for (int c = 0; c < NC; ++c) oacc[c][v] *= cv;
    }
    // O[q][d] += Σ_key P[q][key]·V[key][d]
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) oacc[c] = mfma4(pr[t], vc[c][t], oacc[c]);
    if (more) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        kc[c] = kn[c];
#pragma unroll
        for (int t = 0; t < 4; ++t) vc[c][t] = vn[c][t];
      }
    }
  }
  if (lg == 0) {
    Ms[w * 16 + li] = mrow;
    Ls[w * 16 + li] = lrow;
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) Os[(w * 16 + 4 * lg + v) * PO + 16 * c + li] = oacc[c][v];
  __syncthreads();
  // merge in wave order: M = max_w m_w, L = Σ_w l_w·2^(m_w − M), O = Σ_w O_w·2^(m_w − M) / L
  for (int f = tid; f < 16 * (HD / 4); f += 64 * NW) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gq = q0 + r;
    if (gq >= p.S) continue;
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) M = fmaxf(M, Ms[u * 16 + r]);
    const float Mref = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    floatx4 o = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float wgt = fast_exp2(Ms[u * 16 + r] - Mref);
      L += Ls[u * 16 + r] * wgt;
      o += *reinterpret_cast<const floatx4*>(&Os[(u * 16 + r) * PO + 4 * c4]) * wgt;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<floatx4*>(p.out + (tok0 + gq) * p.out_rs + (int64_t)h * HD + 4 * c4) = o * inv;
    if (c4 == 0) p.lse_out[((int64_t)b * p.Hq + h) * p.S + gq] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
  }
}

// Forward at head_dim 256 (Gemma-3): the same tiling and arithmetic as
// attn_fwd_short, with the workgroup's 16 query rows staged once in LDS and
// read as MFMA operands 16 dims at a time (holding them in registers, with
// the K and V tiles and the O accumulator, would not fit two waves per
// SIMD), and the key tile's K and V rows loaded per tile without a prefetch
// set.  The waves' partial O rows are merged through the same LDS, after a
// barrier that ends every wave's reads of the staged queries.
template <int NW>
__global__ __launch_bounds__(64 * NW) void attn_fwd_short256(AttnP p) {
  constexpr int HD = 256, NC = HD / 16, PO = HD + 4;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* Qs = smem;               // [16][PO] during the key loop
  float* Os = smem;               // [NW][16][PO] after it
  float* Ms = Os + NW * 16 * PO;  // [NW][16]
  float* Ls = Ms + NW * 16;       // [NW][16]
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int nqt = (p.S + 15) / 16;
  const int hb = blockIdx.x % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int qt = nqt - 1 - (int)blockIdx.x / (p.Hq * p.B);  // heaviest (last) tiles first
  const int q0 = 16 * qt;
  const int kh = h / (p.Hq / p.Hkv);
  const int qi = q0 + li;
  const bool qok = qi < p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const int64_t tok0 = (int64_t)b * p.S;
  const int qlast = min(q0 + 15, p.S - 1);
  const int kt_hi = (p.causal ? qlast : p.S - 1) / 16;
  const int kt_lo = p.window > 0 ? max(0, q0 - p.window + 1) / 16 : 0;
  const int jhi = qok ? (p.causal ? qi : p.S - 1) : -1;  // keys visible to query qi
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;

  const float qscale = p.scale * kLog2e;  // scores in base-2 units
  for (int f = tid; f < 16 * (HD / 4); f += 64 * NW) {
    const int r = f / (HD / 4), c4 = f % (HD / 4), q = q0 + r;
    const floatx4 x = *reinterpret_cast<const floatx4*>(p.q + (tok0 + min(q, p.S - 1)) * p.q_rs + (int64_t)h * HD + 4 * c4);
    *reinterpret_cast<floatx4*>(&Qs[r * PO + 4 * c4]) = q < p.S ? x * qscale : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();
  floatx4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(p.k + tok0 * p.k_rs + (int64_t)kh * HD);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(p.v + tok0 * p.v_rs + (int64_t)kh * HD);
  const float* qrow = Qs + li * PO + 4 * lg;
  // K of a key tile: this lane's row slice (S operands); the wave's next K
  // tile is loaded while the current one is multiplied (its V column slices,
  // needed only after the softmax, are loaded at the top of the step)
  auto load_k = [&](int kt, floatx4* k) {
    const uint32_t ko = (uint32_t)(((int64_t)min(16 * kt + li, p.S - 1) * p.k_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) k[c] = buf_load4(rk, ko + 64u * c, 0);
  };
  floatx4 kc[NC], kn[NC];
  if (kt_lo + w <= kt_hi) load_k(kt_lo + w, kc);
  for (int kt = kt_lo + w; kt <= kt_hi; kt += NW) {
    float vc[NC][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t vo = (uint32_t)(((int64_t)min(16 * kt + 4 * lg + t, p.S - 1) * p.v_rs + li) * 4);
#pragma unroll
      for (int c = 0; c < NC; ++c) vc[c][t] = buf_load1(rv, vo + 64u * c, 0);
    }
    if (kt + NW <= kt_hi) load_k(kt + NW, kn);
    floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const floatx4 qv = *reinterpret_cast<const floatx4*>(qrow + 16 * c);
#pragma unroll
      for (int t = 0; t < 4; ++t) s = mfma4(kc[c][t], qv[t], s);
    }
    // lane holds S[query qi][key j0 + v]
    const int j0 = 16 * kt + 4 * lg;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = j0 + v;
      bool ok = (j >= jlo) & (j <= jhi) & (j < p.S);
      if (kpb) ok = ok & (kpb[min(j, p.S - 1)] > 0.5f);
      s[v] = ok ? s[v] : -INFINITY;
    }
    float mloc = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mloc = max_xor32(max_xor16(mloc));
    const float mnew = fmaxf(mrow, mloc);
    const float mref = mnew == -INFINITY ? 0.f : mnew;  // nothing visible yet: exact zeros, no NaN
    const float corr = fast_exp2(mrow - mref);
    floatx4 pr;
#pragma unroll
    for (int v = 0; v < 4; ++v) pr[v] = fast_exp2(s[v] - mref);
    const float lsum = add_xor32(add_xor16((pr[0] + pr[1]) + (pr[2] + pr[3])));
    lrow = lrow * corr + lsum;
    mrow = mnew;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float cv = __shfl(corr, 4 * lg + v, 64);
#pragma unroll
      for (int c = 0; c < NC; ++c) oacc[c][v] *= cv;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) oacc[c] = mfma4(pr[t], vc[c][t], oacc[c]);
    if (kt + NW <= kt_hi)
#pragma unroll
      for (int c = 0; c < NC; ++c) kc[c] = kn[c];
  }
  __syncthreads();  // the staged queries are read by every wave before Os overwrites them
  if (lg == 0) {
    Ms[w * 16 + li] = mrow;
    Ls[w * 16 + li] = lrow;
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) Os[(w * 16 + 4 * lg + v) * PO + 16 * c + li] = oacc[c][v];
  __syncthreads();
  for (int f = tid; f < 16 * (HD / 4); f += 64 * NW) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gq = q0 + r;
    if (gq >= p.S) continue;
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) M = fmaxf(M, Ms[u * 16 + r]);
    const float Mref = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    floatx4 o = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float wgt = fast_exp2(Ms[u * 16 + r] - Mref);
      L += Ls[u * 16 + r] * wgt;
      o += *reinterpret_cast<const floatx4*>(&Os[(u * 16 + r) * PO + 4 * c4]) * wgt;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<floatx4*>(p.out + (tok0 + gq) * p.out_rs + (int64_t)h * HD + 4 * c4) = o * inv;
    if (c4 == 0) p.lse_out[((int64_t)b * p.Hq + h) * p.S + gq] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
  }
}

// dK/dV role: workgroup = one 16-key tile of one QUERY head; waves take the
// query tiles that see it round-robin.  K, V of the tile are read from
// global memory once per workgroup (staged in LDS) and stay in registers
// (B operands of S = Q·Kᵀ and dP = dO·Vᵀ); per query tile a wave reads Q,
// dO, O rows (A operands, and delta) and turns its Q and dO rows into the
// column operands of dK += dSᵀ·Q, dV += Pᵀ·dO through its own LDS slot.  The
// partials [key 4g+v][d 16c+i] are summed over the waves through the same
// slots; GQA groups > 1 write per-query-head partials.
template <int HD, int NW>
__device__ __forceinline__ void attn_bwd_short_dkdv(const AttnP& p, int bid, float* smem) {
  constexpr int NC = HD / 16;
  constexpr int PO = HD + 4;
  float* Dk = smem;               // [NW][16][PO]: wave w's Q transpose slot, then its dK partial
  float* Dv = Dk + NW * 16 * PO;  // [NW][16][PO]: wave w's dO transpose slot, then its dV partial
  float* KV = Dv + NW * 16 * PO;  // [2][16][PO]: the tile's K and V rows
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int grp = p.Hq / p.Hkv;
  const int kh = h / grp;
  const int kt = bid / (p.Hq * p.B);  // heaviest (first) key tiles first
  const int k0 = 16 * kt;
  const int kj = k0 + li;  // this lane's key (S column)
  const int64_t tok0 = (int64_t)b * p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const bool kvalid = kj < p.S && (!kpb || kpb[min(kj, p.S - 1)] > 0.5f);
  const int klast = min(k0 + 15, p.S - 1);
  const int qt_lo = (p.causal ? k0 : 0) / 16;
  const int qt_hi = (p.window > 0 ? min(p.S - 1, klast + p.window - 1) : p.S - 1) / 16;

  const float qk2 = p.scale * kLog2e;
  const int64_t lrow0 = ((int64_t)b * p.Hq + h) * p.S;
  // one query tile's operands: Q, dO, O rows (128-bit), lse of query q0 + i
  struct QTile {
    floatx4 qa[NC], ga[NC], oa[NC];
    float lse;
  };
  // Q, dO, O of this sequence and query head through buffer resources
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(p.q + tok0 * p.q_rs + (int64_t)h * HD);
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(p.dout + tok0 * p.do_rs + (int64_t)h * HD);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(p.o + tok0 * p.o_rs + (int64_t)h * HD);
  auto load = [&](int qt, QTile& T) {
    const int q0 = 16 * qt;
    const int64_t r = min(q0 + li, p.S - 1);
    const uint32_t oq = (uint32_t)((r * p.q_rs + 4 * lg) * 4), og = (uint32_t)((r * p.do_rs + 4 * lg) * 4),
                   oo = (uint32_t)((r * p.o_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      T.qa[c] = buf_load4(rq, oq + 64u * c, 0);
      T.ga[c] = buf_load4(rg, og + 64u * c, 0);
      T.oa[c] = buf_load4(ro, oo + 64u * c, 0);
    }
    T.lse = p.lse[lrow0 + r];
  };
  // K, V rows of the tile (rows past S clamped; their keys are masked):
  // one 128-bit item per thread and tensor per pass, issued together with
  // the wave's first query tile
  constexpr int KV_IT = 16 * (HD / 4) / (64 * NW);
  static_assert(KV_IT >= 1 && KV_IT * 64 * NW == 16 * (HD / 4), "K/V staging shape");
  floatx4 kx[KV_IT], vx[KV_IT];
#pragma unroll
  for (int u = 0; u < KV_IT; ++u) {
    const int f = tid + 64 * NW * u, r = f / (HD / 4), c4 = f % (HD / 4);
    const int64_t row = tok0 + min(k0 + r, p.S - 1);
    kx[u] = *reinterpret_cast<const floatx4*>(p.k + row * p.k_rs + (int64_t)kh * HD + 4 * c4);
    vx[u] = *reinterpret_cast<const floatx4*>(p.v + row * p.v_rs + (int64_t)kh * HD + 4 * c4);
  }
  QTile cur;
  int qt = qt_lo + w;
  if (qt <= qt_hi) load(qt, cur);
#pragma unroll
  for (int u = 0; u < KV_IT; ++u) {
    const int f = tid + 64 * NW * u, r = f / (HD / 4), c4 = f % (HD / 4);
    *reinterpret_cast<floatx4*>(KV + r * PO + 4 * c4) = kx[u];
    *reinterpret_cast<floatx4*>(KV + (16 + r) * PO + 4 * c4) = vx[u];
  }
  __syncthreads();
  floatx4 kreg[NC], vreg[NC], dkacc[NC], dvacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    kreg[c] = *reinterpret_cast<const floatx4*>(KV + li * PO + 16 * c + 4 * lg) * qk2;
    vreg[c] = *reinterpret_cast<const floatx4*>(KV + (16 + li) * PO + 16 * c + 4 * lg);
    dkacc[c] = dvacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  // Q and dO by column (rows 4g + t, column 16c + i): the wave's rows
  // written to its LDS slots and read back transposed (a wave's LDS
  // operations complete in issue order, so the slots need no barrier)
  float* sq = Dk + w * 16 * PO;
  float* sg = Dv + w * 16 * PO;
  auto cols = [&](const QTile& T, float (&qb)[NC][4], float (&gb)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      *reinterpret_cast<floatx4*>(sq + li * PO + 16 * c + 4 * lg) = T.qa[c];
      *reinterpret_cast<floatx4*>(sg + li * PO + 16 * c + 4 * lg) = T.ga[c];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        qb[c][t] = sq[(4 * lg + t) * PO + 16 * c + li];
        gb[c][t] = sg[(4 * lg + t) * PO + 16 * c + li];
      }
  };
  auto compute = [&](int qt, const QTile& T, const float (&qb)[NC][4], const float (&gb)[NC][4]) {
    const int q0 = 16 * qt;
    const float l2 = T.lse * kLog2e;  // query q0 + li
    float dl = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) dl = fmaf(T.ga[c][e], T.oa[c][e], dl);
    dl = add_xor32(add_xor16(dl));  // delta of query q0 + li
    floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s4 = mfma4(T.qa[c][t], kreg[c][t], s4);
        dp4 = mfma4(T.ga[c][t], vreg[c][t], dp4);
      }
    // S[q0 + 4g + v][key kj]: P = 2^(S₂ − lse₂), dS/scale = P∘(dP − delta)
    floatx4 pv, ds;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int qv = q0 + 4 * lg + v;
      const float l2v = __shfl(l2, 4 * lg + v, 64);
      const float dlv = __shfl(dl, 4 * lg + v, 64);
      const bool ok = kvalid & (qv < p.S) & (!p.causal | (qv >= kj)) & ((p.window <= 0) | (qv - kj < p.window));
      pv[v] = fast_exp2(ok ? s4[v] - l2v : -INFINITY);
      ds[v] = pv[v] * (dp4[v] - dlv);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        dvacc[c] = mfma4(pv[t], gb[c][t], dvacc[c]);
        dkacc[c] = mfma4(ds[t], qb[c][t], dkacc[c]);
      }
  };
  // One tile of operands in registers at a time: holding the next tile's
  // loads in flight as well (two tiles of registers) lowers the waves per
  // SIMD below what the launch needs to be resident at once.
  for (; qt <= qt_hi; qt += NW) {
    float qb[NC][4], gb[NC][4];
    cols(cur, qb, gb);
    compute(qt, cur, qb, gb);
    if (qt + NW <= qt_hi) load(qt + NW, cur);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      Dk[(w * 16 + 4 * lg + v) * PO + 16 * c + li] = dkacc[c][v];
      Dv[(w * 16 + 4 * lg + v) * PO + 16 * c + li] = dvacc[c][v];
    }
  __syncthreads();
  const bool direct = grp == 1;
  for (int f = tid; f < 16 * (HD / 4); f += 64 * NW) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gk = k0 + r;
    if (gk >= p.S) continue;
    floatx4 sk = floatx4{0.f, 0.f, 0.f, 0.f}, sv = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      sk += *reinterpret_cast<const floatx4*>(&Dk[(u * 16 + r) * PO + 4 * c4]);
      sv += *reinterpret_cast<const floatx4*>(&Dv[(u * 16 + r) * PO + 4 * c4]);
    }
    const int64_t tok = tok0 + gk;
    float* dkr = direct ? p.dk + tok * p.dk_rs + (int64_t)kh * HD : p.pdk + (tok * p.Hq + h) * HD;
    float* dvr = direct ? p.dv + tok * p.dv_rs + (int64_t)kh * HD : p.pdv + (tok * p.Hq + h) * HD;
    *reinterpret_cast<floatx4*>(dkr + 4 * c4) = sk * p.scale;
    *reinterpret_cast<floatx4*>(dvr + 4 * c4) = sv;
  }
}

// dQ role: workgroup = one 16-query tile of one head; waves take its visible
// key tiles round-robin.  Q, dO, O of the tile are read from global memory
// once per workgroup (staged in LDS); Q, dO stay in registers (B operands of
// Sᵀ = K·Qᵀ and dPᵀ = V·dOᵀ, so a lane owns one query's softmax row); per
// key tile a wave reads K, V rows (A operands) and turns its K rows into the
// column operand of dQ += dS·K through its own LDS slot.  The partials
// [query 4g+v][d 16c+i] are summed over the waves through the same slots.
template <int HD, int NW>
__device__ __forceinline__ void attn_bwd_short_dq(const AttnP& p, int bid, float* smem) {
  constexpr int NC = HD / 16;
  constexpr int PO = HD + 4;
  float* Dq = smem;                // [NW][16][PO]: wave w's K transpose slot, then its dQ partial
  float* QG = Dq + NW * 16 * PO;   // [3][16][PO]: the tile's Q, dO and O rows
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int nqt = (p.S + 15) / 16;
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int qt = nqt - 1 - bid / (p.Hq * p.B);  // heaviest (last) query tiles first
  const int q0 = 16 * qt;
  const int kh = h / (p.Hq / p.Hkv);
  const int qi = q0 + li;
  const bool qok = qi < p.S;
  const int64_t tok0 = (int64_t)b * p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const int qlast = min(q0 + 15, p.S - 1);
  const int kt_hi = (p.causal ? qlast : p.S - 1) / 16;
  const int kt_lo = p.window > 0 ? max(0, q0 - p.window + 1) / 16 : 0;
  const int jhi = qok ? (p.causal ? qi : p.S - 1) : -1;
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;

  const float qk2 = p.scale * kLog2e;
  const float* kbase = p.k + (int64_t)kh * HD;
  const float* vbase = p.v + (int64_t)kh * HD;
  const float lse_q = p.lse[((int64_t)b * p.Hq + h) * p.S + min(qi, p.S - 1)];
  float dl = 0.f, l2 = 0.f;  // delta and lse·log2(e) of query qi (formed below)
  // one key tile's operands: K, V rows (128-bit)
  struct KTile {
    floatx4 ka[NC], va[NC];
  };
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kbase + tok0 * p.k_rs);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vbase + tok0 * p.v_rs);
  auto load = [&](int kt, KTile& T) {
    const int64_t r = min(16 * kt + li, p.S - 1);
    const uint32_t ko = (uint32_t)((r * p.k_rs + 4 * lg) * 4), vo = (uint32_t)((r * p.v_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      T.ka[c] = buf_load4(rk, ko + 64u * c, 0);
      T.va[c] = buf_load4(rv, vo + 64u * c, 0);
    }
  };
  // Q, dO, O rows of the tile (rows past S clamped; they are not stored):
  // one 128-bit item per thread and tensor per pass, issued together with
  // the wave's first key tile
  constexpr int QG_IT = 16 * (HD / 4) / (64 * NW);
  static_assert(QG_IT >= 1 && QG_IT * 64 * NW == 16 * (HD / 4), "Q/dO/O staging shape");
  floatx4 qx[QG_IT], gx[QG_IT], ox[QG_IT];
#pragma unroll
  for (int u = 0; u < QG_IT; ++u) {
    const int f = tid + 64 * NW * u, r = f / (HD / 4), c4 = f % (HD / 4);
    const int64_t row = tok0 + min(q0 + r, p.S - 1);
    const int64_t off = (int64_t)h * HD + 4 * c4;
    qx[u] = *reinterpret_cast<const floatx4*>(p.q + row * p.q_rs + off);
    gx[u] = *reinterpret_cast<const floatx4*>(p.dout + row * p.do_rs + off);
    ox[u] = *reinterpret_cast<const floatx4*>(p.o + row * p.o_rs + off);
  }
  KTile cur;
  int kt = kt_lo + w;
  if (kt <= kt_hi) load(kt, cur);
#pragma unroll
  for (int u = 0; u < QG_IT; ++u) {
    const int f = tid + 64 * NW * u, r = f / (HD / 4), c4 = f % (HD / 4);
    *reinterpret_cast<floatx4*>(QG + r * PO + 4 * c4) = qx[u];
    *reinterpret_cast<floatx4*>(QG + (16 + r) * PO + 4 * c4) = gx[u];
    *reinterpret_cast<floatx4*>(QG + (32 + r) * PO + 4 * c4) = ox[u];
  }
  __syncthreads();
  floatx4 qreg[NC], greg[NC], dqacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    qreg[c] = *reinterpret_cast<const floatx4*>(QG + li * PO + 16 * c + 4 * lg);
    greg[c] = *reinterpret_cast<const floatx4*>(QG + (16 + li) * PO + 16 * c + 4 * lg);
    const floatx4 orow = *reinterpret_cast<const floatx4*>(QG + (32 + li) * PO + 16 * c + 4 * lg);
#pragma unroll
    for (int e = 0; e < 4; ++e) dl = fmaf(greg[c][e], orow[e], dl);
    dqacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  // K by column (rows 4g + t, column 16c + i) through the wave's LDS slot
  float* sk = Dq + w * 16 * PO;
  auto cols = [&](const KTile& T, float (&kb)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) *reinterpret_cast<floatx4*>(sk + li * PO + 16 * c + 4 * lg) = T.ka[c];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < NC; ++c) kb[c][t] = sk[(4 * lg + t) * PO + 16 * c + li];
  };
  auto compute = [&](int kt, const KTile& T, const float (&kb)[NC][4]) {
    floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s4 = mfma4(T.ka[c][t], qreg[c][t], s4);
        dp4 = mfma4(T.va[c][t], greg[c][t], dp4);
      }
    // Sᵀ[key 16kt + 4g + v][query qi]
    floatx4 ds;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = 16 * kt + 4 * lg + v;
      bool ok = (j >= jlo) & (j <= jhi) & (j < p.S);
      if (kpb) ok = ok & (kpb[min(j, p.S - 1)] > 0.5f);
      const float pp = fast_exp2(ok ? s4[v] - l2 : -INFINITY);
      ds[v] = pp * (dp4[v] - dl);
    }
    // dQ[q][d] += Σ_key dS[q][key]·K[key][d]
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) dqacc[c] = mfma4(ds[t], kb[c][t], dqacc[c]);
  };
  // each later key tile's loads go out after the previous one is multiplied
  // (one tile of registers, as in the dK/dV role)
#pragma unroll
  for (int c = 0; c < NC; ++c) qreg[c] *= qk2;
  dl = add_xor32(add_xor16(dl));
  l2 = lse_q * kLog2e;
  for (; kt <= kt_hi; kt += NW) {
    float kb[NC][4];
    cols(cur, kb);
    compute(kt, cur, kb);
    if (kt + NW <= kt_hi) load(kt + NW, cur);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) Dq[(w * 16 + 4 * lg + v) * PO + 16 * c + li] = dqacc[c][v];
  __syncthreads();
  for (int f = tid; f < 16 * (HD / 4); f += 64 * NW) {
    const int r = f / (HD / 4), c4 = f % (HD / 4);
    const int gq = q0 + r;
    if (gq >= p.S) continue;
    floatx4 sq = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) sq += *reinterpret_cast<const floatx4*>(&Dq[(u * 16 + r) * PO + 4 * c4]);
    *reinterpret_cast<floatx4*>(p.dq + (tok0 + gq) * p.dq_rs + (int64_t)h * HD + 4 * c4) = sq * p.scale;
  }
}

// Both short-sequence backward roles in one launch: blocks [0, n_dkdv) are
// dK/dV tiles, the rest dQ tiles.
template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void attn_bwd_short(AttnP p, int n_dkdv) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int bid = (int)blockIdx.x;
  if (bid < n_dkdv) attn_bwd_short_dkdv<HD, NW>(p, bid, smem);
  else attn_bwd_short_dq<HD, NW>(p, bid - n_dkdv, smem);
}

// ------------------------------------------------------------------------------
// Short sequences at head_dim 256: the head dimension split over the waves.
// ------------------------------------------------------------------------------
// At head_dim 256 a lane of attn_bwd_short's roles would hold K, V, dK, dV
// and a query tile's Q, dO, O rows at once (about 576 VGPRs).  Here each of
// the four waves of a workgroup owns one 64-wide slice D_w of the head
// dimension for the whole tile loop, and all waves walk the same inner
// tiles: per inner tile every wave forms its partial S and dP (and delta)
// over D_w with its slice of the operands in registers, the partials go
// through LDS, and each wave sums the four in wave order (every wave gets
// the same bits, so P and dS agree across the workgroup) before
// accumulating its own slice of dK/dV (or dQ).  The exchange buffers
// alternate with the tile's parity, so one barrier per tile both publishes
// this tile's partials and (being after the previous tile's reads) frees
// the buffer written next.  delta = rowsum(dO∘O) is formed from the O rows
// the kernel reads anyway; the dQ role owns its query tile's dQ whole (no
// partial rows, no sum pass).  Column operands (Q, dO rows for dK/dV, K
// rows for dQ) are transposed through a wave-private LDS slot, as in
// attn_bwd_short.
constexpr int kS256W = 4;                     // waves per workgroup: one 64-dim slice each
constexpr int kS256X = 2 * 256 + 16;          // exchange record per wave: S, dP (as [lane][v]), delta
constexpr int kS256TP = 256 / kS256W + 4;     // transposition slot pitch
constexpr size_t kS256Lds = sizeof(float) * (2 * kS256W * kS256X + kS256W * 2 * 16 * kS256TP);

// dK/dV role: workgroup = one 16-key tile of one query head.
__device__ __forceinline__ void attn_bwd_s256_dkdv(const AttnP& p, int bid, float* smem) {
  constexpr int HD = 256, NW = kS256W, DW = HD / NW, NC = DW / 16, TP = kS256TP, XS = kS256X;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int d0 = DW * w;
  float* X = smem;                                     // [2][NW][XS]
  float* sq = smem + 2 * NW * XS + w * 2 * 16 * TP;    // this wave's Q slot [16][TP]
  float* sg = sq + 16 * TP;                            // and dO slot
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  const int grp = p.Hq / p.Hkv;
  const int kh = h / grp;
  // With query chunks (nqc > 1, cq = 16·CH queries each) the unit is (key
  // tile, chunk): the last chunk of every key tile first (causal: the
  // fullest), then the earlier chunks, each heaviest key tile first.
  const int nt = (p.S + 15) / 16;
  const int item = bid / (p.Hq * p.B);
  const int kt = item % nt;
  const int qc = p.nqc > 1 ? p.nqc - 1 - item / nt : 0;
  const int k0 = 16 * kt;
  const int kj = k0 + li;  // this lane's key (S column)
  const int64_t tok0 = (int64_t)b * p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const bool kvalid = kj < p.S && (!kpb || kpb[min(kj, p.S - 1)] > 0.5f);
  const int klast = min(k0 + 15, p.S - 1);
  int qt_lo = (p.causal ? k0 : 0) / 16;
  int qt_hi = (p.window > 0 ? min(p.S - 1, klast + p.window - 1) : p.S - 1) / 16;
  if (p.nqc > 1) {  // this chunk's query tiles; an empty chunk is never read back
    qt_lo = max(qt_lo, qc * (p.cq / 16));
    qt_hi = min(qt_hi, (qc + 1) * (p.cq / 16) - 1);
    if (qt_lo > qt_hi) return;  // whole workgroup, before any barrier
  }
  const float qk2 = p.scale * kLog2e;
  const int64_t lrow0 = ((int64_t)b * p.Hq + h) * p.S;

  // this wave's slice of the tile's K (scaled by scale·log2e) and V rows
  floatx4 kreg[NC], vreg[NC], dkacc[NC], dvacc[NC];
  {
    const int64_t row = tok0 + min(kj, p.S - 1);
    const float* kr = p.k + row * p.k_rs + (int64_t)kh * HD + d0 + 4 * lg;
    const float* vr = p.v + row * p.v_rs + (int64_t)kh * HD + d0 + 4 * lg;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kreg[c] = *reinterpret_cast<const floatx4*>(kr + 16 * c) * qk2;
      vreg[c] = *reinterpret_cast<const floatx4*>(vr + 16 * c);
      dkacc[c] = dvacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  struct QTile {
    floatx4 qa[NC], ga[NC], oa[NC];
    float lse;
  };
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(p.q + tok0 * p.q_rs + (int64_t)h * HD + d0);
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(p.dout + tok0 * p.do_rs + (int64_t)h * HD + d0);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(p.o + tok0 * p.o_rs + (int64_t)h * HD + d0);
  auto load = [&](int qt, QTile& T) {
    const int64_t r = min(16 * qt + li, p.S - 1);
    const uint32_t oq = (uint32_t)((r * p.q_rs + 4 * lg) * 4), og = (uint32_t)((r * p.do_rs + 4 * lg) * 4),
                   oo = (uint32_t)((r * p.o_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      T.qa[c] = buf_load4(rq, oq + 64u * c, 0);
      T.ga[c] = buf_load4(rg, og + 64u * c, 0);
      T.oa[c] = buf_load4(ro, oo + 64u * c, 0);
    }
    T.lse = p.lse[lrow0 + r];
  };
  QTile cur, nxt;
  if (qt_lo <= qt_hi) load(qt_lo, cur);
  int par = 0;
  for (int qt = qt_lo; qt <= qt_hi; ++qt, par ^= 1) {
    if (qt < qt_hi) load(qt + 1, nxt);
    floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
    float dl = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s4 = mfma4(cur.qa[c][t], kreg[c][t], s4);
        dp4 = mfma4(cur.ga[c][t], vreg[c][t], dp4);
        dl = fmaf(cur.ga[c][t], cur.oa[c][t], dl);
      }
    dl = add_xor32(add_xor16(dl));  // delta of query q0 + li over this slice
    float* xw = X + (par * NW + w) * XS;
    *reinterpret_cast<floatx4*>(xw + 4 * lane) = s4;
    *reinterpret_cast<floatx4*>(xw + 256 + 4 * lane) = dp4;
    if (lg == 0) xw[512 + li] = dl;
    // Q, dO by column (rows 4g + t, column 16c + i) through the wave's slots
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      *reinterpret_cast<floatx4*>(sq + li * TP + 16 * c + 4 * lg) = cur.qa[c];
      *reinterpret_cast<floatx4*>(sg + li * TP + 16 * c + 4 * lg) = cur.ga[c];
    }
    float qb[NC][4], gb[NC][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        qb[c][t] = sq[(4 * lg + t) * TP + 16 * c + li];
        gb[c][t] = sg[(4 * lg + t) * TP + 16 * c + li];
      }
    const float l2 = cur.lse * kLog2e;  // query q0 + li
    __syncthreads();
    floatx4 S = floatx4{0.f, 0.f, 0.f, 0.f}, dP = floatx4{0.f, 0.f, 0.f, 0.f}, D = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float* xu = X + (par * NW + u) * XS;
      S += *reinterpret_cast<const floatx4*>(xu + 4 * lane);
      dP += *reinterpret_cast<const floatx4*>(xu + 256 + 4 * lane);
      D += *reinterpret_cast<const floatx4*>(xu + 512 + 4 * lg);
    }
    // S[q0 + 4g + v][key kj]: P = 2^(S₂ − lse₂), dS/scale = P∘(dP − delta)
    const int q0 = 16 * qt;
    floatx4 pv, ds;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int qv = q0 + 4 * lg + v;
      const float l2v = __shfl(l2, 4 * lg + v, 64);
      const bool ok = kvalid & (qv < p.S) & (!p.causal | (qv >= kj)) & ((p.window <= 0) | (qv - kj < p.window));
      pv[v] = fast_exp2(ok ? S[v] - l2v : -INFINITY);
      ds[v] = pv[v] * (dP[v] - D[v]);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        dvacc[c] = mfma4(pv[t], gb[c][t], dvacc[c]);
        dkacc[c] = mfma4(ds[t], qb[c][t], dkacc[c]);
      }
    if (qt < qt_hi) cur = nxt;
  }
  // dK, dV [key k0 + 4g + v][dim d0 + 16c + i] of this wave's slice; partial
  // rows [chunk][B·S][Hq][HD] for GQA groups or query chunks
  const bool direct = grp == 1 && p.nqc <= 1;
  const int64_t prow = (int64_t)qc * p.B * p.S;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gk = k0 + 4 * lg + v;
    if (gk >= p.S) continue;
    const int64_t tok = tok0 + gk;
    float* dkr = (direct ? p.dk + tok * p.dk_rs + (int64_t)kh * HD : p.pdk + ((prow + tok) * p.Hq + h) * HD) + d0 + li;
    float* dvr = (direct ? p.dv + tok * p.dv_rs + (int64_t)kh * HD : p.pdv + ((prow + tok) * p.Hq + h) * HD) + d0 + li;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      dkr[16 * c] = dkacc[c][v] * p.scale;
      dvr[16 * c] = dvacc[c][v];
    }
  }
}

// dQ role: workgroup = one 16-query tile of one head.
__device__ __forceinline__ void attn_bwd_s256_dq(const AttnP& p, int bid, float* smem) {
  constexpr int HD = 256, NW = kS256W, DW = HD / NW, NC = DW / 16, TP = kS256TP, XS = kS256X;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int d0 = DW * w;
  float* X = smem;                                   // [2][NW][XS]
  float* sk = smem + 2 * NW * XS + w * 2 * 16 * TP;  // this wave's K slot [16][TP]
  const int hb = bid % (p.Hq * p.B);
  const int h = hb % p.Hq, b = hb / p.Hq;
  // Lightest (first) query tiles first: the launch fits the GPU at once and
  // its second half lands on the CUs of the first, so dQ tile j shares a CU
  // with dK/dV key tile j (heaviest first) — a causal pair sums to S/16 + 1
  // inner tiles wherever it lands, and a heavy tile finishes alone on its CU.
  // With key chunks (nkc > 1, ckq = 16·CH keys each) the unit is (query
  // tile, chunk), the first chunks first.
  const int nt = (p.S + 15) / 16;
  const int item = bid / (p.Hq * p.B);
  const int qt = item % nt;
  const int kc = p.nkc > 1 ? item / nt : 0;
  const int q0 = 16 * qt;
  const int kh = h / (p.Hq / p.Hkv);
  const int qi = q0 + li;
  const bool qok = qi < p.S;
  const int64_t tok0 = (int64_t)b * p.S;
  const float* kpb = p.kpad ? p.kpad + (int64_t)b * p.S : nullptr;
  const int qlast = min(q0 + 15, p.S - 1);
  int kt_hi = (p.causal ? qlast : p.S - 1) / 16;
  int kt_lo = p.window > 0 ? max(0, q0 - p.window + 1) / 16 : 0;
  if (p.nkc > 1) {  // this chunk's key tiles; an empty chunk is never read back
    kt_lo = max(kt_lo, kc * (p.ckq / 16));
    kt_hi = min(kt_hi, (kc + 1) * (p.ckq / 16) - 1);
    if (kt_lo > kt_hi) return;  // whole workgroup, before any barrier
  }
  const int jhi = qok ? (p.causal ? qi : p.S - 1) : -1;
  const int jlo = p.window > 0 ? qi - p.window + 1 : 0;
  const float qk2 = p.scale * kLog2e;

  // this wave's slice of the tile's Q (scaled) and dO rows (B operands of
  // Sᵀ = K·Qᵀ, dPᵀ = V·dOᵀ: the lane owns query qi), delta over the slice
  floatx4 qreg[NC], greg[NC], dqacc[NC];
  float dl = 0.f;
  {
    const int64_t row = tok0 + min(qi, p.S - 1);
    const int64_t off = (int64_t)h * HD + d0 + 4 * lg;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qreg[c] = *reinterpret_cast<const floatx4*>(p.q + row * p.q_rs + off + 16 * c) * qk2;
      greg[c] = *reinterpret_cast<const floatx4*>(p.dout + row * p.do_rs + off + 16 * c);
      const floatx4 orow = *reinterpret_cast<const floatx4*>(p.o + row * p.o_rs + off + 16 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) dl = fmaf(greg[c][e], orow[e], dl);
      dqacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const float l2 = p.lse[((int64_t)b * p.Hq + h) * p.S + min(qi, p.S - 1)] * kLog2e;
  struct KTile {
    floatx4 ka[NC], va[NC];
  };
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(p.k + tok0 * p.k_rs + (int64_t)kh * HD + d0);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(p.v + tok0 * p.v_rs + (int64_t)kh * HD + d0);
  auto load = [&](int kt, KTile& T) {
    const int64_t r = min(16 * kt + li, p.S - 1);
    const uint32_t ko = (uint32_t)((r * p.k_rs + 4 * lg) * 4), vo = (uint32_t)((r * p.v_rs + 4 * lg) * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      T.ka[c] = buf_load4(rk, ko + 64u * c, 0);
      T.va[c] = buf_load4(rv, vo + 64u * c, 0);
    }
  };
  KTile cur, nxt;
  if (kt_lo <= kt_hi) load(kt_lo, cur);
  // delta of query qi: the four slices' sums through the first exchange
  // buffer, summed in wave order (the first tile's barrier orders them)
  dl = add_xor32(add_xor16(dl));
  float dfull = 0.f;
  int par = 0;
  for (int kt = kt_lo; kt <= kt_hi; ++kt, par ^= 1) {
    if (kt < kt_hi) load(kt + 1, nxt);
    floatx4 s4 = floatx4{0.f, 0.f, 0.f, 0.f}, dp4 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s4 = mfma4(cur.ka[c][t], qreg[c][t], s4);
        dp4 = mfma4(cur.va[c][t], greg[c][t], dp4);
      }
    float* xw = X + (par * NW + w) * XS;
    *reinterpret_cast<floatx4*>(xw + 4 * lane) = s4;
    *reinterpret_cast<floatx4*>(xw + 256 + 4 * lane) = dp4;
    if (kt == kt_lo && lg == 0) xw[512 + li] = dl;
    // K by column (rows 4g + t, column 16c + i) through the wave's slot
#pragma unroll
    for (int c = 0; c < NC; ++c) *reinterpret_cast<floatx4*>(sk + li * TP + 16 * c + 4 * lg) = cur.ka[c];
    float kb[NC][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < NC; ++c) kb[c][t] = sk[(4 * lg + t) * TP + 16 * c + li];
    __syncthreads();
    floatx4 S = floatx4{0.f, 0.f, 0.f, 0.f}, dP = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float* xu = X + (par * NW + u) * XS;
      S += *reinterpret_cast<const floatx4*>(xu + 4 * lane);
      dP += *reinterpret_cast<const floatx4*>(xu + 256 + 4 * lane);
      if (kt == kt_lo) dfull += xu[512 + li];
    }
    // Sᵀ[key 16kt + 4g + v][query qi]
    floatx4 ds;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = 16 * kt + 4 * lg + v;
      bool ok = (j >= jlo) & (j <= jhi) & (j < p.S);
      if (kpb) ok = ok & (kpb[min(j, p.S - 1)] > 0.5f);
      const float pp = fast_exp2(ok ? S[v] - l2 : -INFINITY);
      ds[v] = pp * (dP[v] - dfull);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) dqacc[c] = mfma4(ds[t], kb[c][t], dqacc[c]);
    if (kt < kt_hi) cur = nxt;
  }
  // dQ [query q0 + 4g + v][dim d0 + 16c + i] of this wave's slice (with key
  // chunks: the unscaled partial row [chunk][B·S][Hq][HD], summed and scaled
  // by attn_dq_sum_kernel)
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int gq = q0 + 4 * lg + v;
    if (gq >= p.S) continue;
    if (p.nkc > 1) {
      float* dqr = p.pdq + (((int64_t)kc * p.B * p.S + tok0 + gq) * p.Hq + h) * HD + d0 + li;
#pragma unroll
      for (int c = 0; c < NC; ++c) dqr[16 * c] = dqacc[c][v];
    } else {
      float* dqr = p.dq + (tok0 + gq) * p.dq_rs + (int64_t)h * HD + d0 + li;
#pragma unroll
      for (int c = 0; c < NC; ++c) dqr[16 * c] = dqacc[c][v] * p.scale;
    }
  }
}

// Both roles in one launch: blocks [0, n_dkdv) are dK/dV tiles, the rest dQ tiles.
__global__ __launch_bounds__(64 * kS256W) void attn_bwd_short256(AttnP p, int n_dkdv) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int bid = (int)blockIdx.x;
  if (bid < n_dkdv) attn_bwd_s256_dkdv(p, bid, smem);
  else attn_bwd_s256_dq(p, bid - n_dkdv, smem);
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
  const size_t lds = sizeof(float) * std::max<size_t>(BKV * P + HD * (BKV + 4) + BKV, 16 * NW * P);
  const bool split = p.nch > 1;
  auto kern = split ? attn_fwd_mfma<HD, NW, BKV, true> : attn_fwd_mfma<HD, NW, BKV, false>;
  set_lds(kern, lds);
  dim3 grid((unsigned)(cdiv(p.S, 16 * NW) * p.nch * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
  if (split) {
    const int64_t total = (int64_t)p.B * p.Hq * p.S * (HD / 4);
    hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, p, 16 * NW);
    MFT_LAUNCH_CHECK();
  }
}

template <int HD, int NW, bool SQ, bool SK>
void bwd_main_launch(hipStream_t s, AttnP& p) {
  constexpr int P = HD + 4;
  constexpr int BQ = Cfg<HD>::BQ;
  constexpr int BKV = Cfg<HD>::DQBKV;
  const size_t lds_kv = sizeof(float) * (HD > 128 ? 2 * 16 * NW * P + 2 * BQ * P + 2 * BQ
                                                   : 2 * BQ * P + 2 * HD * (BQ + 4) + 2 * BQ);
  const size_t lds_q = sizeof(float) * (2 * BKV * P + (HD > 128 ? 0 : HD * (BKV + 4)) + BKV);
  const size_t lds = std::max(lds_kv, lds_q);
  auto kern = attn_bwd_mfma<HD, NW, BQ, BKV, SQ, SK>;
  set_lds(kern, lds);
  const int64_t blocks = cdiv(p.S, 16 * NW) * (int64_t)p.Hq * p.B;
  const int n_dkdv = (int)(blocks * p.nqc);
  dim3 grid((unsigned)(n_dkdv + blocks * p.nkc));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p, n_dkdv);
  MFT_LAUNCH_CHECK();
}

template <int HD, int NW>
void bwd_main(hipStream_t s, AttnP& p) {
  const bool sq = p.nqc > 1, sk = p.nkc > 1;
  if (sq && sk) bwd_main_launch<HD, NW, true, true>(s, p);
  else if (sq) bwd_main_launch<HD, NW, true, false>(s, p);
  else if (sk) bwd_main_launch<HD, NW, false, true>(s, p);
  else bwd_main_launch<HD, NW, false, false>(s, p);
  if (p.nkc > 1) {
    const int64_t total = (int64_t)p.B * p.S * p.Hq * (HD / 4);
    hipLaunchKernelGGL(attn_dq_sum_kernel<HD>, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, p, 16 * NW);
    MFT_LAUNCH_CHECK();
  }
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

// Splits of the inner loop.  A launch with fewer than ~2 waves per SIMD
// (2048 waves on 256 CUs) leaves most matrix cores idle and each wave's
// softmax unhidden, so the inner range (keys of a query block, or queries of
// a key block) is cut into chunks of `per` loop blocks (≥ 2), one workgroup
// per non-empty (block, chunk), aiming at ~4096 waves (twice that in chunks
// for a causal mask, which empties about half of them), at most max_chunks
// chunks.  Returns blocks per chunk, 0 for no split.  Tuning hook: the
// environment variable `hook` forces blocks per chunk (0 = no split).
int chunk_blocks(const AttnArgs& a, int64_t waves, int nblk, int max_chunks, const char* hook) {
  int per = 0;
  if (const char* forced = getenv(hook)) {
    per = atoi(forced);
  } else if (waves < 2048 && nblk >= 4) {
    const int64_t want = std::min<int64_t>(cdiv(4096, waves) * (a.causal ? 2 : 1), max_chunks);
    per = std::max(2, (int)cdiv(nblk, want));
  }
  if (per <= 0 || per >= nblk) return 0;
  return std::max(per, (int)cdiv(nblk, max_chunks));
}

int64_t launch_waves(const AttnArgs& a, int nw) { return cdiv(a.S, 16 * nw) * nw * (int64_t)a.Hq * a.B; }

struct FwdPlan {
  int nw, nch, ck;
};

int fwd_bkv(int hd) { return hd == 64 ? Cfg<64>::FBKV : hd == 128 ? Cfg<128>::FBKV : Cfg<256>::FBKV; }

FwdPlan fwd_plan(const AttnArgs& a) {
  const int nw = pick_nw(a);
  const int bkv = fwd_bkv(a.hd);
  const int nkb = (int)cdiv(a.S, bkv);
  const int per = chunk_blocks(a, launch_waves(a, nw), nkb, kMaxChunks, "MFT_ATTN_KBPC");
  if (per == 0) return {nw, 1, a.S};
  return {nw, (int)cdiv(nkb, per), per * bkv};
}

// Backward splits (dK/dV over query chunks, dQ over key chunks), at most
// kMaxBwdChunks each: every chunk costs a partial row per (token, head), and
// at Qwen2's S = 1024 two chunks measured faster than four.
constexpr int kMaxBwdChunks = 2;

struct BwdPlan {
  int nw, nqc, cq, nkc, ckq;
};

BwdPlan bwd_plan(const AttnArgs& a) {
  const int nw = pick_nw(a);
  const int bq = a.hd == 64 ? Cfg<64>::BQ : a.hd == 128 ? Cfg<128>::BQ : Cfg<256>::BQ;
  const int bkv = a.hd == 64 ? Cfg<64>::DQBKV : a.hd == 128 ? Cfg<128>::DQBKV : Cfg<256>::DQBKV;
  const int64_t waves = launch_waves(a, nw);
  const int nqb = (int)cdiv(a.S, bq), nkb = (int)cdiv(a.S, bkv);
  // head_dim 256: a dQ split costs more in partial rows and their sums than
  // it returns (Gemma-3 at S = 256)
  const int maxq = kMaxBwdChunks, maxk = a.hd == 256 ? 1 : kMaxBwdChunks;
  const int pq = chunk_blocks(a, waves, nqb, maxq, "MFT_ATTN_BWD_BPC");
  const int pk = chunk_blocks(a, waves, nkb, maxk, "MFT_ATTN_BWD_BPC");
  BwdPlan pl{nw, 1, a.S, 1, a.S};
  if (pq) { pl.nqc = (int)cdiv(nqb, pq); pl.cq = pq * bq; }
  if (pk) { pl.nkc = (int)cdiv(nkb, pk); pl.ckq = pk * bkv; }
  return pl;
}

template <int HD>
void bwd_launch(hipStream_t s, AttnP& p, int nw) {
  if (nw == 4) bwd_main<HD, 4>(s, p);
  else if (nw == 2) bwd_main<HD, 2>(s, p);
  else bwd_main<HD, 1>(s, p);
  if (p.Hq != p.Hkv || p.nqc > 1) {
    const int64_t total = (int64_t)p.B * p.S * p.Hkv * (HD / 4);
    hipLaunchKernelGGL(attn_partial_sum_kernel<HD>, dim3((unsigned)std::min<int64_t>(cdiv(total, 256), 4096)),
                       dim3(256), 0, s, p, 16 * nw);
    MFT_LAUNCH_CHECK();
  }
}

// The short-sequence kernels serve S ≤ 256 at head_dim 64 and 128.  Tuning
// hook: MFT_ATTN_SHORT=0 keeps the blocked kernels, =1 takes the short ones
// at any S (head_dim ≤ 128).
constexpr int kShortWaves = 4;
bool use_short(const AttnArgs& a) {
  if (a.hd > 128) return false;
  if (const char* forced = getenv("MFT_ATTN_SHORT")) return atoi(forced) != 0;
  return a.S <= 256;
}

template <int HD>
void fwd_short_launch(hipStream_t s, AttnP& p) {
  constexpr int NW = kShortWaves;
  const size_t lds = sizeof(float) * (NW * 16 * (HD + 4) + 2 * NW * 16);
  auto kern = attn_fwd_short<HD, NW>;
  set_lds(kern, lds);
  const dim3 grid((unsigned)(cdiv(p.S, 16) * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
}

// The head_dim-256 forward at S ≤ 256 (its backward keeps the blocked
// kernels).  Tuning hook: MFT_ATTN_SHORT256=0 keeps the blocked forward.
bool use_short256_fwd(const AttnArgs& a) {
  static const int mode = [] {
    const char* e = getenv("MFT_ATTN_SHORT256");
    return e ? atoi(e) : 1;
  }();
  return mode != 0 && a.hd == 256 && a.S <= 256;
}

void fwd_short256_launch(hipStream_t s, AttnP& p) {
  constexpr int NW = kShortWaves, PO = 256 + 4;
  const size_t lds = sizeof(float) * (NW * 16 * PO + 2 * NW * 16);
  auto kern = attn_fwd_short256<NW>;
  set_lds(kern, lds);
  const dim3 grid((unsigned)(cdiv(p.S, 16) * p.Hq * p.B));
  hipLaunchKernelGGL(kern, grid, dim3(64 * NW), lds, s, p);
  MFT_LAUNCH_CHECK();
}

// The head_dim-256 backward at S ≤ 256 (attn_bwd_short256).  Tuning hook:
// MFT_ATTN_SHORT256_BWD=0 keeps the blocked kernels.
bool use_short256_bwd(const AttnArgs& a) {
  static const int mode = [] {
    const char* e = getenv("MFT_ATTN_SHORT256_BWD");
    return e ? atoi(e) : 1;
  }();
  return mode != 0 && a.hd == 256 && a.S <= 256;
}

// Causal chains longer than s256_chunk_tiles() tiles (16 rows each) are cut
// into chunks — the dK/dV role's query range, the dQ role's key range — so
// no workgroup runs more than that many dependent tile steps; the chunks'
// partial rows are summed in chunk order by attn_partial_sum_kernel /
// attn_dq_sum_kernel.  Tuning hook: MFT_ATTN_S256_CHUNK = tiles per chunk
// (0: unsplit).
int s256_chunk_tiles() {
  static const int t = [] {
    const char* e = getenv("MFT_ATTN_S256_CHUNK");
    return e ? atoi(e) : 8;
  }();
  return t;
}

void bwd_short256_launch(hipStream_t s, AttnP& p) {
  set_lds(attn_bwd_short256, kS256Lds);
  const int nt = (int)cdiv(p.S, 16);
  const int ch = s256_chunk_tiles();
  const int nch = ch > 0 && nt > ch ? std::min<int>((int)cdiv(nt, ch), kMaxBwdChunks) : 1;
  const int ctiles = (int)cdiv(nt, nch);  // tiles per chunk
  p.nqc = p.nkc = nch;
  p.cq = p.ckq = 16 * ctiles;
  const int tiles = (int)(nt * p.Hq * p.B);
  hipLaunchKernelGGL(attn_bwd_short256, dim3((unsigned)(2 * tiles * nch)), dim3(64 * kS256W), kS256Lds, s, p,
                     tiles * nch);
  MFT_LAUNCH_CHECK();
  const int64_t kv_total = (int64_t)p.B * p.S * p.Hkv * (256 / 4);
  const int nkv = (int)std::min<int64_t>(cdiv(kv_total, 256), 4096);
  if (nch > 1) {  // dK/dV and dQ partials, summed in one launch
    const int64_t q_total = (int64_t)p.B * p.S * p.Hq * (256 / 4);
    hipLaunchKernelGGL(attn_sums_kernel<256>, dim3((unsigned)(nkv + cdiv(q_total, 256))), dim3(256), 0, s, p, 16, 16,
                       nkv);
    MFT_LAUNCH_CHECK();
  } else if (p.Hq != p.Hkv) {
    hipLaunchKernelGGL(attn_partial_sum_kernel<256>, dim3((unsigned)nkv), dim3(256), 0, s, p, 16);
    MFT_LAUNCH_CHECK();
  }
}

template <int HD>
void bwd_short_launch(hipStream_t s, AttnP& p) {
  constexpr int NW = kShortWaves;
  // dK/dV role: 2·NW wave slots + K, V rows; dQ role: NW slots + Q, dO, O rows
  const size_t lds = sizeof(float) * std::max(2 * NW + 2, NW + 3) * 16 * (HD + 4);
  auto kern = attn_bwd_short<HD, NW>;
  set_lds(kern, lds);
  const int tiles = (int)(cdiv(p.S, 16) * p.Hq * p.B);
  hipLaunchKernelGGL(kern, dim3((unsigned)(2 * tiles)), dim3(64 * NW), lds, s, p, tiles);
  MFT_LAUNCH_CHECK();
  if (p.Hq != p.Hkv) {
    const int64_t total = (int64_t)p.B * p.S * p.Hkv * (HD / 4);
    hipLaunchKernelGGL(attn_partial_sum_kernel<HD>, dim3((unsigned)std::min<int64_t>(cdiv(total, 256), 4096)),
                       dim3(256), 0, s, p, 16);
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
  p.nch = p.nqc = p.nkc = 1;  // unsplit unless a plan says otherwise
  p.ck = p.cq = p.ckq = a.S;
  return p;
}

}  // namespace

size_t attn_fwd_scratch_floats(const AttnArgs& a) {
  if (use_short(a) || use_short256_fwd(a)) return 0;
  const FwdPlan pl = fwd_plan(a);
  if (pl.nch == 1) return 0;
  return (size_t)a.B * a.Hq * pl.nch * a.S * (size_t)(a.hd + 2);
}

size_t attn_scratch_bound_floats(int64_t tokens, int Hq, int hd) {
  const size_t rows = (size_t)tokens * Hq;
  const size_t fwd = (size_t)kMaxChunks * rows * (size_t)(hd + 2);
  const size_t bwd = (rows + 3) / 4 * 4 + 3 * (size_t)kMaxBwdChunks * rows * (size_t)hd;
  return std::max(fwd, bwd);
}

void attn_fwd(hipStream_t s, const AttnArgs& a, float* o, int64_t o_rs, float* lse, Scratch ws) {
  AttnP p = make(a);
  MFT_CHECK_ARG(o && lse, "null output");
  MFT_CHECK_ARG(o_rs % 4 == 0 && ((uintptr_t)o & 15) == 0, "o must be 16-byte aligned rows");
  p.out = o;
  p.out_rs = o_rs;
  p.lse_out = lse;
  if (use_short(a)) {
    a.hd == 64 ? fwd_short_launch<64>(s, p) : fwd_short_launch<128>(s, p);
    return;
  }
  if (use_short256_fwd(a)) {
    fwd_short256_launch(s, p);
    return;
  }
  const FwdPlan pl = fwd_plan(a);
  p.nch = pl.nch;
  p.ck = pl.ck;
  if (pl.nch > 1) {
    MFT_CHECK_ARG(ws.ptr && ws.bytes >= attn_fwd_scratch_floats(a) * sizeof(float),
                  "attention forward scratch too small");
    p.opart = ws.ptr;
    p.mlpart = reinterpret_cast<float2*>(ws.ptr + (size_t)a.B * a.Hq * pl.nch * a.S * a.hd);
  }
  switch (pl.nw) {
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
  // the short kernels read O and write dQ/dK/dV as 128-bit rows
  auto rows16 = [](const float* t, int64_t rs) { return rs % 4 == 0 && ((uintptr_t)t & 15) == 0; };
  const bool short_ok = rows16(o, o_rs) && rows16(dq, dq_rs) && rows16(dk, dk_rs) && rows16(dv, dv_rs);
  if (short_ok && use_short(a)) {  // delta formed in-kernel; GQA partials after the delta rows
    if (a.Hq != a.Hkv) {
      p.pdk = ws.ptr + (rows + 3) / 4 * 4;
      p.pdv = p.pdk + rows * a.hd;
    }
    a.hd == 64 ? bwd_short_launch<64>(s, p) : bwd_short_launch<128>(s, p);
    return;
  }
  if (short_ok && use_short256_bwd(a)) {  // delta formed in-kernel; partials after the delta rows
    // dK, dV per (query chunk, query head), then dQ per key chunk: at most
    // kMaxBwdChunks each (attn_bwd_scratch_floats)
    p.pdk = ws.ptr + (rows + 3) / 4 * 4;
    p.pdv = p.pdk + kMaxBwdChunks * rows * a.hd;
    p.pdq = p.pdv + kMaxBwdChunks * rows * a.hd;
    bwd_short256_launch(s, p);
    return;
  }
  const BwdPlan pl = bwd_plan(a);
  p.nqc = pl.nqc; p.cq = pl.cq;
  p.nkc = pl.nkc; p.ckq = pl.ckq;
  p.delta_out = ws.ptr;
  p.delta = ws.ptr;
  // partial rows after delta (padded to a 16-byte boundary): dK, dV per
  // (query chunk, query head), then dQ per key chunk
  float* part = ws.ptr + (rows + 3) / 4 * 4;
  if (a.Hq != a.Hkv || pl.nqc > 1) {
    p.pdk = part;
    p.pdv = part + pl.nqc * rows * a.hd;
    part += 2 * pl.nqc * rows * a.hd;
  }
  if (pl.nkc > 1) p.pdq = part;
  switch (a.hd) {
    case 64: hipLaunchKernelGGL(attn_delta_mfma_kernel<64>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL(attn_delta_mfma_kernel<128>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(attn_delta_mfma_kernel<256>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p); break;
  }
  MFT_LAUNCH_CHECK();
  switch (a.hd) {
    case 64: bwd_launch<64>(s, p, pl.nw); break;
    case 128: bwd_launch<128>(s, p, pl.nw); break;
    default: bwd_launch<256>(s, p, pl.nw); break;
  }
}

size_t attn_bwd_scratch_floats(const AttnArgs& a) {
  const BwdPlan pl = bwd_plan(a);
  const size_t rows = (size_t)a.B * a.S * a.Hq;
  size_t n = (rows + 3) / 4 * 4;  // covers the short kernels' need too
  if (use_short256_bwd(a)) return n + 3 * (size_t)kMaxBwdChunks * rows * (size_t)a.hd;
  if (a.Hq != a.Hkv || pl.nqc > 1) n += 2 * (size_t)pl.nqc * rows * (size_t)a.hd;
  if (pl.nkc > 1) n += (size_t)pl.nkc * rows * (size_t)a.hd;
  return n;
}

}  // namespace mft
