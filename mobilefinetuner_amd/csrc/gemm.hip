// gemm.hip — LoRA-linear GEMMs for gfx950 (CDNA4).
//
// C[M,N] = A[M,K]·op(B) on the fp32 matrix cores (v_mfma_f32_32x32x2_f32).
// A 256-thread workgroup owns a BM×BN tile; its four wave64s each compute a
// 64×64 sub-tile as 2×2 MFMA tiles (four independent accumulation chains per
// wave).  When the workgroup tile is smaller than 2×2 sub-tiles, the waves
// split every K panel instead (KW-way) and their partial tiles are summed
// through LDS in a fixed order at the end, so each LDS element is read by one
// wave only.  K is consumed in panels of BK through a two-stage LDS ring; the
// global loads of panel k+2 are in flight while panel k is multiplied.  The
// epilogue fuses bias, the rank-r LoRA term scale·P[M,r]·Q, a residual add
// and accumulation into C.
//
// B may be [K,N] (frozen W in the forward, tied embedding in the LM-head
// backward) or [N,K] (W in dX = dY·Wᵀ, embedding in the LM-head forward),
// fp32 or fp16; fp16 is widened to fp32 while the panel is staged into LDS,
// so a frozen fp16 weight is read from HBM at 2 bytes/element and never
// materialised as fp32.
//
// LDS layouts (pitch = row length + 4 floats, conflict-free):
//   A       As[m][k]  — fragments read as 128-bit rows;
//   B [N,K] Bs[n][k]  — same;
//   B [K,N] Bs[k][n]  — global rows land with 128-bit stores, fragments are
//                       read as 32-bit columns (consecutive n per lane).
// In-panel k order: wave kw takes k ∈ [kw·KS, (kw+1)·KS) (KS = BK/KW); lane
// half h of a 32×32 tile supplies k = kw·KS + h·KS/2 + j for its KS/2 MFMAs
// (A and B permuted identically, so the sum is unchanged).  Interior tiles
// take an unchecked load path; edge tiles check every element.
#include <cfloat>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include <hip/hip_ext.h>

#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace mft {
namespace {

struct GemmParams {
  const float* A;
  const void* B;
  float* C;
  int64_t lda, ldb, ldc;
  int M, N, K;
  int k_chunk;       // K range per split (multiple of BK)
  int tiles_m, tiles_n, tiles_per_xcd;
  int splits;        // split-K count (the grid is 1-D; see tile_of)
  int spread;        // 1: every K-slice over all 8 XCDs (tuning comparison)
  float* partial;    // split-K: [splits][M][N] raw accumulators
  int b_vec;         // B rows allow 128-bit (fp32) / 64-bit (fp16) loads
  GemmEpilogue ep;
};

constexpr float kLog2eG = 1.4426950408889634f;

// Softmax statistics of one logits row segment of 64 values held in LDS
// (row-major, 16-byte aligned): (max t, Σ 2^(t − max)) with t = value·log2e.
// Entries past the matrix edge hold −FLT_MAX (their terms flush to 0; the
// first entry is always inside).  The max runs over the raw values (scaling
// by log2e is monotonic) as IEEE maximum, which needs no canonicalised
// operands.
__device__ __forceinline__ float2 row_stats64(const float* row) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
  float v[64];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const float4 t = r4[q];
    v[4 * q] = t.x;
    v[4 * q + 1] = t.y;
    v[4 * q + 2] = t.z;
    v[4 * q + 3] = t.w;
  }
  float mx = v[0];
#pragma unroll
  for (int c = 1; c + 1 < 64; c += 2) mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(v[c], v[c + 1]));
  mx = __builtin_elementwise_maximum(mx, v[63]);
  const float ml = mx * kLog2eG;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int c = 0; c < 64; c += 2) {
    s0 += __builtin_amdgcn_exp2f(fmaf(v[c], kLog2eG, -ml));
    s1 += __builtin_amdgcn_exp2f(fmaf(v[c + 1], kLog2eG, -ml));
  }
  return make_float2(ml, s0 + s1);
}

// Workgroup → (tile, split) of a 1-D grid.  Workgroup L runs on XCD L % 8
// (round-robin dispatch), each XCD with its own L2.  With s ≤ 8 splits, the
// s K-slices take 8/s XCDs each and their tiles are cut into contiguous
// ranges among those XCDs, M-fastest, so an XCD reads whole column bands of
// B and the A rows of only its own K-slice (a split-K launch that spread
// every slice over every XCD would fetch the whole of A into each of the 8
// L2s).  With `spread` (used for s > 8) every K-slice covers all 8 XCDs.
// Host side: tiles_per_xcd = ceil(tiles / (8/s)), or ceil(tiles/8) spread.
template <class Params>
__device__ __forceinline__ bool tile_of(const Params& p, int& tile, int& split) {
  const int L = blockIdx.x, xcd = L % 8, idx = L / 8;
  const int tiles = p.tiles_m * p.tiles_n;
  if (p.spread) {
    const int per = 8 * p.tiles_per_xcd, r = L % per;
    split = L / per;
    tile = (r % 8) * p.tiles_per_xcd + r / 8;
  } else {  // s ≤ 8
    const int g = 8 / p.splits;  // XCDs per split
    split = xcd / g;
    tile = (xcd % g) * p.tiles_per_xcd + idx;
  }
  return tile < tiles && split < p.splits;
}

// Bias, residual and β·C; the rank-r term is accumulated on the matrix
// cores before the epilogue.
__device__ __forceinline__ float epilogue_value(const GemmEpilogue& ep, float acc, int m, int n,
                                                const float* C, int64_t ldc) {
  float v = acc;
  if (ep.bias) v += ep.bias[n];
  if (ep.resid) v += ep.resid[(int64_t)m * ldc + n];
  if (ep.beta != 0.f) v = fmaf(ep.beta, C[(int64_t)m * ldc + n], v);
  return v;
}

// Final value of C[m][n] (epilogue_value, then the fused GELU variants) and
// its store; with gelu_out also stores the activation.
__device__ __forceinline__ void epilogue_store(const GemmEpilogue& ep, float acc, int m, int n, float* C,
                                               int64_t ldc) {
  const int64_t at = (int64_t)m * ldc + n;
  float v = epilogue_value(ep, acc, m, n, C, ldc);
  if (ep.gelu_grad_of) v *= gelu_tanh_grad(ep.gelu_grad_of[at]);
  C[at] = v;
  if (ep.gelu_out) ep.gelu_out[at] = gelu_tanh(v);
}

template <int BM, int BN, int BK, bool B_NK, bool B_F16, int SITE>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  constexpr int NWM = BM / 64, NWN = BN / 64;  // 64×64 sub-tiles
  constexpr int KW = 4 / (NWM * NWN);          // waves sharing a sub-tile (K split)
  constexpr int KS = BK / KW;                  // k per wave per panel
  constexpr int HK = KS / 2;                   // k per lane half per panel
  static_assert(NWM * NWN * KW == 4 && HK % 8 == 0, "tile config");
  constexpr int PA = BK + 4;
  constexpr int PB = B_NK ? BK + 4 : BN + 4;
  constexpr int A_ITEMS = BM * BK / 4 / 256;   // float4 per thread per panel
  constexpr int B_ITEMS = BN * BK / 4 / 256;
  constexpr int A_STAGE = BM * PA;
  constexpr int B_STAGE = B_NK ? BN * PB : BK * PB;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int SMEM = (KW > 1 && 4 * 4096 > 2 * STAGE) ? 4 * 4096 : 2 * STAGE;
  __shared__ __attribute__((aligned(16))) float smem[SMEM];

  // XCD-aware tile order (tile_of): every XCD takes a contiguous run of
  // tiles (m fastest), so the workgroups sharing a B column panel share one
  // XCD's L2.
  int tile, split;
  if (!tile_of(p, tile, split)) return;
  const int tm_idx = tile % p.tiles_m;
  const int tn_idx = tile / p.tiles_m;
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kw = wave % KW;                 // K-split index
  const int sub = wave / KW;                // 64×64 sub-tile index
  const int wm = (sub % NWM) * 64, wn = (sub / NWM) * 64;
  const int li = lane & 31, lh = lane >> 5;
  const int klane = kw * KS + lh * HK;      // first in-panel k of this lane

  floatx16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  // Two register staging sets: panel p lives in set p%2 from the issue of its
  // global loads until it is parked in LDS stage p%2.
  floatx4 ra_set[2][A_ITEMS], rb_set[2][B_ITEMS];

  auto load_panel = [&](auto sc, int k0) {
    constexpr int S = decltype(sc)::value;
    floatx4(&ra)[A_ITEMS] = ra_set[S];
    floatx4(&rb)[B_ITEMS] = rb_set[S];
    // Branch-free: every address is clamped into its tensor (rows past M or
    // N only feed outputs that are never stored; an aligned 4-vector at
    // k < K never crosses a row because the pitches are multiples of 4) and
    // k ≥ kend elements are zeroed by selects, so the loads sit in the same
    // basic block as the MFMAs and can be interleaved with them.
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      const int gm = min(m0 + row, p.M - 1), gk = k0 + kq;
      ra[it] = *reinterpret_cast<const floatx4*>(p.A + (int64_t)gm * p.lda + (gk < kend ? gk : 0));
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      floatx4 v;
      if constexpr (B_NK) {
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        const int gn = min(n0 + row, p.N - 1), gk = k0 + kq;
        const int64_t off = (int64_t)gn * p.ldb + (gk < kend ? gk : 0);
        if constexpr (B_F16) v = stash_f16(*reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.B) + off));
        else v = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.B) + off);
      } else {
        const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
        const int gk = k0 + k, gn = n0 + nq;
        const int64_t off = (int64_t)(gk < kend ? gk : kend - 1) * p.ldb + (gn < p.N ? gn : 0);
        if constexpr (B_F16) v = stash_f16(*reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.B) + off));
        else v = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.B) + off);
      }
      rb[it] = v;
    }
  };
  // The K-tail mask (elements at k ≥ kend read as zero) is applied here,
  // at the LDS store, not at the load: a select on the loaded value would
  // make the wave wait for its global loads right after issuing them.
  auto store_panel = [&](auto sc, int k0) {
    constexpr int S = decltype(sc)::value;
    floatx4(&ra)[A_ITEMS] = ra_set[S];
    floatx4(&rb)[B_ITEMS] = rb_set[S];
    float* As = smem + S * STAGE;
    float* Bs = As + A_STAGE;
    const bool tail = k0 + BK > kend;
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      floatx4 v = ra[it];
      if (tail) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (k0 + kq + e < kend) ? v[e] : 0.f;
      }
      *reinterpret_cast<floatx4*>(&As[row * PA + kq]) = v;
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      floatx4 v = rb[it];
      if constexpr (B_F16) v = unstash_f16(v);
      if constexpr (B_NK) {
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        if (tail) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (k0 + kq + e < kend) ? v[e] : 0.f;
        }
        *reinterpret_cast<floatx4*>(&Bs[row * PB + kq]) = v;
      } else {
        const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
        if (tail && k0 + k >= kend) v = floatx4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<floatx4*>(&Bs[k * PB + nq]) = v;
      }
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  auto compute = [&](auto sc) {
    constexpr int S = decltype(sc)::value;
    const float* as = smem + S * STAGE;
    const float* bs = as + A_STAGE;
#pragma unroll
    for (int c8 = 0; c8 < HK / 8; ++c8) {
      const int kl = klane + 8 * c8;
      floatx4 fa[2][2];
      float fb[2][8];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const float* src = as + (wm + a * 32 + li) * PA + kl;
        fa[a][0] = *reinterpret_cast<const floatx4*>(src);
        fa[a][1] = *reinterpret_cast<const floatx4*>(src + 4);
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int col = wn + b * 32 + li;
        if constexpr (B_NK) {
          const floatx4 u = *reinterpret_cast<const floatx4*>(bs + col * PB + kl);
          const floatx4 v = *reinterpret_cast<const floatx4*>(bs + col * PB + kl + 4);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            fb[b][t] = u[t];
            fb[b][4 + t] = v[t];
          }
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) fb[b][t] = bs[(kl + t) * PB + col];
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][t >> 2][t & 3], fb[b][t], acc[a][b], 0, 0, 0);
    }
  };
  // Iteration kt: put panel kt+2 in flight (its register set was emptied when
  // panel kt was parked), multiply panel kt, then park panel kt+1 — whose
  // loads have had two compute phases to land — in the other LDS stage.
  // Loads and stores are unconditional (past the last panel the clamped,
  // masked loads fetch nothing that is used), keeping the step one basic
  // block; the scheduler is then told to put the fragment reads first and to
  // thread the global loads and the LDS stores through the MFMA stream.
  constexpr int N_DSR = (HK / 8) * (4 + (B_NK ? 4 : 16));
  constexpr int N_MFMA = (HK / 8) * 32;
  constexpr int N_VMEM = A_ITEMS + B_ITEMS;
  auto step = [&](auto sc, int kt) {
    constexpr int S = decltype(sc)::value;
    using SN = std::integral_constant<int, 1 - S>;
    load_panel(sc, kbeg + (kt + 2) * BK);
    compute(sc);
    store_panel(SN{}, kbeg + (kt + 1) * BK);
    __builtin_amdgcn_sched_group_barrier(0x100, N_DSR, 0);
#pragma unroll
    for (int i = 0; i < N_VMEM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < N_VMEM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, N_MFMA - 2 * N_VMEM, 0);
    __syncthreads();
  };
  if (nk > 0) load_panel(I0{}, kbeg);
  if (nk > 1) load_panel(I1{}, kbeg + BK);
  if (nk > 0) store_panel(I0{}, kbeg);
  __syncthreads();
  // Both steps run unconditionally (no control flow inside the loop body,
  // so the staged registers need no copies at a merge point): when nk is odd
  // the last step multiplies a panel past kend, which the tail mask zeroed.
  for (int kt = 0; kt < nk; kt += 2) {
    step(I0{}, kt);
    step(I1{}, kt + 1);
  }

  // Rank-r LoRA term on the matrix cores: C += lscale·P[M,r]·Qᵀ is one more
  // K panel of depth r (padded to even), staged in the free LDS ring and
  // multiplied by the waves of K-split slot 0 (split 0 only, so split-K adds
  // it once).  Lane (li, lh) supplies P[row li][2t+lh] and Q[col li][2t+lh].
  if (p.ep.P != nullptr && split == 0) {
    const int r = p.ep.r, rp = (r + 1) & ~1, pr = rp + 1;  // odd pitch: conflict-free column reads
    float* Ps = smem;
    float* Qs = smem + BM * pr;
    for (int i = tid; i < BM * rp; i += 256) {
      const int row = i / rp, j = i % rp, m = m0 + row;
      Ps[row * pr + j] = (m < p.M && j < r) ? p.ep.P[(int64_t)m * r + j] : 0.f;
    }
    for (int i = tid; i < BN * rp; i += 256) {
      const int col = i / rp, j = i % rp, n = n0 + col;
      Qs[col * pr + j] = (n < p.N && j < r) ? p.ep.lscale * p.ep.Q[(int64_t)n * p.ep.qsn + (int64_t)j * p.ep.qsj] : 0.f;
    }
    __syncthreads();
    if (kw == 0) {
      for (int t = 0; t < rp / 2; ++t) {
        const int k = 2 * t + lh;
        float fp[2], fq[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) fp[a] = Ps[(wm + a * 32 + li) * pr + k];
#pragma unroll
        for (int b = 0; b < 2; ++b) fq[b] = Qs[(wn + b * 32 + li) * pr + k];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fp[a], fq[b], acc[a][b], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  const bool split_out = p.partial != nullptr;
  // K-split: every wave parks its partial sub-tile in LDS (the ring is free
  // after the final barrier), then all 256 threads sum the KW partials of
  // each element in kw order (timing-independent) and run the epilogue with
  // coalesced row stores.
  if constexpr (KW > 1) {
    float* red = smem;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[wave * 4096 + ((a * 2 + b) * 16 + e) * 64 + lane] = acc[a][b][e];
    __syncthreads();
#pragma unroll 4
    for (int i = 0; i < BM * BN / 256; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx / BN, col = idx % BN;
      const int s2 = (col / 64) * NWM + row / 64;   // sub-tile
      const int rr = row % 64, cc = col % 64;
      const int a = rr / 32, r = rr % 32, b = cc / 32;
      const int e = 4 * (r / 8) + (r % 4), lh2 = (r / 4) % 2;
      const int slot = ((a * 2 + b) * 16 + e) * 64 + (cc % 32) + 32 * lh2;
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < KW; ++w2) v += red[(s2 * KW + w2) * 4096 + slot];
      const int m = m0 + row, n = n0 + col;
      if (m < p.M && n < p.N) {
        if (split_out)
          p.partial[((int64_t)split * p.M + m) * p.N + n] = v;
        else
          epilogue_store(p.ep, v, m, n, p.C, p.ldc);
      }
    }
    return;
  }

  // Row statistics of the LM head's logits for the cross-entropy: one
  // (max, Σ) pair per row and 64-column block of the values stored below
  // (the LM head's epilogue adds nothing); a block wholly past N writes none.
  // Each wave transposes its 64×64 sub-tile through its own region of the
  // (now idle) LDS ring, row pitch 68 floats, so lane L reads row L whole
  // with conflict-free 128-bit reads and reduces it alone; a wave's LDS
  // operations complete in issue order, so no barrier is needed.
  if constexpr (SITE == 1 && BM == 128 && BN == 128) {
    constexpr int SP = 68;
    static_assert(4 * 64 * SP <= SMEM, "LDS ring too small for the statistics transpose");
    const int nb = n0 + wn;
    if (p.ep.stats && !split_out && nb < p.N) {
      float* ws = smem + wave * 64 * SP;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const bool in = nb + b * 32 + li < p.N;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            ws[(a * 32 + 8 * (e >> 2) + 4 * lh + (e & 3)) * SP + b * 32 + li] = in ? acc[a][b][e] : -FLT_MAX;
      }
      const float2 st = row_stats64(ws + lane * SP);
      const int m = m0 + wm + lane;
      if (m < p.M) p.ep.stats[(int64_t)m * p.ep.stats_ld + nb / 64] = st;
    }
  }

  // Output: lane (li, lh) of a 32×32 tile holds column li, rows
  // 8*(e/4) + 4*lh + e%4 for e = 0..15.
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int n = n0 + wn + b * 32 + li;
      if (n >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm + a * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
        if (m >= p.M) continue;
        if (split_out)
          p.partial[((int64_t)split * p.M + m) * p.N + n] = acc[a][b][e];
        else
          epilogue_store(p.ep, acc[a][b][e], m, n, p.C, p.ldc);
      }
    }
}

// 64×64 workgroup tile for the layer GEMMs: each of the four waves owns a
// 32×32 quadrant as 2×2 tiles of v_mfma_f32_16x16x4_f32 (four independent
// accumulation chains, 16 accumulator VGPRs), so no wave shares output
// elements and the tile needs no LDS reduction at the end.  Lane (i, g) of a
// 16×16×4 MFMA supplies A[row i][k g] and B[k g][col i] and holds D[row
// 4g+v][col i]; over four consecutive MFMAs lane group g takes k = 4g..4g+3
// of a 16-wide k block (the same order for A and B), so every A fragment and
// every [N,K] B fragment is one 128-bit LDS read; with B as [K,N] the
// wave's two column tiles interleave (tile b holds columns 2i + b), so one
// 64-bit read gives a lane its B values of both tiles.  Panels of BK are staged
// through two register sets and a two-stage LDS ring exactly like
// gemm_kernel; the small register and LDS footprint allows four resident
// workgroups per CU.
template <int BM, int BK, bool B_NK, bool B_F16, int SITE>
__global__ __launch_bounds__(256) void gemm_q_kernel(GemmParams p) {
  constexpr int BN = 64;
  constexpr int WA = BM / 32;  // 16-row MFMA tiles per wave (waves are 2 × 2)
  constexpr int PA = BK + 4;
  // [K,N] B: 4·PB ≡ 32 (mod 64) puts lane groups g and g+1 of a 64-bit
  // fragment read in disjoint LDS bank halves.
  constexpr int PB = B_NK ? BK + 4 : BN + 8;
  constexpr int A_ITEMS = BM * BK / 4 / 256;
  constexpr int B_ITEMS = BN * BK / 4 / 256;
  constexpr int A_STAGE = BM * PA;
  constexpr int B_STAGE = B_NK ? BN * PB : BK * PB;
  constexpr int STAGE = A_STAGE + B_STAGE;
  static_assert(BK % 16 == 0 && A_ITEMS >= 1 && B_ITEMS >= 1, "tile config");
  __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];

  int tile, split;
  if (!tile_of(p, tile, split)) return;
  const int tm_idx = tile % p.tiles_m;
  const int tn_idx = tile / p.tiles_m;
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave & 1) * (BM / 2), wn = (wave >> 1) * 32;
  const int li = lane & 15, lg = lane >> 4;

  floatx4 acc[WA][2];
#pragma unroll
  for (int a = 0; a < WA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  floatx4 ra_set[2][A_ITEMS], rb_set[2][B_ITEMS];
  auto load_panel = [&](auto sc, int k0) {
    constexpr int S = decltype(sc)::value;
    floatx4(&ra)[A_ITEMS] = ra_set[S];
    floatx4(&rb)[B_ITEMS] = rb_set[S];
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      const int gm = min(m0 + row, p.M - 1), gk = k0 + kq;
      ra[it] = *reinterpret_cast<const floatx4*>(p.A + (int64_t)gm * p.lda + (gk < kend ? gk : 0));
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      floatx4 v;
      if constexpr (B_NK) {
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        const int gn = min(n0 + row, p.N - 1), gk = k0 + kq;
        const int64_t off = (int64_t)gn * p.ldb + (gk < kend ? gk : 0);
        if constexpr (B_F16) v = stash_f16(*reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.B) + off));
        else v = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.B) + off);
      } else {
        const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
        const int gk = k0 + k, gn = n0 + nq;
        const int64_t off = (int64_t)(gk < kend ? gk : kend - 1) * p.ldb + (gn < p.N ? gn : 0);
        if constexpr (B_F16) v = stash_f16(*reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.B) + off));
        else v = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(p.B) + off);
      }
      rb[it] = v;
    }
  };
  // The K-tail mask (elements at k ≥ kend read as zero) is applied here,
  // at the LDS store, not at the load: a select on the loaded value would
  // make the wave wait for its global loads right after issuing them.
  auto store_panel = [&](auto sc, int k0) {
    constexpr int S = decltype(sc)::value;
    floatx4(&ra)[A_ITEMS] = ra_set[S];
    floatx4(&rb)[B_ITEMS] = rb_set[S];
    float* As = smem + S * STAGE;
    float* Bs = As + A_STAGE;
    const bool tail = k0 + BK > kend;
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      floatx4 v = ra[it];
      if (tail) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (k0 + kq + e < kend) ? v[e] : 0.f;
      }
      *reinterpret_cast<floatx4*>(&As[row * PA + kq]) = v;
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      floatx4 v = rb[it];
      if constexpr (B_F16) v = unstash_f16(v);
      if constexpr (B_NK) {
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        if (tail) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (k0 + kq + e < kend) ? v[e] : 0.f;
        }
        *reinterpret_cast<floatx4*>(&Bs[row * PB + kq]) = v;
      } else {
        const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
        if (tail && k0 + k >= kend) v = floatx4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<floatx4*>(&Bs[k * PB + nq]) = v;
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  auto compute = [&](auto sc) {
    constexpr int S = decltype(sc)::value;
    const float* as = smem + S * STAGE;
    const float* bs = as + A_STAGE;
#pragma unroll
    for (int kb = 0; kb < BK; kb += 16) {
      floatx4 fa[WA], fb[2];
#pragma unroll
      for (int a = 0; a < WA; ++a) fa[a] = *reinterpret_cast<const floatx4*>(as + (wm + 16 * a + li) * PA + kb + 4 * lg);
      if constexpr (B_NK) {
#pragma unroll
        for (int b = 0; b < 2; ++b) fb[b] = *reinterpret_cast<const floatx4*>(bs + (wn + 16 * b + li) * PB + kb + 4 * lg);
      } else {
        // [K,N] B: the two 16-column tiles interleave (tile b takes columns
        // wn + 2i + b), so one 64-bit read per k feeds both MFMAs.
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float2 v = *reinterpret_cast<const float2*>(bs + (kb + 4 * lg + t) * PB + wn + 2 * li);
          fb[0][t] = v.x;
          fb[1][t] = v.y;
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int a = 0; a < WA; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a][t], fb[b][t], acc[a][b], 0, 0, 0);
    }
  };
  constexpr int N_DSR = (BK / 16) * (WA + (B_NK ? 2 : 4));
  constexpr int N_MFMA = (BK / 16) * 8 * WA;
  constexpr int N_VMEM = A_ITEMS + B_ITEMS;
  static_assert(N_MFMA >= 2 * N_VMEM, "schedule");
  auto step = [&](auto sc, int kt) {
    constexpr int S = decltype(sc)::value;
    using SN = std::integral_constant<int, 1 - S>;
    load_panel(sc, kbeg + (kt + 2) * BK);
    compute(sc);
    store_panel(SN{}, kbeg + (kt + 1) * BK);
    __builtin_amdgcn_sched_group_barrier(0x100, N_DSR, 0);
#pragma unroll
    for (int i = 0; i < N_VMEM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < N_VMEM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, N_MFMA - 2 * N_VMEM, 0);
    __syncthreads();
  };
  if ((kend - kbeg) % BK == 0) {
    // Whole panels only (the common case): every thread's global addresses
    // are fixed per tile up to the panel offset, so they are formed once
    // here and a panel adds one uniform offset (clamped to the last panel,
    // so the prefetches past the end stay in bounds; those panels are
    // stored as zeros).  No per-element masks in the loop.
    constexpr int BES = B_F16 ? 2 : 4;
    // buffer resources at the tile's first row / column and kbeg (as in
    // gemm_p_kernel): 32-bit per-lane offsets, panel offsets in SGPRs
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(p.A + (int64_t)m0 * p.lda + kbeg);
    const __amdgpu_buffer_rsrc_t rsb =
        buf_rsrc(static_cast<const char*>(p.B) + (B_NK ? (int64_t)n0 * p.ldb + kbeg : (int64_t)kbeg * p.ldb + n0) * BES);
    uint32_t a_off[A_ITEMS], b_off[B_ITEMS];
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      a_off[it] = (uint32_t)(((int64_t)(min(m0 + row, p.M - 1) - m0) * p.lda + kq) * 4);
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      if constexpr (B_NK) {
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        b_off[it] = (uint32_t)(((int64_t)(min(n0 + row, p.N - 1) - n0) * p.ldb + kq) * BES);
      } else {
        const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
        b_off[it] = (uint32_t)(((int64_t)k * p.ldb + (n0 + nq < p.N ? nq : 0)) * BES);
      }
    }
    auto load_fast = [&](auto sc, int k0) {
      constexpr int S = decltype(sc)::value;
      const int kc = min(k0, kend - BK) - kbeg;
#pragma unroll
      for (int it = 0; it < A_ITEMS; ++it) ra_set[S][it] = buf_load4(rsa, a_off[it], (uint32_t)kc * 4u);
      const uint32_t boff = (uint32_t)((B_NK ? (int64_t)kc : (int64_t)kc * p.ldb) * BES);
#pragma unroll
      for (int it = 0; it < B_ITEMS; ++it) {
        if constexpr (B_F16) rb_set[S][it] = stash_f16(buf_load2u(rsb, b_off[it], boff));
        else rb_set[S][it] = buf_load4(rsb, b_off[it], boff);
      }
    };
    auto store_fast = [&](auto sc, int k0) {
      constexpr int S = decltype(sc)::value;
      float* As = smem + S * STAGE;
      float* Bs = As + A_STAGE;
      // A panel past kend (only multiplied when nk is odd) is stored as
      // zeros; the scale keeps this a multiply, not a per-element select.
      const float keep = k0 >= kend ? 0.f : 1.f;
#pragma unroll
      for (int it = 0; it < A_ITEMS; ++it) {
        const int flat = tid + 256 * it;
        const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
        *reinterpret_cast<floatx4*>(&As[row * PA + kq]) = ra_set[S][it] * keep;
      }
#pragma unroll
      for (int it = 0; it < B_ITEMS; ++it) {
        const int flat = tid + 256 * it;
        floatx4 v = rb_set[S][it];
        if constexpr (B_F16) v = unstash_f16(v);
        if constexpr (B_NK) {
          const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
          *reinterpret_cast<floatx4*>(&Bs[row * PB + kq]) = v;
        } else {
          const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
          *reinterpret_cast<floatx4*>(&Bs[k * PB + nq]) = v;
        }
      }
    };
    auto step_fast = [&](auto sc, int kt) {
      using SN = std::integral_constant<int, 1 - decltype(sc)::value>;
      load_fast(sc, kbeg + (kt + 2) * BK);
      compute(sc);
      store_fast(SN{}, kbeg + (kt + 1) * BK);
      __builtin_amdgcn_sched_group_barrier(0x100, N_DSR, 0);
#pragma unroll
      for (int i = 0; i < N_VMEM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < N_VMEM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, N_MFMA - 2 * N_VMEM, 0);
      __syncthreads();
    };
    if (nk > 0) {
      load_fast(I0{}, kbeg);
      load_fast(I1{}, kbeg + BK);
      store_fast(I0{}, kbeg);
      __syncthreads();
      for (int kt = 0; kt < nk; kt += 2) {
        step_fast(I0{}, kt);
        step_fast(I1{}, kt + 1);
      }
    }
  } else {
    if (nk > 0) load_panel(I0{}, kbeg);
    if (nk > 1) load_panel(I1{}, kbeg + BK);
    if (nk > 0) store_panel(I0{}, kbeg);
    __syncthreads();
    // Both steps run unconditionally (no control flow inside the loop body,
    // so the staged registers need no copies at a merge point): when nk is
    // odd the last step multiplies a panel past kend, which the tail mask
    // zeroed.
    for (int kt = 0; kt < nk; kt += 2) {
      step(I0{}, kt);
      step(I1{}, kt + 1);
    }
  }

  // Rank-r LoRA term: one more K panel of depth r (padded to a multiple of
  // 4) from the free LDS ring; split 0 only.
  if (p.ep.P != nullptr && split == 0) {
    const int r = p.ep.r, rp = (r + 3) & ~3, pr = rp + 1;
    float* Ps = smem;
    float* Qs = smem + BM * pr;
    for (int i = tid; i < BM * rp; i += 256) {
      const int row = i / rp, j = i % rp, m = m0 + row;
      Ps[row * pr + j] = (m < p.M && j < r) ? p.ep.P[(int64_t)m * r + j] : 0.f;
    }
    for (int i = tid; i < BN * rp; i += 256) {
      const int col = i / rp, j = i % rp, n = n0 + col;
      Qs[col * pr + j] = (n < p.N && j < r) ? p.ep.lscale * p.ep.Q[(int64_t)n * p.ep.qsn + (int64_t)j * p.ep.qsj] : 0.f;
    }
    __syncthreads();
    for (int t = 0; t < rp / 4; ++t) {
      float fp[WA], fq[2];
#pragma unroll
      for (int a = 0; a < WA; ++a) fp[a] = Ps[(wm + 16 * a + li) * pr + 4 * t + lg];
#pragma unroll
      for (int b = 0; b < 2; ++b) fq[b] = Qs[(wn + (B_NK ? 16 * b + li : 2 * li + b)) * pr + 4 * t + lg];
#pragma unroll
      for (int a = 0; a < WA; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fp[a], fq[b], acc[a][b], 0, 0, 0);
    }
  }

  const bool split_out = p.partial != nullptr;
#pragma unroll
  for (int a = 0; a < WA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int n = n0 + wn + (B_NK ? 16 * b + li : 2 * li + b);
      if (n >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm + 16 * a + 4 * lg + v;
        if (m >= p.M) continue;
        if (split_out)
          p.partial[((int64_t)split * p.M + m) * p.N + n] = acc[a][b][v];
        else
          epilogue_store(p.ep, acc[a][b][v], m, n, p.C, p.ldc);
      }
    }
}

// Pipelined GEMM for whole BK-deep panels (BK = 32 or 64), with an optional
// rank-r LoRA panel after the last one.  Workgroup tile BM×64 (BM = 32, 64 or 128), four waves as 2×2, each
// owning (BM/2)×32 outputs as 16×16 v_mfma_f32_16x16x4_f32 tiles.  Panel
// entry j lives in LDS stage j % 3 of a three-stage ring and is stored two
// steps before it is multiplied, so during step j every wave already holds
// the fragments of the first 16-wide k block of entry j+1 (read after the
// barrier that ended step j-1): within a step, the fragments of k block q+1
// are read while block q is multiplied, and a step's MFMAs never wait on an
// LDS read issued in the same step.  Global loads run four entries ahead
// through two register sets (entry j in set j % 2, stored two steps after it
// was loaded), interleaved with the MFMAs of the step's last k block
// together with the LDS stores.  One barrier per step orders both the
// stores of entry j+2 before their reads and the reads of stage j % 3
// before it is rewritten.
//
// The loop runs two steps per iteration (the register sets alternate), so
// an odd panel count is padded at the front with a virtual entry of zeros
// stored by the prologue; loads past the last panel re-read the last panel
// (in bounds) and are never multiplied.  No per-step masks or selects.
template <int BM, int BK, bool B_NK, bool B_F16, int SITE, bool RANK>
__global__ __launch_bounds__(256) void gemm_p_kernel(GemmParams p) {
  constexpr int BN = 64;
  constexpr int WA = BM / 32;
  constexpr int Q = BK / 16;  // 16-wide k blocks per panel
  constexpr int PA = BK + 4;
  constexpr int PB = B_NK ? BK + 4 : BN + 8;  // as in gemm_q_kernel
  constexpr int A_ITEMS = BM * BK / 4 / 256;
  constexpr int B_ITEMS = BN * BK / 4 / 256;
  constexpr int A_STAGE = BM * PA;
  constexpr int B_STAGE = B_NK ? BN * PB : BK * PB;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int BES = B_F16 ? 2 : 4;
  static_assert(A_ITEMS >= 1 && B_ITEMS >= 1 && (Q == 2 || Q == 4), "tile config");
  __shared__ __attribute__((aligned(16))) float smem[3 * STAGE];

  int tile, split;
  if (!tile_of(p, tile, split)) return;
  const int tm_idx = tile % p.tiles_m;
  const int tn_idx = tile / p.tiles_m;
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nk = (kend - kbeg) / BK;  // whole panels (checked on the host)
  const int odd = nk & 1;             // entry 0 is a zero panel when nk is odd
  const int T = nk + odd;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave & 1) * (BM / 2), wn = (wave >> 1) * 32;
  const int li = lane & 15, lg = lane >> 4;

  floatx4 acc[WA][2];
#pragma unroll
  for (int a = 0; a < WA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Operands through raw buffer resources based at this workgroup's tile
  // (A at row m0, column kbeg; B at its first row or column of the K-slice):
  // a load takes one 32-bit per-lane byte offset fixed per tile plus a
  // wave-uniform panel offset in an SGPR, instead of a 64-bit address pair
  // and its 64-bit arithmetic per load (the c_fc-shaped GEMM of GPT-2 small,
  // M = 512: 24.8 → 22.2 µs).  Offsets stay within the tile's K-slice, far
  // below 2^32 bytes (checked on the host).
  const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(p.A + (int64_t)m0 * p.lda + kbeg);
  const __amdgpu_buffer_rsrc_t rsb =
      buf_rsrc(static_cast<const char*>(p.B) + (B_NK ? (int64_t)n0 * p.ldb + kbeg : (int64_t)kbeg * p.ldb + n0) * BES);
  uint32_t a_off[A_ITEMS], b_off[B_ITEMS];
  int a_lds[A_ITEMS], b_lds[B_ITEMS];  // LDS offsets (floats) within a stage
#pragma unroll
  for (int it = 0; it < A_ITEMS; ++it) {
    const int flat = tid + 256 * it;
    const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
    a_off[it] = (uint32_t)(((int64_t)(min(m0 + row, p.M - 1) - m0) * p.lda + kq) * 4);
    a_lds[it] = row * PA + kq;
  }
#pragma unroll
  for (int it = 0; it < B_ITEMS; ++it) {
    const int flat = tid + 256 * it;
    if constexpr (B_NK) {
      const int row = flat / (BK / 4), kq = (flat % (BK / 4)) * 4;
      b_off[it] = (uint32_t)(((int64_t)(min(n0 + row, p.N - 1) - n0) * p.ldb + kq) * BES);
      b_lds[it] = A_STAGE + row * PB + kq;
    } else {
      const int k = flat / (BN / 4), nq = (flat % (BN / 4)) * 4;
      b_off[it] = (uint32_t)(((int64_t)k * p.ldb + (n0 + nq < p.N ? nq : 0)) * BES);
      b_lds[it] = A_STAGE + k * PB + nq;
    }
  }

  floatx4 rs[2][A_ITEMS + B_ITEMS];  // register staging sets
  // Entry j holds panel j - odd, clamped into [0, nk-1].
  auto gload = [&](auto sc, int j) {
    constexpr int S = decltype(sc)::value;
    const int kc = min(max(j - odd, 0), nk - 1) * BK;  // within the K-slice
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) rs[S][it] = buf_load4(rsa, a_off[it], (uint32_t)kc * 4u);
    const uint32_t boff = (uint32_t)((B_NK ? (int64_t)kc : (int64_t)kc * p.ldb) * BES);
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      if constexpr (B_F16) rs[S][A_ITEMS + it] = stash_f16(buf_load2u(rsb, b_off[it], boff));
      else rs[S][A_ITEMS + it] = buf_load4(rsb, b_off[it], boff);
    }
  };
  auto lstore = [&](auto sc, int stage) {
    constexpr int S = decltype(sc)::value;
    float* st = smem + stage * STAGE;
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) *reinterpret_cast<floatx4*>(st + a_lds[it]) = rs[S][it];
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      floatx4 v = rs[S][A_ITEMS + it];
      if constexpr (B_F16) v = unstash_f16(v);
      *reinterpret_cast<floatx4*>(st + b_lds[it]) = v;
    }
  };
  struct Frags {
    floatx4 a[WA], b[2];
  };
  auto read_frags = [&](Frags& f, int stage, int kb) {
    const float* as = smem + stage * STAGE;
    const float* bs = as + A_STAGE;
#pragma unroll
    for (int a = 0; a < WA; ++a)
      f.a[a] = *reinterpret_cast<const floatx4*>(as + (wm + 16 * a + li) * PA + kb + 4 * lg);
    if constexpr (B_NK) {
#pragma unroll
      for (int b = 0; b < 2; ++b) f.b[b] = *reinterpret_cast<const floatx4*>(bs + (wn + 16 * b + li) * PB + kb + 4 * lg);
    } else {  // interleaved column tiles, one 64-bit read per k (as in gemm_q_kernel)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float2 v = *reinterpret_cast<const float2*>(bs + (kb + 4 * lg + t) * PB + wn + 2 * li);
        f.b[0][t] = v.x;
        f.b[1][t] = v.y;
      }
    }
  };
  auto mfmas = [&](const Frags& f) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int a = 0; a < WA; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[a][t], f.b[b][t], acc[a][b], 0, 0, 0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // Schedule of one step, per k block q: the next block's fragment reads,
  // then the block's MFMAs; in the last block the LDS stores and global loads
  // alternate with the MFMAs.
  constexpr int N_RD = WA + (B_NK ? 2 : 4);  // LDS read instructions per read_frags
  constexpr int N_ST = A_ITEMS + B_ITEMS;
  constexpr int N_MF = 4 * WA * 2;           // MFMAs per 16-wide k block
  Frags F[2];
  int s_cur = 0, s_nxt = 1, s_st = 2;  // stages of entries j, j+1, j+2 (wave-uniform)
  auto step = [&](auto sc, int j) {
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (q + 1 < Q) read_frags(F[(q + 1) & 1], s_cur, 16 * (q + 1));
      else read_frags(F[(q + 1) & 1], s_nxt, 0);  // entry j+1, visible since the last barrier
      if (q == Q - 1) {
        lstore(sc, s_st);  // entry j+2, loaded two steps ago
        gload(sc, j + 4);  // into the same register set
      }
      mfmas(F[q & 1]);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, N_RD, 0);
      if (q == Q - 1 && N_MF >= 2 * N_ST) {
#pragma unroll
        for (int i = 0; i < N_ST; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < N_ST; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, N_MF - 2 * N_ST, 0);
      } else if (q == Q - 1) {
        __builtin_amdgcn_sched_group_barrier(0x200, N_ST, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, N_ST, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, N_MF, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, N_MF, 0);
      }
    }
    __syncthreads();
    const int t = s_cur;
    s_cur = s_nxt;
    s_nxt = s_st;
    s_st = t;
  };
  gload(I0{}, 0);
  gload(I1{}, 1);
  if (odd) {  // the virtual entry 0: a stage of zeros (no garbage NaN·0 either)
    for (int i = tid; i < STAGE / 4; i += 256) reinterpret_cast<floatx4*>(smem)[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  } else {
    lstore(I0{}, 0);
  }
  lstore(I1{}, 1);
  gload(I0{}, 2);
  gload(I1{}, 3);
  __syncthreads();
  read_frags(F[0], 0, 0);
  for (int j = 0; j < T; j += 2) {
    step(I0{}, j);
    step(I1{}, j + 1);
  }

  // Rank-r LoRA term: one more K panel of depth r (padded to a multiple of
  // 4), staged in the ring's LDS once the last step's barrier has passed;
  // split 0 only.
  if (RANK && split == 0) {
    const int r = p.ep.r, rp = (r + 3) & ~3, pr = rp + 1;
    float* Ps = smem;
    float* Qs = smem + BM * pr;
    for (int i = tid; i < BM * rp; i += 256) {
      const int row = i / rp, j = i % rp, m = m0 + row;
      Ps[row * pr + j] = (m < p.M && j < r) ? p.ep.P[(int64_t)m * r + j] : 0.f;
    }
    for (int i = tid; i < BN * rp; i += 256) {
      const int col = i / rp, j = i % rp, n = n0 + col;
      Qs[col * pr + j] = (n < p.N && j < r) ? p.ep.lscale * p.ep.Q[(int64_t)n * p.ep.qsn + (int64_t)j * p.ep.qsj] : 0.f;
    }
    __syncthreads();
    for (int t = 0; t < rp / 4; ++t) {
      float fp[WA], fq[2];
#pragma unroll
      for (int a = 0; a < WA; ++a) fp[a] = Ps[(wm + 16 * a + li) * pr + 4 * t + lg];
#pragma unroll
      for (int b = 0; b < 2; ++b) fq[b] = Qs[(wn + (B_NK ? 16 * b + li : 2 * li + b)) * pr + 4 * t + lg];
#pragma unroll
      for (int a = 0; a < WA; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fp[a], fq[b], acc[a][b], 0, 0, 0);
    }
  }

  const bool split_out = p.partial != nullptr;
#pragma unroll
  for (int a = 0; a < WA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int n = n0 + wn + (B_NK ? 16 * b + li : 2 * li + b);
      if (n >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm + 16 * a + 4 * lg + v;
        if (m >= p.M) continue;
        if (split_out)
          p.partial[((int64_t)split * p.M + m) * p.N + n] = acc[a][b][v];
        else
          epilogue_store(p.ep, acc[a][b][v], m, n, p.C, p.ldc);
      }
    }
}

// Sum of the split-K partials in split order plus the epilogue.  Rows are
// blockIdx.y; each thread takes four consecutive columns (128-bit partial
// loads when N is a multiple of 4).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int splits,
                                                            int M, int N, float* C, int64_t ldc,
                                                            GemmEpilogue ep) {
  const int n0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n0 >= N) return;
  const int64_t total = (int64_t)M * N;
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const float* src = partial + (int64_t)m * N + n0;
    if ((N & 3) == 0) {
      floatx4 s = *reinterpret_cast<const floatx4*>(src);
      for (int z = 1; z < splits; ++z) s += *reinterpret_cast<const floatx4*>(src + (int64_t)z * total);
#pragma unroll
      for (int e = 0; e < 4; ++e) epilogue_store(ep, s[e], m, n0 + e, C, ldc);
    } else {
      for (int e = 0; e < 4 && n0 + e < N; ++e) {
        float s = 0.f;
        for (int z = 0; z < splits; ++z) s += src[(int64_t)z * total + e];
        epilogue_store(ep, s, m, n0 + e, C, ldc);
      }
    }
  }
}

// ---- fp16 matrix-core path ---------------------------------------------------
// Frozen W stored as fp16 is exact in fp16, so y = x·W can run on the fp16
// matrix cores (v_mfma_f32_16x16x32_f16: 8× the fp32 MFMA rate) once the fp32
// operand x is carried by two fp16 values.  Row m of x is scaled by
// s_m = 2^(14 − ⌊log2 max|x_m|⌋), so that max|x_m·s_m| ∈ [2^14, 2^15) sits
// inside fp16's range, and split into hi = fp16(x·s) and lo = fp16(x·s − hi),
// both rounded to nearest even (x·s and x·s − hi are exact in fp32).  The
// pair keeps x·s to within 2^-22·|x·s| (or 2^-25 absolute where lo is
// subnormal, far below the row maximum): 22 of fp32's 24 significand bits.
// Products of fp16 values are exact in fp32 and the matrix cores accumulate
// in fp32, so diag(1/s)·(hi·W + lo·W) differs from the fp32 product by a few
// units of 2^-22 relative.  The GEMM splits its A tiles while staging them
// into LDS; the row scales come from a pass that already reads every row
// (the rank-r projections of the LoRA branch, rank_batch) or from
// row_scale_kernel.  inv_s[m] = 1/s_m is a power of two.
// inv_s[m] of rows x[m, 0:K) (K a multiple of 4), one workgroup per row.
// fmaxf drops NaN operands; NaN and ±inf entries pass through the split
// unchanged (their rows' products are NaN / inf as in fp32).
__global__ __launch_bounds__(256) void row_scale_kernel(const float* __restrict__ x, int64_t ldx, int K,
                                                        float* __restrict__ inv_s) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const float* xr = x + (int64_t)m * ldx;
  float mx = 0.f;
  for (int k = 4 * tid; k < K; k += 1024) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(xr + k);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) inv_s[m] = row_inv_scale(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
}

// hi/lo split of two fp32 values x0, x1 scaled by s, packed two fp16 per
// register: hi = fp16(x·s), lo = fp16(x·s − hi), both rounded to nearest
// even from the exact fp32 value (the fma forms x·s − hi exactly).  Four
// mixed-precision fmas write each half in place (mixlo keeps the high half,
// mixhi the low), instead of converts plus shift-and-or packing.
__device__ __forceinline__ void split2_f16(float x0, float x1, float s, uint32_t& hi, uint32_t& lo) {
  asm("v_fma_mixlo_f16 %0, %2, %4, 0\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0\n\t"
      "v_fma_mixlo_f16 %1, %2, %4, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %1, %3, %4, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(hi), "=&v"(lo)
      : "v"(x0), "v"(x1), "v"(s));
}

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

// A column segment of a segmented launch: output columns [n0, next n0) of
// the launch take their own B, C and rank-r panel (P, Q) — the q, k and v
// (or gate and up) projections of one shared input in one launch.
struct GemmHSegment {
  int n0;
  const uint16_t* B;
  int64_t ldb;
  float* C;
  int64_t ldc;
  const float* P;
  const float* Q;
};
constexpr int kMaxGemmHSegments = 3;
// A K segment of a K-segmented launch ([N,K] B only): reduction indices
// [k0, next k0) take their own B (fp16 [N][ldb]), the row scales of their A
// columns and their rank-r panel — dX = Σ_g dY_g·W_gᵀ over the q, k and v (or
// gate and up) projections, whose dY are column blocks of one A.
struct GemmHKSegment {
  int k0;
  const uint16_t* B;
  int64_t ldb;
  const float* inv_s;
  const float* P;
  const float* Q;
};

struct GemmHParams {
  const float* A;      // fp32 [M][lda]
  const float* inv_s;  // [M] row scales 1/s_m (powers of two), or null (s = 1)
  const uint16_t* B;   // fp16 [N][ldb] (B_NK) or [K][ldb]
  float* C;
  int64_t lda, ldb, ldc;
  int M, N, K;
  int k_chunk;
  int tiles_m, tiles_n, tiles_per_xcd;
  int splits, spread;
  float* partial;
  GemmEpilogue ep;
  int nseg;  // > 1: column segments (unsplit K, every segment a whole number of BN-wide tiles)
  GemmHSegment seg[kMaxGemmHSegments];
  int nkseg;  // > 1: K segments (B_NK; every segment a whole number of 32-deep panels)
  GemmHKSegment kseg[kMaxGemmHSegments];
};

// C = diag(inv_s)·(hi + lo)·op(B) (+ the rank-r panel and epilogue of
// gemm_p_kernel), hi/lo the fp16 split of diag(s)·A made while A's fp32
// panel is staged into LDS.  Workgroup tile BM×BN, four waves as 2×2, each
// owning (BM/2)×(BN/2) outputs as 16×16 tiles; K in panels of 32 (one
// v_mfma_f32_16x16x32_f16 k-block: lane l holds row l%16, k 8(l/16)..+7 of
// each operand).  LDS per stage: the hi and lo A planes [BM][32] and B as
// [BN][32] (B_NK) or [32][BN] (k-major, as W [K,N] is stored): k-major B
// fragments come out of LDS through ds_read_b64_tr_b16, which hands lane
// 4a+e of every 16-lane group element e of the 8-byte rows addressed by
// lanes a, a+4, a+8, a+12 — lanes addressing rows k..k+3 at columns
// n0 + 4·(0..3) give each lane four consecutive k of its own column, so W
// needs no transposed copy.  Pipeline as in gemm_p_kernel: a three-stage
// LDS ring stored two steps ahead, global loads four steps ahead in two
// register sets, fragments of the next stage read at the top of each step,
// one barrier per step.  Row pitches: 40 halves (A, [N,K] B: 16-byte
// fragment reads conflict-free over 8 lanes), BN + 16 halves (k-major B:
// the four rows of a 16-lane transposed read fall in disjoint banks).
template <int BM, int BN, bool B_NK, bool RANK, int PIPE>
__global__ __launch_bounds__(256) void gemm_h_kernel(GemmHParams p) {
  constexpr int BK = 32;
  constexpr int TA = BM / 32, TB = BN / 32;  // 16×16 tiles per wave along M and N
  constexpr int PA = BK + 8;
  constexpr int PT = BN + 16;
  constexpr int A_PL = BM * PA;
  constexpr int B_PL = B_NK ? BN * PA : BK * PT;
  constexpr int STAGE = 2 * A_PL + B_PL;  // halves
  constexpr int A_ITEMS = BM * BK / 4 / 256;  // 16-byte fp32 chunks of A per thread
  constexpr int B_ITEMS = BN * BK / 8 / 256;  // 16-byte fp16 chunks of B per thread
  constexpr int N_ST = A_ITEMS + B_ITEMS;     // global loads per panel
  constexpr int N_WR = 2 * A_ITEMS + B_ITEMS; // LDS stores per panel
  static_assert(A_ITEMS >= 1 && B_ITEMS >= 1 && TA >= 1 && TB >= 1, "tile config");
  __shared__ __attribute__((aligned(16))) uint16_t smem[3 * STAGE];

  int tile, split;
  if (!tile_of(p, tile, split)) return;
  const int tm_idx = tile % p.tiles_m;
  const int tn_idx = tile / p.tiles_m;
  const int m0 = tm_idx * BM;
  int n0 = tn_idx * BN;
  static_assert(kMaxGemmHSegments == 3, "segment selects below");
  if (p.nseg > 1) {  // the tile's column segment (uniform): its operands, columns relative to it
    // selects over constant indices only: a computed index into the kernel
    // arguments would copy them to scratch memory
    const int g = p.nseg > 2 && n0 >= p.seg[2].n0 ? 2 : n0 >= p.seg[1].n0 ? 1 : 0;
#define MFT_SEG(f) (g == 0 ? p.seg[0].f : g == 1 ? p.seg[1].f : p.seg[2].f)
    const int nb = MFT_SEG(n0);
    const int ne = g == 0 ? p.seg[1].n0 : g == 1 && p.nseg > 2 ? p.seg[2].n0 : p.N;
    p.B = MFT_SEG(B);
    p.ldb = MFT_SEG(ldb);
    p.C = MFT_SEG(C);
    p.ldc = MFT_SEG(ldc);
    p.ep.P = MFT_SEG(P);
    p.ep.Q = MFT_SEG(Q);
#undef MFT_SEG
    n0 -= nb;
    p.N = ne - nb;
  }
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nk = (kend - kbeg) / BK;  // whole panels (checked on the host)
  const int pad = (PIPE - nk % PIPE) % PIPE;  // leading zero entries: the step loop runs PIPE steps per iteration
  const int T = nk + pad;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave & 1) * (BM / 2), wn = (wave >> 1) * (BN / 2);
  const int li = lane & 15, lg = lane >> 4;

  floatx4 acc[TA][TB];
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int b = 0; b < TB; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  // buffer resources based at the tile's first row / column of its K-slice
  const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(p.A + (int64_t)m0 * p.lda + kbeg);
  const __amdgpu_buffer_rsrc_t rsb =
      buf_rsrc(p.B + (B_NK ? (int64_t)n0 * p.ldb + kbeg : (int64_t)kbeg * p.ldb + n0));
  // K segments: every segment's B based at the tile's first column (its own
  // pitch); a panel takes the segment holding its first k (selects over
  // constant indices keep the kernel arguments in scalar registers)
  static_assert(kMaxGemmHSegments == 3, "K-segment selects below");
  const bool kseg = B_NK && p.nkseg > 1;

  const int64_t kldb1 = p.kseg[1].ldb, kldb2 = p.kseg[2].ldb;
  const int kk1 = p.kseg[1].k0, kk2 = p.kseg[2].k0;
  // 1/s_m of row m: with K segments the largest of the segments' scales
  // (their A blocks share one row scale, so the products sum in one accumulator)
  auto row_isc = [&](int m) {
    if (!kseg) return p.inv_s[m];
    float v = fmaxf(p.kseg[0].inv_s[m], p.kseg[1].inv_s[m]);
    return p.nkseg > 2 ? fmaxf(v, p.kseg[2].inv_s[m]) : v;
  };
  uint32_t a_off[A_ITEMS], b_off[B_ITEMS];
  int b_row[B_ITEMS], b_kq[B_ITEMS];   // [N,K] B chunk: row within the tile, k within the panel
  int a_lds[A_ITEMS], b_lds[B_ITEMS];  // LDS offsets (halves) within a stage
  float a_sc[A_ITEMS];                 // s_m of each A chunk's row
#pragma unroll
  for (int it = 0; it < A_ITEMS; ++it) {
    const int flat = tid + 256 * it;
    const int row = flat / 8, kq = (flat % 8) * 4;
    const int mr = min(m0 + row, p.M - 1);
    a_off[it] = (uint32_t)(((int64_t)(mr - m0) * p.lda + kq) * 4);
    a_lds[it] = row * PA + kq;
    a_sc[it] = p.inv_s ? 1.f / row_isc(mr) : 1.f;  // exact: a power of two
  }
#pragma unroll
  for (int it = 0; it < B_ITEMS; ++it) {
    const int flat = tid + 256 * it;
    if constexpr (B_NK) {
      const int row = flat / 4, kq = (flat % 4) * 8;
      b_row[it] = min(n0 + row, p.N - 1) - n0;
      b_kq[it] = kq;
      b_off[it] = (uint32_t)(((int64_t)b_row[it] * p.ldb + kq) * 2);
      b_lds[it] = 2 * A_PL + row * PA + kq;
    } else {
      const int k = flat / (BN / 8), nq = (flat % (BN / 8)) * 8;
      b_off[it] = (uint32_t)(((int64_t)k * p.ldb + (n0 + nq < p.N ? nq : 0)) * 2);
      b_lds[it] = 2 * A_PL + k * PT + nq;
    }
  }

  floatx4 rs[PIPE][N_ST];  // register staging sets (16-byte chunks as floats); entry e in set e % PIPE
  auto gload = [&](auto sc, int j) {
    constexpr int S = decltype(sc)::value;
    const int kc = min(max(j - pad, 0), nk - 1) * BK;
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) rs[S][it] = buf_load4(rsa, a_off[it], (uint32_t)kc * 4u);
    if constexpr (B_NK) {
      // selects only (no branch): the panel's segment — always 0 without K
      // segments, where segment 0's B is the whole of B
      const int kg = kbeg + kc;  // the panel's first k in the whole reduction
      const int g = !kseg ? 0 : p.nkseg > 2 && kg >= kk2 ? 2 : kg >= kk1 ? 1 : 0;
      // the pointer is selected, then made a resource (selecting among three
      // resources, or among pointers computed ahead of the loop, puts them in
      // scratch memory)
      const __amdgpu_buffer_rsrc_t rb = buf_rsrc(
          g == 0 ? (kseg ? p.kseg[0].B + (int64_t)n0 * p.kseg[0].ldb : p.B + (int64_t)n0 * p.ldb)
                 : g == 1 ? p.kseg[1].B + (int64_t)n0 * kldb1 : p.kseg[2].B + (int64_t)n0 * kldb2);
      const int64_t ldb = g == 1 ? kldb1 : kldb2;
      const uint32_t boff = (uint32_t)(kg - (g == 0 ? 0 : g == 1 ? kk1 : kk2)) * 2u;
#pragma unroll
      for (int it = 0; it < B_ITEMS; ++it)
        rs[S][A_ITEMS + it] =
            buf_load4(rb, g == 0 ? b_off[it] : (uint32_t)(((int64_t)b_row[it] * ldb + b_kq[it]) * 2), boff);
    } else {
      const uint32_t boff = (uint32_t)((int64_t)kc * p.ldb * 2);
#pragma unroll
      for (int it = 0; it < B_ITEMS; ++it) rs[S][A_ITEMS + it] = buf_load4(rsb, b_off[it], boff);
    }
  };
  auto lstore = [&](auto sc, int stage) {
    constexpr int S = decltype(sc)::value;
    uint16_t* st = smem + stage * STAGE;
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      uint2 h, l;
      split2_f16(rs[S][it][0], rs[S][it][1], a_sc[it], h.x, l.x);
      split2_f16(rs[S][it][2], rs[S][it][3], a_sc[it], h.y, l.y);
      *reinterpret_cast<uint2*>(st + a_lds[it]) = h;
      *reinterpret_cast<uint2*>(st + A_PL + a_lds[it]) = l;
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) *reinterpret_cast<floatx4*>(st + b_lds[it]) = rs[S][A_ITEMS + it];
  };
  struct Frags {
    halfx8 h[TA], l[TA], b[TB];
  };
  auto read_frags = [&](Frags& f, int stage) {
    const uint16_t* st = smem + stage * STAGE;
#pragma unroll
    for (int a = 0; a < TA; ++a) {
      const int o = (wm + 16 * a + li) * PA + 8 * lg;
      f.h[a] = *reinterpret_cast<const halfx8*>(st + o);
      f.l[a] = *reinterpret_cast<const halfx8*>(st + A_PL + o);
    }
    const uint16_t* bs = st + 2 * A_PL;
    if constexpr (B_NK) {
#pragma unroll
      for (int b = 0; b < TB; ++b) f.b[b] = *reinterpret_cast<const halfx8*>(bs + (wn + 16 * b + li) * PA + 8 * lg);
    } else {
      const int r = 8 * lg + (li >> 2);
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        const int c = wn + 16 * b + 4 * (li & 3);
        const shortx4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(bs + r * PT + c));
        const shortx4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(bs + (r + 4) * PT + c));
        f.b[b] = __builtin_bit_cast(halfx8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  auto mfmas = [&](const Frags& f) {
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
      for (int b = 0; b < TB; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.h[a], f.b[b], acc[a][b], 0, 0, 0);
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
      for (int b = 0; b < TB; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.l[a], f.b[b], acc[a][b], 0, 0, 0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  constexpr int N_RD = 2 * TA + (B_NK ? TB : 2 * TB);  // LDS read instructions per read_frags
  constexpr int N_MF = 2 * TA * TB;                     // MFMAs per step
  Frags F[PIPE];                                        // entry e's fragments in F[e % PIPE]
  int s_nxt = 1, s_st = 2;  // stages of entries j+1, j+2 (wave-uniform); entry j sits in the third
  // Step j (fc = j % PIPE, sc = (j + 2) % PIPE): read entry j+1's fragments,
  // store entry j+2 (loaded PIPE steps ago) and load entry j+2+PIPE into its
  // register set, multiply entry j.
  auto step = [&](auto fc, auto sc, int j) {
    constexpr int FC = decltype(fc)::value;
    read_frags(F[(FC + 1) % PIPE], s_nxt);  // entry j+1, visible since the last barrier
    lstore(sc, s_st);
    gload(sc, j + 2 + PIPE);
    mfmas(F[FC]);
    __builtin_amdgcn_sched_group_barrier(0x100, N_RD, 0);
    if constexpr (N_MF >= N_WR + N_ST) {
#pragma unroll
      for (int i = 0; i < N_WR; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < N_ST; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, N_MF - N_WR - N_ST, 0);
    } else {
      __builtin_amdgcn_sched_group_barrier(0x200, N_WR, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, N_ST, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, N_MF, 0);
    }
    __syncthreads();
    const int t = s_nxt;  // the stage of entry j (just multiplied) takes entry j+3
    s_nxt = s_st;
    s_st = (t + 2) % 3;
  };
  // Prologue: entries 0 .. PIPE-1 into their sets, entries 0 and 1 stored
  // (zero stages for leading pad entries), then entries PIPE, PIPE+1.
  auto zero_stage = [&](int stage) {
    for (int i = tid; i < STAGE / 8; i += 256)
      reinterpret_cast<floatx4*>(smem + stage * STAGE)[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  };
  gload(I0{}, 0);
  gload(I1{}, 1);
  if constexpr (PIPE == 3) gload(I2{}, 2);
  if (pad > 0) zero_stage(0);
  else lstore(I0{}, 0);
  if (pad > 1) zero_stage(1);
  else lstore(I1{}, 1);
  gload(I0{}, PIPE);
  gload(I1{}, PIPE + 1);
  __syncthreads();
  read_frags(F[0], 0);
  if constexpr (PIPE == 2) {
    for (int j = 0; j < T; j += 2) {
      step(I0{}, I0{}, j);
      step(I1{}, I1{}, j + 1);
    }
  } else {
    for (int j = 0; j < T; j += 3) {
      step(I0{}, I2{}, j);
      step(I1{}, I0{}, j + 1);
      step(I2{}, I1{}, j + 2);
    }
  }

  // undo the row scale
  if (p.inv_s) {
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float f = row_isc(min(m0 + wm + 16 * a + 4 * lg + v, p.M - 1));
#pragma unroll
        for (int b = 0; b < TB; ++b) acc[a][b][v] *= f;
      }
  }

  // Rank-r LoRA term in fp32 (v_mfma_f32_16x16x4_f32), split 0 only, staged
  // in the ring's LDS after the last step's barrier.
  if (RANK && split == 0) {
    // with K segments the panels of the segments side by side: rank index
    // j = g·r + jj takes segment g's P[m][jj] and Q(n, jj)
    const int r = p.ep.r, rt = kseg ? p.nkseg * r : r, rp = (rt + 3) & ~3, pr = rp + 1;
    const float *kP0 = p.kseg[0].P, *kP1 = p.kseg[1].P, *kP2 = p.kseg[2].P;
    const float *kQ0 = p.kseg[0].Q, *kQ1 = p.kseg[1].Q, *kQ2 = p.kseg[2].Q;
    float* Ps = reinterpret_cast<float*>(smem);
    float* Qs = Ps + BM * pr;
    for (int i = tid; i < BM * rp; i += 256) {
      const int row = i / rp, j = i % rp, m = m0 + row;
      const int g = j / r, jj = j % r;
      const float* P = !kseg ? p.ep.P : g == 0 ? kP0 : g == 1 ? kP1 : kP2;
      Ps[row * pr + j] = (m < p.M && j < rt) ? P[(int64_t)m * r + jj] : 0.f;
    }
    for (int i = tid; i < BN * rp; i += 256) {
      const int col = i / rp, j = i % rp, n = n0 + col;
      const int g = j / r, jj = j % r;
      const float* Q = !kseg ? p.ep.Q : g == 0 ? kQ0 : g == 1 ? kQ1 : kQ2;
      Qs[col * pr + j] = (n < p.N && j < rt) ? p.ep.lscale * Q[(int64_t)n * p.ep.qsn + (int64_t)jj * p.ep.qsj] : 0.f;
    }
    __syncthreads();
    for (int t = 0; t < rp / 4; ++t) {
      float fp[TA], fq[TB];
#pragma unroll
      for (int a = 0; a < TA; ++a) fp[a] = Ps[(wm + 16 * a + li) * pr + 4 * t + lg];
#pragma unroll
      for (int b = 0; b < TB; ++b) fq[b] = Qs[(wn + 16 * b + li) * pr + 4 * t + lg];
#pragma unroll
      for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fp[a], fq[b], acc[a][b], 0, 0, 0);
    }
  }

  const bool split_out = p.partial != nullptr;
  // Row statistics of the LM head's logits for the cross-entropy, as in
  // gemm_kernel's: each wave's (BM/2)×64 sub-tile is one 64-column block;
  // the wave transposes it through its own region of the idle LDS ring (row
  // pitch 68 floats) and lane L < BM/2 reduces row L alone (row_stats64);
  // a block wholly past N writes none.
  if constexpr (BN == 128) {
    constexpr int SP = 68;
    static_assert(4 * (BM / 2) * SP * 4 <= 3 * STAGE * 2, "LDS ring too small for the statistics transpose");
    const int nb = n0 + wn;
    if (p.ep.stats && !split_out) {  // uniform over the workgroup
      __syncthreads();  // every wave is done with the ring
    }
    if (p.ep.stats && !split_out && nb < p.N) {
      float* ws = reinterpret_cast<float*>(smem) + wave * (BM / 2) * SP;
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        const bool in = nb + 16 * b + li < p.N;
#pragma unroll
        for (int a = 0; a < TA; ++a)
#pragma unroll
          for (int v = 0; v < 4; ++v) ws[(16 * a + 4 * lg + v) * SP + 16 * b + li] = in ? acc[a][b][v] : -FLT_MAX;
      }
      if (lane < BM / 2) {
        const float2 st = row_stats64(ws + lane * SP);
        const int m = m0 + wm + lane;
        if (m < p.M) p.ep.stats[(int64_t)m * p.ep.stats_ld + nb / 64] = st;
      }
    }
  }
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int b = 0; b < TB; ++b) {
      const int n = n0 + wn + 16 * b + li;
      if (n >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm + 16 * a + 4 * lg + v;
        if (m >= p.M) continue;
        if (split_out)
          p.partial[((int64_t)split * p.M + m) * p.N + n] = acc[a][b][v];
        else
          epilogue_store(p.ep, acc[a][b][v], m, n, p.C, p.ldc);
      }
    }
}

// Launch of the GEMM kernel proper.  With timing events set, the dispatch
// itself records them (hipExtLaunchKernel: the timestamps bracket the
// kernel's execution), so timing adds no event packets to the stream and the
// measured span matches a kernel trace's duration.
thread_local const KernelEvents* t_gemm_events = nullptr;
}  // namespace
thread_local hipEvent_t t_tail_start = nullptr, t_tail_stop = nullptr;
namespace {

template <typename Kern, class Params>
void launch_gemm_kernel(Kern kernel, dim3 grid, dim3 block, hipStream_t s, const Params& p) {
  if (t_gemm_events)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, t_gemm_events->start, t_gemm_events->stop, 0, p);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, s, p);
}

template <int BM, int BN, int BK, int SITE>
void launch_variant(hipStream_t s, const GemmParams& p, dim3 grid, bool b_nk, bool b_f16) {
  const dim3 block(256);
  if (b_nk) {
    if (b_f16) launch_gemm_kernel(gemm_kernel<BM, BN, BK, true, true, SITE>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_kernel<BM, BN, BK, true, false, SITE>, grid, block, s, p);
  } else {
    if (b_f16) launch_gemm_kernel(gemm_kernel<BM, BN, BK, false, true, SITE>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_kernel<BM, BN, BK, false, false, SITE>, grid, block, s, p);
  }
}

template <int BM, int BK, int SITE>
void launch_q_variant(hipStream_t s, const GemmParams& p, dim3 grid, bool b_nk, bool b_f16) {
  const dim3 block(256);
  if (b_nk) {
    if (b_f16) launch_gemm_kernel(gemm_q_kernel<BM, BK, true, true, SITE>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_q_kernel<BM, BK, true, false, SITE>, grid, block, s, p);
  } else {
    if (b_f16) launch_gemm_kernel(gemm_q_kernel<BM, BK, false, true, SITE>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_q_kernel<BM, BK, false, false, SITE>, grid, block, s, p);
  }
}

template <int BM, int BK, int SITE, bool RANK>
void launch_p_rank(hipStream_t s, const GemmParams& p, dim3 grid, bool b_nk, bool b_f16) {
  const dim3 block(256);
  if (b_nk) {
    if (b_f16) launch_gemm_kernel(gemm_p_kernel<BM, BK, true, true, SITE, RANK>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_p_kernel<BM, BK, true, false, SITE, RANK>, grid, block, s, p);
  } else {
    if (b_f16) launch_gemm_kernel(gemm_p_kernel<BM, BK, false, true, SITE, RANK>, grid, block, s, p);
    else       launch_gemm_kernel(gemm_p_kernel<BM, BK, false, false, SITE, RANK>, grid, block, s, p);
  }
}

// The rank-r panel is a template switch, so GEMMs without it keep the
// register allocation of the plain kernel.
template <int BM, int BK, int SITE>
void launch_p_variant(hipStream_t s, const GemmParams& p, dim3 grid, bool b_nk, bool b_f16) {
  if (p.ep.P != nullptr) launch_p_rank<BM, BK, SITE, true>(s, p, grid, b_nk, b_f16);
  else launch_p_rank<BM, BK, SITE, false>(s, p, grid, b_nk, b_f16);
}

// The 1-D grid of tile_of for `splits` K-slices.
template <class Params>
dim3 xcd_grid(Params& p, int splits) {
  static const int spread = [] {  // tuning hook: MFT_GEMM_SPREAD=1 spreads every K-slice over all XCDs
    const char* e = getenv("MFT_GEMM_SPREAD");
    return e ? atoi(e) : 0;
  }();
  const int tiles = p.tiles_m * p.tiles_n;
  p.splits = splits;
  // vocabulary-deep reductions (the LM head's dH, 16 splits) measured 1.4%
  // faster with every slice over all XCDs; layer GEMMs keep one K-slice per
  // XCD group (43% less L2 fetch on GPT-2 small, same time)
  p.spread = spread || splits > 8;
  if (p.spread) {
    p.tiles_per_xcd = (int)cdiv(tiles, 8);
    return dim3((unsigned)(p.tiles_per_xcd * 8 * splits), 1);
  }
  p.tiles_per_xcd = (int)cdiv(tiles, 8 / splits);
  return dim3((unsigned)(p.tiles_per_xcd * 8), 1);
}

template <int BM, int BK>
void launch_q(hipStream_t s, GemmParams& p, bool b_nk, bool b_f16, int splits) {
  p.tiles_m = (int)cdiv(p.M, BM);
  p.tiles_n = (int)cdiv(p.N, 64);
  const dim3 grid = xcd_grid(p, splits);
  // The pipelined kernel takes whole BK-deep panels in every split (and
  // the rank-r panel); gemm_q_kernel covers K tails.  Tuning hook:
  // MFT_GEMM_PIPE=0 keeps gemm_q_kernel everywhere.
  static const int pipe_mode = [] {
    const char* e = getenv("MFT_GEMM_PIPE");
    return e ? atoi(e) : 1;
  }();
  const bool whole = p.k_chunk % BK == 0 && p.K % BK == 0;
  if (pipe_mode != 0 && whole) {
    if (p.ep.site == 1) launch_p_variant<BM, BK, 1>(s, p, grid, b_nk, b_f16);
    else launch_p_variant<BM, BK, 0>(s, p, grid, b_nk, b_f16);
    MFT_LAUNCH_CHECK();
    return;
  }
  if (p.ep.site == 1) launch_q_variant<BM, BK, 1>(s, p, grid, b_nk, b_f16);
  else launch_q_variant<BM, BK, 0>(s, p, grid, b_nk, b_f16);
  MFT_LAUNCH_CHECK();
}

template <int BM, int BN, int BK>
void launch_tile(hipStream_t s, GemmParams& p, bool b_nk, bool b_f16, int splits) {
  p.tiles_m = (int)cdiv(p.M, BM);
  p.tiles_n = (int)cdiv(p.N, BN);
  const dim3 grid = xcd_grid(p, splits);
  if (p.ep.site == 1) launch_variant<BM, BN, BK, 1>(s, p, grid, b_nk, b_f16);
  else launch_variant<BM, BN, BK, 0>(s, p, grid, b_nk, b_f16);
  MFT_LAUNCH_CHECK();
}

// bm = 64, bn = 64 → gemm_kernel 64×64 (K split over the waves);
// bm = 64, bn = 0 → gemm_q_kernel (64×64, wave quadrants).
struct Plan {
  int bm, bn, splits;
};

int plan_bk(int bm, int bn) { return ((bm == 64 || bm == 128) && bn == 64) || bn == 1 ? 64 : 32; }

// Tile shape and split-K.  Very large grids (the LM head's forward over the
// vocabulary) use the 128×128 kernel.  Reductions over a vocabulary
// (K ≥ 16384: the LM head's dH = dlogits·E) double split-K up to 16 splits
// and 2048 workgroups — 1.2–1.45× faster than 2–4 splits at the Gemma-3 /
// Qwen2.5 / GPT-2 vocabularies.  Every other GEMM takes the cheapest of
// 64- or 32-row tiles with 1, 2, 4 or 8 splits under a wave-quantisation
// cost model: a launch runs in ceil(workgroups / capacity) rounds, capacity
// = 256 CUs × resident workgroups per CU (2 for 64-row tiles, 3 for 32-row
// tiles, from their LDS and VGPR use), a round costs the per-CU matrix work
// of those workgroups (32-row tiles at 0.8 of the 64-row rate), and a split
// adds 8 µs plus 2 µs per MB of partials written and read back.  Fitted to
// cold-cache sweeps of the 41 layer shapes of the five benchmark
// configurations on MI355X, it lands within 0.8% of the best measured plan
// in total (a 576-workgroup plan, one full round plus an eighth of a
// second, was the costliest miss of the previous rule).
Plan plan_gemm(int M, int N, int K, size_t ws_bytes) {
  if (gemm_wide_plan(M, N)) return {128, 128, 1};
  if (K >= 16384) {
    const int64_t tiles = cdiv(M, 64) * cdiv(N, 64);
    int sp = 1;
    while (tiles * sp < 2048 && K / (2 * sp) >= 512 && sp < 16 &&
           (size_t)(2 * sp) * M * N * sizeof(float) <= ws_bytes)
      sp *= 2;
    return {64, 0, sp};
  }
  Plan best{32, 0, 1};
  double best_t = 1e30;
  for (int bm : {64, 32}) {
    const int occ = bm == 64 ? 2 : 3;
    const double eff = bm == 64 ? 1.0 : 0.8;
    const int64_t tiles = cdiv(M, bm) * cdiv(N, 64);
    for (int sp : {1, 2, 4, 8}) {
      const int64_t kc = cdiv(cdiv(K, sp), 32) * 32;
      if (cdiv(K, kc) != sp) continue;
      if (sp > 1 && (kc < 256 || (size_t)sp * M * N * sizeof(float) > ws_bytes)) continue;
      const int64_t rounds = cdiv(tiles * sp, 256 * occ);
      // µs: 2·(rows·64·k) FLOPs per workgroup at 80% of a CU's 157.3/256 TFLOP/s
      double t = (double)rounds * occ * bm * 64 * kc / eff * 2.0 / (157.3e12 / 256) * 1e6 * 1.25;
      if (sp > 1) t += 8.0 + 2.0 * sp * (double)M * N * 4 / 1e6;
      if (t < best_t) {
        best_t = t;
        best = {bm, 0, sp};
      }
    }
  }
  return best;
}

// After the main launch: the split-K reduction with the epilogue (and the
// row norm, fused into it where splitk_norm can), or the row norm alone.
void gemm_finish(hipStream_t s, int splits, bool dispatch_events, const KernelEvents* ev, const float* partial,
                 int M, int N, float* C, int64_t ldc, const GemmEpilogue& ep, const RowNorm* nm) {
  MFT_CHECK_ARG(!nm || ldc == N, "a row norm needs ldc == N");
  if (splits > 1) {
    // The split-K reduction (with the epilogue and, when fused, the row
    // norm) belongs to the GEMM's time: bracket it with the tail events.
    const bool tail = ev && ev->tail_start && ev->tail_stop;
    if (tail) {
      ev->tail_used = true;
      if (dispatch_events) {
        t_tail_start = ev->tail_start;
        t_tail_stop = ev->tail_stop;
      } else {
        MFT_HIP(hipEventRecord(ev->tail_start, s));
      }
    }
    struct TailReset {
      ~TailReset() { t_tail_start = t_tail_stop = nullptr; }
    } tail_reset;
    const bool fused = nm && splitk_norm(s, partial, splits, M, N, C, ldc, ep, *nm);
    if (!fused) {
      MFT_LAUNCH_TAIL(splitk_reduce_kernel, dim3((unsigned)cdiv(N, 1024), (unsigned)std::min(M, 65535)), dim3(256),
                      0, s, partial, splits, M, N, C, ldc, ep);
    }
    t_tail_start = t_tail_stop = nullptr;
    if (tail && !dispatch_events) MFT_HIP(hipEventRecord(ev->tail_stop, s));
    MFT_LAUNCH_CHECK();
    if (!fused && nm) row_norm(s, C, M, N, *nm);
  } else if (nm) {
    row_norm(s, C, M, N, *nm);
  }
}


// ---- fp16 matrix-core GEMM launch ----
template <int BM, int BN, bool RANK>
void launch_h_rank(hipStream_t s, GemmHParams& p, bool b_nk, int splits) {
  p.tiles_m = (int)cdiv(p.M, BM);
  p.tiles_n = (int)cdiv(p.N, BN);
  const dim3 grid = xcd_grid(p, splits), block(256);
  static const int pipe = [] {  // tuning hook: MFT_GEMMH_PIPE = 2 or 3 register staging sets
    const char* e = getenv("MFT_GEMMH_PIPE");
    return e && atoi(e) == 2 ? 2 : 3;
  }();
  if (pipe == 3) {
    if (b_nk) launch_gemm_kernel(gemm_h_kernel<BM, BN, true, RANK, 3>, grid, block, s, p);
    else launch_gemm_kernel(gemm_h_kernel<BM, BN, false, RANK, 3>, grid, block, s, p);
  } else {
    if (b_nk) launch_gemm_kernel(gemm_h_kernel<BM, BN, true, RANK, 2>, grid, block, s, p);
    else launch_gemm_kernel(gemm_h_kernel<BM, BN, false, RANK, 2>, grid, block, s, p);
  }
  MFT_LAUNCH_CHECK();
}
template <int BM, int BN>
void launch_h(hipStream_t s, GemmHParams& p, bool b_nk, int splits) {
  if (p.ep.P != nullptr) launch_h_rank<BM, BN, true>(s, p, b_nk, splits);
  else launch_h_rank<BM, BN, false>(s, p, b_nk, splits);
}

// Tile shape and split-K of the fp16 GEMM.  A panel step's time is the
// larger of a per-shape latency floor and the step's operand bytes (fp32 A,
// fp16 B) times the workgroups resident at once over an effective L2 rate;
// a launch runs ceil(workgroups / capacity) rounds of k_chunk/32 steps
// (capacity = 256 CUs × 1, 2 or 3 workgroups of the 128×128, 64×128 and
// 64×64 tiles, from their LDS rings), plus 5 µs per launch and, split, 2 µs
// plus the partials at 3 MB/µs.  Fitted to MI355X sweeps of the Gemma-3 1B
// linear shapes (M = 1024, 18 plans each), it picks within 6% of the best
// measured plan in total; K-slices deeper than 1024 measured slower than
// the model says (the fp32 A rows of a deep slice fall out of L2), so deep
// reductions split until a slice is at most 1024 deep.
struct PlanH {
  int bm, bn, splits;
};
PlanH plan_gemm_h(int M, int N, int K, size_t ws_bytes, bool stats) {
  struct Shape {
    int bm, bn, occ;
    double lat_us;
  };
  static const Shape shapes[] = {{128, 128, 1, 1.0}, {64, 128, 2, 0.4}, {64, 64, 3, 0.3}};
  PlanH best{64, 64, 1};
  double best_t = 1e30;
  for (const Shape& sh : shapes) {
    if (stats && sh.bn != 128) continue;  // row statistics: 64-column blocks per wave, unsplit K
    const int64_t tiles = cdiv(M, sh.bm) * cdiv(N, sh.bn);
    for (int sp : {1, 2, 3, 4, 6, 8, 16, 32}) {
      const int64_t kc = cdiv(cdiv(K, sp), 32) * 32;
      if (cdiv(K, kc) != sp) continue;
      if (stats && sp > 1) continue;
      if (sp > 1 && (kc < 128 || (size_t)sp * M * N * sizeof(float) > ws_bytes)) continue;
      if (K >= 4096 && kc > 1024 && sp < 8) continue;
      const int64_t wgs = tiles * sp, cap = 256 * sh.occ;
      const double conc = (double)std::min<int64_t>(wgs, cap);
      const double step_bytes = sh.bm * 32.0 * 4 + sh.bn * 32.0 * 2;
      const double tau = std::max(sh.lat_us, conc * step_bytes / 11e6);  // µs per panel step
      double t = 5.0 + (double)cdiv(wgs, cap) * (double)(kc / 32) * tau;
      if (sp > 1) t += 2.0 + sp * (double)M * N * 8 / 3e6;
      if (t < best_t) {
        best_t = t;
        best = {sh.bm, sh.bn, sp};
      }
    }
  }
  return best;
}
}  // namespace

bool gemm_wide_plan(int M, int N) { return cdiv(M, 128) * cdiv(N, 128) >= 1024; }

// Tuning hooks MFT_GEMM_PLAN / MFT_GEMMH_PLAN: "bm,bn,splits" forces every
// launch; "M,N,K:bm,bn,splits;..." forces the listed shapes only.  Returns
// false when the variable forces nothing for this shape.
static bool forced_plan(const char* env, int M, int N, int K, int& bm, int& bn, int& sp) {
  if (!env) return false;
  if (!strchr(env, ':')) return sscanf(env, "%d,%d,%d", &bm, &bn, &sp) == 3;
  for (const char* e = env; e && *e; e = strchr(e, ';') ? strchr(e, ';') + 1 : nullptr) {
    int m = 0, n = 0, k = 0;
    if (sscanf(e, "%d,%d,%d:%d,%d,%d", &m, &n, &k, &bm, &bn, &sp) == 6 && m == M && n == N && k == K) return true;
  }
  return false;
}

void gemm(hipStream_t s, const float* A, int64_t lda, const void* B, int64_t ldb, bool b_nk,
          bool b_f16, float* C, int64_t ldc, int M, int N, int K, const GemmEpilogue& ep,
          Scratch ws, const KernelEvents* ev) {
  MFT_CHECK_ARG(M > 0 && N > 0 && K > 0, "empty GEMM");
  MFT_CHECK_ARG(lda % 4 == 0 && lda >= K, "lda must be a multiple of 4 and >= K");
  MFT_CHECK_ARG(!b_nk || ldb >= K, "ldb must be >= K for [N,K] B");
  MFT_CHECK_ARG(b_nk || ldb >= N, "ldb must be >= N for [K,N] B");
  MFT_CHECK_ARG(ldc >= N, "ldc must be >= N");
  MFT_CHECK_ARG(ep.r <= 32, "LoRA rank > 32 unsupported");
  MFT_CHECK_ARG(((uintptr_t)A & 15) == 0, "A must be 16-byte aligned");
  GemmParams p;
  p.A = A; p.B = B; p.C = C;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K;
  p.ep = ep;
  p.partial = nullptr;
  p.b_vec = (ldb % 4 == 0) && (((uintptr_t)B & (b_f16 ? 7 : 15)) == 0);
  if (!p.b_vec) {
    // The kernel reads B as aligned 4-vectors; repack an unaligned or
    // odd-pitch B into the workspace with a padded pitch first.
    const size_t esz = b_f16 ? 2 : 4;
    const int64_t rows = b_nk ? N : K, cols = b_nk ? K : N;
    const int64_t pitch = (cols + 3) / 4 * 4;
    const size_t need = (size_t)rows * pitch * esz;
    MFT_CHECK_ARG(ws.ptr && ws.bytes >= need + 256, "unaligned B needs a workspace for repacking");
    char* dst = reinterpret_cast<char*>(ws.ptr);
    MFT_HIP(hipMemcpy2DAsync(dst, pitch * esz, B, ldb * esz, cols * esz, rows, hipMemcpyDeviceToDevice, s));
    p.B = dst;
    p.ldb = pitch;
    p.b_vec = 1;
    const size_t used = (need + 255) / 256 * 256;
    ws.ptr = reinterpret_cast<float*>(dst + used);
    ws.bytes -= used;
  }

  Plan pl = plan_gemm(M, N, K, ws.ptr ? ws.bytes : 0);
  // Tuning hook: MFT_GEMM_PLAN="bm,bn,splits" (or per shape, "M,N,K:bm,bn,splits;...") forces the launch shape
  // (bm×bn ∈ {128×128, 64×128, 64×64}, or "64,0,s" for the quadrant kernel);
  // same arithmetic, other tiling.
  static const char* forced_env = getenv("MFT_GEMM_PLAN");
  int bm = 0, bn = 0, sp = 0;
  const bool forced = forced_plan(forced_env, M, N, K, bm, bn, sp);
  if (forced && !ep.stats) {
    if (sp >= 1 &&
        ((bm == 128 && bn == 128) || (bm == 64 && bn == 128) || (bm == 64 && bn == 64) ||
         ((bm == 32 || bm == 64 || bm == 128) && (bn == 0 || bn == 1))) &&
        (sp == 1 || (size_t)sp * M * N * sizeof(float) <= ws.bytes))
      pl = {bm, bn, sp};
  }
  const RowNorm* nm = ep.norm && ep.norm->kind != NORM_NONE ? ep.norm : nullptr;
  // A row norm after the GEMM costs nothing extra in a split-K reduction and
  // a launch of its own otherwise: an unsplit plan with K >= 512 becomes
  // 32-row tiles split in two (GPT-2 medium's attention c_proj: 53.3k vs
  // 52.9k tokens/s on MI355X; GPT-2 small's, K = 768: +1.1%).  Tuning hooks: MFT_GEMM_NORM_PLAN="bm,0,splits",
  // MFT_GEMM_NORM_MINK (the K threshold).
  static const int norm_min_k = [] {
    const char* e = getenv("MFT_GEMM_NORM_MINK");
    return e ? atoi(e) : 512;
  }();
  if (nm && !forced && pl.splits == 1 && K >= norm_min_k && N % 4 == 0 && N <= 4096 && ldc == N) {
    static const char* nplan = getenv("MFT_GEMM_NORM_PLAN");
    int bm = 32, bn = 0, sp = 2;
    if (nplan && !(sscanf(nplan, "%d,%d,%d", &bm, &bn, &sp) == 3 && sp >= 1 && (bm == 32 || bm == 64) && bn == 0))
      bm = 32, bn = 0, sp = 2;
    if ((size_t)sp * M * N * sizeof(float) <= ws.bytes) pl = {bm, bn, sp};
  }
  // Wave quantisation of the 128×128 plan: two such workgroups fit a CU, so
  // the launch runs in rounds of 512 tiles.  When its last round would be
  // under a quarter full (GPT-2's 50257-entry vocabulary at M = 512: 1572
  // tiles, 36 of them in a fourth round), the trailing column tiles become
  // an unsplit 32-row-tile launch instead, which spreads that work over the
  // whole GPU for a fraction of a round.  Plain epilogues only (bias allowed).
  MFT_CHECK_ARG(!ep.stats || (pl.bm == 128 && pl.bn == 128 && ep.site == 1 && ep.stats_ld >= cdiv(N, 64)),
                "row statistics need the 128x128 LM-head plan");
  MFT_CHECK_ARG(!ep.stats || (!ep.bias && !ep.resid && ep.beta == 0.f && !ep.gelu_out && !ep.gelu_grad_of &&
                              !ep.P && !(ep.norm && ep.norm->kind != NORM_NONE)),
                "row statistics describe plain logits (no epilogue terms)");
  int n_main = 0;
  if (pl.bm == 128 && pl.bn == 128 && !forced && !nm && ep.P == nullptr && !ep.resid && ep.beta == 0.f &&
      !ep.gelu_out && !ep.gelu_grad_of && !ep.stats) {
    const int64_t tm = cdiv(M, 128), tn = cdiv(N, 128), tiles = tm * tn;
    const int64_t rem = tiles % 512;
    if (tiles > 512 && rem > 0 && rem * 4 <= 512) n_main = (int)((tn - cdiv(rem, tm)) * 128);
  }
  const int bk = plan_bk(pl.bm, pl.bn);
  int splits = pl.splits;
  p.k_chunk = (int)(cdiv(cdiv(K, splits), bk) * bk);
  splits = (int)cdiv(K, p.k_chunk);
  static const bool log_plans = getenv("MFT_GEMM_PLAN_LOG") != nullptr;  // tuning hook: print each launch's plan
  if (log_plans) fprintf(stderr, "gemm %d,%d,%d:%d,%d,%d norm=%d main=%d\n", M, N, K, pl.bm, pl.bn, splits, nm ? 1 : 0, n_main);
  MFT_CHECK_ARG(!ep.stats || splits == 1, "row statistics need an unsplit K");
  // The whole-panel kernels address a tile's K-slice through 32-bit buffer
  // offsets from the tile's first row / column.
  MFT_CHECK_ARG(((int64_t)128 * lda + p.k_chunk) * 4 < (int64_t(1) << 32) &&
                    (b_nk ? (int64_t)128 * p.ldb + p.k_chunk : (int64_t)p.k_chunk * p.ldb + 128) * (b_f16 ? 2 : 4) <
                        (int64_t(1) << 32),
                "GEMM operand too large for 32-bit buffer offsets");
  if (splits > 1) p.partial = ws.ptr;

  // Timing: events recorded by the dispatch itself, except under stream
  // capture, where they are separate event records around the launch.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (ev) MFT_HIP(hipStreamIsCapturing(s, &cap));
  const bool dispatch_events = ev && ev->start && ev->stop && cap == hipStreamCaptureStatusNone;
  if (ev && ev->start && !dispatch_events) MFT_HIP(hipEventRecord(ev->start, s));
  t_gemm_events = dispatch_events ? ev : nullptr;
  if (n_main > 0) {
    GemmParams pm = p;
    pm.N = n_main;
    launch_tile<128, 128, 32>(s, pm, b_nk, b_f16, 1);
    t_gemm_events = nullptr;
    if (ev && ev->stop && !dispatch_events) MFT_HIP(hipEventRecord(ev->stop, s));
    // columns [n_main, N): the tail events time this launch
    GemmParams pt = p;
    const size_t esz = b_f16 ? 2 : 4;
    pt.B = static_cast<const char*>(p.B) + (b_nk ? (size_t)n_main * p.ldb : (size_t)n_main) * esz;
    pt.C = C + n_main;
    pt.N = N - n_main;
    if (pt.ep.bias) pt.ep.bias += n_main;
    pt.k_chunk = (int)(cdiv(K, 32) * 32);
    const bool tail = ev && ev->tail_start && ev->tail_stop;
    KernelEvents tev;
    if (tail) {
      ev->tail_used = true;
      tev.start = ev->tail_start;
      tev.stop = ev->tail_stop;
      if (!dispatch_events) MFT_HIP(hipEventRecord(ev->tail_start, s));
    }
    t_gemm_events = tail && dispatch_events ? &tev : nullptr;
    launch_q<32, 32>(s, pt, b_nk, b_f16, 1);
    t_gemm_events = nullptr;
    if (tail && !dispatch_events) MFT_HIP(hipEventRecord(ev->tail_stop, s));
    return;
  }
  if (pl.bm == 128 && pl.bn == 0) launch_q<128, 32>(s, p, b_nk, b_f16, splits);
  else if (pl.bm == 128 && pl.bn == 1) launch_q<128, 64>(s, p, b_nk, b_f16, splits);
  else if (pl.bm == 128) launch_tile<128, 128, 32>(s, p, b_nk, b_f16, splits);
  else if (pl.bn == 128) launch_tile<64, 128, 32>(s, p, b_nk, b_f16, splits);
  else if (pl.bn == 64) launch_tile<64, 64, 64>(s, p, b_nk, b_f16, splits);
  else if (pl.bm == 64 && pl.bn == 1) launch_q<64, 64>(s, p, b_nk, b_f16, splits);
  else if (pl.bm == 32 && pl.bn == 1) launch_q<32, 64>(s, p, b_nk, b_f16, splits);
  else if (pl.bm == 32) launch_q<32, 32>(s, p, b_nk, b_f16, splits);
  else launch_q<64, 32>(s, p, b_nk, b_f16, splits);
  t_gemm_events = nullptr;
  if (ev && ev->stop && !dispatch_events) MFT_HIP(hipEventRecord(ev->stop, s));

  gemm_finish(s, splits, dispatch_events, ev, ws.ptr, M, N, C, ldc, ep, nm);
}


void row_scales(hipStream_t s, const float* x, int64_t ldx, int M, int K, float* inv_s) {
  MFT_CHECK_ARG(M > 0 && K > 0 && K % 4 == 0 && ldx % 4 == 0 && ((uintptr_t)x & 15) == 0, "row_scales shape");
  hipLaunchKernelGGL(row_scale_kernel, dim3((unsigned)M), dim3(256), 0, s, x, ldx, K, inv_s);
  MFT_LAUNCH_CHECK();
}

bool gemm_h_ok(int N, int K, bool b_nk, int r) { return K % 32 == 0 && (b_nk || N % 8 == 0) && r <= 32; }

void gemm_h(hipStream_t s, const float* A, int64_t lda, const float* inv_s, const uint16_t* B, int64_t ldb, bool b_nk,
            float* C, int64_t ldc, int M, int N, int K, const GemmEpilogue& ep, Scratch ws, const KernelEvents* ev) {
  MFT_CHECK_ARG(M > 0 && N > 0 && K > 0, "empty GEMM");
  MFT_CHECK_ARG(gemm_h_ok(N, K, b_nk, ep.r), "fp16 GEMM takes K % 32 == 0, N % 8 == 0 for [K,N] B, r <= 32");
  MFT_CHECK_ARG(A && lda >= K && lda % 4 == 0, "lda must be a multiple of 4 and >= K");
  MFT_CHECK_ARG(b_nk ? ldb >= K : ldb >= N, "ldb too small");
  MFT_CHECK_ARG(ldb % 8 == 0, "ldb must be a multiple of 8");
  MFT_CHECK_ARG(ldc >= N, "ldc must be >= N");
  MFT_CHECK_ARG((((uintptr_t)A | (uintptr_t)B) & 15) == 0, "GEMM operands must be 16-byte aligned");
  MFT_CHECK_ARG(!ep.stats || (ep.stats_ld >= cdiv(N, 64) && !ep.bias && !ep.resid && ep.beta == 0.f && !ep.gelu_out &&
                              !ep.gelu_grad_of && !ep.P && !(ep.norm && ep.norm->kind != NORM_NONE)),
                "row statistics describe plain logits (no epilogue terms)");
  GemmHParams p{};
  p.A = A; p.inv_s = inv_s; p.B = B; p.C = C;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K;
  p.ep = ep;
  p.partial = nullptr;
  PlanH pl = plan_gemm_h(M, N, K, ws.ptr ? ws.bytes : 0, ep.stats != nullptr);
  // Tuning hook: MFT_GEMMH_PLAN="bm,bn,splits" (or per shape, "M,N,K:bm,bn,splits;...") forces the launch shape.
  static const char* forced_env = getenv("MFT_GEMMH_PLAN");
  int bm = 0, bn = 0, sp = 0;
  const bool forced = forced_plan(forced_env, M, N, K, bm, bn, sp);
  if (forced && !ep.stats) {
    if (sp >= 1 && sp <= 64 &&
        ((bm == 128 && bn == 128) || (bm == 64 && bn == 128) || (bm == 64 && bn == 64)) &&
        (sp == 1 || (size_t)sp * M * N * sizeof(float) <= ws.bytes))
      pl = {bm, bn, sp};
  }
  const RowNorm* nm = ep.norm && ep.norm->kind != NORM_NONE ? ep.norm : nullptr;
  // as in gemm(): a row norm rides in the split-K reduction for free
  if (nm && !forced && !ep.stats && pl.splits == 1 && K >= 512 && N % 4 == 0 && N <= 4096 && ldc == N &&
      (size_t)2 * M * N * sizeof(float) <= ws.bytes)
    pl.splits = 2;
  int splits = pl.splits;
  p.k_chunk = (int)(cdiv(cdiv(K, splits), 32) * 32);
  splits = (int)cdiv(K, p.k_chunk);
  static const bool log_plans = getenv("MFT_GEMM_PLAN_LOG") != nullptr;
  if (log_plans) fprintf(stderr, "gemm_h %d,%d,%d:%d,%d,%d norm=%d\n", M, N, K, pl.bm, pl.bn, splits, nm ? 1 : 0);
  MFT_CHECK_ARG(((int64_t)pl.bm * p.lda + p.k_chunk) * 4 < (int64_t(1) << 32) &&
                    (b_nk ? (int64_t)pl.bn * p.ldb + p.k_chunk : (int64_t)p.k_chunk * p.ldb + pl.bn) * 2 <
                        (int64_t(1) << 32),
                "GEMM operand too large for 32-bit buffer offsets");
  if (splits > 1) p.partial = ws.ptr;

  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (ev) MFT_HIP(hipStreamIsCapturing(s, &cap));
  const bool dispatch_events = ev && ev->start && ev->stop && cap == hipStreamCaptureStatusNone;
  if (ev && ev->start && !dispatch_events) MFT_HIP(hipEventRecord(ev->start, s));
  t_gemm_events = dispatch_events ? ev : nullptr;
  if (pl.bm == 128) launch_h<128, 128>(s, p, b_nk, splits);
  else if (pl.bn == 128) launch_h<64, 128>(s, p, b_nk, splits);
  else launch_h<64, 64>(s, p, b_nk, splits);
  t_gemm_events = nullptr;
  if (ev && ev->stop && !dispatch_events) MFT_HIP(hipEventRecord(ev->stop, s));
  gemm_finish(s, splits, dispatch_events, ev, ws.ptr, M, N, C, ldc, ep, nm);
}

bool gemm_h_segments(hipStream_t s, const float* A, int64_t lda, const float* inv_s, bool b_nk,
                     const GemmHSegmentArg* seg, int nseg, int M, int K, const GemmEpilogue& ep,
                     const KernelEvents* ev) {
  MFT_CHECK_ARG(seg && nseg >= 2 && nseg <= kMaxGemmHSegments && M > 0 && K > 0, "segmented GEMM: 2 or 3 segments");
  MFT_CHECK_ARG(A && lda >= K && lda % 4 == 0 && ((uintptr_t)A & 15) == 0, "segmented GEMM: A");
  MFT_CHECK_ARG(!ep.bias && !ep.resid && ep.beta == 0.f && !ep.gelu_out && !ep.gelu_grad_of && !ep.stats &&
                    !(ep.norm && ep.norm->kind != NORM_NONE),
                "segmented GEMM: plain outputs plus the rank-r panel only");
  int N = 0;
  bool all64 = true, all128 = true;
  for (int g = 0; g < nseg; ++g) {
    const GemmHSegmentArg& a = seg[g];
    MFT_CHECK_ARG(a.B && a.C && a.N > 0 && gemm_h_ok(a.N, K, b_nk, ep.r) && a.ldb % 8 == 0 &&
                      (b_nk ? a.ldb >= K : a.ldb >= a.N) && a.ldc >= a.N && ((uintptr_t)a.B & 15) == 0,
                  "segmented GEMM: segment shape");
    MFT_CHECK_ARG((ep.r > 0) == (a.P != nullptr && a.Q != nullptr), "segmented GEMM: rank panel per segment");
    all64 = all64 && a.N % 64 == 0;
    all128 = all128 && a.N % 128 == 0;
    N += a.N;
  }
  PlanH pl = plan_gemm_h(M, N, K, 0, false);  // no workspace: unsplit
  static const char* forced_env = getenv("MFT_GEMMH_PLAN");
  int bm = 0, bn = 0, sp = 0;
  if (forced_plan(forced_env, M, N, K, bm, bn, sp) && sp == 1 &&
      ((bm == 128 && bn == 128) || (bm == 64 && bn == 128) || (bm == 64 && bn == 64)))
    pl = {bm, bn, 1};
  if (pl.bn == 128 && !all128) pl = {64, 64, 1};
  if (!all64) return false;
  GemmHParams p{};
  p.A = A; p.inv_s = inv_s; p.B = seg[0].B; p.C = seg[0].C;
  p.lda = lda; p.ldb = seg[0].ldb; p.ldc = seg[0].ldc;
  p.M = M; p.N = N; p.K = K;
  p.ep = ep;
  p.ep.P = seg[0].P;  // selects the rank-panel kernel; each tile takes its segment's panel
  p.ep.Q = seg[0].Q;
  p.partial = nullptr;
  p.k_chunk = K;
  p.nseg = nseg;
  for (int g = 0, n0 = 0; g < nseg; n0 += seg[g].N, ++g) {
    p.seg[g] = GemmHSegment{n0, seg[g].B, seg[g].ldb, seg[g].C, seg[g].ldc, seg[g].P, seg[g].Q};
    MFT_CHECK_ARG((b_nk ? (int64_t)pl.bn * seg[g].ldb + K : (int64_t)K * seg[g].ldb + pl.bn) * 2 < (int64_t(1) << 32),
                  "GEMM operand too large for 32-bit buffer offsets");
  }
  MFT_CHECK_ARG(((int64_t)pl.bm * lda + K) * 4 < (int64_t(1) << 32), "GEMM operand too large for 32-bit buffer offsets");
  static const bool log_plans = getenv("MFT_GEMM_PLAN_LOG") != nullptr;
  if (log_plans) fprintf(stderr, "gemm_h_seg %d,%d,%d:%d,%d,1 nseg=%d\n", M, N, K, pl.bm, pl.bn, nseg);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (ev) MFT_HIP(hipStreamIsCapturing(s, &cap));
  const bool dispatch_events = ev && ev->start && ev->stop && cap == hipStreamCaptureStatusNone;
  if (ev && ev->start && !dispatch_events) MFT_HIP(hipEventRecord(ev->start, s));
  t_gemm_events = dispatch_events ? ev : nullptr;
  if (pl.bm == 128) launch_h<128, 128>(s, p, b_nk, 1);
  else if (pl.bn == 128) launch_h<64, 128>(s, p, b_nk, 1);
  else launch_h<64, 64>(s, p, b_nk, 1);
  t_gemm_events = nullptr;
  if (ev && ev->stop && !dispatch_events) MFT_HIP(hipEventRecord(ev->stop, s));
  return true;
}

void gemm_h_ksegments(hipStream_t s, const float* A, int64_t lda, const GemmHKSegmentArg* seg, int nseg, float* C,
                      int64_t ldc, int M, int N, const GemmEpilogue& ep, Scratch ws, const KernelEvents* ev) {
  MFT_CHECK_ARG(seg && nseg >= 2 && nseg <= kMaxGemmHSegments && M > 0 && N > 0, "K-segmented GEMM: 2 or 3 segments");
  MFT_CHECK_ARG(A && lda % 4 == 0 && ((uintptr_t)A & 15) == 0, "K-segmented GEMM: A");
  MFT_CHECK_ARG(ldc >= N && nseg * ep.r <= 32, "K-segmented GEMM: ldc or rank");
  MFT_CHECK_ARG(!ep.stats && !ep.gelu_out && !ep.gelu_grad_of, "K-segmented GEMM: no statistics or GELU terms");
  int K = 0;
  for (int g = 0; g < nseg; ++g) {
    const GemmHKSegmentArg& a = seg[g];
    MFT_CHECK_ARG(a.B && a.inv_s && a.K > 0 && a.K % 32 == 0 && a.ldb >= a.K && a.ldb % 8 == 0 &&
                      ((uintptr_t)a.B & 15) == 0,
                  "K-segmented GEMM: segment shape");
    MFT_CHECK_ARG((ep.r > 0) == (a.P != nullptr && a.Q != nullptr), "K-segmented GEMM: rank panel per segment");
    K += a.K;
  }
  MFT_CHECK_ARG(lda >= K, "K-segmented GEMM: lda < K");
  GemmHParams p{};
  p.A = A; p.inv_s = seg[0].inv_s; p.B = seg[0].B; p.C = C;
  p.lda = lda; p.ldb = seg[0].ldb; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K;
  p.ep = ep;
  p.ep.P = seg[0].P;  // selects the rank-panel kernel; the panel reads every segment's P, Q
  p.ep.Q = seg[0].Q;
  p.partial = nullptr;
  p.nkseg = nseg;
  for (int g = 0, k0 = 0; g < nseg; k0 += seg[g].K, ++g)
    p.kseg[g] = GemmHKSegment{k0, seg[g].B, seg[g].ldb, seg[g].inv_s, seg[g].P, seg[g].Q};
  for (int g = nseg; g < kMaxGemmHSegments; ++g) p.kseg[g] = p.kseg[nseg - 1];  // never selected
  PlanH pl = plan_gemm_h(M, N, K, ws.ptr ? ws.bytes : 0, false);
  static const char* forced_env = getenv("MFT_GEMMH_PLAN");
  int bm = 0, bn = 0, sp = 0;
  const bool forced = forced_plan(forced_env, M, N, K, bm, bn, sp);
  if (forced && sp >= 1 && sp <= 64 && ((bm == 128 && bn == 128) || (bm == 64 && bn == 128) || (bm == 64 && bn == 64)) &&
      (sp == 1 || (size_t)sp * M * N * sizeof(float) <= ws.bytes))
    pl = {bm, bn, sp};
  const RowNorm* nm = ep.norm && ep.norm->kind != NORM_NONE ? ep.norm : nullptr;
  if (nm && !forced && pl.splits == 1 && K >= 512 && N % 4 == 0 && N <= 4096 && ldc == N &&
      (size_t)2 * M * N * sizeof(float) <= ws.bytes)
    pl.splits = 2;  // a row norm rides in the split-K reduction
  p.k_chunk = (int)(cdiv(cdiv(K, pl.splits), 32) * 32);
  const int splits = (int)cdiv(K, p.k_chunk);
  for (int g = 0; g < nseg; ++g)
    MFT_CHECK_ARG(((int64_t)pl.bn * seg[g].ldb + seg[g].K) * 2 < (int64_t(1) << 32),
                  "GEMM operand too large for 32-bit buffer offsets");
  MFT_CHECK_ARG(((int64_t)pl.bm * lda + p.k_chunk) * 4 < (int64_t(1) << 32), "GEMM operand too large for 32-bit buffer offsets");
  if (splits > 1) p.partial = ws.ptr;
  static const bool log_plans = getenv("MFT_GEMM_PLAN_LOG") != nullptr;
  if (log_plans) fprintf(stderr, "gemm_h_kseg %d,%d,%d:%d,%d,%d nseg=%d norm=%d\n", M, N, K, pl.bm, pl.bn, splits, nseg, nm ? 1 : 0);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (ev) MFT_HIP(hipStreamIsCapturing(s, &cap));
  const bool dispatch_events = ev && ev->start && ev->stop && cap == hipStreamCaptureStatusNone;
  if (ev && ev->start && !dispatch_events) MFT_HIP(hipEventRecord(ev->start, s));
  t_gemm_events = dispatch_events ? ev : nullptr;
  if (pl.bm == 128) launch_h<128, 128>(s, p, true, splits);
  else if (pl.bn == 128) launch_h<64, 128>(s, p, true, splits);
  else launch_h<64, 64>(s, p, true, splits);
  t_gemm_events = nullptr;
  if (ev && ev->stop && !dispatch_events) MFT_HIP(hipEventRecord(ev->stop, s));
  gemm_finish(s, splits, dispatch_events, ev, ws.ptr, M, N, C, ldc, ep, nm);
}

bool gemm_f16w(hipStream_t s, const float* x, int64_t ldx, const void* W, int64_t ldw, bool b_nk, float* C,
               int64_t ldc, int M, int N, int K, const GemmEpilogue& ep, Scratch ws, const KernelEvents* ev) {
  static const int mode = [] {  // tuning hook: MFT_GEMM_F16=0 keeps fp16 W on the fp32 kernels
    const char* e = getenv("MFT_GEMM_F16");
    return e ? atoi(e) : 1;
  }();
  if (!mode || ep.stats || !gemm_h_ok(N, K, b_nk, ep.r) || ldx % 4 != 0 || ldx < K || ((uintptr_t)x & 15) != 0 ||
      ldw % 8 != 0 || ((uintptr_t)W & 15) != 0)
    return false;
  const size_t need = ((size_t)M * sizeof(float) + 255) / 256 * 256;
  const size_t pad = ws.ptr ? (256 - ((uintptr_t)ws.ptr & 255)) & 255 : 0;
  if (!ws.ptr || ws.bytes < need + pad) return false;
  char* base = reinterpret_cast<char*>(ws.ptr) + pad;
  float* inv_s = reinterpret_cast<float*>(base);
  row_scales(s, x, ldx, M, K, inv_s);
  Scratch rest;
  rest.ptr = reinterpret_cast<float*>(base + need);
  rest.bytes = ws.bytes - need - pad;
  gemm_h(s, x, ldx, inv_s, static_cast<const uint16_t*>(W), ldw, b_nk, C, ldc, M, N, K, ep, rest, ev);
  return true;
}

}  // namespace mft
