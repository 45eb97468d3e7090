// rank.hip — the skinny rank-r products of the LoRA branch.
//
//   rank_proj:  out[M,r] = X[M,K] · Y          (xa = x·Aᵀ, U = dy·B)
//   rank_outer: out(j,c) (+)= s · Σ_m P[m,j] X[m,c]   (dA = s·Uᵀx, dB = s·dyᵀxa)
//
// Both are HBM/latency-bound passes over X (2–28 MB at the benchmark
// shapes).  rank_proj spreads each row's K over a whole workgroup (128-bit
// chunks, the r×K or K×r factor re-read from L1/L2) and reduces by
// recursive halving; rank_outer runs on
// the matrix cores, one launch for both gradients of a layer, with M split
// over the waves of a workgroup and summed in wave order (deterministic, no
// atomics, no second pass).
#include <type_traits>

#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace mft {
namespace {

// Reduce NV per-lane partial sums over a wave64 by recursive halving: at
// offset o each lane keeps one half of its values and adds the partner's
// copy of that half, so a wave needs NV-1 + log2(64/NV) shuffles instead of
// 6·NV.  Afterwards lane l holds the wave total of value l / (64/NV).
template <int NV>
__device__ __forceinline__ float wave_reduce_spread(float (&v)[NV], int lane) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "NV must be a power of two <= 64");
  int o = 32;
#pragma unroll
  for (int half = NV / 2; half >= 1; half /= 2, o /= 2) {
    const bool up = (lane & o) != 0;
#pragma unroll
    for (int q = 0; q < half; ++q) {
      const float send = up ? v[q] : v[q + half];
      const float keep = up ? v[q + half] : v[q];
      v[q] = keep + __shfl_xor(send, o, 64);
    }
  }
  float t = v[0];
#pragma unroll
  for (; o >= 1; o /= 2) t += __shfl_xor(t, o, 64);
  return t;
}

// acc[i·R + j] += Σ_k X[row i, k]·Y(k, j) over this thread's share of K for
// the RB rows xr[i], and with MX mx[i] = max |X[row i, k]| over that share.
// Y_RK: Y stored [R][K] (xa = x·Aᵀ with A [r,K]); thread t takes the 128-bit
// chunks k = 4t + 1024i and reads each Y row with one 128-bit load per chunk.
// Otherwise Y is [K][R] (U = dy·B with B [N,r]); thread t takes single
// columns k = t + 256i, E at a time, so that a wave's Y reads (R contiguous
// floats per k) are contiguous across lanes.  128-bit X chunks there would
// put 4R floats between the lanes' Y reads, one cache line per lane per load
// (2.3x slower at K = 6912, 1.5x at K = 1152).
template <int R, int RB, bool Y_RK, bool MX>
__device__ __forceinline__ void proj_accumulate(const float* const (&xr)[RB], const float* __restrict__ Y, int K,
                                                int tid, float (&acc)[RB * R], float (&mx)[RB]) {
  if constexpr (Y_RK) {
    for (int k = tid * 4; k < K; k += 1024) {
      floatx4 xv[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        xv[i] = *reinterpret_cast<const floatx4*>(xr[i] + k);
        if constexpr (MX)
          mx[i] = fmaxf(mx[i], fmaxf(fmaxf(fabsf(xv[i][0]), fabsf(xv[i][1])), fmaxf(fabsf(xv[i][2]), fabsf(xv[i][3]))));
      }
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const floatx4 y = *reinterpret_cast<const floatx4*>(Y + (int64_t)j * K + k);
#pragma unroll
        for (int i = 0; i < RB; ++i)
          acc[i * R + j] += xv[i][0] * y[0] + xv[i][1] * y[1] + xv[i][2] * y[2] + xv[i][3] * y[3];
      }
    }
  } else {
    constexpr int E = R <= 8 ? 4 : R == 16 ? 2 : 1;
    for (int k0 = tid; k0 < K; k0 += 256 * E) {
      float xs[E][RB];
      floatx4 ys[E][R / 4];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int k = k0 + 256 * e;
        if (k < K) {
#pragma unroll
          for (int i = 0; i < RB; ++i) xs[e][i] = xr[i][k];
#pragma unroll
          for (int q = 0; q < R / 4; ++q) ys[e][q] = *reinterpret_cast<const floatx4*>(Y + (int64_t)k * R + 4 * q);
        } else {
#pragma unroll
          for (int i = 0; i < RB; ++i) xs[e][i] = 0.f;
#pragma unroll
          for (int q = 0; q < R / 4; ++q) ys[e][q] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e)
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          if constexpr (MX) mx[i] = fmaxf(mx[i], fabsf(xs[e][i]));
#pragma unroll
          for (int q = 0; q < R / 4; ++q)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[i * R + 4 * q + u] = fmaf(xs[e][i], ys[e][q][u], acc[i * R + 4 * q + u]);
        }
    }
  }
}

// out[m, j] = Σ_k X[m,k]·Y(k,j), one row per 256-thread workgroup; the R
// partial sums are reduced within each wave by recursive halving and across
// the four waves in LDS.
template <int R, bool Y_RK>
__global__ __launch_bounds__(256) void rank_proj_vec_kernel(const float* __restrict__ X, int64_t ldx,
                                                             const float* __restrict__ Y, int M, int K,
                                                             float* __restrict__ out) {
  __shared__ float red[4][R];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = blockIdx.x;
  float acc[R], mx[1];
#pragma unroll
  for (int q = 0; q < R; ++q) acc[q] = 0.f;
  const float* const xr[1] = {X + (int64_t)m * ldx};
  proj_accumulate<R, 1, Y_RK, false>(xr, Y, K, tid, acc, mx);
  const float t = wave_reduce_spread<R>(acc, lane);
  constexpr int SPREAD = 64 / R;
  if ((lane % SPREAD) == 0) red[wave][lane / SPREAD] = t;
  __syncthreads();
  if (tid < R) out[(int64_t)m * R + tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
}

// Up to three projection jobs of one launch, passed by value (no job table
// to read before the first load): workgroup b runs RB rows of job b / nb
// (nb = ⌈M/RB⌉ row blocks per job) with proj_accumulate, and with inv_s set
// also writes each row's fp16-GEMM scale row_inv_scale(max_k |X[m,k]|).
// RB = 2 shares each read of Y among two rows (deep K: every workgroup reads
// all K·r floats of Y).  The per-layer batches of the rank-r panel path (xa
// of a group's shared input, U of its dY blocks) take this form.
template <int R, int RB, bool Y_RK>
__global__ __launch_bounds__(256) void rank_proj_jobs_kernel(ProjJobs jb, int M) {
  static_assert(kMaxProjJobs == 3, "job selects below");
  constexpr int NV = RB * R;
  __shared__ float red[4][NV];
  __shared__ float rmx[4][RB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nb = (M + RB - 1) / RB;
  const int g = (int)blockIdx.x / nb, m0 = ((int)blockIdx.x % nb) * RB;
  // selects over constant indices keep the arguments in scalar registers
  const float* X = g == 0 ? jb.j[0].X : g == 1 ? jb.j[1].X : jb.j[2].X;
  const int64_t ldx = g == 0 ? jb.j[0].ldx : g == 1 ? jb.j[1].ldx : jb.j[2].ldx;
  const float* Y = g == 0 ? jb.j[0].Y : g == 1 ? jb.j[1].Y : jb.j[2].Y;
  const int K = g == 0 ? jb.j[0].K : g == 1 ? jb.j[1].K : jb.j[2].K;
  float* out = g == 0 ? jb.j[0].out : g == 1 ? jb.j[1].out : jb.j[2].out;
  float* inv_s = g == 0 ? jb.j[0].inv_s : g == 1 ? jb.j[1].inv_s : jb.j[2].inv_s;
  float acc[NV], mx[RB];
#pragma unroll
  for (int q = 0; q < NV; ++q) acc[q] = 0.f;
  const float* xr[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    xr[i] = X + (int64_t)min(m0 + i, M - 1) * ldx;
    mx[i] = 0.f;
  }
  proj_accumulate<R, RB, Y_RK, true>(xr, Y, K, tid, acc, mx);
  const float t = wave_reduce_spread<NV>(acc, lane);
  constexpr int SPREAD = 64 / NV;
  if ((lane % SPREAD) == 0) red[wave][lane / SPREAD] = t;
  if (inv_s) {  // uniform per job
#pragma unroll
    for (int i = 0; i < RB; ++i) {
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], d, 64));
      if (lane == 0) rmx[wave][i] = mx[i];
    }
  }
  __syncthreads();
  if (tid < NV) {
    const int i = tid / R, j = tid % R;
    const float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    if (m0 + i < M) out[(int64_t)(m0 + i) * R + j] = v;
  }
  if (inv_s && tid < RB && m0 + tid < M)
    inv_s[m0 + tid] = row_inv_scale(fmaxf(fmaxf(rmx[0][tid], rmx[1][tid]), fmaxf(rmx[2][tid], rmx[3][tid])));
}

// Generic fallback (any r ≤ 32, any alignment).
template <int RMAX>
__global__ __launch_bounds__(256) void rank_proj_scalar_kernel(const float* X, int64_t ldx,
                                                                const float* Y, int64_t ysk,
                                                                int64_t ysj, int M, int K, int r,
                                                                float* out) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  float acc[RMAX];
#pragma unroll
  for (int j = 0; j < RMAX; ++j) acc[j] = 0.f;
  const float* xr = X + (int64_t)m * ldx;
  for (int k = lane; k < K; k += 64) {
    const float xv = xr[k];
    const float* yk = Y + (int64_t)k * ysk;
#pragma unroll
    for (int j = 0; j < RMAX; ++j)
      if (j < r) acc[j] = fmaf(xv, yk[j * ysj], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    float v = acc[j];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[j] = v;
  }
  if (lane < r) {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < RMAX; ++j)
      if (j == lane) v = acc[j];
    out[(int64_t)m * r + lane] = v;
  }
}

// out(j,c) (+)= scale·Σ_m P[m,j]·X[m,c] on the matrix cores
// (v_mfma_f32_16x16x4_f32): D[c][j] += A[c][m]·B[m][j] with A = Xᵀ, B = P,
// so lane (i, g) feeds X[m+g][c0+i] and P[m+g][16·jt+i] and ends holding
// D[c0+4g+v][16·jt+i].  A workgroup owns 16 columns c of one product; its
// 16 waves take consecutive sixteenths of M in chunks of 32 rows, each
// chunk's loads issued while the previous chunk is multiplied, and are
// summed through LDS in wave order (deterministic, no atomics).  Column
// blocks are dealt to the eight XCDs in contiguous runs, so the workgroups
// sharing a 128-byte line of X share one L2.  Two independent products (dA
// and dB of one LoRA layer) share one launch.
struct OuterJob {
  const float* P;
  const float* X;
  int64_t ldx;
  int C, blocks;  // blocks: launched for this job (a multiple of 8)
  float* out;
  int64_t osj, osc;
};
struct OuterArgs {
  OuterJob job[2];
  int M, r, accumulate;
  float scale;
};

constexpr int kOuterWaves = 16;

template <int JT>
struct OuterChunk {
  float x[8], p[JT][8];
};

template <int JT>
__device__ __forceinline__ void outer_load(OuterChunk<JT>& ch, const OuterJob& jb, int r, int m, int me, int mb,
                                           int ci, bool cok, int i, int g) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int mr = m + 4 * t + g;
    const bool ok = mr < me;
    const int mc = ok ? mr : mb;
    const float x = jb.X[(int64_t)mc * jb.ldx + ci];
    ch.x[t] = (ok && cok) ? x : 0.f;
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      const int jj = 16 * jt + i;
      const float pp = jb.P[(int64_t)mc * r + min(jj, r - 1)];
      ch.p[jt][t] = (ok && jj < r) ? pp : 0.f;
    }
  }
}

template <int JT>
__device__ __forceinline__ void outer_mfma(floatx4 (&acc)[JT], const OuterChunk<JT>& ch) {
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
      acc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ch.x[t], ch.p[jt][t], acc[jt], 0, 0, 0);
}

template <int JT>
__global__ __launch_bounds__(64 * kOuterWaves) void rank_outer_mfma(OuterArgs a) {
  __shared__ floatx4 red[kOuterWaves - 1][JT][64];
  const bool second = (int)blockIdx.x >= a.job[0].blocks;
  const OuterJob jb = second ? a.job[1] : a.job[0];
  const int raw = second ? (int)blockIdx.x - a.job[0].blocks : (int)blockIdx.x;
  const int blk = (raw % 8) * (jb.blocks / 8) + raw / 8;  // contiguous column runs per XCD
  const int c0 = blk * 16;
  if (c0 >= jb.C) return;  // whole workgroup, before any barrier
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int ci = min(c0 + i, jb.C - 1);
  const bool cok = c0 + i < jb.C;
  // rows per wave, a multiple of 32
  const int per = ((a.M + kOuterWaves * 32 - 1) / (kOuterWaves * 32)) * 32;
  const int mb = min(a.M, w * per), me = min(a.M, mb + per);
  floatx4 acc[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) acc[jt] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (mb < me) {
    OuterChunk<JT> c0v, c1v;
    outer_load(c0v, jb, a.r, mb, me, mb, ci, cok, i, g);
    for (int m = mb; m < me; m += 64) {
      // chunks past me load clamped rows and are multiplied as zeros
      outer_load(c1v, jb, a.r, m + 32, me, mb, ci, cok, i, g);
      outer_mfma(acc, c0v);
      if (m + 32 >= me) break;
      outer_load(c0v, jb, a.r, m + 64, me, mb, ci, cok, i, g);
      outer_mfma(acc, c1v);
    }
  }
  if (w > 0) {
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) red[w - 1][jt][lane] = acc[jt];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) {
    floatx4 v = acc[jt];
#pragma unroll
    for (int q = 0; q < kOuterWaves - 1; ++q) v += red[q][jt][lane];
    const int j = 16 * jt + i;
    if (j >= a.r) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = c0 + 4 * g + e;
      if (c >= jb.C) continue;
      float* o = jb.out + (int64_t)j * jb.osj + (int64_t)c * jb.osc;
      *o = a.accumulate ? fmaf(a.scale, v[e], *o) : a.scale * v[e];
    }
  }
}

// ---- batched LoRA work ---------------------------------------------------------
// W_eff[k][n] = W[k][n] + scale·Σ_j A[j][k]·B[n][j].  A workgroup owns
// kMergeRows·4 rows × 256 columns of one job; a thread takes kMergeRows rows ×
// 4 columns (the A values of its rows are wave-uniform, the B values of its
// columns come from the tile's B rows staged in LDS, reused over all its
// rows).  HBM-bound: reads W once, writes W_eff once.
constexpr int kMergeRows = 8;
template <int R>
__global__ __launch_bounds__(256) void lora_merge_kernel(const MergeJob* __restrict__ jobs, int njobs, float scale) {
  const int t = blockIdx.x;
  int lo = 0, hi = njobs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (jobs[mid].tile0 <= t) lo = mid;
    else hi = mid - 1;
  }
  const MergeJob jb = jobs[lo];
  const int tiles_n = (jb.N + 255) / 256;
  const int tt = t - jb.tile0;
  const int k0 = (tt / tiles_n) * (4 * kMergeRows) + kMergeRows * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = (tt % tiles_n) * 256, n = nb + 4 * (threadIdx.x & 63);
  const bool nok = n < jb.N;  // N is a multiple of 4
  // All rows' W loads are issued before any is used (rows past K re-read
  // row K-1 and are not stored), so each thread has kMergeRows loads in flight.
  floatx4 w[kMergeRows];
#pragma unroll
  for (int q = 0; q < kMergeRows; ++q) {
    const int k = min(k0 + q, jb.K - 1);
    const int64_t at = (int64_t)k * jb.N + (nok ? n : 0);
    if (jb.f16)
      w[q] = widen4(*reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(jb.W) + at));
    else
      w[q] = *reinterpret_cast<const floatx4*>(static_cast<const float*>(jb.W) + at);
  }
  // The tile's 256 rows of B ([N][R]) are read once, coalesced, and staged
  // transposed (bt[j][column]); a lane then takes its four columns of rank j
  // as one 128-bit LDS read (read straight from B, the lanes' four rows sit
  // 4·R floats apart: a cache line per lane per load).
  __shared__ float bt[R][256 + 4];
  for (int f = threadIdx.x; f < 64 * R; f += 256) {
    const int c = (4 * f) / R, j0 = (4 * f) % R;
    const floatx4 v = nb + c < jb.N ? *reinterpret_cast<const floatx4*>(jb.B + (int64_t)(nb + c) * R + j0)
                                    : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) bt[j0 + u][c] = v[u];
  }
  __syncthreads();
  if (!nok) return;
  float bv[4][R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const floatx4 b4 = *reinterpret_cast<const floatx4*>(&bt[j][4 * (threadIdx.x & 63)]);
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e][j] = b4[e];
  }
#pragma unroll
  for (int q = 0; q < kMergeRows; ++q) {
    const int k = k0 + q;
    if (k >= jb.K) break;
    float a[R];
#pragma unroll
    for (int j = 0; j < R; ++j) a[j] = jb.A[(int64_t)j * jb.K + k];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < R; ++j) d = fmaf(a[j], bv[e][j], d);
      w[q][e] = fmaf(scale, d, w[q][e]);
    }
    *reinterpret_cast<floatx4*>(jb.out + (int64_t)k * jb.ldo + n) = w[q];
  }
}

// Batched rank-r products: each 256-thread workgroup runs one job's share.
// Both roles are HBM-bound streams over X (every byte read once); they run on
// the vector units with full-width loads rather than on the matrix cores
// (r = 8 would fill half a 16-wide MFMA tile and the K split it needs left
// 1024-thread workgroups with a few KB of loads each).
//
// Projection role (out[M,r] = X·Y, Y(k,j) = Y[j·K+k] or Y[k·r+j]): a wave
// owns RW consecutive rows (RW·r = 32 or 64 values) and strides K with one
// 128-bit load per row per lane (a wave reads 1 KB of a row per step); Y's
// four k rows of the step are the same for every wave of the GPU and come
// from the caches.  The RW·r per-lane partial sums are combined across the
// wave by a halving butterfly (each xor-shuffle step hands half of the
// remaining values to the partner lane), after which value v sits in lanes
// with lane >> (6 − log2(RW·r)) == v.
//
// Outer role (out(j,c) (+)= s·Σ_m P[m,j]·X[m,c]): 128 columns per
// workgroup (two per lane, one 64-bit load per row: 2.4% faster than one
// column per lane on the Gemma-3 1B panel path, 4% on GPT-2; 256 columns
// leave too few workgroups for GPT-2's 768-wide products), the rows split
// over the four waves and read in chunks of 8 rows in flight; P's row is
// uniform across the wave.  Wave
// partials are added through LDS in wave order (deterministic), column runs
// per XCD.
// Job tables hold generic pointers; loads through them are marked global
// (vector memory instructions instead of flat ones), and a row that is the
// same for the whole wave is read through the scalar cache.
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ T lds_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

constexpr int kBatchThreads = 256;
constexpr int kBatchCols = 128;  // outer-product columns per workgroup

template <int R>
constexpr int batch_rows_per_wave() { return R <= 16 ? 4 : 2; }

// KS = 1: each wave owns RW rows and the whole of K.  KS = 4: the four
// waves share RW rows and take interleaved 256-wide slices of K (for batches
// with few jobs, where one wave per RW rows leaves the GPU mostly idle), and
// their sums are added in wave order through LDS.
template <int R, int KS>
__device__ __forceinline__ void batch_proj(const RankJob& jb, int b, int M, float* lds) {
  constexpr int RW = batch_rows_per_wave<R>();
  constexpr int V = RW * R;  // 16 .. 64 partial sums per lane
  static_assert(V >= 2 && V <= 64 && (V & (V - 1)) == 0, "butterfly size");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m0 = (KS == 1 ? b * 4 + w : b) * RW;
  if (m0 >= M) return;  // the same m0 for every wave when KS > 1: no wave waits at the barrier
  const int K = jb.K;
  const float* xr[RW];
#pragma unroll
  for (int q = 0; q < RW; ++q) xr[q] = jb.X + (int64_t)min(m0 + q, M - 1) * jb.ldx;
  float acc[RW][R];
  float mx[RW];  // max |x| of each row (row scales for the fp16 GEMM, when asked for)
#pragma unroll
  for (int q = 0; q < RW; ++q) {
    mx[q] = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) acc[q][j] = 0.f;
  }
  // K is a multiple of 4 (checked on the host), so a 4-vector never crosses a row.
  // The K-split form unrolls deeper: its few workgroups (one job of 4-row
  // groups) leave the loads of several steps to cover the memory latency.
  if (jb.y_rk) {  // Y [r, K]: a lane takes 4-wide chunks of K, one 128-bit Y load per rank
#pragma unroll(KS == 1 ? 2 : 4)
    for (int k = 4 * lane + (KS == 1 ? 0 : 256 * w); k < K; k += 256 * KS) {
      floatx4 xv[RW];
#pragma unroll
      for (int q = 0; q < RW; ++q) {
        xv[q] = ldg(reinterpret_cast<const floatx4*>(xr[q] + k));
        mx[q] = fmaxf(mx[q], fmaxf(fmaxf(fabsf(xv[q][0]), fabsf(xv[q][1])), fmaxf(fabsf(xv[q][2]), fabsf(xv[q][3]))));
      }
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const floatx4 y = ldg(reinterpret_cast<const floatx4*>(jb.Y + (int64_t)j * K + k));
#pragma unroll
        for (int q = 0; q < RW; ++q)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[q][j] = fmaf(xv[q][t], y[t], acc[q][j]);
      }
    }
  } else {
    // Y [K, r]: a lane takes single columns k, E at a time, so that a wave's
    // Y reads (r consecutive floats per column) are contiguous across lanes;
    // with 4-wide chunks the lanes' Y reads would sit 4·r floats apart, a
    // cache line per lane per load
    constexpr int E = 4, KSTEP = 64 * KS;
    for (int k0 = lane + (KS == 1 ? 0 : 64 * w); k0 < K; k0 += KSTEP * E) {
      float xs[E][RW];
      floatx4 ys[E][R / 4];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int k = k0 + KSTEP * e;
        if (k < K) {
#pragma unroll
          for (int q = 0; q < RW; ++q) xs[e][q] = ldg(xr[q] + k);
#pragma unroll
          for (int jq = 0; jq < R / 4; ++jq) ys[e][jq] = ldg(reinterpret_cast<const floatx4*>(jb.Y + (int64_t)k * R) + jq);
        } else {
#pragma unroll
          for (int q = 0; q < RW; ++q) xs[e][q] = 0.f;
#pragma unroll
          for (int jq = 0; jq < R / 4; ++jq) ys[e][jq] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e)
#pragma unroll
        for (int q = 0; q < RW; ++q) {
          mx[q] = fmaxf(mx[q], fabsf(xs[e][q]));
#pragma unroll
          for (int jq = 0; jq < R / 4; ++jq)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[q][4 * jq + u] = fmaf(xs[e][q], ys[e][jq][u], acc[q][4 * jq + u]);
        }
    }
  }
  float v[V];
#pragma unroll
  for (int q = 0; q < RW; ++q)
#pragma unroll
    for (int j = 0; j < R; ++j) v[q * R + j] = acc[q][j];
  int n = V;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    if (n > 1) {
      const bool upper = (lane & d) != 0;
#pragma unroll
      for (int i = 0; i < V / 2; ++i) {
        if (i < n / 2) {
          const float send = upper ? v[i] : v[i + n / 2];
          const float keep = upper ? v[i + n / 2] : v[i];
          v[i] = keep + __shfl_xor(send, d, 64);
        }
      }
      n /= 2;
    } else {
      v[0] += __shfl_xor(v[0], d, 64);
    }
  }
  constexpr int SH = V == 64 ? 0 : V == 32 ? 1 : V == 16 ? 2 : V == 8 ? 3 : V == 4 ? 4 : 5;
  const int vi = lane >> SH;
  if (jb.inv_s) {  // uniform per job
#pragma unroll
    for (int q = 0; q < RW; ++q)
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], d, 64));
  }
  if constexpr (KS == 1) {
    if ((lane & ((1 << SH) - 1)) == 0) {
      const int q = vi / R, j = vi % R, m = m0 + q;
      if (m < M) jb.out[(int64_t)m * R + j] = v[0];
    }
    if (jb.inv_s && lane < RW && m0 + lane < M) {
      float t = mx[0];
#pragma unroll
      for (int q = 1; q < RW; ++q) t = lane == q ? mx[q] : t;
      jb.inv_s[m0 + lane] = row_inv_scale(t);
    }
  } else {
    if ((lane & ((1 << SH) - 1)) == 0) lds[w * V + vi] = v[0];
    if (jb.inv_s && lane == 0) {
#pragma unroll
      for (int q = 0; q < RW; ++q) lds[KS * V + w * RW + q] = mx[q];
    }
    __syncthreads();
    if (w == 0 && lane < V) {
      float t = lds[lane];
#pragma unroll
      for (int u = 1; u < KS; ++u) t += lds[u * V + lane];
      const int q = lane / R, j = lane % R, m = m0 + q;
      if (m < M) jb.out[(int64_t)m * R + j] = t;
    }
    if (jb.inv_s && w == 0 && lane < RW && m0 + lane < M) {
      float t = lds[KS * V + lane];
#pragma unroll
      for (int u = 1; u < KS; ++u) t = fmaxf(t, lds[KS * V + u * RW + lane]);
      jb.inv_s[m0 + lane] = row_inv_scale(t);
    }
  }
}

template <int R>
__device__ __forceinline__ void batch_outer(const RankJob& jb, int raw, int M, float* lds) {
  constexpr int CPL = kBatchCols / 64;  // columns per lane
  typedef float colv __attribute__((ext_vector_type(CPL)));
  const int blk = (raw % 8) * (jb.blocks / 8) + raw / 8;
  const int c0 = blk * kBatchCols;
  if (c0 >= jb.K) return;  // whole workgroup, before any barrier
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = c0 + CPL * lane;
  const bool cok = c < jb.K;  // C is a multiple of 4 (checked on the host)
  const int per = (M + 3) / 4;
  const int mb = w * per, me = min(M, mb + per);
  float acc[R][CPL];
#pragma unroll
  for (int j = 0; j < R; ++j)
#pragma unroll
    for (int e = 0; e < CPL; ++e) acc[j][e] = 0.f;
  const float* xp = jb.X + (cok ? c : 0);
  // rows in chunks of CH, every row load of a chunk issued before its first
  // use (a wave's rows are one chain of chunk latencies); P's row is the
  // same for the whole wave and comes through the scalar cache
  auto rows = [&](int m, auto nc) {
    constexpr int NCH = decltype(nc)::value;
    colv xs[NCH];
#pragma unroll
    for (int u = 0; u < NCH; ++u) xs[u] = ldg(reinterpret_cast<const colv*>(xp + (int64_t)(m + u) * jb.ldx));
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const floatx4* pp = reinterpret_cast<const floatx4*>(jb.Y + (int64_t)(m + u) * R);
#pragma unroll
      for (int jq = 0; jq < R / 4; ++jq) {
        const floatx4 pv = lds_uniform(pp + jq);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int t = 0; t < CPL; ++t) acc[4 * jq + e][t] = fmaf(pv[e], xs[u][t], acc[4 * jq + e][t]);
      }
    }
  };
  constexpr int CH = 16 / CPL;
  int m = mb;
  for (; m + CH <= me; m += CH) rows(m, std::integral_constant<int, CH>{});
  for (; m < me; ++m) rows(m, std::integral_constant<int, 1>{});
  // wave-ordered sum through LDS: lds[j][kBatchCols columns]
  for (int q = 0; q < 4; ++q) {
    if (w == q) {
#pragma unroll
      for (int j = 0; j < R; ++j)
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          float& d = lds[j * kBatchCols + CPL * lane + e];
          d = q == 0 ? acc[j][e] : d + acc[j][e];
        }
    }
    __syncthreads();
  }
  if (w != 0 || !cok) return;
#pragma unroll
  for (int j = 0; j < R; ++j)
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      float* out = jb.out + (int64_t)j * jb.osj + (int64_t)(c + e) * jb.osc;
      const float v = lds[j * kBatchCols + CPL * lane + e];
      *out = jb.accumulate ? fmaf(jb.scale, v, *out) : jb.scale * v;
    }
}

template <int R, int KS>
__global__ __launch_bounds__(kBatchThreads) void rank_batch_kernel(const RankJob* __restrict__ jobs, int njobs,
                                                                   int nproj, int M) {
  __shared__ float lds[R * kBatchCols];
  constexpr int ROWS = (KS == 1 ? 4 : 1) * batch_rows_per_wave<R>();  // rows per workgroup
  const int pb = (M + ROWS - 1) / ROWS;
  int b = blockIdx.x;
  if (b < nproj * pb) {
    const int ji = b / pb;
    batch_proj<R, KS>(jobs[ji], b - ji * pb, M, lds);
    return;
  }
  b -= nproj * pb;
  int lo = nproj, hi = njobs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (jobs[mid].block0 <= b) lo = mid;
    else hi = mid - 1;
  }
  batch_outer<R>(jobs[lo], b - jobs[lo].block0, M, lds);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int R>
void proj_vec(hipStream_t s, const float* X, int64_t ldx, const float* Y, bool y_rk, int M, int K,
              float* out) {
  const dim3 grid((unsigned)M), block(256);
  if (y_rk) hipLaunchKernelGGL((rank_proj_vec_kernel<R, true>), grid, block, 0, s, X, ldx, Y, M, K, out);
  else      hipLaunchKernelGGL((rank_proj_vec_kernel<R, false>), grid, block, 0, s, X, ldx, Y, M, K, out);
}

void outer_launch(hipStream_t s, OuterArgs& a) {
  // column blocks of 16, padded to a multiple of 8 (one run per XCD)
  a.job[0].blocks = (int)cdiv(cdiv(a.job[0].C, 16), 8) * 8;
  a.job[1].blocks = a.job[1].out ? (int)cdiv(cdiv(a.job[1].C, 16), 8) * 8 : 0;
  const dim3 grid((unsigned)(a.job[0].blocks + a.job[1].blocks)), block(64 * kOuterWaves);
  if (a.r <= 16) hipLaunchKernelGGL(rank_outer_mfma<1>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(rank_outer_mfma<2>, grid, block, 0, s, a);
  MFT_LAUNCH_CHECK();
}

}  // namespace

size_t merge_tiles(int K, int N) { return (size_t)cdiv(K, 4 * kMergeRows) * (size_t)cdiv(N, 256); }

void lora_merge(hipStream_t s, const MergeJob* jobs, int njobs, int total_tiles, int r, float scale) {
  MFT_CHECK_ARG(jobs && njobs > 0 && total_tiles > 0, "empty merge");
  const dim3 grid((unsigned)total_tiles), block(256);
  switch (r) {
    case 4: hipLaunchKernelGGL(lora_merge_kernel<4>, grid, block, 0, s, jobs, njobs, scale); break;
    case 8: hipLaunchKernelGGL(lora_merge_kernel<8>, grid, block, 0, s, jobs, njobs, scale); break;
    case 16: hipLaunchKernelGGL(lora_merge_kernel<16>, grid, block, 0, s, jobs, njobs, scale); break;
    case 32: hipLaunchKernelGGL(lora_merge_kernel<32>, grid, block, 0, s, jobs, njobs, scale); break;
    default: MFT_CHECK_ARG(false, "merged LoRA takes r in {4, 8, 16, 32}");
  }
  MFT_LAUNCH_CHECK();
}

int rank_outer_blocks(int C) { return (int)cdiv(cdiv(C, kBatchCols), 8) * 8; }

template <int KS>
void rank_batch_launch(hipStream_t s, const RankJob* jobs, int njobs, int nproj, int outer_blocks, int M, int r) {
  const int rows_per_wg = (KS == 1 ? 4 : 1) * (r <= 16 ? 4 : 2);
  const int64_t blocks = (int64_t)nproj * cdiv(M, rows_per_wg) + outer_blocks;
  const dim3 grid((unsigned)blocks), block(kBatchThreads);
  switch (r) {
    case 4: hipLaunchKernelGGL((rank_batch_kernel<4, KS>), grid, block, 0, s, jobs, njobs, nproj, M); break;
    case 8: hipLaunchKernelGGL((rank_batch_kernel<8, KS>), grid, block, 0, s, jobs, njobs, nproj, M); break;
    case 16: hipLaunchKernelGGL((rank_batch_kernel<16, KS>), grid, block, 0, s, jobs, njobs, nproj, M); break;
    case 32: hipLaunchKernelGGL((rank_batch_kernel<32, KS>), grid, block, 0, s, jobs, njobs, nproj, M); break;
    default: MFT_CHECK_ARG(false, "batched rank-r work takes r in {4, 8, 16, 32}");
  }
  MFT_LAUNCH_CHECK();
}

void rank_proj_jobs(hipStream_t s, const ProjJobs& jb, int M, int r) {
  MFT_CHECK_ARG(jb.n >= 1 && jb.n <= kMaxProjJobs && M > 0 && (r == 4 || r == 8 || r == 16 || r == 32),
                "projection jobs: 1-3 jobs, r in {4, 8, 16, 32}");
  bool y_rk = jb.j[0].y_rk != 0;
  for (int g = 0; g < jb.n; ++g) {
    const ProjJob& j = jb.j[g];
    MFT_CHECK_ARG(j.X && j.Y && j.out && j.K > 0 && j.K % 4 == 0 && j.ldx % 4 == 0 && aligned16(j.X) &&
                      aligned16(j.Y) && (j.y_rk != 0) == y_rk,
                  "projection job: shape, alignment or Y layout");
  }
  int kmax = 0;
  for (int g = 0; g < jb.n; ++g) kmax = std::max(kmax, jb.j[g].K);
  ProjJobs b = jb;
  for (int g = jb.n; g < kMaxProjJobs; ++g) b.j[g] = b.j[jb.n - 1];  // never selected
  // two rows per workgroup share the Y reads of deep [K][r] Y (a row per
  // workgroup otherwise: 2.4 TB/s at K = 6912 with one job, 30% slower at two
  // rows; [K][r] at K = 6912, two jobs: 22.5 -> 19.2 us)
  const bool two = !y_rk && kmax > 2048 && r <= 8;
  const dim3 grid((unsigned)(jb.n * (two ? cdiv(M, 2) : M))), block(256);
#define MFT_PJ(R, RB)                                                                       \
  if (y_rk) hipLaunchKernelGGL((rank_proj_jobs_kernel<R, RB, true>), grid, block, 0, s, b, M); \
  else hipLaunchKernelGGL((rank_proj_jobs_kernel<R, RB, false>), grid, block, 0, s, b, M)
  switch (r) {
    case 4: if (two) { MFT_PJ(4, 2); } else { MFT_PJ(4, 1); } break;
    case 8: if (two) { MFT_PJ(8, 2); } else { MFT_PJ(8, 1); } break;
    case 16: { MFT_PJ(16, 1); } break;
    default: { MFT_PJ(32, 1); } break;
  }
#undef MFT_PJ
  MFT_LAUNCH_CHECK();
}

void rank_batch(hipStream_t s, const RankJob* jobs, int njobs, int nproj, int outer_blocks, int M, int r) {
  MFT_CHECK_ARG(jobs && njobs > 0 && M > 0, "empty rank batch");
  // Projection-only batches of under 256 workgroups (the per-layer groups
  // of the rank-r panel path) split K over the four waves of a workgroup.
  const int rows_per_wg = 4 * (r <= 16 ? 4 : 2);
  if (outer_blocks == 0 && (int64_t)nproj * cdiv(M, rows_per_wg) < 256)
    rank_batch_launch<4>(s, jobs, njobs, nproj, outer_blocks, M, r);
  else
    rank_batch_launch<1>(s, jobs, njobs, nproj, outer_blocks, M, r);
}

void rank_proj(hipStream_t s, const float* X, int64_t ldx, const float* Y, int64_t ysk,
               int64_t ysj, int M, int K, int r, float* out) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  MFT_CHECK_ARG(M > 0 && K > 0, "empty");
  const bool y_rk = ysk == 1 && ysj == K;
  const bool y_kr = ysj == 1 && ysk == r;
  const bool vec = (r == 4 || r == 8 || r == 16 || r == 32) && (y_rk || y_kr) && K % 4 == 0 && ldx % 4 == 0 &&
                   aligned16(X) && aligned16(Y);
  if (vec) {
    if (r == 4) proj_vec<4>(s, X, ldx, Y, y_rk, M, K, out);
    else if (r == 8) proj_vec<8>(s, X, ldx, Y, y_rk, M, K, out);
    else if (r == 16) proj_vec<16>(s, X, ldx, Y, y_rk, M, K, out);
    else proj_vec<32>(s, X, ldx, Y, y_rk, M, K, out);
  } else {
    dim3 grid((unsigned)cdiv(M, 4)), block(256);
    if (r <= 8)       hipLaunchKernelGGL(rank_proj_scalar_kernel<8>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
    else if (r <= 16) hipLaunchKernelGGL(rank_proj_scalar_kernel<16>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
    else              hipLaunchKernelGGL(rank_proj_scalar_kernel<32>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
  }
  MFT_LAUNCH_CHECK();
}

namespace {
OuterJob make_job(const float* P, const float* X, int64_t ldx, int C, float* out, int64_t osj,
                  int64_t osc) {
  MFT_CHECK_ARG(P && X && out && C > 0, "rank_outer: null tensor or empty");
  OuterJob j{};
  j.P = P; j.X = X; j.ldx = ldx; j.C = C; j.out = out; j.osj = osj; j.osc = osc;
  return j;
}

}  // namespace

void rank_outer(hipStream_t s, const float* P, const float* X, int64_t ldx, int M, int C, int r,
                float scale, float* out, int64_t osj, int64_t osc, bool accumulate, Scratch) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  MFT_CHECK_ARG(M > 0, "empty");
  OuterArgs a{};
  a.job[0] = make_job(P, X, ldx, C, out, osj, osc);
  a.M = M; a.r = r; a.accumulate = accumulate ? 1 : 0; a.scale = scale;
  outer_launch(s, a);
}

void rank_outer_pair(hipStream_t s, int M, int r, float scale, bool accumulate,
                     const float* P0, const float* X0, int64_t ldx0, int C0, float* out0, int64_t osj0,
                     int64_t osc0, const float* P1, const float* X1, int64_t ldx1, int C1, float* out1,
                     int64_t osj1, int64_t osc1) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  MFT_CHECK_ARG(M > 0, "empty");
  OuterArgs a{};
  a.job[0] = make_job(P0, X0, ldx0, C0, out0, osj0, osc0);
  a.job[1] = make_job(P1, X1, ldx1, C1, out1, osj1, osc1);
  a.M = M; a.r = r; a.accumulate = accumulate ? 1 : 0; a.scale = scale;
  outer_launch(s, a);
}

}  // namespace mft
