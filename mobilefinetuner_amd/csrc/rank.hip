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

// out[m, j] = Σ_k X[m,k]·Y(k,j) for RB rows per 256-thread workgroup; every
// thread takes 128-bit chunks of K for all RB rows (so X is streamed once),
// the RB·R partial sums are reduced within each wave by recursive halving
// and across the four waves in LDS.
// Y_RK: Y stored [R][K] (xa = x·Aᵀ with A [r,K]); otherwise [K][R]
// (U = dy·B with B [N,r]).
template <int R, int RB, bool Y_RK>
__global__ __launch_bounds__(256) void rank_proj_vec_kernel(const float* __restrict__ X, int64_t ldx,
                                                             const float* __restrict__ Y, int M, int K,
                                                             float* __restrict__ out) {
  constexpr int NV = RB * R;
  __shared__ float red[4][NV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.x * RB;
  float acc[NV];
#pragma unroll
  for (int q = 0; q < NV; ++q) acc[q] = 0.f;
  for (int k = tid * 4; k < K; k += 1024) {
    floatx4 xv[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int m = min(m0 + i, M - 1);
      xv[i] = *reinterpret_cast<const floatx4*>(X + (int64_t)m * ldx + k);
    }
    if constexpr (Y_RK) {
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const floatx4 y = *reinterpret_cast<const floatx4*>(Y + (int64_t)j * K + k);
#pragma unroll
        for (int i = 0; i < RB; ++i)
          acc[i * R + j] += xv[i][0] * y[0] + xv[i][1] * y[1] + xv[i][2] * y[2] + xv[i][3] * y[3];
      }
    } else {
      const float* yk = Y + (int64_t)k * R;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jq = 0; jq < R / 4; ++jq) {
          const floatx4 y = *reinterpret_cast<const floatx4*>(yk + e * R + 4 * jq);
#pragma unroll
          for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[i * R + 4 * jq + u] = fmaf(xv[i][e], y[u], acc[i * R + 4 * jq + u]);
        }
    }
  }
  const float t = wave_reduce_spread<NV>(acc, lane);
  constexpr int SPREAD = 64 / NV;
  if ((lane % SPREAD) == 0) red[wave][lane / SPREAD] = t;
  __syncthreads();
  if (tid < NV) {
    const int i = tid / R, j = tid % R;
    const float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    if (m0 + i < M) out[(int64_t)(m0 + i) * R + j] = v;
  }
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
// D[c0+4g+v][16·jt+i].  A workgroup owns 16 columns c of one product; its 8
// waves take consecutive eighths of M (loads of 8 MFMA steps issued ahead of
// the MFMAs) and are summed through LDS in wave order.  Two independent
// products (dA and dB of one LoRA layer) share one launch.
struct OuterJob {
  const float* P;
  const float* X;
  int64_t ldx;
  int C, blocks;
  float* out;
  int64_t osj, osc;
};
struct OuterArgs {
  OuterJob job[2];
  int M, r, accumulate;
  float scale;
};

template <int JT>
__global__ __launch_bounds__(512) void rank_outer_mfma(OuterArgs a) {
  __shared__ floatx4 red[7][JT][64];
  const bool second = (int)blockIdx.x >= a.job[0].blocks;
  const OuterJob jb = second ? a.job[1] : a.job[0];
  const int blk = second ? (int)blockIdx.x - a.job[0].blocks : (int)blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int c0 = blk * 16;
  const int ci = min(c0 + i, jb.C - 1);
  const bool cok = c0 + i < jb.C;
  const int per = ((a.M + 8 * 32 - 1) / (8 * 32)) * 32;  // rows per wave, multiple of 32
  const int mb = w * per, me = min(a.M, mb + per);
  floatx4 acc[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) acc[jt] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int m = mb; m < me; m += 32) {
    float xv[8], pv[JT][8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int mr = m + 4 * t + g;
      const bool ok = mr < me;
      const int mc = ok ? mr : mb;
      const float x = jb.X[(int64_t)mc * jb.ldx + ci];
      xv[t] = (ok && cok) ? x : 0.f;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const int jj = 16 * jt + i;
        const float pp = jb.P[(int64_t)mc * a.r + min(jj, a.r - 1)];
        pv[jt][t] = (ok && jj < a.r) ? pp : 0.f;
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
        acc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t], pv[jt][t], acc[jt], 0, 0, 0);
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
    for (int q = 0; q < 7; ++q) v += red[q][jt][lane];
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

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int R, int RB>
void proj_vec(hipStream_t s, const float* X, int64_t ldx, const float* Y, bool y_rk, int M, int K,
              float* out) {
  const dim3 grid((unsigned)cdiv(M, RB)), block(256);
  if (y_rk) hipLaunchKernelGGL((rank_proj_vec_kernel<R, RB, true>), grid, block, 0, s, X, ldx, Y, M, K, out);
  else      hipLaunchKernelGGL((rank_proj_vec_kernel<R, RB, false>), grid, block, 0, s, X, ldx, Y, M, K, out);
}

void outer_launch(hipStream_t s, OuterArgs& a) {
  a.job[0].blocks = (int)cdiv(a.job[0].C, 16);
  a.job[1].blocks = a.job[1].out ? (int)cdiv(a.job[1].C, 16) : 0;
  const dim3 grid((unsigned)(a.job[0].blocks + a.job[1].blocks)), block(512);
  if (a.r <= 16) hipLaunchKernelGGL(rank_outer_mfma<1>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(rank_outer_mfma<2>, grid, block, 0, s, a);
  MFT_LAUNCH_CHECK();
}

}  // namespace

void rank_proj(hipStream_t s, const float* X, int64_t ldx, const float* Y, int64_t ysk,
               int64_t ysj, int M, int K, int r, float* out) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  MFT_CHECK_ARG(M > 0 && K > 0, "empty");
  const bool y_rk = ysk == 1 && ysj == K;
  const bool y_kr = ysj == 1 && ysk == r;
  const bool vec = (r == 4 || r == 8 || r == 16 || r == 32) && (y_rk || y_kr) && K % 4 == 0 && ldx % 4 == 0 &&
                   aligned16(X) && aligned16(Y);
  if (vec) {
    // one row per workgroup (measured fastest at M = 512–1024 for r = 8)
    if (r == 4) proj_vec<4, 1>(s, X, ldx, Y, y_rk, M, K, out);
    else if (r == 8) proj_vec<8, 1>(s, X, ldx, Y, y_rk, M, K, out);
    else if (r == 16) proj_vec<16, 1>(s, X, ldx, Y, y_rk, M, K, out);
    else proj_vec<32, 1>(s, X, ldx, Y, y_rk, M, K, out);
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
