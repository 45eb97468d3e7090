// rank.hip — the skinny rank-r products of the LoRA branch.
//
//   rank_proj:  out[M,r] = X[M,K] · Y          (xa = x·Aᵀ, U = dy·B)
//   rank_outer: out(j,c) (+)= s · Σ_m P[m,j] X[m,c]   (dA = s·Uᵀx, dB = s·dyᵀxa)
//
// Both are HBM/latency-bound passes over X (2–16 MB at the benchmark
// shapes).  rank_proj gives each wave two rows and has every lane stream
// 128-bit chunks of K, so a wave keeps ~20 independent 16-byte loads in
// flight; the r×K (or K×r) factor is re-read from L1/L2.  rank_outer splits M
// into slices (≥ ~256 workgroups), keeps r partial sums per column in
// registers, reduces the four waves of a workgroup in LDS and finishes the
// slices in a fixed order (deterministic, no atomics).
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace mft {
namespace {

constexpr int RW = 2;  // rows per wave in rank_proj

// Y_RK: Y stored [R][K] (row j contiguous in k)  — xa = x·Aᵀ with A [r,K]
// Y_KR: Y stored [K][R] (row k contiguous in j)  — U = dy·B with B [N,r]
template <int R, bool Y_RK>
__global__ __launch_bounds__(256) void rank_proj_vec_kernel(const float* __restrict__ X,
                                                             int64_t ldx,
                                                             const float* __restrict__ Y,
                                                             int M, int K,
                                                             float* __restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = (blockIdx.x * 4 + wave) * RW;
  if (m0 >= M) return;
  float acc[RW][R];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < R; ++j) acc[i][j] = 0.f;
  const bool two = m0 + 1 < M;
#pragma unroll 2
  for (int k = lane * 4; k < K; k += 256) {
    floatx4 xv[RW];
    xv[0] = *reinterpret_cast<const floatx4*>(X + (int64_t)m0 * ldx + k);
    xv[1] = two ? *reinterpret_cast<const floatx4*>(X + (int64_t)(m0 + 1) * ldx + k)
                : floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (Y_RK) {
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const floatx4 y = *reinterpret_cast<const floatx4*>(Y + (int64_t)j * K + k);
#pragma unroll
        for (int i = 0; i < RW; ++i)
          acc[i][j] += xv[i][0] * y[0] + xv[i][1] * y[1] + xv[i][2] * y[2] + xv[i][3] * y[3];
      }
    } else {
      const float* yk = Y + (int64_t)k * R;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jq = 0; jq < R / 4; ++jq) {
          const floatx4 y = *reinterpret_cast<const floatx4*>(yk + e * R + 4 * jq);
#pragma unroll
          for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[i][4 * jq + u] = fmaf(xv[i][e], y[u], acc[i][4 * jq + u]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < R; ++j) {
      float v = acc[i][j];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[i][j] = v;
    }
  if (lane < R) {
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      if (m0 + i >= M) break;
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < R; ++j)
        if (j == lane) v = acc[i][j];
      out[(int64_t)(m0 + i) * R + lane] = v;
    }
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

// Partial Σ_m P[m,j] X[m,c] over one row slice: 64 columns per workgroup
// (one per lane), the 4 waves interleave rows.  part[slice][j][c].
template <int R>
__global__ __launch_bounds__(256) void rank_outer_kernel(const float* __restrict__ P,
                                                          const float* __restrict__ X,
                                                          int64_t ldx, int M, int C,
                                                          int rows_per_slice, float scale,
                                                          float* part, float* out, int64_t osj,
                                                          int64_t osc, int direct,
                                                          int accumulate) {
  __shared__ float red[3][R][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int slice = blockIdx.y;
  const int mb = slice * rows_per_slice, me = min(M, mb + rows_per_slice);
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.f;
  if (c < C) {
#pragma unroll 4
    for (int m = mb + w; m < me; m += 4) {
      const float xv = X[(int64_t)m * ldx + c];
      const floatx4* pr = reinterpret_cast<const floatx4*>(P + (int64_t)m * R);
#pragma unroll
      for (int jq = 0; jq < R / 4; ++jq) {
        const floatx4 p4 = pr[jq];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[4 * jq + u] = fmaf(p4[u], xv, acc[4 * jq + u]);
      }
    }
  }
  if (w > 0) {
#pragma unroll
    for (int j = 0; j < R; ++j) red[w - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (w == 0 && c < C) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const float v = ((acc[j] + red[0][j][lane]) + red[1][j][lane]) + red[2][j][lane];
      if (direct) {
        float* o = out + (int64_t)j * osj + (int64_t)c * osc;
        *o = accumulate ? fmaf(scale, v, *o) : scale * v;
      } else {
        part[((int64_t)slice * R + j) * C + c] = v;
      }
    }
  }
}

__global__ void rank_outer_finish(const float* __restrict__ part, int slices, int C, int r,
                                  float scale, float* out, int64_t osj, int64_t osc,
                                  int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)C * r) return;
  const int j = (int)(idx / C), c = (int)(idx % C);
  float s = 0.f;
  for (int z = 0; z < slices; ++z) s += part[((int64_t)z * r + j) * C + c];
  float* o = out + (int64_t)j * osj + (int64_t)c * osc;
  *o = accumulate ? fmaf(scale, s, *o) : scale * s;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int R>
void proj_vec(hipStream_t s, const float* X, int64_t ldx, const float* Y, bool y_rk, int M, int K,
              float* out) {
  dim3 grid((unsigned)cdiv(M, 4 * RW)), block(256);
  if (y_rk) hipLaunchKernelGGL((rank_proj_vec_kernel<R, true>), grid, block, 0, s, X, ldx, Y, M, K, out);
  else      hipLaunchKernelGGL((rank_proj_vec_kernel<R, false>), grid, block, 0, s, X, ldx, Y, M, K, out);
}

template <int R>
void outer_launch(hipStream_t s, const float* P, const float* X, int64_t ldx, int M, int C,
                  float scale, float* out, int64_t osj, int64_t osc, bool accumulate, Scratch ws) {
  const int64_t cblocks = cdiv(C, 64);
  int64_t slices = std::max<int64_t>(1, std::min<int64_t>(cdiv(256, cblocks), cdiv(M, 16)));
  while (slices > 1 && (size_t)slices * R * C * sizeof(float) > ws.bytes) slices /= 2;
  if (!ws.ptr) slices = 1;
  const int rows = (int)cdiv(M, slices);
  slices = cdiv(M, rows);
  const int direct = slices == 1;
  dim3 grid((unsigned)cblocks, (unsigned)slices), block(256);
  hipLaunchKernelGGL((rank_outer_kernel<R>), grid, block, 0, s, P, X, ldx, M, C, rows, scale, ws.ptr,
                     out, osj, osc, direct, accumulate ? 1 : 0);
  MFT_LAUNCH_CHECK();
  if (!direct) {
    hipLaunchKernelGGL(rank_outer_finish, dim3((unsigned)cdiv((int64_t)C * R, 256)), dim3(256), 0, s,
                       (const float*)ws.ptr, (int)slices, C, R, scale, out, osj, osc,
                       accumulate ? 1 : 0);
    MFT_LAUNCH_CHECK();
  }
}

}  // namespace

void rank_proj(hipStream_t s, const float* X, int64_t ldx, const float* Y, int64_t ysk,
               int64_t ysj, int M, int K, int r, float* out) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  MFT_CHECK_ARG(M > 0 && K > 0, "empty");
  const bool y_rk = ysk == 1 && ysj == K;
  const bool y_kr = ysj == 1 && ysk == r;
  const bool vec = (r == 4 || r == 8 || r == 16) && (y_rk || y_kr) && K % 4 == 0 && ldx % 4 == 0 &&
                   aligned16(X) && aligned16(Y);
  if (vec) {
    if (r == 4) proj_vec<4>(s, X, ldx, Y, y_rk, M, K, out);
    else if (r == 8) proj_vec<8>(s, X, ldx, Y, y_rk, M, K, out);
    else proj_vec<16>(s, X, ldx, Y, y_rk, M, K, out);
  } else {
    dim3 grid((unsigned)cdiv(M, 4)), block(256);
    if (r <= 8)       hipLaunchKernelGGL(rank_proj_scalar_kernel<8>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
    else if (r <= 16) hipLaunchKernelGGL(rank_proj_scalar_kernel<16>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
    else              hipLaunchKernelGGL(rank_proj_scalar_kernel<32>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
  }
  MFT_LAUNCH_CHECK();
}

void rank_outer(hipStream_t s, const float* P, const float* X, int64_t ldx, int M, int C, int r,
                float scale, float* out, int64_t osj, int64_t osc, bool accumulate, Scratch ws) {
  MFT_CHECK_ARG(r == 4 || r == 8 || r == 16 || r == 32, "rank must be 4, 8, 16 or 32");
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  MFT_CHECK_ARG(aligned16(P), "P must be 16-byte aligned");
  if (r == 4) outer_launch<4>(s, P, X, ldx, M, C, scale, out, osj, osc, accumulate, ws);
  else if (r == 8) outer_launch<8>(s, P, X, ldx, M, C, scale, out, osj, osc, accumulate, ws);
  else if (r == 16) outer_launch<16>(s, P, X, ldx, M, C, scale, out, osj, osc, accumulate, ws);
  else outer_launch<32>(s, P, X, ldx, M, C, scale, out, osj, osc, accumulate, ws);
}

}  // namespace mft
