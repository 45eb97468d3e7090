// gemm.hip — LoRA-linear GEMMs for gfx950 (CDNA4).
//
// C[M,N] = A[M,K]·op(B) on the fp32 matrix cores (v_mfma_f32_32x32x2_f32),
// 256-thread workgroups = 4 wave64s in a 2×2 grid, LDS double-buffered K
// panels (BK = 16), epilogue fusing bias, the rank-r LoRA term
// scale·P[M,r]·Q, a residual add, and accumulation into C.  B may be [K,N]
// (frozen W in the forward, tied embedding in the LM-head backward) or [N,K]
// (W in dX = dY·Wᵀ, embedding in the LM-head forward), fp32 or fp16; fp16 is
// widened to fp32 while the tile is staged into LDS, so the frozen weight is
// read from HBM at 2 bytes/element and never materialised as fp32.
//
// LDS holds both panels k-contiguous (As[m][k], Bs[n][k], row pitch BK+4
// floats) so every MFMA operand fetch is a ds_read_b128 without bank
// conflicts: within one BK=16 panel, lane (i, h) of a 32×32 tile consumes
// k = 8h .. 8h+7 over eight MFMAs (the k order inside a panel is permuted the
// same way for A and B, which leaves the sum unchanged).
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace mft {
namespace {

constexpr int BK = 16;
constexpr int PITCH = BK + 4;  // floats per LDS row

struct GemmParams {
  const float* A;
  const void* B;
  float* C;
  int64_t lda, ldb, ldc;
  int M, N, K;
  int k_chunk;       // K range per split (multiple of BK)
  int tiles_m, tiles_n, tiles_per_xcd;
  float* partial;    // split-K: [splits][M][N] raw accumulators
  GemmEpilogue ep;
};

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float epilogue_value(const GemmEpilogue& ep,
                                                float acc, int m, int n,
                                                const float* C, int64_t ldc) {
  float v = acc;
  if (ep.bias) v += ep.bias[n];
  if (ep.P) {
    float s = 0.f;
    const float* pr = ep.P + (int64_t)m * ep.r;
    const float* qn = ep.Q + (int64_t)n * ep.qsn;
    for (int j = 0; j < ep.r; ++j) s = fmaf(pr[j], qn[j * ep.qsj], s);
    v = fmaf(ep.lscale, s, v);
  }
  if (ep.resid) v += ep.resid[(int64_t)m * ldc + n];
  if (ep.beta != 0.f) v = fmaf(ep.beta, C[(int64_t)m * ldc + n], v);
  return v;
}

template <int BM, int BN, bool B_NK, bool B_F16>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;    // 32×32 MFMA tiles per wave
  constexpr int A_ITEMS = BM / 64;             // float4 per thread per panel
  constexpr int B_ITEMS = BN / 64;
  __shared__ __attribute__((aligned(16))) float As[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * PITCH];

  // XCD-aware tile order: consecutive workgroup ids land on different XCDs
  // (round-robin dispatch), so tile = xcd-major chunk + local index keeps the
  // workgroups that share a B column panel on one XCD's L2.
  const int wg = blockIdx.x;
  const int tile = (wg % 8) * p.tiles_per_xcd + wg / 8;
  if (tile >= p.tiles_m * p.tiles_n) return;
  const int tm_idx = tile % p.tiles_m;
  const int tn_idx = tile / p.tiles_m;
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int split = blockIdx.y;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wave_m = wave & 1, wave_n = wave >> 1;
  const int li = lane & 31, lh = lane >> 5;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  floatx4 ra[A_ITEMS], rb[B_ITEMS];

  auto load_panel = [&](int k0) {
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat >> 2, kq = (flat & 3) * 4;
      const int gm = m0 + row, gk = k0 + kq;
      ra[it] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (gm < p.M) {
        const float* src = p.A + (int64_t)gm * p.lda + gk;
        if (gk + 4 <= kend) {
          ra[it] = *reinterpret_cast<const floatx4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (gk + e < kend) ra[it][e] = src[e];
        }
      }
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      if constexpr (B_NK) {
        const int row = flat >> 2, kq = (flat & 3) * 4;
        const int gn = n0 + row, gk = k0 + kq;
        rb[it] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (gn < p.N) {
          if constexpr (B_F16) {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)gn * p.ldb + gk;
            if (gk + 4 <= kend) {
              const uint2 u = *reinterpret_cast<const uint2*>(src);
              rb[it] = floatx4{half_bits_to_float(u.x & 0xffff), half_bits_to_float(u.x >> 16),
                               half_bits_to_float(u.y & 0xffff), half_bits_to_float(u.y >> 16)};
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gk + e < kend) rb[it][e] = half_bits_to_float(src[e]);
            }
          } else {
            const float* src = reinterpret_cast<const float*>(p.B) + (int64_t)gn * p.ldb + gk;
            if (gk + 4 <= kend) {
              rb[it] = *reinterpret_cast<const floatx4*>(src);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gk + e < kend) rb[it][e] = src[e];
            }
          }
        }
      } else {
        // [K,N]: lanes walk n (coalesced rows of W); each thread gathers 4 k.
        const int n = flat % BN, kq = (flat / BN) * 4;
        const int gn = n0 + n;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gk = k0 + kq + e;
          float val = 0.f;
          if (gn < p.N && gk < kend) {
            if constexpr (B_F16)
              val = half_bits_to_float(reinterpret_cast<const uint16_t*>(p.B)[(int64_t)gk * p.ldb + gn]);
            else
              val = reinterpret_cast<const float*>(p.B)[(int64_t)gk * p.ldb + gn];
          }
          rb[it][e] = val;
        }
      }
    }
  };
  auto store_panel = [&](int buf) {
#pragma unroll
    for (int it = 0; it < A_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      const int row = flat >> 2, kq = (flat & 3) * 4;
      *reinterpret_cast<floatx4*>(&As[buf][row * PITCH + kq]) = ra[it];
    }
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      const int flat = tid + 256 * it;
      int row, kq;
      if constexpr (B_NK) {
        row = flat >> 2;
        kq = (flat & 3) * 4;
      } else {
        row = flat % BN;
        kq = (flat / BN) * 4;
      }
      *reinterpret_cast<floatx4*>(&Bs[buf][row * PITCH + kq]) = rb[it];
    }
  };

  if (nk > 0) {
    load_panel(kbeg);
    store_panel(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_panel(kbeg + (kt + 1) * BK);
    floatx4 fa[TM][2], fb[TN][2];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const float* src = &As[buf][(wave_m * WM + a * 32 + li) * PITCH + 8 * lh];
      fa[a][0] = *reinterpret_cast<const floatx4*>(src);
      fa[a][1] = *reinterpret_cast<const floatx4*>(src + 4);
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float* src = &Bs[buf][(wave_n * WN + b * 32 + li) * PITCH + 8 * lh];
      fb[b][0] = *reinterpret_cast<const floatx4*>(src);
      fb[b][1] = *reinterpret_cast<const floatx4*>(src + 4);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][t >> 2][t & 3],
                                                           fb[b][t >> 2][t & 3],
                                                           acc[a][b], 0, 0, 0);
    if (kt + 1 < nk) store_panel(buf ^ 1);
    __syncthreads();
  }

  // Output: lane (li, lh) of a 32×32 tile holds column li, rows
  // 8*(e/4) + 4*lh + e%4 for e = 0..15.
  const bool split_out = p.partial != nullptr;
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int n = n0 + wave_n * WN + b * 32 + li;
      if (n >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wave_m * WM + a * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
        if (m >= p.M) continue;
        if (split_out) {
          p.partial[((int64_t)split * p.M + m) * p.N + n] = acc[a][b][e];
        } else {
          p.C[(int64_t)m * p.ldc + n] = epilogue_value(p.ep, acc[a][b][e], m, n, p.C, p.ldc);
        }
      }
    }
}

__global__ void splitk_reduce_kernel(const float* partial, int splits, int M,
                                     int N, float* C, int64_t ldc,
                                     GemmEpilogue ep) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)M * N;
  if (idx >= total) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  float s = 0.f;
  for (int z = 0; z < splits; ++z) s += partial[(int64_t)z * total + idx];
  C[(int64_t)m * ldc + n] = epilogue_value(ep, s, m, n, C, ldc);
}

template <int BM, int BN>
void launch_tile(hipStream_t s, GemmParams& p, bool b_nk, bool b_f16, int splits) {
  p.tiles_m = (int)cdiv(p.M, BM);
  p.tiles_n = (int)cdiv(p.N, BN);
  const int tiles = p.tiles_m * p.tiles_n;
  p.tiles_per_xcd = (int)cdiv(tiles, 8);
  dim3 grid(p.tiles_per_xcd * 8, splits), block(256);
  if (b_nk) {
    if (b_f16) hipLaunchKernelGGL((gemm_kernel<BM, BN, true, true>), grid, block, 0, s, p);
    else       hipLaunchKernelGGL((gemm_kernel<BM, BN, true, false>), grid, block, 0, s, p);
  } else {
    if (b_f16) hipLaunchKernelGGL((gemm_kernel<BM, BN, false, true>), grid, block, 0, s, p);
    else       hipLaunchKernelGGL((gemm_kernel<BM, BN, false, false>), grid, block, 0, s, p);
  }
  MFT_LAUNCH_CHECK();
}

// ---- skinny rank-r kernels --------------------------------------------------
// out[m, j] = Σ_k X[m,k] · Y(k,j); one wave per row, lanes stride k.
template <int R>
__global__ __launch_bounds__(256) void rank_proj_kernel(const float* X, int64_t ldx,
                                                         const float* Y, int64_t ysk,
                                                         int64_t ysj, int M, int K,
                                                         int r, float* out) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.f;
  const float* xr = X + (int64_t)m * ldx;
  for (int k = lane; k < K; k += 64) {
    const float xv = xr[k];
    const float* yk = Y + (int64_t)k * ysk;
#pragma unroll
    for (int j = 0; j < R; ++j)
      if (j < r) acc[j] = fmaf(xv, yk[j * ysj], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < R; ++j) {
    float v = acc[j];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[j] = v;
  }
  if (lane < r) {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j)
      if (j == lane) v = acc[j];
    out[(int64_t)m * r + lane] = v;
  }
}

// Partial sums of Σ_m P[m,j] X[m,c] over a row slice; 64 columns × 4 row
// groups per workgroup.  Writes part[slice][j][c].
template <int R>
__global__ __launch_bounds__(256) void rank_outer_kernel(const float* P, const float* X,
                                                          int64_t ldx, int M, int C, int r,
                                                          int rows_per_slice, float* part) {
  __shared__ float red[4][R][64];
  const int c = blockIdx.x * 64 + (threadIdx.x & 63);
  const int g = threadIdx.x >> 6;
  const int slice = blockIdx.y;
  const int mb = slice * rows_per_slice, me = min(M, mb + rows_per_slice);
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.f;
  if (c < C) {
    for (int m = mb + g; m < me; m += 4) {
      const float xv = X[(int64_t)m * ldx + c];
      const float* pr = P + (int64_t)m * r;
#pragma unroll
      for (int j = 0; j < R; ++j)
        if (j < r) acc[j] = fmaf(pr[j], xv, acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < R; ++j) red[g][j][threadIdx.x & 63] = acc[j];
  __syncthreads();
  if (g == 0 && c < C) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (j >= r) break;
      const float v = red[0][j][threadIdx.x] + red[1][j][threadIdx.x] +
                      red[2][j][threadIdx.x] + red[3][j][threadIdx.x];
      part[((int64_t)slice * r + j) * C + c] = v;
    }
  }
}

__global__ void rank_outer_finish(const float* part, int slices, int C, int r,
                                  float scale, float* out, int64_t osj,
                                  int64_t osc, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)C * r) return;
  const int j = (int)(idx / C), c = (int)(idx % C);
  float s = 0.f;
  for (int z = 0; z < slices; ++z) s += part[((int64_t)z * r + j) * C + c];
  float* o = out + (int64_t)j * osj + (int64_t)c * osc;
  *o = accumulate ? fmaf(scale, s, *o) : scale * s;
}

}  // namespace

void gemm(hipStream_t s, const float* A, int64_t lda, const void* B,
          int64_t ldb, bool b_nk, bool b_f16, float* C, int64_t ldc, int M,
          int N, int K, const GemmEpilogue& ep, Scratch ws,
          const KernelEvents* ev) {
  float* workspace = ws.ptr;
  const size_t workspace_bytes = ws.bytes;
  MFT_CHECK_ARG(M > 0 && N > 0 && K > 0, "empty GEMM");
  MFT_CHECK_ARG(lda % 4 == 0 && lda >= K, "lda must be a multiple of 4 and >= K");
  MFT_CHECK_ARG(!b_nk || (ldb % 4 == 0 && ldb >= K), "ldb must be a multiple of 4 and >= K for [N,K] B");
  MFT_CHECK_ARG(b_nk || ldb >= N, "ldb must be >= N for [K,N] B");
  MFT_CHECK_ARG(ldc >= N, "ldc must be >= N");
  MFT_CHECK_ARG(ep.r <= 32, "LoRA rank > 32 unsupported");
  MFT_CHECK_ARG(((uintptr_t)A & 15) == 0, "A must be 16-byte aligned");
  MFT_CHECK_ARG(!b_nk || ((uintptr_t)B & (b_f16 ? 7 : 15)) == 0, "B misaligned");
  GemmParams p;
  p.A = A; p.B = B; p.C = C;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K;
  p.ep = ep;
  p.partial = nullptr;

  // Tile choice: the largest tile that still yields ≥ one workgroup per CU;
  // otherwise 64×64 plus split-K until the grid covers the 256 CUs.
  const int64_t t128 = cdiv(M, 128) * cdiv(N, 128);
  const int64_t t64x128 = cdiv(M, 64) * cdiv(N, 128);
  const int64_t t64 = cdiv(M, 64) * cdiv(N, 64);
  int bm = 64, bn = 64, splits = 1;
  if (t128 >= 256) { bm = 128; bn = 128; }
  else if (t64x128 >= 256) { bm = 64; bn = 128; }
  else {
    const int64_t want = cdiv(256, t64);
    const int64_t kmax = K / 128;  // keep ≥ 128 of K per split
    splits = (int)std::max<int64_t>(1, std::min<int64_t>(want, kmax));
    if (splits > 1 && (size_t)splits * M * N * sizeof(float) > workspace_bytes) splits = 1;
  }
  p.k_chunk = (int)(cdiv(cdiv(K, splits), BK) * BK);
  splits = (int)cdiv(K, p.k_chunk);
  if (splits > 1) p.partial = workspace;

  if (ev && ev->start) MFT_HIP(hipEventRecord(ev->start, s));
  if (bm == 128) launch_tile<128, 128>(s, p, b_nk, b_f16, splits);
  else if (bn == 128) launch_tile<64, 128>(s, p, b_nk, b_f16, splits);
  else launch_tile<64, 64>(s, p, b_nk, b_f16, splits);
  if (ev && ev->stop) MFT_HIP(hipEventRecord(ev->stop, s));

  if (splits > 1) {
    const int64_t total = (int64_t)M * N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s,
                       (const float*)workspace, splits, M, N, C, ldc, ep);
    MFT_LAUNCH_CHECK();
  }
}

void rank_proj(hipStream_t s, const float* X, int64_t ldx, const float* Y,
               int64_t ysk, int64_t ysj, int M, int K, int r, float* out) {
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  dim3 grid((unsigned)cdiv(M, 4)), block(256);
  if (r <= 8)       hipLaunchKernelGGL(rank_proj_kernel<8>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
  else if (r <= 16) hipLaunchKernelGGL(rank_proj_kernel<16>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
  else              hipLaunchKernelGGL(rank_proj_kernel<32>, grid, block, 0, s, X, ldx, Y, ysk, ysj, M, K, r, out);
  MFT_LAUNCH_CHECK();
}

void rank_outer(hipStream_t s, const float* P, const float* X, int64_t ldx,
                int M, int C, int r, float scale, float* out, int64_t osj,
                int64_t osc, bool accumulate, Scratch ws) {
  float* workspace = ws.ptr;
  const size_t ws_bytes = ws.bytes;
  MFT_CHECK_ARG(r >= 1 && r <= 32, "rank must be in [1,32]");
  int slices = (int)std::min<int64_t>(cdiv(M, 64), 16);
  while (slices > 1 && (size_t)slices * r * C * sizeof(float) > ws_bytes) slices /= 2;
  if (!workspace) slices = 1;
  MFT_CHECK_ARG(workspace && (size_t)slices * r * C * sizeof(float) <= ws_bytes,
                "rank_outer needs a workspace of r*C floats");
  const int rows = (int)cdiv(M, slices);
  dim3 grid((unsigned)cdiv(C, 64), slices), block(256);
  if (r <= 8)       hipLaunchKernelGGL(rank_outer_kernel<8>, grid, block, 0, s, P, X, ldx, M, C, r, rows, workspace);
  else if (r <= 16) hipLaunchKernelGGL(rank_outer_kernel<16>, grid, block, 0, s, P, X, ldx, M, C, r, rows, workspace);
  else              hipLaunchKernelGGL(rank_outer_kernel<32>, grid, block, 0, s, P, X, ldx, M, C, r, rows, workspace);
  MFT_LAUNCH_CHECK();
  hipLaunchKernelGGL(rank_outer_finish, dim3((unsigned)cdiv((int64_t)C * r, 256)), dim3(256), 0, s,
                     (const float*)workspace, slices, C, r, scale, out, osj, osc, accumulate ? 1 : 0);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
