// ce.hip — shifted LM cross-entropy over the full vocabulary, forward and
// backward in one pass structure:
//   1. count the valid targets (label != ignore_index, shifted by one),
//   2. one workgroup per logits row: online max/sum-exp over V in registers
//      (each thread keeps its own running max and rescaled sum, merged by a
//      wave64 shuffle tree and an LDS step), NLL = lse − x[label], then a
//      second sweep writes dlogits = (exp(x − lse) − onehot)·upstream/n in
//      place (the row is re-read from L2/MALL, not HBM, at these row sizes),
//   3. a single-workgroup fixed-order reduction of the per-row NLLs into the
//      fp64 loss sum (deterministic).
// Algorithmic HBM traffic: read logits once + write dlogits once
// (8·rows·V bytes).
#include "common.h"

namespace mft {
namespace {

__global__ void zero_i64_kernel(int64_t* p) { *p = 0; }

__global__ __launch_bounds__(256) void ce_count_kernel(const int32_t* __restrict__ labels,
                                                       int B, int S, int ignore_index,
                                                       int64_t* cnt) {
  __shared__ int red[4];
  int c = 0;
  const int64_t total = (int64_t)B * S;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int s = (int)(i % S);
    if (s + 1 < S && labels[i + 1] != ignore_index) c++;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int v = red[0] + red[1] + red[2] + red[3];
    if (v) atomicAdd((unsigned long long*)cnt, (unsigned long long)v);
  }
}

__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  if (m2 > m) {
    s = s * __expf(m - m2) + s2;
    m = m2;
  } else if (m2 > -INFINITY) {
    s += s2 * __expf(m2 - m);
  }
}

template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void ce_row_kernel(
    const float* logits, const int32_t* __restrict__ labels, int B, int S,
    int64_t V, int64_t ld, int ignore_index, float upstream, int64_t norm_count,
    const int64_t* __restrict__ cnt, float* dlogits, float* __restrict__ row_nll) {
  constexpr int NW = BLOCK / 64;
  __shared__ float sm[NW], ss[NW];
  const int64_t row = blockIdx.x;
  const int s = (int)(row % S);
  const int label = (s + 1 < S) ? labels[row + 1] : ignore_index;
  const float* x = logits + row * ld;
  float* dx = dlogits ? dlogits + row * ld : nullptr;
  if (label == ignore_index || label < 0 || (int64_t)label >= V) {
    if (dx)
      for (int64_t j = threadIdx.x; j < V; j += BLOCK) dx[j] = 0.f;
    if (threadIdx.x == 0) row_nll[row] = 0.f;
    return;
  }
  float m = -INFINITY, sum = 0.f;
  for (int64_t j = threadIdx.x; j < V; j += BLOCK) {
    const float v = x[j];
    if (v > m) {
      sum = sum * __expf(m - v) + 1.f;
      m = v;
    } else {
      sum += __expf(v - m);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(sum, off, 64);
    merge_ms(m, sum, m2, s2);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = m;
    ss[w] = sum;
  }
  __syncthreads();
  m = sm[0];
  sum = ss[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) merge_ms(m, sum, sm[i], ss[i]);
  const float lse = m + logf(sum);
  const float xl = x[label];
  if (threadIdx.x == 0) row_nll[row] = lse - xl;
  if (dx) {
    const int64_t n = norm_count > 0 ? norm_count : *cnt;
    const float g = n > 0 ? upstream / (float)n : 0.f;
    // dx may alias x: every element is read before it is written by the
    // same thread, and the label logit was read above the barrier.
    __syncthreads();
    for (int64_t j = threadIdx.x; j < V; j += BLOCK) {
      const float p = __expf(x[j] - lse);
      dx[j] = (j == label ? p - 1.f : p) * g;
    }
  }
}

__global__ __launch_bounds__(256) void ce_sum_kernel(const float* __restrict__ row_nll,
                                                     int64_t rows, double* loss_sum,
                                                     const int64_t* cnt, int64_t* n_valid) {
  __shared__ double red[4];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < rows; i += 256) s += (double)row_nll[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    if (loss_sum) *loss_sum += (red[0] + red[1]) + (red[2] + red[3]);
    if (n_valid) *n_valid += *cnt;
  }
}

}  // namespace

void ce_fwd_bwd(hipStream_t s, const float* logits, const int32_t* labels,
                int B, int S, int64_t V, int64_t ld, int ignore_index, float upstream,
                int64_t norm_count, double* loss_sum, int64_t* n_valid,
                float* dlogits, float* row_nll, int64_t* count_scratch) {
  MFT_CHECK_ARG(B > 0 && S > 0 && V > 0 && ld >= V, "empty or bad row stride");
  MFT_CHECK_ARG(count_scratch && row_nll, "scratch required");
  const int64_t rows = (int64_t)B * S;
  // A fill kernel rather than hipMemsetAsync keeps the sequence capturable
  // in a HIP graph.
  hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(1), 0, s, count_scratch);
  MFT_LAUNCH_CHECK();
  hipLaunchKernelGGL(ce_count_kernel, dim3((unsigned)std::min<int64_t>(cdiv(rows, 256), 64)), dim3(256),
                     0, s, labels, B, S, ignore_index, count_scratch);
  MFT_LAUNCH_CHECK();
  hipLaunchKernelGGL(ce_row_kernel<512>, dim3((unsigned)rows), dim3(512), 0, s, logits, labels, B, S, V, ld,
                     ignore_index, upstream, norm_count, (const int64_t*)count_scratch, dlogits, row_nll);
  MFT_LAUNCH_CHECK();
  hipLaunchKernelGGL(ce_sum_kernel, dim3(1), dim3(256), 0, s, (const float*)row_nll, rows, loss_sum,
                     (const int64_t*)count_scratch, n_valid);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
