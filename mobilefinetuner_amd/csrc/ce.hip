// ce.hip — shifted LM cross-entropy over the full vocabulary, forward and
// backward in one pass structure:
//   1. count the valid targets (label != ignore_index, shifted by one) —
//      inside every row workgroup for up to kCountInRowMax rows, else once
//      by a one-workgroup launch ahead of the rows (per-row counting reads
//      the whole label array once per row: rows² work),
//   2. one workgroup per logits row: online max/sum-exp over V in registers
//      (base 2 on x·log2e; each thread keeps its own running max and
//      rescaled sum over 128-bit loads, merged by a wave64 shuffle tree and
//      an LDS step), NLL = lse − x[label], then a second sweep writes
//      dlogits = (exp(x − lse) − onehot)·upstream/n in place (the row is
//      re-read from L2/MALL, not HBM, at these row sizes),
//   3. a single-workgroup fixed-order reduction of the per-row NLLs into the
//      fp64 loss sum (deterministic).
// Algorithmic HBM traffic: read logits once + write dlogits once
// (8·rows·V bytes).
#include <algorithm>
#include <cfloat>

#include "common.h"

namespace mft {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Running (max, Σ 2^(t − max)) pairs over base-2 scaled logits t = x·log2e.
// The max starts at −FLT_MAX (not −inf) so that merging two empty pairs
// gives 0·2^0 = 0 rather than NaN.
__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = s * __builtin_amdgcn_exp2f(m - mm) + s2 * __builtin_amdgcn_exp2f(m2 - mm);
  m = mm;
}

// The micro-batch's valid shifted targets, counted by every row workgroup:
// position s < S−1 whose next label is neither ignore_index nor outside
// [0, V) — the test the row itself applies, so an out-of-range label is
// excluded from both the loss and its normaliser (and flagged in *bad).
// This thread's share over i = tid, tid + BLOCK, …; `oor` is set when the
// share met an out-of-range label.  The loads are independent of the row's,
// so they overlap its reads.  The count is stored (by workgroup 0), not
// accumulated, so no clearing launch precedes it.
__device__ __forceinline__ int count_share(const int32_t* __restrict__ labels, int B, int S, int64_t V,
                                           int ignore_index, int tid, int block, bool& oor) {
  int c = 0;
  const int64_t total = (int64_t)B * S;
  for (int64_t i = tid; i < total; i += block) {
    const int s = (int)(i % S);
    if (s + 1 >= S) continue;
    const int lab = labels[i + 1];
    if (lab == ignore_index) continue;
    if (lab >= 0 && (int64_t)lab < V) c++;
    else oor = true;
  }
  return c;
}

// Workgroup 0 publishes the count (for the loss sum) and the bad-label flag.
// red: NW ints of LDS; a full workgroup reduction with its own barrier, for a
// workgroup whose row takes no other reduction.
template <int NW>
__device__ __forceinline__ void publish_count(int c, bool oor, int* red, int64_t* cnt, int* bad) {
  if (blockIdx.x != 0) return;
  if (oor && bad) atomicOr(bad, 1);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t v = 0;
    for (int w = 0; w < NW; ++w) v += red[w];
    *cnt = v;
  }
}

// The micro-batch's valid-target count formed once (batches above
// kCountInRowMax rows): one workgroup strides the labels, stores the count
// in *cnt and raises *bad for an out-of-range label.
__global__ __launch_bounds__(1024) void ce_count_kernel(const int32_t* __restrict__ labels, int B, int S,
                                                        int64_t V, int ignore_index, int64_t* cnt, int* bad) {
  __shared__ int red[16];
  bool oor = false;
  int c = count_share(labels, B, S, V, ignore_index, threadIdx.x, 1024, oor);
  if (oor && bad) atomicOr(bad, 1);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t v = 0;
    for (int w = 0; w < 16; ++w) v += red[w];
    *cnt = v;
  }
}

// One workgroup per logits row.  The row is walked as an aligned float4 body
// (rows start at any 4-byte offset when V is odd) plus a scalar head and
// tail.  The first H·BLOCK float4 of the body stay in registers from the
// statistics sweep to the gradient sweep (each thread issues its H loads at
// once), so only the rest of the row is read twice: a row of up to
// 4·H·BLOCK values (GPT-2's 50257 with H = 13) moves through HBM once
// each way.  The rest is streamed with U float4 loads in flight per thread,
// each group of 4·U values folded into the thread's running (max, Σ) pair
// with one rescale, and re-read by the gradient sweep, which writes dlogits
// in place.
// The micro-batch's target count is formed in every workgroup beside the
// row's statistics (workgroup 0 stores it in *cnt and raises *bad), or, with
// `counted`, read from *cnt where ce_count_kernel stored it.
template <int BLOCK, int H>
__global__ __launch_bounds__(BLOCK) void ce_row_kernel(
    const float* logits, const int32_t* __restrict__ labels, int B, int S,
    int64_t V, int64_t ld, int ignore_index, float upstream, int64_t norm_count,
    int64_t* __restrict__ cnt, int* bad, float* dlogits, float* __restrict__ row_nll, int counted,
    float* __restrict__ dl_inv_s) {
  constexpr int NW = BLOCK / 64, U = 4;
  __shared__ float sm[NW], ss[NW];
  __shared__ int sc[NW];
  const int64_t row = blockIdx.x;
  const int s = (int)(row % S);
  const int label = (s + 1 < S) ? labels[row + 1] : ignore_index;
  const float* x = logits + row * ld;
  float* dx = dlogits ? dlogits + row * ld : nullptr;
  const int tid = threadIdx.x;
  bool oor = false;
  int c = counted ? 0 : count_share(labels, B, S, V, ignore_index, tid, BLOCK, oor);
  if (label == ignore_index || label < 0 || (int64_t)label >= V) {
    if (!counted) publish_count<NW>(c, oor, sc, cnt, bad);
    if (dx)
      for (int64_t j = tid; j < V; j += BLOCK) dx[j] = 0.f;
    if (tid == 0) row_nll[row] = 0.f;
    if (dx && dl_inv_s && tid == 0) dl_inv_s[row] = 1.f;  // a zero row
    return;
  }
  if (blockIdx.x == 0 && oor && bad) atomicOr(bad, 1);
  const float xl = x[label];  // read before any thread writes (dx may alias x)
  const int64_t head = std::min<int64_t>((4 - (((uintptr_t)x >> 2) & 3)) & 3, V);
  const int64_t n4 = (V - head) / 4;
  const int64_t tail0 = head + 4 * n4;
  const floatx4* x4 = reinterpret_cast<const floatx4*>(x + head);

  float m = -FLT_MAX, sum = 0.f;
  for (int64_t j = tid; j < head; j += BLOCK) merge_ms(m, sum, x[j] * kLog2e, 1.f);
  // held part: float4 q = tid + BLOCK·i, i < H
  floatx4 hv[H];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int64_t q = tid + (int64_t)BLOCK * i;
    hv[i] = q < n4 ? x4[q] : floatx4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  {
    float mx = m;
#pragma unroll
    for (int i = 0; i < H; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) mx = fmaxf(mx, hv[i][e] * kLog2e);
    float acc = sum * __builtin_amdgcn_exp2f(m - mx);
#pragma unroll
    for (int i = 0; i < H; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc += __builtin_amdgcn_exp2f(fmaf(hv[i][e], kLog2e, -mx));
    sum = acc;
    m = mx;
  }
  const int64_t rest0 = (int64_t)BLOCK * H;  // first streamed float4
  for (int64_t b = rest0 + tid; b < n4; b += (int64_t)BLOCK * U) {
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = b + (int64_t)u * BLOCK;
      v[u] = q < n4 ? x4[q] : floatx4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    float mx = m;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[u][e] *= kLog2e;
        mx = fmaxf(mx, v[u][e]);
      }
    float acc = sum * __builtin_amdgcn_exp2f(m - mx);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc += __builtin_amdgcn_exp2f(v[u][e] - mx);
    sum = acc;
    m = mx;
  }
  for (int64_t j = tail0 + tid; j < V; j += BLOCK) merge_ms(m, sum, x[j] * kLog2e, 1.f);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(sum, off, 64);
    merge_ms(m, sum, m2, s2);
    c += __shfl_xor(c, off, 64);
  }
  const int w = tid >> 6;
  if ((tid & 63) == 0) {
    sm[w] = m;
    ss[w] = sum;
    sc[w] = c;
  }
  __syncthreads();
  m = sm[0];
  sum = ss[0];
  int64_t n_valid = sc[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    merge_ms(m, sum, sm[i], ss[i]);
    n_valid += sc[i];
  }
  if (counted) n_valid = *cnt;
  else if (blockIdx.x == 0 && tid == 0) *cnt = n_valid;
  const float lse2 = m + __builtin_amdgcn_logf(sum);  // log2 Σ 2^t (sum ≥ 1)
  if (tid == 0) row_nll[row] = lse2 * kLn2 - xl;
  if (!dx) return;
  const int64_t n = norm_count > 0 ? norm_count : n_valid;
  const float g = n > 0 ? upstream / (float)n : 0.f;
  if (dl_inv_s && tid == 0) {
    // row scale of the dlogits for the fp16 GEMM that consumes them, from a
    // bound on the row's max |dlogit| = |g|·max(max_j p_j, 1 − p_label)
    const float pmax = __builtin_amdgcn_exp2f(m - lse2);
    const float plab = __builtin_amdgcn_exp2f(fmaf(xl, kLog2e, -lse2));
    dl_inv_s[row] = row_inv_scale(fabsf(g) * fmaxf(pmax, 1.f - plab));
  }
  // dlogits = (softmax − onehot(label))·g; every element is read before the
  // same thread writes it.
  for (int64_t j = tid; j < head; j += BLOCK) {
    const float p = __builtin_amdgcn_exp2f(fmaf(x[j], kLog2e, -lse2));
    dx[j] = (j == label ? p - 1.f : p) * g;
  }
  floatx4* d4 = reinterpret_cast<floatx4*>(dx + head);
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int64_t q = tid + (int64_t)BLOCK * i;
    if (q >= n4) continue;
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(fmaf(hv[i][e], kLog2e, -lse2));
      o[e] = (head + 4 * q + e == label ? p - 1.f : p) * g;
    }
    d4[q] = o;
  }
  for (int64_t b = rest0 + tid; b < n4; b += (int64_t)BLOCK * U) {
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = b + (int64_t)u * BLOCK;
      if (q < n4) v[u] = x4[q];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = b + (int64_t)u * BLOCK;
      if (q >= n4) continue;
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(fmaf(v[u][e], kLog2e, -lse2));
        o[e] = (head + 4 * q + e == label ? p - 1.f : p) * g;
      }
      d4[q] = o;
    }
  }
  for (int64_t j = tail0 + tid; j < V; j += BLOCK) {
    const float p = __builtin_amdgcn_exp2f(fmaf(x[j], kLog2e, -lse2));
    dx[j] = (j == label ? p - 1.f : p) * g;
  }
}

// Rows whose base-2 softmax statistics the LM-head GEMM wrote per 64-column
// block (stats[row·stats_ld + j] = (max, Σ)): the row's log-sum-exp is merged
// from those pairs, so the gradient sweep is the only pass over the logits —
// each value read once and its dlogit written in place.
template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void ce_row_stats_kernel(
    const float* logits, const int32_t* __restrict__ labels, int B, int S, int64_t V, int64_t ld,
    int ignore_index, float upstream, int64_t norm_count, int64_t* __restrict__ cnt, int* bad, float* dlogits,
    float* __restrict__ row_nll, const float2* __restrict__ stats, int64_t stats_ld, int counted,
    float* __restrict__ dl_inv_s) {
  constexpr int NW = BLOCK / 64, U = 4;
  __shared__ float sm[NW], ss[NW];
  __shared__ int sc[NW];
  const int64_t row = blockIdx.x;
  const int s = (int)(row % S);
  const int label = (s + 1 < S) ? labels[row + 1] : ignore_index;
  const float* x = logits + row * ld;
  float* dx = dlogits ? dlogits + row * ld : nullptr;
  const int tid = threadIdx.x;
  bool oor = false;
  int c = counted ? 0 : count_share(labels, B, S, V, ignore_index, tid, BLOCK, oor);
  if (label == ignore_index || label < 0 || (int64_t)label >= V) {
    if (!counted) publish_count<NW>(c, oor, sc, cnt, bad);
    if (dx)
      for (int64_t j = tid; j < V; j += BLOCK) dx[j] = 0.f;
    if (tid == 0) row_nll[row] = 0.f;
    if (dx && dl_inv_s && tid == 0) dl_inv_s[row] = 1.f;  // a zero row
    return;
  }
  if (blockIdx.x == 0 && oor && bad) atomicOr(bad, 1);
  const float xl = x[label];  // read before any thread writes (dx may alias x)
  const int64_t nb = (V + 63) / 64;
  const float2* st = stats + row * stats_ld;
  float m = -FLT_MAX, sum = 0.f;
  for (int64_t j = tid; j < nb; j += BLOCK) {
    const float2 p = st[j];
    merge_ms(m, sum, p.x, p.y);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(sum, off, 64);
    merge_ms(m, sum, m2, s2);
    c += __shfl_xor(c, off, 64);
  }
  const int w = tid >> 6;
  if ((tid & 63) == 0) {
    sm[w] = m;
    ss[w] = sum;
    sc[w] = c;
  }
  __syncthreads();
  m = sm[0];
  sum = ss[0];
  int64_t n_valid = sc[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    merge_ms(m, sum, sm[i], ss[i]);
    n_valid += sc[i];
  }
  if (counted) n_valid = *cnt;
  else if (blockIdx.x == 0 && tid == 0) *cnt = n_valid;
  const float lse2 = m + __builtin_amdgcn_logf(sum);
  if (tid == 0) row_nll[row] = lse2 * kLn2 - xl;
  if (!dx) return;
  const int64_t n = norm_count > 0 ? norm_count : n_valid;
  const float g = n > 0 ? upstream / (float)n : 0.f;
  if (dl_inv_s && tid == 0) {
    // row scale of the dlogits for the fp16 GEMM that consumes them, from a
    // bound on the row's max |dlogit| = |g|·max(max_j p_j, 1 − p_label)
    const float pmax = __builtin_amdgcn_exp2f(m - lse2);
    const float plab = __builtin_amdgcn_exp2f(fmaf(xl, kLog2e, -lse2));
    dl_inv_s[row] = row_inv_scale(fabsf(g) * fmaxf(pmax, 1.f - plab));
  }
  const int64_t head = std::min<int64_t>((4 - (((uintptr_t)x >> 2) & 3)) & 3, V);
  const int64_t n4 = (V - head) / 4;
  const int64_t tail0 = head + 4 * n4;
  const floatx4* x4 = reinterpret_cast<const floatx4*>(x + head);
  floatx4* d4 = reinterpret_cast<floatx4*>(dx + head);
  for (int64_t j = tid; j < head; j += BLOCK) {
    const float p = __builtin_amdgcn_exp2f(fmaf(x[j], kLog2e, -lse2));
    dx[j] = (j == label ? p - 1.f : p) * g;
  }
  for (int64_t b = tid; b < n4; b += (int64_t)BLOCK * U) {
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = b + (int64_t)u * BLOCK;
      if (q < n4) v[u] = x4[q];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = b + (int64_t)u * BLOCK;
      if (q >= n4) continue;
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(fmaf(v[u][e], kLog2e, -lse2));
        o[e] = (head + 4 * q + e == label ? p - 1.f : p) * g;
      }
      d4[q] = o;
    }
  }
  for (int64_t j = tail0 + tid; j < V; j += BLOCK) {
    const float p = __builtin_amdgcn_exp2f(fmaf(x[j], kLog2e, -lse2));
    dx[j] = (j == label ? p - 1.f : p) * g;
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
                float* dlogits, float* row_nll, int64_t* count_scratch, int* bad_label,
                const float2* row_stats, int64_t stats_ld, float* dl_inv_s) {
  if (!dlogits) dl_inv_s = nullptr;
  MFT_CHECK_ARG(B > 0 && S > 0 && V > 0 && ld >= V, "empty or bad row stride");
  MFT_CHECK_ARG(count_scratch && row_nll, "scratch required");
  const int64_t rows = (int64_t)B * S;
  // Up to kCountInRowMax rows every row workgroup counts the targets beside
  // its own statistics (no launch of its own); beyond, a count launch forms it
  // once (per-row counting grows with rows²: 4.3G label reads at 65536 rows).
  constexpr int64_t kCountInRowMax = 4096;
  const int counted = rows > kCountInRowMax ? 1 : 0;
  if (counted) {
    hipLaunchKernelGGL(ce_count_kernel, dim3(1), dim3(1024), 0, s, labels, B, S, V, ignore_index, count_scratch,
                       bad_label);
    MFT_LAUNCH_CHECK();
  }
  // rows of up to 13·4096 values are held whole in registers (GPT-2's
  // 50257); wider rows take the LM head's row statistics when it wrote them
  // (one sweep), else keep their first 16·4096 values in registers
  if (row_stats && V > 13 * 4096) {
    MFT_CHECK_ARG(stats_ld >= cdiv(V, 64), "row statistics pitch");
    hipLaunchKernelGGL((ce_row_stats_kernel<1024>), dim3((unsigned)rows), dim3(1024), 0, s, logits, labels, B, S, V,
                       ld, ignore_index, upstream, norm_count, count_scratch, bad_label, dlogits, row_nll,
                       row_stats, stats_ld, counted, dl_inv_s);
  } else if (V <= 13 * 4096)
    hipLaunchKernelGGL((ce_row_kernel<1024, 13>), dim3((unsigned)rows), dim3(1024), 0, s, logits, labels, B, S, V,
                       ld, ignore_index, upstream, norm_count, count_scratch, bad_label, dlogits, row_nll, counted,
                       dl_inv_s);
  else
    hipLaunchKernelGGL((ce_row_kernel<1024, 16>), dim3((unsigned)rows), dim3(1024), 0, s, logits, labels, B, S, V,
                       ld, ignore_index, upstream, norm_count, count_scratch, bad_label, dlogits, row_nll, counted,
                       dl_inv_s);
  MFT_LAUNCH_CHECK();
  if (!loss_sum && !n_valid) return;  // dlogits only
  hipLaunchKernelGGL(ce_sum_kernel, dim3(1), dim3(256), 0, s, (const float*)row_nll, rows, loss_sum,
                     (const int64_t*)count_scratch, n_valid);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
