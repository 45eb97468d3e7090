// elementwise.hip — HBM-bound support kernels of the LoRA step: norms,
// activations, RoPE, embedding gather, fp16 widening, Adam, grad-norm/clip,
// and deterministic initialisers.  Row reductions use one wave64 per row
// (4 rows per 256-thread workgroup) with shuffle reductions; streaming
// kernels use 128-bit accesses where the tensor length allows.
#include "common.h"

namespace mft {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Round-to-nearest-even fp32 → fp16 via the hardware conversion
// (v_cvt_f16_f32 rounds to nearest even under the default rounding mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- LayerNorm (GPT-2) -------------------------------------------------------
__global__ __launch_bounds__(256) void layernorm_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ b, int64_t M, int C, float eps,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + row * C;
  float s = 0.f;
  for (int j = lane; j < C; j += 64) s += xr[j];
  const float mu = wave_sum(s) / (float)C;
  float v = 0.f;
  for (int j = lane; j < C; j += 64) {
    const float d = xr[j] - mu;
    v = fmaf(d, d, v);
  }
  const float rs = rsqrtf(wave_sum(v) / (float)C + eps);
  float* yr = y + row * C;
  for (int j = lane; j < C; j += 64) yr[j] = fmaf((xr[j] - mu) * rs, g[j], b[j]);
  if (lane == 0) {
    if (mean) mean[row] = mu;
    if (rstd) rstd[row] = rs;
  }
}

__global__ __launch_bounds__(256) void layernorm_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ g, const float* __restrict__ mean,
    const float* __restrict__ rstd, int64_t M, int C, float* dx,
    const float* resid) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + row * C;
  const float* dyr = dy + row * C;
  const float mu = mean[row], rs = rstd[row];
  float s1 = 0.f, s2 = 0.f;
  for (int j = lane; j < C; j += 64) {
    const float xh = (xr[j] - mu) * rs;
    const float dxh = dyr[j] * g[j];
    s1 += dxh;
    s2 = fmaf(dxh, xh, s2);
  }
  s1 = wave_sum(s1) / (float)C;
  s2 = wave_sum(s2) / (float)C;
  float* dxr = dx + row * C;
  for (int j = lane; j < C; j += 64) {
    const float xh = (xr[j] - mu) * rs;
    const float r = rs * (dyr[j] * g[j] - s1 - xh * s2);
    dxr[j] = resid ? resid[row * C + j] + r : r;
  }
}

// ---- RMSNorm (Qwen2: w; Gemma3: 1+w) ------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ w, int64_t M, int C,
    float eps, int unit_offset, float* __restrict__ y, float* __restrict__ rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + row * C;
  float s = 0.f;
  for (int j = lane; j < C; j += 64) s = fmaf(xr[j], xr[j], s);
  const float rs = rsqrtf(wave_sum(s) / (float)C + eps);
  float* yr = y + row * C;
  for (int j = lane; j < C; j += 64) {
    const float wj = unit_offset ? 1.f + w[j] : w[j];
    yr[j] = xr[j] * rs * wj;
  }
  if (lane == 0 && rstd) rstd[row] = rs;
}

__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ rstd, int64_t M,
    int C, int unit_offset, float* dx, const float* resid) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + row * C;
  const float* dyr = dy + row * C;
  const float rs = rstd[row];
  float s = 0.f;
  for (int j = lane; j < C; j += 64) {
    const float wj = unit_offset ? 1.f + w[j] : w[j];
    s = fmaf(dyr[j] * wj, xr[j] * rs, s);
  }
  s = wave_sum(s) / (float)C;
  float* dxr = dx + row * C;
  for (int j = lane; j < C; j += 64) {
    const float wj = unit_offset ? 1.f + w[j] : w[j];
    const float r = rs * (dyr[j] * wj - xr[j] * rs * s);
    dxr[j] = resid ? resid[row * C + j] + r : r;
  }
}

// ---- activations ---------------------------------------------------------------
__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }
__device__ __forceinline__ float silu_grad(float x) {
  const float s = 1.f / (1.f + expf(-x));
  return s * (1.f + x * (1.f - s));
}

// Element i of a [rows, cols] view: gate/up (and dgate/dup) rows ld_gu
// apart, out/dout rows cols apart (ld_gu == cols: one flat array).
__device__ __forceinline__ int64_t gu_index(int64_t i, int64_t cols, int64_t ld_gu) {
  if (ld_gu == cols) return i;
  const int64_t r = i / cols;
  return r * ld_gu + (i - r * cols);
}

__global__ void glu_fwd_kernel(const float* __restrict__ gate,
                               const float* __restrict__ up, int64_t n, int64_t cols, int64_t ld_gu, int act,
                               float* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = gu_index(i, cols, ld_gu);
    const float a = act == 0 ? gelu_tanh(gate[j]) : silu(gate[j]);
    out[i] = up ? a * up[j] : a;
  }
}

__global__ void glu_bwd_kernel(const float* __restrict__ dout,
                               const float* __restrict__ gate,
                               const float* __restrict__ up, int64_t n, int64_t cols, int64_t ld_gu, int act,
                               float* __restrict__ dgate, float* __restrict__ dup) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = gu_index(i, cols, ld_gu);
    const float gv = gate[j];
    const float a = act == 0 ? gelu_tanh(gv) : silu(gv);
    const float da = act == 0 ? gelu_tanh_grad(gv) : silu_grad(gv);
    const float u = up ? up[j] : 1.f;
    const float d = dout[i];
    dgate[j] = d * u * da;
    if (up && dup) dup[j] = d * a;
  }
}

// 128-bit forms: one run of 4 consecutive elements of a row per thread
// (cols % 4 == 0, every operand 16-byte aligned and n/4 < 2^31, checked on
// the host), the run's row found with one 32-bit division.
typedef float glux4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int64_t gu_run(unsigned q, unsigned cq, unsigned ldq) {
  if (ldq == cq) return q;
  const unsigned r = q / cq;
  return (int64_t)r * ldq + (q - r * cq);
}

__global__ __launch_bounds__(256) void glu_fwd_vec(const glux4* __restrict__ gate, const glux4* __restrict__ up,
                                                   unsigned nq, unsigned cq, unsigned ldq, int act,
                                                   glux4* __restrict__ out) {
  const unsigned q = blockIdx.x * 256u + threadIdx.x;
  if (q >= nq) return;
  const int64_t j = gu_run(q, cq, ldq);
  const glux4 g = gate[j];
  const glux4 u = up ? up[j] : glux4{1.f, 1.f, 1.f, 1.f};
  glux4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (act == 0 ? gelu_tanh(g[e]) : silu(g[e])) * u[e];
  out[q] = o;
}

__global__ __launch_bounds__(256) void glu_bwd_vec(const glux4* __restrict__ dout, const glux4* __restrict__ gate,
                                                   const glux4* __restrict__ up, unsigned nq, unsigned cq,
                                                   unsigned ldq, int act, glux4* __restrict__ dgate,
                                                   glux4* __restrict__ dup) {
  const unsigned q = blockIdx.x * 256u + threadIdx.x;
  if (q >= nq) return;
  const int64_t j = gu_run(q, cq, ldq);
  const glux4 d = dout[q];
  const glux4 g = gate[j];
  const glux4 u = up ? up[j] : glux4{1.f, 1.f, 1.f, 1.f};
  glux4 dg, du;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float gv = g[e];
    const float a = act == 0 ? gelu_tanh(gv) : silu(gv);
    const float da = act == 0 ? gelu_tanh_grad(gv) : silu_grad(gv);
    dg[e] = d[e] * u[e] * da;
    du[e] = d[e] * a;
  }
  dgate[j] = dg;
  if (up && dup) dup[j] = du;
}

// ---- RoPE (HF rotate_half) ---------------------------------------------------
__global__ void rope_kernel(float* x, int64_t rs, int B, int S, int H, int hd,
                            double theta, int inverse) {
  const int half = hd / 2;
  const int64_t total = (int64_t)B * S * H * half;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(idx % half);
    const int64_t t = idx / half;
    const int h = (int)(t % H);
    const int64_t tok = t / H;  // b*S + s
    const int s = (int)(tok % S);
    const double inv = pow(theta, -2.0 * i / (double)hd);
    double sn, cs;
    sincos((double)s * inv, &sn, &cs);
    const float c = (float)cs, sgn = (float)(inverse ? -sn : sn);
    float* xp = x + tok * rs + (int64_t)h * hd;
    const float x1 = xp[i], x2 = xp[i + half];
    xp[i] = x1 * c - x2 * sgn;
    xp[i + half] = x2 * c + x1 * sgn;
  }
}

// ---- embedding ------------------------------------------------------------------
// A token id outside [0, V) reads nothing: its row is written as zeros and
// *bad (when given) is set to 1, for the host to report.
template <bool F16>
__global__ void embed_kernel(const int32_t* __restrict__ ids, int64_t M, int S,
                             const void* __restrict__ wte, int64_t V, const float* __restrict__ wpe,
                             int C, float scale, float* __restrict__ out, int* bad) {
  const int64_t row = blockIdx.x;
  if (row >= M) return;
  const int64_t id = ids[row];
  const int s = (int)(row % S);
  if (id < 0 || id >= V) {
    for (int j = threadIdx.x; j < C; j += blockDim.x) out[row * C + j] = 0.f;
    if (bad && threadIdx.x == 0) atomicOr(bad, 1);
    return;
  }
  for (int j = threadIdx.x; j < C; j += blockDim.x) {
    float e;
    if constexpr (F16)
      e = half_bits_to_float(reinterpret_cast<const uint16_t*>(wte)[id * C + j]);
    else
      e = reinterpret_cast<const float*>(wte)[id * C + j];
    float v = e * scale;
    if (wpe) v += wpe[(int64_t)s * C + j];
    out[row * C + j] = v;
  }
}

__global__ void add_kernel(float* a, const float* b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    a[i] += b[i];
}

// ---- fp16 <-> fp32 -----------------------------------------------------------
// 8 halves (16 B) in, 8 floats (32 B) out per chunk; each thread issues the
// loads of four grid-strided chunks before converting and storing them, so
// four 16-byte reads per thread are in flight at once.
__global__ void dequant_f16_kernel(const uint16_t* __restrict__ src,
                                   float* __restrict__ dst, int64_t n) {
  constexpr int U = 4;
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  float4* d4 = reinterpret_cast<float4*>(dst);
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < nvec; i0 += U * stride) {
    uint4 u[U];
#pragma unroll
    for (int j = 0; j < U; ++j)
      if (i0 + j * stride < nvec) u[j] = s4[i0 + j * stride];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t i = i0 + j * stride;
      if (i >= nvec) break;
      float4 a, b;
      a.x = half_bits_to_float(u[j].x & 0xffff); a.y = half_bits_to_float(u[j].x >> 16);
      a.z = half_bits_to_float(u[j].y & 0xffff); a.w = half_bits_to_float(u[j].y >> 16);
      b.x = half_bits_to_float(u[j].z & 0xffff); b.y = half_bits_to_float(u[j].z >> 16);
      b.z = half_bits_to_float(u[j].w & 0xffff); b.w = half_bits_to_float(u[j].w >> 16);
      d4[2 * i] = a;
      d4[2 * i + 1] = b;
    }
  }
  for (int64_t i = nvec * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = half_bits_to_float(src[i]);
}

__global__ void dequant_f16_scalar_kernel(const uint16_t* __restrict__ src,
                                          float* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = half_bits_to_float(src[i]);
}

__global__ void quant_f16_kernel(const float* __restrict__ src,
                                 uint16_t* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = float_to_half_bits(src[i]);
}

// ---- Adam / grad norm ------------------------------------------------------------
__global__ void adam_kernel(float* __restrict__ p, float* __restrict__ g,
                            float* __restrict__ m, float* __restrict__ v,
                            int64_t n, float lr, float b1, float b2, float eps,
                            float wd, double bc1, double bc2,
                            const float* __restrict__ clip_scale, int zero_grad) {
  const float cs = clip_scale ? *clip_scale : 1.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gi = g[i] * cs;
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const double mh = mi / bc1, vh = vi / bc2;
    double pi = p[i];
    if (wd != 0.f) pi -= (double)lr * wd * pi;
    pi -= (double)lr * mh / (sqrt(vh) + eps);
    p[i] = (float)pi;
    if (zero_grad) g[i] = 0.f;
  }
}

// Same update with the hyper-parameters and the 1-based step count read
// from device memory (hp = {lr, b1, b2, eps, wd, max_norm}), so a captured
// step graph can be replayed with a new learning rate and step.  The clip
// factor comes from Σg² (ss) in every thread: max_norm/(norm + 1e-6) when
// norm > max_norm > 0, else 1; thread 0 also stores it and the clipped norm
// (out[0], out[1]).
__global__ void adam_dev_kernel(float* __restrict__ p, float* __restrict__ g,
                                float* __restrict__ m, float* __restrict__ v, int64_t n,
                                const float* __restrict__ hp, const int* __restrict__ tstep,
                                const double* __restrict__ ss, float* __restrict__ out, int zero_grad) {
  const float lr = hp[0], b1 = hp[1], b2 = hp[2], eps = hp[3], wd = hp[4], max_norm = hp[5];
  const int t = *tstep;
  const double bc1 = 1.0 - pow((double)b1, (double)t);
  const double bc2 = 1.0 - pow((double)b2, (double)t);
  float nv = (float)sqrt(*ss);
  float cs = 1.f;
  if (max_norm > 0.f && nv > max_norm) {
    cs = max_norm / (nv + 1e-6f);
    nv = max_norm;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = cs;
    out[1] = nv;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gi = g[i] * cs;
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const double mh = mi / bc1, vh = vi / bc2;
    double pi = p[i];
    if (wd != 0.f) pi -= (double)lr * wd * pi;
    pi -= (double)lr * mh / (sqrt(vh) + eps);
    p[i] = (float)pi;
    if (zero_grad) g[i] = 0.f;
  }
}

// Start of a device-side optimizer step: hp = {lr, b1, b2, eps, wd,
// max_norm} from the arguments (no host staging buffer for a captured graph
// to read), the step counter advanced, the Σg² accumulator cleared.
__global__ void set_hparams_kernel(float* hp, float lr, float b1, float b2, float eps, float wd,
                                   float max_norm, double* ss, int* tstep) {
  if (threadIdx.x == 0) {
    hp[0] = lr; hp[1] = b1; hp[2] = b2; hp[3] = eps; hp[4] = wd; hp[5] = max_norm;
    *ss = 0.0;
    *tstep += 1;
  }
}

__global__ void add_out_kernel(float* __restrict__ out, const float* __restrict__ a,
                               const float* __restrict__ b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ g,
                                                    int64_t n, double* out) {
  __shared__ double red[4];
  double s = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const double x = g[i];
    s += x * x;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(out, red[0] + red[1] + red[2] + red[3]);
}

__global__ __launch_bounds__(256) void opt_partials_kernel(const float* __restrict__ g, int64_t n,
                                                           double* __restrict__ partials, HpArgs a, int write_hp,
                                                           float* __restrict__ hp, int* __restrict__ tstep) {
  __shared__ double red[4];
  if (write_hp && blockIdx.x == 0 && threadIdx.x == 0) {
    hp[0] = a.lr; hp[1] = a.b1; hp[2] = a.b2; hp[3] = a.eps; hp[4] = a.wd; hp[5] = a.max_norm;
    *tstep += 1;
  }
  double s = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const double x = g[i];
    s += x * x;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// Adam with the clip factor from kOptBlocks Σg² partials, summed by every
// workgroup in the same order (one per thread, then a fixed tree).
__global__ __launch_bounds__(256) void adam_partials_kernel(float* __restrict__ p, float* __restrict__ g,
                                                            float* __restrict__ m, float* __restrict__ v, int64_t n,
                                                            const float* __restrict__ hp,
                                                            const int* __restrict__ tstep,
                                                            const double* __restrict__ partials,
                                                            float* __restrict__ out, int zero_grad) {
  static_assert(kOptBlocks == 256, "one partial per thread");
  __shared__ double red[4];
  double ps = partials[threadIdx.x];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ps;
  __syncthreads();
  const double ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float lr = hp[0], b1 = hp[1], b2 = hp[2], eps = hp[3], wd = hp[4], max_norm = hp[5];
  const int t = *tstep;
  const double bc1 = 1.0 - pow((double)b1, (double)t);
  const double bc2 = 1.0 - pow((double)b2, (double)t);
  float nv = (float)sqrt(ss);
  float cs = 1.f;
  if (max_norm > 0.f && nv > max_norm) {
    cs = max_norm / (nv + 1e-6f);
    nv = max_norm;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = cs;
    out[1] = nv;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float gi = g[i] * cs;
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const double mh = mi / bc1, vh = vi / bc2;
    double pi = p[i];
    if (wd != 0.f) pi -= (double)lr * wd * pi;
    pi -= (double)lr * mh / (sqrt(vh) + eps);
    p[i] = (float)pi;
    if (zero_grad) g[i] = 0.f;
  }
}

__global__ void clip_kernel(const double* ss, float max_norm, float* scale,
                            float* norm) {
  float nv = (float)sqrt(*ss);
  float sc = 1.f;
  if (max_norm > 0.f && nv > max_norm) {
    sc = max_norm / (nv + 1e-6f);
    nv = max_norm;
  }
  if (scale) *scale = sc;
  if (norm) *norm = nv;
}

// ---- deterministic initialisers (splitmix64 counter hash + Box-Muller) ------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float normal_at(uint64_t seed, int64_t i) {
  const uint64_t a = splitmix64(seed ^ splitmix64((uint64_t)i * 2 + 1));
  const uint64_t b = splitmix64(a);
  const double u1 = ((a >> 11) + 1) * (1.0 / 9007199254740993.0);  // (0,1]
  const double u2 = (b >> 11) * (1.0 / 9007199254740992.0);        // [0,1)
  return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

__global__ void fill_normal_kernel(float* p, int64_t n, uint64_t seed, float std,
                                   float mean) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = mean + std * normal_at(seed, i);
}
__global__ void fill_normal_f16_kernel(uint16_t* p, int64_t n, uint64_t seed,
                                       float std) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = float_to_half_bits(std * normal_at(seed, i));
}
__global__ void fill_const_kernel(float* p, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}
__global__ void scale_kernel(const float* x, int64_t n, float a, float* y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = a * x[i];
}
__global__ void axpy_kernel(float a, const float* x, float* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = fmaf(a, x[i], y[i]);
}
__global__ void fill_uniform_int_kernel(int32_t* p, int64_t n, uint64_t seed,
                                        int32_t hi) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = (int32_t)(splitmix64(seed ^ splitmix64((uint64_t)i)) % (uint64_t)hi);
}

// One workgroup per per_block work items up to `cap` workgroups (the
// kernels are grid-stride loops, so any grid is correct): one item per
// thread keeps the most loads in flight; a capped grid that loops measured
// 20% below the copy rate on the HBM-bound kernels.
// ---- layout ops of the operators API (off the training hot path) ---------------
// dst (contiguous, row-major in `shape`) = src read at Σ_d coord_d·stride_d
// (strides in elements; 0 repeats a dimension).  Covers permute, transpose,
// repeat_kv_heads and contiguous copies of views.
struct StridedShape {
  int ndim;
  int64_t shape[kMaxCopyDims];
  int64_t stride[kMaxCopyDims];
};
__global__ void strided_copy_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n,
                                    StridedShape sh) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, off = 0;
    for (int d = sh.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % sh.shape[d];
      rem /= sh.shape[d];
      off += c * sh.stride[d];
    }
    dst[i] = src[off];
  }
}

// C[b] = A[b]·B[b] for row-major A [M,K], B [K,N], C [M,N] per batch entry
// (batch strides M·K, K·N, M·N): 16×16 output tiles through LDS, fp32 FMA
// (debug and analysis products; the training GEMMs use the MFMA kernels).
__global__ __launch_bounds__(256) void batched_matmul_kernel(const float* __restrict__ A,
                                                             const float* __restrict__ B, float* __restrict__ C,
                                                             int M, int K, int N) {
  __shared__ float As[16][17], Bs[16][17];
  const int b = blockIdx.z;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
  const float* a = A + (int64_t)b * M * K;
  const float* bb = B + (int64_t)b * K * N;
  float acc = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    As[ty][tx] = row < M && k0 + tx < K ? a[(int64_t)row * K + k0 + tx] : 0.f;
    Bs[ty][tx] = k0 + ty < K && col < N ? bb[(int64_t)(k0 + ty) * N + col] : 0.f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = fmaf(As[ty][k], Bs[k][tx], acc);
    __syncthreads();
  }
  if (row < M && col < N) C[(int64_t)b * M * N + (int64_t)row * N + col] = acc;
}

inline unsigned grid_for(int64_t n, int per_block = 256, int64_t cap = 1 << 20) {
  int64_t g = cdiv(n, per_block);
  if (g < 1) g = 1;
  return (unsigned)(g > cap ? cap : g);
}

}  // namespace

// Row-loop versions for shapes the vectorised kernels (norms.hip) do not
// take: C not a multiple of 4, unaligned rows, or C > 4096.
void layernorm_fwd_rowloop(hipStream_t s, const float* x, const float* g,
                           const float* b, int64_t M, int64_t C, float eps, float* y,
                           float* mean, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  hipLaunchKernelGGL(layernorm_fwd_kernel, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s,
                     x, g, b, M, (int)C, eps, y, mean, rstd);
  MFT_LAUNCH_CHECK();
}
void layernorm_bwd_rowloop(hipStream_t s, const float* dy, const float* x,
                           const float* g, const float* mean, const float* rstd,
                           int64_t M, int64_t C, float* dx, const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  hipLaunchKernelGGL(layernorm_bwd_kernel, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s,
                     dy, x, g, mean, rstd, M, (int)C, dx, resid);
  MFT_LAUNCH_CHECK();
}
void rmsnorm_fwd_rowloop(hipStream_t s, const float* x, const float* w, int64_t M,
                         int64_t C, float eps, bool unit_offset, float* y, float* rstd) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s,
                     x, w, M, (int)C, eps, unit_offset ? 1 : 0, y, rstd);
  MFT_LAUNCH_CHECK();
}
void rmsnorm_bwd_rowloop(hipStream_t s, const float* dy, const float* x,
                         const float* w, const float* rstd, int64_t M, int64_t C,
                         bool unit_offset, float* dx, const float* resid) {
  MFT_CHECK_ARG(M > 0 && C > 0, "empty");
  hipLaunchKernelGGL(rmsnorm_bwd_kernel, dim3((unsigned)cdiv(M, 4)), dim3(256), 0, s,
                     dy, x, w, rstd, M, (int)C, unit_offset ? 1 : 0, dx, resid);
  MFT_LAUNCH_CHECK();
}
void glu_fwd(hipStream_t s, const float* gate, const float* up, int64_t n,
             int act, float* out) {
  glu_fwd_rows(s, gate, up, 1, n, n, act, out);
}
void glu_bwd(hipStream_t s, const float* dout, const float* gate,
             const float* up, int64_t n, int act, float* dgate, float* dup) {
  glu_bwd_rows(s, dout, gate, up, 1, n, n, act, dgate, dup);
}
// The 128-bit GLU kernels' preconditions (null operands pass).
static bool glu_vec_ok(int64_t n, int64_t cols, int64_t ld_gu, std::initializer_list<const void*> ptrs) {
  if (cols % 4 != 0 || ld_gu % 4 != 0 || n / 4 >= ((int64_t)1 << 31)) return false;
  for (const void* p : ptrs)
    if (((uintptr_t)p & 15) != 0) return false;
  return true;
}

void glu_fwd_rows(hipStream_t s, const float* gate, const float* up, int64_t rows, int64_t cols, int64_t ld_gu,
                  int act, float* out) {
  const int64_t n = rows * cols;
  if (n <= 0) return;
  MFT_CHECK_ARG(ld_gu >= cols, "glu: gate/up row pitch below the row length");
  if (glu_vec_ok(n, cols, ld_gu, {gate, up, out})) {
    const unsigned nq = (unsigned)(n / 4);
    hipLaunchKernelGGL(glu_fwd_vec, dim3(cdiv(nq, 256)), dim3(256), 0, s, reinterpret_cast<const glux4*>(gate),
                       reinterpret_cast<const glux4*>(up), nq, (unsigned)(cols / 4), (unsigned)(ld_gu / 4), act,
                       reinterpret_cast<glux4*>(out));
    MFT_LAUNCH_CHECK();
    return;
  }
  hipLaunchKernelGGL(glu_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, s, gate, up, n, cols, ld_gu, act, out);
  MFT_LAUNCH_CHECK();
}
void glu_bwd_rows(hipStream_t s, const float* dout, const float* gate, const float* up, int64_t rows,
                  int64_t cols, int64_t ld_gu, int act, float* dgate, float* dup) {
  const int64_t n = rows * cols;
  if (n <= 0) return;
  MFT_CHECK_ARG(ld_gu >= cols, "glu: gate/up row pitch below the row length");
  if (glu_vec_ok(n, cols, ld_gu, {dout, gate, up, dgate, dup})) {
    const unsigned nq = (unsigned)(n / 4);
    hipLaunchKernelGGL(glu_bwd_vec, dim3(cdiv(nq, 256)), dim3(256), 0, s, reinterpret_cast<const glux4*>(dout),
                       reinterpret_cast<const glux4*>(gate), reinterpret_cast<const glux4*>(up), nq,
                       (unsigned)(cols / 4), (unsigned)(ld_gu / 4), act, reinterpret_cast<glux4*>(dgate),
                       reinterpret_cast<glux4*>(dup));
    MFT_LAUNCH_CHECK();
    return;
  }
  hipLaunchKernelGGL(glu_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, s, dout, gate, up, n, cols, ld_gu, act, dgate,
                     dup);
  MFT_LAUNCH_CHECK();
}
void rope(hipStream_t s, float* x, int64_t rs, int B, int S, int H, int hd,
          double theta, bool inverse) {
  MFT_CHECK_ARG(hd % 2 == 0, "head_dim must be even");
  const int64_t n = (int64_t)B * S * H * (hd / 2);
  if (n <= 0) return;
  hipLaunchKernelGGL(rope_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, rs, B, S, H, hd, theta,
                     inverse ? 1 : 0);
  MFT_LAUNCH_CHECK();
}
void embed(hipStream_t s, const int32_t* ids, int64_t M, int S,
           const void* wte, int64_t V, bool w_f16, const float* wpe, int64_t C,
           float scale, float* out, int* bad) {
  MFT_CHECK_ARG(M > 0 && C > 0 && S > 0 && V > 0, "empty");
  if (w_f16)
    hipLaunchKernelGGL(embed_kernel<true>, dim3((unsigned)M), dim3(256), 0, s, ids, M, S, wte, V, wpe, (int)C, scale,
                       out, bad);
  else
    hipLaunchKernelGGL(embed_kernel<false>, dim3((unsigned)M), dim3(256), 0, s, ids, M, S, wte, V, wpe, (int)C, scale,
                       out, bad);
  MFT_LAUNCH_CHECK();
}
void add_inplace(hipStream_t s, float* a, const float* b, int64_t n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, b, n);
  MFT_LAUNCH_CHECK();
}
void dequant_f16(hipStream_t s, const uint16_t* src, float* dst, int64_t n) {
  if (n <= 0) return;
  const bool aligned = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
  if (aligned)
    hipLaunchKernelGGL(dequant_f16_kernel, dim3(grid_for(cdiv(n, 8))), dim3(256), 0, s, src, dst, n);
  else
    hipLaunchKernelGGL(dequant_f16_scalar_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n);
  MFT_LAUNCH_CHECK();
}
void quant_f16(hipStream_t s, const float* src, uint16_t* dst, int64_t n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(quant_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n);
  MFT_LAUNCH_CHECK();
}
void adam_step(hipStream_t s, float* p, float* g, float* m, float* v,
               int64_t n, float lr, float b1, float b2, float eps, float wd,
               int t, const float* clip_scale, bool zero_grad) {
  MFT_CHECK_ARG(t >= 1, "Adam step count is 1-based");
  if (n <= 0) return;
  const double bc1 = 1.0 - std::pow((double)b1, t);
  const double bc2 = 1.0 - std::pow((double)b2, t);
  hipLaunchKernelGGL(adam_kernel, dim3(grid_for(n, 256, 2048)), dim3(256), 0, s, p, g, m, v, n, lr, b1,
                     b2, eps, wd, bc1, bc2, clip_scale, zero_grad ? 1 : 0);
  MFT_LAUNCH_CHECK();
}
void adam_step_dev(hipStream_t s, float* p, float* g, float* m, float* v, int64_t n,
                   const float* hp, const int* tstep, const double* ss, float* clip_out, bool zero_grad) {
  if (n <= 0) return;
  hipLaunchKernelGGL(adam_dev_kernel, dim3(grid_for(n, 256, 2048)), dim3(256), 0, s, p, g, m, v, n, hp,
                     tstep, ss, clip_out, zero_grad ? 1 : 0);
  MFT_LAUNCH_CHECK();
}
void set_hparams(hipStream_t s, float* hp, float lr, float b1, float b2, float eps, float wd,
                 float max_norm, double* ss, int* tstep) {
  hipLaunchKernelGGL(set_hparams_kernel, dim3(1), dim3(64), 0, s, hp, lr, b1, b2, eps, wd, max_norm, ss, tstep);
  MFT_LAUNCH_CHECK();
}
void add_out(hipStream_t s, float* out, const float* a, const float* b, int64_t n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_out_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, a, b, n);
  MFT_LAUNCH_CHECK();
}
void sumsq(hipStream_t s, const float* g, int64_t n, double* out) {
  if (n <= 0) return;
  hipLaunchKernelGGL(sumsq_kernel, dim3(grid_for(n, 256, 1024)), dim3(256), 0, s, g, n, out);
  MFT_LAUNCH_CHECK();
}
void opt_partials(hipStream_t s, const float* g, int64_t n, double* partials, const HpArgs* hp_args, float* hp,
                  int* tstep) {
  const HpArgs a = hp_args ? *hp_args : HpArgs{};
  hipLaunchKernelGGL(opt_partials_kernel, dim3(kOptBlocks), dim3(256), 0, s, g, n, partials, a, hp_args ? 1 : 0, hp,
                     tstep);
  MFT_LAUNCH_CHECK();
}
void adam_partials(hipStream_t s, float* p, float* g, float* m, float* v, int64_t n, const float* hp,
                   const int* tstep, const double* partials, float* clip_out, bool zero_grad) {
  if (n <= 0) return;
  hipLaunchKernelGGL(adam_partials_kernel, dim3(grid_for(n, 256, 2048)), dim3(256), 0, s, p, g, m, v, n, hp, tstep,
                     partials, clip_out, zero_grad ? 1 : 0);
  MFT_LAUNCH_CHECK();
}
void clip_scale(hipStream_t s, const double* ss, float max_norm, float* scale,
                float* norm) {
  hipLaunchKernelGGL(clip_kernel, dim3(1), dim3(1), 0, s, ss, max_norm, scale, norm);
  MFT_LAUNCH_CHECK();
}
void fill_normal(hipStream_t s, float* p, int64_t n, uint64_t seed, float std,
                 float mean) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, seed, std, mean);
  MFT_LAUNCH_CHECK();
}
void fill_normal_f16(hipStream_t s, uint16_t* p, int64_t n, uint64_t seed,
                     float std) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_normal_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, seed, std);
  MFT_LAUNCH_CHECK();
}
void fill_const(hipStream_t s, float* p, int64_t n, float v) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_const_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, v);
  MFT_LAUNCH_CHECK();
}
void scale(hipStream_t s, const float* x, int64_t n, float a, float* y) {
  if (n <= 0) return;
  hipLaunchKernelGGL(scale_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, n, a, y);
  MFT_LAUNCH_CHECK();
}
void axpy(hipStream_t s, float a, const float* x, float* y, int64_t n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(axpy_kernel, dim3(grid_for(n)), dim3(256), 0, s, a, x, y, n);
  MFT_LAUNCH_CHECK();
}
void fill_uniform_int(hipStream_t s, int32_t* p, int64_t n, uint64_t seed,
                      int32_t hi) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_uniform_int_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, seed, hi);
  MFT_LAUNCH_CHECK();
}

void strided_copy(hipStream_t s, const float* src, float* dst, int ndim, const int64_t* shape,
                  const int64_t* stride) {
  MFT_CHECK_ARG(ndim >= 1 && ndim <= kMaxCopyDims, "1 to 8 dimensions");
  StridedShape sh{};
  sh.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    MFT_CHECK_ARG(shape[d] >= 0 && stride[d] >= 0, "negative shape or stride");
    sh.shape[d] = shape[d];
    sh.stride[d] = stride[d];
    n *= shape[d];
  }
  if (n == 0) return;
  hipLaunchKernelGGL(strided_copy_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n, sh);
  MFT_LAUNCH_CHECK();
}
void batched_matmul(hipStream_t s, const float* A, const float* B, float* C, int batch, int M, int K, int N) {
  MFT_CHECK_ARG(batch > 0 && M > 0 && K > 0 && N > 0, "empty matmul");
  const dim3 grid((unsigned)cdiv(N, 16), (unsigned)cdiv(M, 16), (unsigned)batch);
  hipLaunchKernelGGL(batched_matmul_kernel, grid, dim3(256), 0, s, A, B, C, M, K, N);
  MFT_LAUNCH_CHECK();
}

}  // namespace mft
