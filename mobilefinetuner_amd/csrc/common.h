// common.h — shared plumbing for the gfx950 kernel library.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "mft_hip.h"

struct mft_handle_s {
  hipStream_t stream = nullptr;
  int device = 0;
  int num_cu = 256;
};

namespace mft {

// Thrown inside the library, converted to a status code at the C-ABI.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);

#define MFT_CHECK_ARG(cond, msg)                                            \
  do {                                                                      \
    if (!(cond)) throw ::mft::Error(MFT_EINVAL, std::string(__func__) + ": " + (msg)); \
  } while (0)

#define MFT_HIP(call)                                                       \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess)                                                   \
      throw ::mft::Error(MFT_EHIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

// Kernel launch error check (catches invalid launch configurations).  In
// sync-check mode (mft_set_sync_check, or MFT_SYNC_CHECK=1 in the
// environment) every check also waits for the library's streams and reports
// an execution error with the launch site that precedes it — except while
// one of them is being captured into a graph, where waiting would break the
// capture.
extern int g_sync_check;
void sync_check(const char* file, int line);
// Streams the sync check waits for (every stream the library launches on).
void register_stream(hipStream_t s);
void unregister_stream(hipStream_t s);
#define MFT_LAUNCH_CHECK()                                   \
  do {                                                       \
    MFT_HIP(hipGetLastError());                              \
    if (::mft::g_sync_check) ::mft::sync_check(__FILE__, __LINE__); \
  } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// GELU, tanh approximation (GPT-2's gelu_new), and its derivative.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.f + tanhf(c * fmaf(0.044715f * x, x * x, x)));
}
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float c = 0.7978845608028654f;
  const float t = tanhf(c * fmaf(0.044715f * x, x * x, x));
  const float du = c * fmaf(3.f * 0.044715f, x * x, 1.f);
  return 0.5f * (1.f + t) + 0.5f * x * (1.f - t * t) * du;
}

// IEEE fp16 bits → fp32 (exact), one value and four packed in a uint2.
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float __attribute__((ext_vector_type(4))) widen4(uint2 u) {
  return {half_bits_to_float(u.x & 0xffff), half_bits_to_float(u.x >> 16), half_bits_to_float(u.y & 0xffff),
          half_bits_to_float(u.y >> 16)};
}
// fp16 operand staging in the GEMMs: the raw 64 bits ride in lanes 0–1 of a
// float4 register set from the global load until the LDS store, which
// widens them; widening at the load would make the wave wait for the load
// right after issuing it and lose the prefetch distance.
__device__ __forceinline__ float __attribute__((ext_vector_type(4))) stash_f16(uint2 u) {
  return {__uint_as_float(u.x), __uint_as_float(u.y), 0.f, 0.f};
}
__device__ __forceinline__ float __attribute__((ext_vector_type(4))) unstash_f16(
    float __attribute__((ext_vector_type(4))) v) {
  return widen4(uint2{__float_as_uint(v[0]), __float_as_uint(v[1])});
}

// Raw buffer resource over [base, base + 4 GiB): a load takes a 32-bit
// per-lane byte offset (one VGPR) plus a wave-uniform offset (an SGPR)
// instead of a 64-bit address pair and its 64-bit arithmetic — on the
// operand loads of the GEMM and attention loops that issue cost showed as
// matrix-core idle time.  No range checking is relied on: every offset the
// kernels form stays inside its operand.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ float __attribute__((ext_vector_type(4))) buf_load4(__amdgpu_buffer_rsrc_t r,
                                                                              uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float __attribute__((ext_vector_type(4))),
                            __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint2 buf_load2u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

// ---- launchers shared by the C-ABI and the step engine ----------------------
// A row norm applied to the finished rows of a GEMM output C[M,N] (N = the
// normalised width, ldc = N):
//   NORM_LN_FWD:  y = LayerNorm(C row)·w + b, mean and rstd stored;
//   NORM_RMS_FWD: y = C row · rstd · (w + unit_offset), rstd stored;
//   NORM_LN_BWD / NORM_RMS_BWD: C is the gradient of the norm's output for
//     input rows x (with the stored mean / rstd); y = resid + ∂x (resid may
//     be null or alias y).  skip_c: C itself is not needed afterwards.
//   NORM_RMS_RES_RMS (Gemma3's sandwich: post-norm, residual add, the next
//     pre-norm): y = resid + C row · rstd · (w + unit_offset), rstd stored;
//     y2 = y · rstd2 · (w2 + unit_offset), rstd2 stored.
//   NORM_RMS_BWD_POST (its backward): y as NORM_RMS_BWD, then y2 = the
//     gradient of the post-norm's input for its input rows x2 (w2, stored
//     rstd2) given output gradient y.
// With split-K the reduction, the epilogue and the norm run as one pass
// (the row is finished in registers); otherwise the norm runs after the GEMM.
enum { NORM_NONE = 0, NORM_LN_FWD, NORM_RMS_FWD, NORM_LN_BWD, NORM_RMS_BWD, NORM_RMS_RES_RMS, NORM_RMS_BWD_POST };
struct RowNorm {
  int kind = NORM_NONE;
  const float* w = nullptr;
  const float* b = nullptr;
  float eps = 0.f;
  int unit_offset = 0;
  float* y = nullptr;
  float* mean = nullptr;  // LN forward: written; LN backward: read
  float* rstd = nullptr;  // forward: written; backward: read
  const float* x = nullptr;
  const float* resid = nullptr;
  bool skip_c = false;
  const float* w2 = nullptr;  // NORM_RMS_RES_RMS / NORM_RMS_BWD_POST: the second norm
  float* y2 = nullptr;
  float* rstd2 = nullptr;
  const float* x2 = nullptr;  // NORM_RMS_BWD_POST: the second norm's input rows
};

struct GemmEpilogue {
  const float* bias = nullptr;   // [N]
  const float* resid = nullptr;  // [M,N] row stride ldc; may alias C
  float beta = 0.f;              // C = ... + beta * C_old
  // rank-r update: C += lscale * P[M,r] · Q,  Q(n,j) = Q[n*qsn + j*qsj]
  const float* P = nullptr;
  const float* Q = nullptr;
  int r = 0;
  int64_t qsn = 0, qsj = 0;
  float lscale = 0.f;
  // GELU (tanh form) fused into the output, for GPT-2's MLP:
  //   gelu_out:     C keeps the pre-activation v, gelu_out[m·ldc + n] = gelu(v);
  //   gelu_grad_of: C = v · gelu'(gelu_grad_of[m·ldc + n]), i.e. the gradient
  //                 of the activation's input from that of its output.
  float* gelu_out = nullptr;
  const float* gelu_grad_of = nullptr;
  // Call site: 0 = a layer's linear GEMM, 1 = the LM head.  Selects a
  // separately named (otherwise identical) kernel instantiation so kernel
  // traces and counter profiles attribute the two apart.
  int site = 0;
  // LM head (128×128 plan only): per row and 64-column block of C, the
  // base-2 softmax statistics (max of C·log2e, Σ 2^(C·log2e − max)) of the
  // stored values, at stats[row·stats_ld + n/64]; the cross-entropy then
  // reads the logits once.
  float2* stats = nullptr;
  int64_t stats_ld = 0;
  // Host-side only: row norm of the finished output (never read by kernels).
  const RowNorm* norm = nullptr;
};
// Row scales of an fp32 operand x [M,K] for the fp16 matrix-core GEMM:
// inv_s[m] = 2^(⌊log2 max|x_m|⌋ − 14) (1 for a zero or non-finite maximum;
// at most 2^126 below), so that x_m/inv_s[m] splits into two fp16 values per
// element without leaving fp16's range.
__device__ __forceinline__ float row_inv_scale(float mx) {
  int e = 0;
  if (mx > 0.f && mx <= 3.402823466e38f) e = min(14 - ilogbf(mx), 126);  // ilogb ≤ 127: e ≥ −113
  return __int_as_float((127 - e) << 23);
}
void row_scales(hipStream_t s, const float* x, int64_t ldx, int M, int K, float* inv_s);
// Shapes gemm_h takes (K in whole 32-deep panels; 8-wide column chunks of a [K,N] B).
bool gemm_h_ok(int N, int K, bool b_nk, int r);
// Whether gemm() runs an M×N×K product (the LM head's logits) on the
// 128×128 kernel, the one that can emit row statistics.
bool gemm_wide_plan(int M, int N);

// Device scratch handed to launchers (split-K partials, rank-r temporaries).
struct Scratch {
  float* ptr = nullptr;
  size_t bytes = 0;
  Scratch offset(size_t nfloats) const {
    Scratch s;
    if (ptr && nfloats * sizeof(float) <= bytes) {
      s.ptr = ptr + nfloats;
      s.bytes = bytes - nfloats * sizeof(float);
    }
    return s;
  }
};

// Optional events for live per-kernel timing of a GEMM: start/stop bracket
// the main GEMM kernel; tail_start/tail_stop bracket the split-K reduction
// (with its fused epilogue and row norm) when the plan splits K, and the
// GEMM then sets tail_used.  The GEMM's time is (start→stop) plus
// (tail_start→tail_stop) when tail_used.
struct KernelEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  hipEvent_t tail_start = nullptr, tail_stop = nullptr;
  mutable bool tail_used = false;
};
// Set by gemm() around the launch of its split-K reduction: the reduction
// launchers (splitk_reduce in gemm.hip, splitk_norm_vec in norms.hip) pass
// these events to the dispatch (hipExtLaunchKernel) when non-null.
extern thread_local hipEvent_t t_tail_start, t_tail_stop;
#define MFT_LAUNCH_TAIL(KERNEL, GRID, BLOCK, SHMEM, STREAM, ...)                                   \
  do {                                                                                             \
    if (::mft::t_tail_start)                                                                       \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, ::mft::t_tail_start,               \
                            ::mft::t_tail_stop, 0, __VA_ARGS__);                                   \
    else                                                                                           \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, __VA_ARGS__);                         \
  } while (0)

// C[M,N] = A[M,K] · op(B) (+ epilogue).  b_nk=false: B is [K,N] (ldb = row
// stride); b_nk=true: B is [N,K].  b_f16: B holds IEEE fp16 values.
void gemm(hipStream_t s, const float* A, int64_t lda, const void* B,
          int64_t ldb, bool b_nk, bool b_f16, float* C, int64_t ldc, int M,
          int N, int K, const GemmEpilogue& ep, Scratch ws = Scratch(),
          const KernelEvents* ev = nullptr);
// C[M,N] = A·op(B) (+ epilogue, as gemm()) on the fp16 matrix cores: A fp32
// with its row scales (row_scales; null: rows used unscaled), split into two
// fp16 values per element in the tile load; B fp16 [N,K] (b_nk) or [K,N].
void gemm_h(hipStream_t s, const float* A, int64_t lda, const float* inv_s, const uint16_t* B, int64_t ldb, bool b_nk,
            float* C, int64_t ldc, int M, int N, int K, const GemmEpilogue& ep, Scratch ws = Scratch(),
            const KernelEvents* ev = nullptr);
// Column-segmented gemm_h: one launch computes C_g = A·op(B_g) (+ the
// rank-r panel lscale·P_g·Q_g) for every segment g over the shared fp32 input
// A — the q, k and v (or gate and up) projections of one input.  The
// epilogue's r / qsn / qsj / lscale apply to every segment; no bias,
// residual, beta, GELU, norm or statistics; K is not split.  Returns false
// (nothing launched) when the segments' widths do not fit a tile plan.
struct GemmHSegmentArg {
  const uint16_t* B;
  int64_t ldb;
  int N;
  float* C;
  int64_t ldc;
  const float* P;
  const float* Q;
};
bool gemm_h_segments(hipStream_t s, const float* A, int64_t lda, const float* inv_s, bool b_nk,
                     const GemmHSegmentArg* seg, int nseg, int M, int K, const GemmEpilogue& ep,
                     const KernelEvents* ev = nullptr);
// K-segmented gemm_h over [N,K] B: C = Σ_g A[:, k0_g : k0_g + K_g]·B_gᵀ
// (+ Σ_g lscale·P_g·Q_g, ep.r per segment), with A's column blocks scaled by
// the largest of the segments' row scales — the dX of the q, k and v (or gate
// and up) projections, their dY side by side in A.  The epilogue, split-K and
// a row norm as in gemm_h.  Segments' K in whole 32-deep panels; nseg·r ≤ 32.
struct GemmHKSegmentArg {
  const uint16_t* B;  // fp16 [N][ldb]
  int64_t ldb;
  int K;
  const float* inv_s;  // row scales of A's column block
  const float* P;
  const float* Q;
};
void gemm_h_ksegments(hipStream_t s, const float* A, int64_t lda, const GemmHKSegmentArg* seg, int nseg, float* C,
                      int64_t ldc, int M, int N, const GemmEpilogue& ep, Scratch ws,
                      const KernelEvents* ev = nullptr);
// C = x·op(W) for fp16 W: row_scales into the front of ws, then gemm_h.
// Returns false (nothing launched) when the shape, alignment or workspace
// does not fit; the caller then runs gemm() with W widened.
bool gemm_f16w(hipStream_t s, const float* x, int64_t ldx, const void* W, int64_t ldw, bool b_nk, float* C,
               int64_t ldc, int M, int N, int K, const GemmEpilogue& ep, Scratch ws, const KernelEvents* ev = nullptr);
// out[M,r] = X[M,K] · Y with Y(k,j) = Y[k*ysk + j*ysj]
void rank_proj(hipStream_t s, const float* X, int64_t ldx, const float* Y,
               int64_t ysk, int64_t ysj, int M, int K, int r, float* out);
// out(j,c) (+)= scale · Σ_m P[m,j] X[m,c];  out(j,c) = out[j*osj + c*osc]
void rank_outer(hipStream_t s, const float* P, const float* X, int64_t ldx,
                int M, int C, int r, float scale, float* out, int64_t osj,
                int64_t osc, bool accumulate, Scratch ws);
// Two rank_outer products with the same M, r, scale in one launch.
void rank_outer_pair(hipStream_t s, int M, int r, float scale, bool accumulate,
                     const float* P0, const float* X0, int64_t ldx0, int C0, float* out0, int64_t osj0,
                     int64_t osc0, const float* P1, const float* X1, int64_t ldx1, int C1, float* out1,
                     int64_t osj1, int64_t osc1);

// ---- batched LoRA work of the step engine (job tables in device memory) ----
// W_eff = W + scale·Aᵀ·Bᵀ for one LoRA linear: W [K,N] fp32 or fp16 (f16 = 1),
// A [r,K], B [N,r], out [K,N] fp32.  N must be a multiple of 4.
struct MergeJob {
  const void* W;
  const float* A;
  const float* B;
  float* out;  // [K, N] rows ldo apart (ldo > N: a column block of a fused W_eff)
  int K, N, f16;
  int tile0;  // first tile of this job (tiles of merge_tiles' size: 32 rows × 256 columns)
  int ldo;
};
size_t merge_tiles(int K, int N);
// jobs: device array of njobs MergeJobs with increasing tile0; r ∈ {4, 8, 16, 32}.
void lora_merge(hipStream_t s, const MergeJob* jobs, int njobs, int total_tiles, int r, float scale);

// One rank-r product of a batched launch.
//   kind 0 (projection): out[M,r] = X[M,K]·Y, Y = A [r,K] (y_rk) or B [K,r];
//   kind 1 (outer):      out(j,c) (+)= scale·Σ_m P[m,j]·X[m,c], c < C.
// Projection jobs come first in a table and take cdiv(M, 16) workgroups
// each; outer jobs take `blocks` = rank_outer_blocks(C) workgroups (a
// multiple of 8) from `block0`, counted after the projections.
struct RankJob {
  int kind;
  int K;  // projection: K; outer: C
  int y_rk;
  int accumulate;
  int blocks, block0;
  const float* X;
  int64_t ldx;
  const float* Y;  // projection: Y; outer: P [M, r]
  float* out;
  int64_t osj, osc;
  float scale;
  float* inv_s;  // projection: when set, also the row scales of X (row_scales) for the fp16 GEMM
};
int rank_outer_blocks(int C);
// Up to three projections out[M,r] = X·Y of one launch, by value (the per-layer
// batches of the rank-r panel path); inv_s (nullable): the rows' fp16-GEMM scales.
struct ProjJob {
  const float* X;
  int64_t ldx;
  const float* Y;  // [r][K] (y_rk) or [K][r]
  int K, y_rk;
  float* out;
  float* inv_s;
};
constexpr int kMaxProjJobs = 3;
struct ProjJobs {
  ProjJob j[kMaxProjJobs];
  int n;
};
void rank_proj_jobs(hipStream_t s, const ProjJobs& jb, int M, int r);
// Runs jobs[0, njobs) (the first nproj are projections) over M rows.
void rank_batch(hipStream_t s, const RankJob* jobs, int njobs, int nproj, int outer_blocks, int M, int r);

void lora_linear_fwd(hipStream_t s, const float* x, int64_t M, int64_t K,
                     const void* W, bool w_f16, int64_t N, const float* bias,
                     const float* A, const float* B, int r, float scale,
                     float* y, float* xa, const float* resid, Scratch ws,
                     const KernelEvents* ev = nullptr);
void lora_linear_bwd(hipStream_t s, const float* dy, const float* x,
                     const void* W, bool w_f16, const float* A, const float* B,
                     const float* xa, int64_t M, int64_t K, int64_t N, int r,
                     float scale, float* dx, float* dA, float* dB,
                     bool accumulate, bool dx_accumulate, Scratch ws,
                     const KernelEvents* ev = nullptr);
// Scratch floats lora_linear_bwd needs for its rank-r temporaries.
size_t lora_bwd_scratch_floats(int64_t M, int64_t K, int64_t N, int r);
// LoRA dropout (lora.hip).  A DropStream covers n_fwd training forwards
// launched as one (rows_per_fwd rows each) whose last one is step *step.
struct DropStream {
  float p;
  uint64_t seed;
  const int* step;
  int n_fwd;
  int64_t rows_per_fwd;
};
// keep threshold on the top 24 bits of the mask hash: floor(p·2^24)
uint32_t dropout_threshold(float p);
// *step += n (n training forwards start)
void dropout_step(hipStream_t s, int* step, int n);
// xd = x∘mask of stream `lid` (x rows ldx apart, xd dense [M,K])
void dropout_apply(hipStream_t s, const float* x, int64_t ldx, int64_t M, int64_t K, const DropStream& d, int lid,
                   float* xd);
// dx += scale·(U·A)∘mask; gelu_grad_scale: x *= gelu'(pre) elementwise
void dropout_dx(hipStream_t s, float* dx, int64_t M, int64_t K, const float* U, const float* A, int r, float scale,
                const DropStream& d, int lid);
void gelu_grad_scale(hipStream_t s, float* x, const float* pre, int64_t n);

struct AttnArgs {
  const float *q, *k, *v;
  int64_t q_rs, k_rs, v_rs;
  int B, Hq, Hkv, S, hd;
  float scale;
  int causal, window;
  const float* kpad;
};
// ws: scratch of attn_fwd_scratch_floats(a) floats (0 when the launch is not
// split over keys).
void attn_fwd(hipStream_t s, const AttnArgs& a, float* o, int64_t o_rs,
              float* lse, Scratch ws);
size_t attn_fwd_scratch_floats(const AttnArgs& a);
// Upper bound of attn_fwd / attn_bwd scratch over every shape with
// B·S ≤ tokens.
size_t attn_scratch_bound_floats(int64_t tokens, int Hq, int hd);
void attn_bwd(hipStream_t s, const AttnArgs& a, const float* o, int64_t o_rs,
              const float* dout, int64_t do_rs, const float* lse, float* dq,
              int64_t dq_rs, float* dk, int64_t dk_rs, float* dv,
              int64_t dv_rs, Scratch ws);
// Scratch floats attn_bwd needs: delta rows, plus per-query-head dK/dV
// partials when heads are grouped (Hq != Hkv).
size_t attn_bwd_scratch_floats(const AttnArgs& a);

// logits rows have stride ld (>= V); dlogits (may alias logits) uses the same.
// dl_inv_s (nullable; with dlogits): per row, the row_inv_scale of a bound on
// the row's max |dlogit|, for the fp16 matrix-core GEMM that reads dlogits.
// A target is valid iff label != ignore_index and 0 <= label < V; other
// labels count as ignored, and set *bad_label (device int, nullable) to 1.
void ce_fwd_bwd(hipStream_t s, const float* logits, const int32_t* labels,
                int B, int S, int64_t V, int64_t ld, int ignore_index, float upstream,
                int64_t norm_count, double* loss_sum, int64_t* n_valid,
                float* dlogits, float* row_nll, int64_t* count_scratch, int* bad_label = nullptr,
                const float2* row_stats = nullptr, int64_t stats_ld = 0, float* dl_inv_s = nullptr);

void dequant_f16(hipStream_t s, const uint16_t* src, float* dst, int64_t n);
void quant_f16(hipStream_t s, const float* src, uint16_t* dst, int64_t n);
void adam_step(hipStream_t s, float* p, float* g, float* m, float* v,
               int64_t n, float lr, float b1, float b2, float eps, float wd,
               int t, const float* clip_scale, bool zero_grad);
// Device-parameterised variants for captured step graphs:
// hp = {lr, b1, b2, eps, wd, max_norm}; *tstep is the 1-based Adam step.
// set_hparams writes hp, advances *tstep and clears the Σg² accumulator *ss;
// adam_step_dev clips by the norm in *ss (clip factor and clipped norm to
// clip_out[0..1]) and applies Adam.
void adam_step_dev(hipStream_t s, float* p, float* g, float* m, float* v, int64_t n,
                   const float* hp, const int* tstep, const double* ss, float* clip_out, bool zero_grad);
void set_hparams(hipStream_t s, float* hp, float lr, float b1, float b2, float eps, float wd,
                 float max_norm, double* ss, int* tstep);
void add_out(hipStream_t s, float* out, const float* a, const float* b, int64_t n);
void sumsq(hipStream_t s, const float* g, int64_t n, double* out);
// The step engine's optimizer in two launches: opt_partials writes one
// Σg² partial per workgroup (kOptBlocks of them, fixed order, no atomics)
// and, given hp_args (the eager step), the hyper-parameters and the step
// count as set_hparams does; adam_partials sums the partials in a fixed
// order in every workgroup, clips and applies Adam as adam_step_dev.
constexpr int kOptBlocks = 256;
struct HpArgs {
  float lr, b1, b2, eps, wd, max_norm;
};
void opt_partials(hipStream_t s, const float* g, int64_t n, double* partials, const HpArgs* hp_args, float* hp,
                  int* tstep);
void adam_partials(hipStream_t s, float* p, float* g, float* m, float* v, int64_t n, const float* hp,
                   const int* tstep, const double* partials, float* clip_out, bool zero_grad);
void clip_scale(hipStream_t s, const double* ss, float max_norm, float* scale,
                float* norm);
void layernorm_fwd(hipStream_t s, const float* x, const float* g,
                   const float* b, int64_t M, int64_t C, float eps, float* y,
                   float* mean, float* rstd);
// dx = LayerNorm backward of dy (+ resid[M,C] when resid is not null; resid
// may alias dx for in-place accumulation).
void layernorm_bwd(hipStream_t s, const float* dy, const float* x,
                   const float* g, const float* mean, const float* rstd,
                   int64_t M, int64_t C, float* dx, const float* resid);
void rmsnorm_fwd(hipStream_t s, const float* x, const float* w, int64_t M,
                 int64_t C, float eps, bool unit_offset, float* y,
                 float* rstd);
// dx = RMSNorm backward of dy (+ resid, as layernorm_bwd).
void rmsnorm_bwd(hipStream_t s, const float* dy, const float* x,
                 const float* w, const float* rstd, int64_t M, int64_t C,
                 bool unit_offset, float* dx, const float* resid);
// The norm of nm applied to finished rows c[M,C] (one of the four launchers).
// RMSNorm over rows grouped seg per token (row r at (r/seg)·ld + (r%seg)·C):
// per-head norms reading or writing head rows of a fused q|k|v buffer.
void rmsnorm_fwd_seg(hipStream_t s, const float* x, int64_t x_ld, const float* w, int64_t M, int64_t C, int seg,
                     float eps, bool unit_offset, float* y, int64_t y_ld, float* rstd);
void rmsnorm_bwd_seg(hipStream_t s, const float* dy, int64_t dy_ld, const float* x, int64_t x_ld, const float* w,
                     const float* rstd, int64_t M, int64_t C, int seg, bool unit_offset, float* dx, int64_t dx_ld);
void row_norm(hipStream_t s, const float* c, int64_t M, int64_t C, const RowNorm& nm);
// RoPE angle table: tab[p·hd/2 + i] = (cos, sin)(p·θ^(−2i/hd)) for positions
// p < npos, computed in double and rounded to float (the values the
// per-element rope computes).
void rope_table(hipStream_t s, double theta, int hd, int npos, float2* tab);
// The head rows of q or k around attention: row r = (token t, head h) at
// t·ld + h·hd (a strided view of a fused q|k|v buffer works).  With a norm
// (w != null, Gemma3's per-head RMSNorm with the (1 + w) scale): x is the
// projection output the norm reads (forward) or its input saved for the
// backward, rstd its per-row 1/rms.
// ---- alignment-dump debug mode (debug.hip) ------------------------------------
// Dense attention scores / probabilities [B, Hq, S, S] and their gradients
// of one layer (token-major q/k/v/o/dout rows; lse from the forward); any
// output may be null, gradients need dout, v and o.
struct DebugAttn {
  const float *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *dout = nullptr, *lse = nullptr;
  const float* kpad = nullptr;
  int64_t q_rs = 0, k_rs = 0, v_rs = 0, o_rs = 0, do_rs = 0;
  int B = 0, Hq = 0, Hkv = 0, S = 0, hd = 0, causal = 1, window = 0;
  float scale = 1.f;
  float *scores = nullptr, *probs = nullptr, *dprobs = nullptr, *dscores = nullptr;
};
void debug_attn(hipStream_t s, const DebugAttn& a);
// out = a∘b and out = GELU(x) (tanh form) over rows × cols.
void debug_mul(hipStream_t s, const float* a, int64_t lda, const float* b, int64_t ldb, float* out, int64_t ldo,
               int64_t rows, int64_t cols);
void debug_gelu(hipStream_t s, const float* x, int64_t ldx, float* out, int64_t ldo, int64_t rows, int64_t cols);

struct HeadRows {
  const float* in = nullptr;
  int64_t in_ld = 0;
  float* out = nullptr;
  int64_t out_ld = 0;
  int H = 0;
  const float* w = nullptr;
  float* rstd = nullptr;
  const float* x = nullptr;
  int64_t x_ld = 0;
};
// Forward: out = RoPE(RMSNorm(in)) (RoPE(in) without a norm; out may alias
// in), q and k rows in one launch; position of token t is t mod S.
void qk_rope_fwd(hipStream_t s, const HeadRows& q, const HeadRows& k, int64_t M, int S, int hd, float eps,
                 const float2* tab, int npos);
// Backward: out = RMSNormᵀ(RoPE⁻¹(in)) (RoPE⁻¹(in) without a norm).
void qk_rope_bwd(hipStream_t s, const HeadRows& q, const HeadRows& k, int64_t M, int S, int hd,
                 const float2* tab, int npos);
// Split-K reduction (partials [splits][M][N], summed in split order) + the
// GEMM epilogue + the row norm in one pass.  Returns false, launching
// nothing, when the shape or alignment does not fit the fused kernel.
bool splitk_norm(hipStream_t s, const float* partial, int splits, int M, int N, float* C, int64_t ldc,
                 const GemmEpilogue& ep, const RowNorm& nm);
// Row-loop fallbacks of the four norm launchers (elementwise.hip).
void layernorm_fwd_rowloop(hipStream_t s, const float* x, const float* g, const float* b,
                           int64_t M, int64_t C, float eps, float* y, float* mean, float* rstd);
void layernorm_bwd_rowloop(hipStream_t s, const float* dy, const float* x, const float* g,
                           const float* mean, const float* rstd, int64_t M, int64_t C,
                           float* dx, const float* resid);
void rmsnorm_fwd_rowloop(hipStream_t s, const float* x, const float* w, int64_t M, int64_t C,
                         float eps, bool unit_offset, float* y, float* rstd);
void rmsnorm_bwd_rowloop(hipStream_t s, const float* dy, const float* x, const float* w,
                         const float* rstd, int64_t M, int64_t C, bool unit_offset, float* dx,
                         const float* resid);
void glu_fwd(hipStream_t s, const float* gate, const float* up, int64_t n,
             int act, float* out);
void glu_bwd(hipStream_t s, const float* dout, const float* gate,
             const float* up, int64_t n, int act, float* dgate, float* dup);
// The same over [rows, cols] views whose gate/up (and dgate/dup) rows are
// ld_gu apart (a fused gate|up projection: ld_gu = 2·cols); out and dout
// are [rows, cols] arrays.
void glu_fwd_rows(hipStream_t s, const float* gate, const float* up, int64_t rows, int64_t cols, int64_t ld_gu,
                  int act, float* out);
void glu_bwd_rows(hipStream_t s, const float* dout, const float* gate, const float* up, int64_t rows,
                  int64_t cols, int64_t ld_gu, int act, float* dgate, float* dup);
void rope(hipStream_t s, float* x, int64_t rs, int B, int S, int H, int hd,
          double theta, bool inverse);
// Ids outside [0, V) give zero rows and set *bad (device int, nullable).
void embed(hipStream_t s, const int32_t* ids, int64_t M, int S,
           const void* wte, int64_t V, bool w_f16, const float* wpe, int64_t C,
           float scale, float* out, int* bad);
// embed() followed by row_norm(x, nm) (LayerNorm or RMSNorm forward) in one
// launch; workgroup 0 also zeroes `zero` (nzero 8-byte words, nullable).
// Returns false, launching nothing, when the row layout does not allow it
// (C % 4, C > 4096, unaligned rows).
bool embed_norm(hipStream_t s, const int32_t* ids, int64_t M, int S, const void* wte, int64_t V, bool w_f16,
                const float* wpe, int64_t C, float scale, float* x, int* bad, const RowNorm& nm, void* zero,
                int nzero);
void add_inplace(hipStream_t s, float* a, const float* b, int64_t n);
void fill_normal(hipStream_t s, float* p, int64_t n, uint64_t seed, float std,
                 float mean);
void fill_normal_f16(hipStream_t s, uint16_t* p, int64_t n, uint64_t seed,
                     float std);
void fill_const(hipStream_t s, float* p, int64_t n, float v);
void scale(hipStream_t s, const float* x, int64_t n, float a, float* y);
void axpy(hipStream_t s, float a, const float* x, float* y, int64_t n);
void fill_uniform_int(hipStream_t s, int32_t* p, int64_t n, uint64_t seed,
                      int32_t hi);
// Layout ops of the operators API (off the hot path).
constexpr int kMaxCopyDims = 8;
void strided_copy(hipStream_t s, const float* src, float* dst, int ndim, const int64_t* shape,
                  const int64_t* stride);
void batched_matmul(hipStream_t s, const float* A, const float* B, float* C, int batch, int M, int K, int N);

}  // namespace mft
