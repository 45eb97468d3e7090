/*
 * mft_hip.h — C-ABI of the MI355X (gfx950) kernel library libmft_hip.so.
 *
 * This is the layer under MobileFineTuner's C++ `operators` API
 * (operators/finetune_ops/{core,nn,graph,optim}; the library itself is not in
 * the published reference tree, its interface is reconstructed from the
 * drivers' call sites, cited per entry point below).
 *
 * Conventions
 *   - extern "C", plain pointers and sizes, no C++ or torch types.
 *   - All tensor pointers are DEVICE pointers owned by the caller; all
 *     tensors are fp32, row-major, unless the argument says otherwise.
 *   - Every call is asynchronous on the handle's stream; calls on one handle
 *     are ordered.  Handles are not thread-safe; use one per host thread.
 *   - Return value 0 = success; otherwise a nonzero MFT_E* code, with a
 *     message available from mft_last_error() (thread-local).  Invalid
 *     shapes are rejected on the host before any kernel is launched.
 *   - Linear weights are [in, out] = [K, N] (the reference's internal layout:
 *     gpt2_small_lora_finetune/src/main.cpp:211-214 loads GPT-2 Conv1D weights
 *     untransposed; qwen_lora_finetune/src/wikitext_main.cpp:67-74 transposes
 *     HF [out,in] at load time).  LoRA A is [r, K], B is [N, r] (PEFT layout,
 *     README.md:282,296).
 */
#ifndef MFT_HIP_H
#define MFT_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mft_handle_s* mft_handle;

enum mft_status {
  MFT_OK = 0,
  MFT_EINVAL = 1,   /* bad argument / shape */
  MFT_EHIP = 2,     /* HIP runtime error */
  MFT_ENOMEM = 3,   /* device allocation failed */
  MFT_EUNSUP = 4    /* unsupported configuration */
};

enum mft_dtype { MFT_F32 = 0, MFT_F16 = 1 };

/* ---- handle / runtime --------------------------------------------------- */
/* stream: a hipStream_t (NULL = the legacy default stream). */
int         mft_create(mft_handle* out, void* stream);
int         mft_destroy(mft_handle h);
int         mft_set_stream(mft_handle h, void* stream);
void*       mft_get_stream(mft_handle h);
int         mft_synchronize(mft_handle h);
const char* mft_last_error(void);
const char* mft_version(void);
/* Debug mode: with on != 0 every kernel launch is followed by a device
 * synchronisation, and an execution error is reported (MFT_EHIP, message
 * naming the source line of the launch) by the call that made it.  Also set
 * by MFT_SYNC_CHECK=1 in the environment at library load.  A captured
 * training-step graph is not used while it is on (steps run eagerly).
 * No counterpart in the reference (it runs on the CPU); the debug build mode
 * for the GPU path. */
int         mft_set_sync_check(int on);
/* Device memory helpers for hosts without their own allocator (the C++
 * operators layer, ctypes tests). */
int mft_malloc(void** ptr, size_t bytes);
int mft_free(void* ptr);
int mft_memcpy_h2d(mft_handle h, void* dst, const void* src, size_t bytes);
int mft_memcpy_d2h(mft_handle h, void* dst, const void* src, size_t bytes);
int mft_memset(mft_handle h, void* dst, int value, size_t bytes);

/* ---- a1: LoRA-linear forward ----------------------------------------------
 * y[M,N] = x[M,K]·W[K,N] + bias[N] + scale·(x·Aᵀ)·Bᵀ,  scale = alpha/r.
 * Replaces LoRALinear::forward (operators/finetune_ops/nn, absent; used via
 * blk.qkv_lin / blk.proj_lin, gpt2_small_lora_finetune/src/main.cpp:231-232,
 * and blk.{q,k,v,o}_proj_lora, gemma_3_270m_lora_finetune/src/main.cpp:411-414).
 * W is fp32 or fp16 (w_dtype); fp16 W is widened inside the GEMM's tile load
 * (the FP16 shard store of opt_ops/sharding, README.md:307-318).
 * bias, A, B may be NULL (plain frozen linear; r ignored).  xa [M,r] receives
 * x·Aᵀ for the backward (may be NULL only when A is NULL).
 * resid (nullable, [M,N], may alias y): y += resid (fused residual add). */
int mft_lora_linear_fwd(mft_handle h, const float* x, int64_t M, int64_t K,
                        const void* W, int w_dtype, int64_t N,
                        const float* bias, const float* A, const float* B,
                        int r, float scale, float* y, float* xa,
                        const float* resid);

/* ---- a2: LoRA-linear backward (W frozen) -----------------------------------
 * U = dy·B [M,r];  dx = dy·Wᵀ + scale·U·A  (overwritten; dx may be NULL);
 * dA (+)= scale·Uᵀ·x [r,K];  dB (+)= scale·dyᵀ·xa [N,r].
 * accumulate != 0 adds into dA/dB (grad accumulation across micro-batches,
 * gpt2_small_lora_finetune/src/main.cpp:471-487).  dx_accumulate != 0 adds
 * into dx instead of overwriting it.  Replaces the LoRALinear autograd node. */
int mft_lora_linear_bwd(mft_handle h, const float* dy, const float* x,
                        const void* W, int w_dtype, const float* A,
                        const float* B, const float* xa, int64_t M, int64_t K,
                        int64_t N, int r, float scale, float* dx, float* dA,
                        float* dB, int accumulate, int dx_accumulate);

/* ---- a3/a4: causal attention with GQA ---------------------------------------
 * q [B,S,Hq,hd], k/v [B,S,Hkv,hd] token-major with row strides *_rs (elements
 * between consecutive tokens; lets q/k/v be views into a fused QKV buffer).
 * P = softmax(scale·Q·Kᵀ + causal + window + key-padding), O = P·V.
 * window > 0: key j visible from query i iff i-j < window.  kpad [B,S]
 * (nullable): key j visible iff kpad[b,j] > 0.5.  lse [B,Hq,S] is saved for
 * the backward.  Query head h reads KV head h/(Hq/Hkv) — the same values the
 * reference's repeat_kv_heads copy produces
 * (gemma_3_270m_lora_finetune/src/main.cpp:623-626), without the copy.
 * hd ∈ {64, 128, 256}. */
int mft_attn_fwd(mft_handle h, const float* q, int64_t q_rs, const float* k,
                 int64_t k_rs, const float* v, int64_t v_rs, int B, int Hq,
                 int Hkv, int S, int hd, float scale, int causal, int window,
                 const float* kpad, float* o, int64_t o_rs, float* lse);
/* dV = Pᵀ·dO; dP = dO·Vᵀ; dS = P∘(dP − rowsum(dO∘O)); dQ = scale·dS·K;
 * dK = scale·dSᵀ·Q; dK/dV summed over each GQA group (formulas restated at
 * gemma_3_270m_lora_finetune/src/main.cpp:605-657).  dq/dk/dv overwritten. */
int mft_attn_bwd(mft_handle h, const float* q, int64_t q_rs, const float* k,
                 int64_t k_rs, const float* v, int64_t v_rs, const float* o,
                 int64_t o_rs, const float* dout, int64_t do_rs,
                 const float* lse, int B, int Hq, int Hkv, int S, int hd,
                 float scale, int causal, int window, const float* kpad,
                 float* dq, int64_t dq_rs, float* dk, int64_t dk_rs, float* dv,
                 int64_t dv_rs);

/* ---- a5/a6: shifted LM cross-entropy, forward + backward ---------------------
 * lm_cross_entropy(logits, labels, -100, "mean")
 * (gpt2_small_lora_finetune/src/main.cpp:475; closed form restated at
 * gemma_3_270m_lora_finetune/src/main.cpp:100-133): row (b,s), s < S-1,
 * predicts labels[b,s+1]; NLL = logsumexp(row) − row[label]; mean over
 * valid targets (label != ignore_index and 0 <= label < V; any other label
 * counts as ignored in both the loss and its normaliser).  logits [B*S, V]
 * fp32, labels [B,S] int32.
 * dlogits (nullable; may equal logits for in-place) = (softmax − onehot) ·
 * upstream / n, where n = norm_count if > 0, else the number of valid
 * targets counted on the device.  Ignored and last-position rows get 0.
 * loss_sum (device double*, nullable) += Σ NLL;  n_valid (device int64*,
 * nullable) += valid-target count;  row_nll (nullable) [B*S]. */
int mft_ce_fwd_bwd(mft_handle h, const float* logits, const int32_t* labels,
                   int B, int S, int64_t V, int ignore_index, float upstream,
                   int64_t norm_count, double* loss_sum, int64_t* n_valid,
                   float* dlogits, float* row_nll);

/* The same computation as mft_ce_fwd_bwd, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Its scratch (the
 * valid-target counter and, when row_nll is NULL, the per-row NLLs) is a
 * fixed device array of 256 KiB + 256 B inside the library, held by each
 * device until the process ends; the call allocates nothing.  B*S must not
 * exceed 65536 rows (MFT_EINVAL otherwise, nothing launched).  Every call on
 * one device shares that array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. */
int mft_ce_fwd_bwd_noalloc(mft_handle h, const float* logits,
                           const int32_t* labels, int B, int S, int64_t V,
                           int ignore_index, float upstream,
                           int64_t norm_count, double* loss_sum,
                           int64_t* n_valid, float* dlogits, float* row_nll);

/* ---- a7: fp16 → fp32 widening ------------------------------------------------
 * The FP16 shard store's require() path (ParameterSharder, opt_ops/sharding;
 * --shard_fp16_disk, README.md:311,318).  Exact for every bit pattern. */
int mft_dequant_f16(mft_handle h, const uint16_t* src, float* dst, int64_t n);
/* fp32 → fp16, round-to-nearest-even (how config-5 weights are stored). */
int mft_quant_f16(mft_handle h, const float* src, uint16_t* dst, int64_t n);

/* ---- a8/a9: Adam + global grad-norm clip -------------------------------------
 * Adam(AdamConfig{lr, b1, b2, eps, wd})::step (gpt2_small_lora_finetune/src/
 * main.cpp:341-348,497-502): bias-corrected, t 1-based, decoupled weight
 * decay.  clip_scale (device float*, nullable) multiplies g first, as
 * clip_and_get_grad_norm does in place (main.cpp:384-409).  When zero_grad
 * != 0 the gradient is zeroed after use (main.cpp:503-505). */
int mft_adam_step(mft_handle h, float* p, float* g, float* m, float* v,
                  int64_t n, float lr, float b1, float b2, float eps, float wd,
                  int t, const float* clip_scale, int zero_grad);
/* *out (device double) += Σ g² (fp64 accumulation, main.cpp:385-391). */
int mft_sumsq(mft_handle h, const float* g, int64_t n, double* out);
/* From a device Σg²: norm = sqrt(ss); scale = max_norm/(norm+1e-6) if
 * max_norm > 0 and norm > max_norm else 1; writes scale and the reported norm
 * (clipped value, as main.cpp:404 returns) to device floats. */
int mft_clip_scale(mft_handle h, const double* sumsq, float max_norm,
                   float* scale_out, float* norm_out);

/* ---- autograd support ---------------------------------------------------------
 * y = a·x (y may alias x): ops::mul(TensorPtr, float) and the loss scaling of
 * gpt2_small_lora_finetune/src/main.cpp:481-485 applied to a device tensor.
 * mft_axpy: y += a·x, gradient accumulation into a leaf's grad across
 * backward() calls (gpt2_small_lora_finetune/src/main.cpp:471-487).
 * mft_fill: p[i] = v, the device side of Tensor::zero_grad()
 * (gpt2_small_lora_finetune/src/main.cpp:503-505). */
int mft_scale(mft_handle h, const float* x, int64_t n, float a, float* y);
int mft_axpy(mft_handle h, float a, const float* x, float* y, int64_t n);
int mft_fill(mft_handle h, float* p, int64_t n, float v);

/* ---- layout ops of the operators API (not on the training path) ----------------
 * The free functions matmul / transpose / permute / repeat_kv_heads the Gemma
 * driver applies to dumped gradients in its alignment mode
 * (gemma_3_270m_lora_finetune/src/main.cpp:626-651).
 * mft_strided_copy: dst (contiguous in `shape`, ndim ≤ 8) = src read at
 * Σ_d coord_d·src_strides[d] (elements; a stride of 0 repeats that dimension).
 * mft_batched_matmul: C[b] = A[b]·B[b], row-major A [M,K], B [K,N], C [M,N]
 * packed per batch entry (fp32 FMA, not the MFMA training kernels). */
int mft_strided_copy(mft_handle h, const float* src, float* dst, int ndim,
                     const int64_t* shape, const int64_t* src_strides);
int mft_batched_matmul(mft_handle h, const float* A, const float* B, float* C,
                       int batch, int M, int K, int N);

/* ---- a10: support ops of the three graphs -------------------------------------
 * LayerNorm (GPT-2, γ/β frozen): saves mean/rstd [M]. */
int mft_layernorm_fwd(mft_handle h, const float* x, const float* g,
                      const float* b, int64_t M, int64_t C, float eps,
                      float* y, float* mean, float* rstd);
/* dx (+)= LayerNorm backward w.r.t. x. */
int mft_layernorm_bwd(mft_handle h, const float* dy, const float* x,
                      const float* g, const float* mean, const float* rstd,
                      int64_t M, int64_t C, float* dx, int accumulate);
/* RMSNorm: unit_offset=1 → x·rstd·(1+w) (Gemma3), 0 → x·rstd·w (Qwen2).
 * Also used per head over head_dim for Gemma3's QK-norm (M = tokens·heads). */
int mft_rmsnorm_fwd(mft_handle h, const float* x, const float* w, int64_t M,
                    int64_t C, float eps, int unit_offset, float* y,
                    float* rstd);
int mft_rmsnorm_bwd(mft_handle h, const float* dy, const float* x,
                    const float* w, const float* rstd, int64_t M, int64_t C,
                    int unit_offset, float* dx, int accumulate);
/* act 0 = GELU(tanh), 1 = SiLU.  out = act(gate)·up, or act(gate) if up is
 * NULL. */
int mft_glu_fwd(mft_handle h, const float* gate, const float* up, int64_t n,
                int act, float* out);
int mft_glu_bwd(mft_handle h, const float* dout, const float* gate,
                const float* up, int64_t n, int act, float* dgate,
                float* dup);
/* In-place HF rotate-half RoPE over [B,S,H,hd] (row stride rs), position = s,
 * inv_freq_i = theta^(-2i/hd).  inverse != 0 applies the transpose rotation
 * (the backward). */
int mft_rope(mft_handle h, float* x, int64_t rs, int B, int S, int H, int hd,
             double theta, int inverse);
/* h[m] = wte[ids[m]]·scale (+ wpe[m % S]); wte [vocab, C] fp32 or fp16
 * (w_dtype).  An id outside [0, vocab) reads nothing: its row of h is zeros
 * and *bad_ids (device int32, nullable) is set to 1. */
int mft_embed(mft_handle h, const int32_t* ids, int64_t M, int S,
              const void* wte, int64_t vocab, int w_dtype, const float* wpe,
              int64_t C, float scale, float* out, int32_t* bad_ids);

#ifdef __cplusplus
}
#endif
#endif
