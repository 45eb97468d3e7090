// capi.cpp — extern "C" entry points of libmft_hip.so (declared in
// include/mft_hip.h).  Each call validates shapes on the host, launches on
// the handle's stream and converts C++ exceptions into status codes plus a
// thread-local message.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace mft {
namespace {
thread_local std::string g_last_error;

// Per-handle device scratch used by the standalone entry points (split-K
// partials, rank-r temporaries, CE counters).  The step engine brings its
// own preallocated workspace instead.
struct HandleScratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }

int g_sync_check = [] {
  const char* e = getenv("MFT_SYNC_CHECK");
  return e && atoi(e) != 0 ? 1 : 0;
}();

// Streams the library launches on (handles, models, their copy and capture
// streams), reference-counted.  The sync check waits for these streams only,
// and not at all while any of them is being captured into a graph: a device
// or stream wait inside a capture would invalidate it.  (So the mode reports
// nothing for launches made under capture; they run when the graph does.)
std::mutex g_streams_mu;
std::vector<std::pair<hipStream_t, int>> g_streams;

void register_stream(hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_streams_mu);
  for (auto& e : g_streams)
    if (e.first == s) {
      ++e.second;
      return;
    }
  g_streams.emplace_back(s, 1);
}

void unregister_stream(hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_streams_mu);
  for (size_t i = 0; i < g_streams.size(); ++i)
    if (g_streams[i].first == s) {
      if (--g_streams[i].second == 0) g_streams.erase(g_streams.begin() + (std::ptrdiff_t)i);
      return;
    }
}

void sync_check(const char* file, int line) {
  std::vector<hipStream_t> streams;
  {
    std::lock_guard<std::mutex> lock(g_streams_mu);
    for (const auto& e : g_streams) streams.push_back(e.first);
  }
  for (hipStream_t s : streams) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone) return;
  }
  for (hipStream_t s : streams) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess)
      throw Error(MFT_EHIP, std::string("sync check after the launch at ") + file + ":" + std::to_string(line) +
                                ": " + hipGetErrorString(e));
  }
}

}  // namespace mft

namespace {
// A handle is allocated with its scratch descriptor right after it.
struct HandleImpl {
  mft_handle_s h;
  mft::HandleScratch scratch;
};

HandleImpl* impl(mft_handle h) { return reinterpret_cast<HandleImpl*>(h); }

// Returns device scratch of at least `bytes`, growing it (after draining the
// stream, so no in-flight kernel still uses the old buffer).
void* scratch(mft_handle h, size_t bytes) {
  HandleImpl* hi = impl(h);
  if (hi->scratch.bytes >= bytes) return hi->scratch.ptr;
  MFT_HIP(hipStreamSynchronize(h->stream));
  if (hi->scratch.ptr) MFT_HIP(hipFree(hi->scratch.ptr));
  hi->scratch.ptr = nullptr;
  hi->scratch.bytes = 0;
  size_t want = bytes < (size_t(64) << 20) ? (size_t(64) << 20) : bytes;
  if (hipMalloc(&hi->scratch.ptr, want) != hipSuccess)
    throw mft::Error(MFT_ENOMEM, "scratch allocation of " + std::to_string(want) + " bytes failed");
  hi->scratch.bytes = want;
  return hi->scratch.ptr;
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return MFT_OK;
  } catch (const mft::Error& e) {
    mft::set_last_error(e.what());
    return e.code;
  } catch (const std::exception& e) {
    mft::set_last_error(e.what());
    return MFT_EHIP;
  }
}

void require_handle(mft_handle h) {
  if (!h) throw mft::Error(MFT_EINVAL, "null handle");
}
}  // namespace

extern "C" {

const char* mft_last_error(void) { return mft::g_last_error.c_str(); }

int mft_set_sync_check(int on) {
  return guarded([&] { mft::g_sync_check = on ? 1 : 0; });
}
const char* mft_version(void) { return "mft_hip 0.1 gfx950"; }

int mft_create(mft_handle* out, void* stream) {
  return guarded([&] {
    if (!out) throw mft::Error(MFT_EINVAL, "null out");
    HandleImpl* hi = new HandleImpl();
    hi->h.stream = reinterpret_cast<hipStream_t>(stream);
    mft::register_stream(hi->h.stream);
    MFT_HIP(hipGetDevice(&hi->h.device));
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, hi->h.device) == hipSuccess && ncu > 0)
      hi->h.num_cu = ncu;
    *out = &hi->h;
  });
}

int mft_destroy(mft_handle h) {
  return guarded([&] {
    if (!h) return;
    HandleImpl* hi = impl(h);
    if (hi->scratch.ptr) {
      (void)hipStreamSynchronize(h->stream);
      (void)hipFree(hi->scratch.ptr);
    }
    mft::unregister_stream(h->stream);
    delete hi;
  });
}

int mft_set_stream(mft_handle h, void* stream) {
  return guarded([&] {
    require_handle(h);
    mft::register_stream(reinterpret_cast<hipStream_t>(stream));
    mft::unregister_stream(h->stream);
    h->stream = reinterpret_cast<hipStream_t>(stream);
  });
}
void* mft_get_stream(mft_handle h) { return h ? reinterpret_cast<void*>(h->stream) : nullptr; }

int mft_synchronize(mft_handle h) {
  return guarded([&] {
    require_handle(h);
    MFT_HIP(hipStreamSynchronize(h->stream));
  });
}

int mft_malloc(void** ptr, size_t bytes) {
  return guarded([&] {
    if (!ptr) throw mft::Error(MFT_EINVAL, "null ptr");
    if (hipMalloc(ptr, bytes ? bytes : 1) != hipSuccess)
      throw mft::Error(MFT_ENOMEM, "hipMalloc failed for " + std::to_string(bytes) + " bytes");
  });
}
int mft_free(void* ptr) {
  return guarded([&] {
    if (ptr) MFT_HIP(hipFree(ptr));
  });
}
int mft_memcpy_h2d(mft_handle h, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    require_handle(h);
    // Default: the runtime reads the pointer kinds (a streamed model's
    // frozen tensors live in pinned host memory)
    MFT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, h->stream));
    MFT_HIP(hipStreamSynchronize(h->stream));
  });
}
int mft_memcpy_d2h(mft_handle h, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    require_handle(h);
    MFT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, h->stream));
    MFT_HIP(hipStreamSynchronize(h->stream));
  });
}
int mft_memset(mft_handle h, void* dst, int value, size_t bytes) {
  return guarded([&] {
    require_handle(h);
    MFT_HIP(hipMemsetAsync(dst, value, bytes, h->stream));
  });
}

int mft_lora_linear_fwd(mft_handle h, const float* x, int64_t M, int64_t K,
                        const void* W, int w_dtype, int64_t N,
                        const float* bias, const float* A, const float* B,
                        int r, float scale, float* y, float* xa,
                        const float* resid) {
  return guarded([&] {
    require_handle(h);
    if (M <= 0 || K <= 0 || N <= 0) throw mft::Error(MFT_EINVAL, "mft_lora_linear_fwd: empty shape");
    if (w_dtype != MFT_F32 && w_dtype != MFT_F16) throw mft::Error(MFT_EINVAL, "bad w_dtype");
    if ((A == nullptr) != (B == nullptr)) throw mft::Error(MFT_EINVAL, "A and B must both be set or both NULL");
    const size_t ws = (size_t)16 * M * N * sizeof(float) + (size_t)M * sizeof(float) + 512;
    mft::Scratch s{reinterpret_cast<float*>(scratch(h, ws)), ws};
    mft::lora_linear_fwd(h->stream, x, M, K, W, w_dtype == MFT_F16, N, bias, A, B, A ? r : 0, scale,
                         y, xa, resid, s);
  });
}

int mft_lora_linear_bwd(mft_handle h, const float* dy, const float* x,
                        const void* W, int w_dtype, const float* A,
                        const float* B, const float* xa, int64_t M, int64_t K,
                        int64_t N, int r, float scale, float* dx, float* dA,
                        float* dB, int accumulate, int dx_accumulate) {
  return guarded([&] {
    require_handle(h);
    if (M <= 0 || K <= 0 || N <= 0) throw mft::Error(MFT_EINVAL, "mft_lora_linear_bwd: empty shape");
    if (w_dtype != MFT_F32 && w_dtype != MFT_F16) throw mft::Error(MFT_EINVAL, "bad w_dtype");
    if ((A == nullptr) != (B == nullptr)) throw mft::Error(MFT_EINVAL, "A and B must both be set or both NULL");
    const size_t ws = mft::lora_bwd_scratch_floats(M, K, N, A ? r : 0) * sizeof(float) +
                      (size_t)16 * M * K * sizeof(float) + (size_t)M * sizeof(float) + 512;
    mft::Scratch s{reinterpret_cast<float*>(scratch(h, ws)), ws};
    mft::lora_linear_bwd(h->stream, dy, x, W, w_dtype == MFT_F16, A, B, xa, M, K, N, A ? r : 0, scale,
                         dx, dA, dB, accumulate != 0, dx_accumulate != 0, s);
  });
}

int mft_attn_fwd(mft_handle h, const float* q, int64_t q_rs, const float* k,
                 int64_t k_rs, const float* v, int64_t v_rs, int B, int Hq,
                 int Hkv, int S, int hd, float scale, int causal, int window,
                 const float* kpad, float* o, int64_t o_rs, float* lse) {
  return guarded([&] {
    require_handle(h);
    mft::AttnArgs a{q, k, v, q_rs, k_rs, v_rs, B, Hq, Hkv, S, hd, scale, causal, window, kpad};
    const size_t ws = mft::attn_fwd_scratch_floats(a) * sizeof(float);
    mft::Scratch s{ws ? reinterpret_cast<float*>(scratch(h, ws)) : nullptr, ws};
    mft::attn_fwd(h->stream, a, o, o_rs, lse, s);
  });
}

int mft_attn_bwd(mft_handle h, const float* q, int64_t q_rs, const float* k,
                 int64_t k_rs, const float* v, int64_t v_rs, const float* o,
                 int64_t o_rs, const float* dout, int64_t do_rs,
                 const float* lse, int B, int Hq, int Hkv, int S, int hd,
                 float scale, int causal, int window, const float* kpad,
                 float* dq, int64_t dq_rs, float* dk, int64_t dk_rs, float* dv,
                 int64_t dv_rs) {
  return guarded([&] {
    require_handle(h);
    mft::AttnArgs a{q, k, v, q_rs, k_rs, v_rs, B, Hq, Hkv, S, hd, scale, causal, window, kpad};
    const size_t ws = mft::attn_bwd_scratch_floats(a) * sizeof(float);
    mft::Scratch s{reinterpret_cast<float*>(scratch(h, ws)), ws};
    mft::attn_bwd(h->stream, a, o, o_rs, dout, do_rs, lse, dq, dq_rs, dk, dk_rs, dv, dv_rs, s);
  });
}

int mft_ce_fwd_bwd(mft_handle h, const float* logits, const int32_t* labels,
                   int B, int S, int64_t V, int ignore_index, float upstream,
                   int64_t norm_count, double* loss_sum, int64_t* n_valid,
                   float* dlogits, float* row_nll) {
  return guarded([&] {
    require_handle(h);
    if (B <= 0 || S <= 0 || V <= 0) throw mft::Error(MFT_EINVAL, "mft_ce_fwd_bwd: empty shape");
    const size_t rows = (size_t)B * S;
    const size_t ws = 256 + rows * sizeof(float);
    char* base = reinterpret_cast<char*>(scratch(h, ws));
    int64_t* cnt = reinterpret_cast<int64_t*>(base);
    float* nll = row_nll ? row_nll : reinterpret_cast<float*>(base + 256);
    mft::ce_fwd_bwd(h->stream, logits, labels, B, S, V, V, ignore_index, upstream, norm_count, loss_sum,
                    n_valid, dlogits, nll, cnt);
  });
}

int mft_dequant_f16(mft_handle h, const uint16_t* src, float* dst, int64_t n) {
  return guarded([&] {
    require_handle(h);
    if (n < 0) throw mft::Error(MFT_EINVAL, "negative n");
    mft::dequant_f16(h->stream, src, dst, n);
  });
}
int mft_quant_f16(mft_handle h, const float* src, uint16_t* dst, int64_t n) {
  return guarded([&] {
    require_handle(h);
    if (n < 0) throw mft::Error(MFT_EINVAL, "negative n");
    mft::quant_f16(h->stream, src, dst, n);
  });
}

int mft_adam_step(mft_handle h, float* p, float* g, float* m, float* v,
                  int64_t n, float lr, float b1, float b2, float eps, float wd,
                  int t, const float* clip_scale, int zero_grad) {
  return guarded([&] {
    require_handle(h);
    if (n < 0) throw mft::Error(MFT_EINVAL, "negative n");
    mft::adam_step(h->stream, p, g, m, v, n, lr, b1, b2, eps, wd, t, clip_scale, zero_grad != 0);
  });
}
int mft_sumsq(mft_handle h, const float* g, int64_t n, double* out) {
  return guarded([&] {
    require_handle(h);
    mft::sumsq(h->stream, g, n, out);
  });
}
int mft_clip_scale(mft_handle h, const double* sumsq, float max_norm,
                   float* scale_out, float* norm_out) {
  return guarded([&] {
    require_handle(h);
    mft::clip_scale(h->stream, sumsq, max_norm, scale_out, norm_out);
  });
}

int mft_scale(mft_handle h, const float* x, int64_t n, float a, float* y) {
  return guarded([&] {
    require_handle(h);
    if (n < 0 || (n > 0 && (!x || !y))) throw mft::Error(MFT_EINVAL, "mft_scale: bad arguments");
    mft::scale(h->stream, x, n, a, y);
  });
}

int mft_axpy(mft_handle h, float a, const float* x, float* y, int64_t n) {
  return guarded([&] {
    require_handle(h);
    if (n < 0 || (n > 0 && (!x || !y))) throw mft::Error(MFT_EINVAL, "mft_axpy: bad arguments");
    mft::axpy(h->stream, a, x, y, n);
  });
}

int mft_fill(mft_handle h, float* p, int64_t n, float v) {
  return guarded([&] {
    require_handle(h);
    if (n < 0 || (n > 0 && !p)) throw mft::Error(MFT_EINVAL, "mft_fill: bad arguments");
    mft::fill_const(h->stream, p, n, v);
  });
}

int mft_strided_copy(mft_handle h, const float* src, float* dst, int ndim,
                     const int64_t* shape, const int64_t* src_strides) {
  return guarded([&] {
    require_handle(h);
    if (!src || !dst || !shape || !src_strides) throw mft::Error(MFT_EINVAL, "mft_strided_copy: null argument");
    mft::strided_copy(h->stream, src, dst, ndim, shape, src_strides);
  });
}

int mft_batched_matmul(mft_handle h, const float* A, const float* B, float* C,
                       int batch, int M, int K, int N) {
  return guarded([&] {
    require_handle(h);
    if (!A || !B || !C) throw mft::Error(MFT_EINVAL, "mft_batched_matmul: null argument");
    mft::batched_matmul(h->stream, A, B, C, batch, M, K, N);
  });
}

int mft_layernorm_fwd(mft_handle h, const float* x, const float* g,
                      const float* b, int64_t M, int64_t C, float eps,
                      float* y, float* mean, float* rstd) {
  return guarded([&] {
    require_handle(h);
    mft::layernorm_fwd(h->stream, x, g, b, M, C, eps, y, mean, rstd);
  });
}
int mft_layernorm_bwd(mft_handle h, const float* dy, const float* x,
                      const float* g, const float* mean, const float* rstd,
                      int64_t M, int64_t C, float* dx, int accumulate) {
  return guarded([&] {
    require_handle(h);
    mft::layernorm_bwd(h->stream, dy, x, g, mean, rstd, M, C, dx, accumulate != 0 ? dx : nullptr);
  });
}
int mft_rmsnorm_fwd(mft_handle h, const float* x, const float* w, int64_t M,
                    int64_t C, float eps, int unit_offset, float* y,
                    float* rstd) {
  return guarded([&] {
    require_handle(h);
    mft::rmsnorm_fwd(h->stream, x, w, M, C, eps, unit_offset != 0, y, rstd);
  });
}
int mft_rmsnorm_bwd(mft_handle h, const float* dy, const float* x,
                    const float* w, const float* rstd, int64_t M, int64_t C,
                    int unit_offset, float* dx, int accumulate) {
  return guarded([&] {
    require_handle(h);
    mft::rmsnorm_bwd(h->stream, dy, x, w, rstd, M, C, unit_offset != 0, dx, accumulate != 0 ? dx : nullptr);
  });
}
int mft_glu_fwd(mft_handle h, const float* gate, const float* up, int64_t n,
                int act, float* out) {
  return guarded([&] {
    require_handle(h);
    if (act != 0 && act != 1) throw mft::Error(MFT_EINVAL, "act must be 0 (gelu_tanh) or 1 (silu)");
    mft::glu_fwd(h->stream, gate, up, n, act, out);
  });
}
int mft_glu_bwd(mft_handle h, const float* dout, const float* gate,
                const float* up, int64_t n, int act, float* dgate,
                float* dup) {
  return guarded([&] {
    require_handle(h);
    if (act != 0 && act != 1) throw mft::Error(MFT_EINVAL, "act must be 0 (gelu_tanh) or 1 (silu)");
    mft::glu_bwd(h->stream, dout, gate, up, n, act, dgate, dup);
  });
}
int mft_rope(mft_handle h, float* x, int64_t rs, int B, int S, int H, int hd,
             double theta, int inverse) {
  return guarded([&] {
    require_handle(h);
    mft::rope(h->stream, x, rs, B, S, H, hd, theta, inverse != 0);
  });
}
int mft_embed(mft_handle h, const int32_t* ids, int64_t M, int S,
              const void* wte, int64_t vocab, int w_dtype, const float* wpe,
              int64_t C, float scale, float* out, int32_t* bad_ids) {
  return guarded([&] {
    require_handle(h);
    if (w_dtype != MFT_F32 && w_dtype != MFT_F16) throw mft::Error(MFT_EINVAL, "bad w_dtype");
    if (vocab <= 0) throw mft::Error(MFT_EINVAL, "mft_embed: vocab must be positive");
    mft::embed(h->stream, ids, M, S, wte, vocab, w_dtype == MFT_F16, wpe, C, scale, out, bad_ids);
  });
}

}  // extern "C"
