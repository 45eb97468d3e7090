// ce_noalloc.hip — mft_ce_fwd_bwd_noalloc: the shifted LM cross-entropy of
// mft_ce_fwd_bwd (same kernels, ce.hip) with its scratch in a fixed device
// array, for callers that cannot allocate device memory.
#include <mutex>
#include <string>

#include "common.h"

namespace mft {
// The valid-target counter and the per-row NLLs live in a file-scope device
// array instead of handle scratch, so the call never allocates.  Layout:
// bytes [0, 8) the int64 counter, [256, 256 + 4·rows) the row NLLs.
namespace {
constexpr int64_t kCeNoAllocMaxRows = int64_t(1) << 16;
constexpr size_t kCeNoAllocBytes = 256 + (size_t)kCeNoAllocMaxRows * sizeof(float);  // 256 KiB + 256 B
}  // namespace

static __device__ __align__(256) char scratch[kCeNoAllocBytes];

namespace {
// Device address of `scratch` per device, looked up once per device (with
// that device current) on the first call there.  The host-side name of the
// array is a stand-in, not a device address: only these pointers are passed.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

char* scratch_on_current_device() {
  int dev = 0;
  MFT_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) throw Error(MFT_EUNSUP, "device ordinal beyond the no-allocation table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      throw Error(MFT_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  return static_cast<char*>(g_scratch_ptr[dev]);
}
}  // namespace

}  // namespace mft

extern "C" int mft_ce_fwd_bwd_noalloc(mft_handle h, const float* logits, const int32_t* labels, int B, int S,
                                      int64_t V, int ignore_index, float upstream, int64_t norm_count,
                                      double* loss_sum, int64_t* n_valid, float* dlogits, float* row_nll) {
  try {
    if (!h) throw mft::Error(MFT_EINVAL, "null handle");
    if (B <= 0 || S <= 0 || V <= 0) throw mft::Error(MFT_EINVAL, "mft_ce_fwd_bwd_noalloc: empty shape");
    const int64_t rows = (int64_t)B * S;
    if (rows > mft::kCeNoAllocMaxRows)
      throw mft::Error(MFT_EINVAL, "mft_ce_fwd_bwd_noalloc: B*S = " + std::to_string(rows) +
                                       " rows exceeds the no-allocation maximum of " +
                                       std::to_string(mft::kCeNoAllocMaxRows));
    char* base = mft::scratch_on_current_device();
    int64_t* cnt = reinterpret_cast<int64_t*>(base);  // stored (not accumulated) inside ce_fwd_bwd
    float* nll = row_nll ? row_nll : reinterpret_cast<float*>(base + 256);
    mft::ce_fwd_bwd(h->stream, logits, labels, B, S, V, V, ignore_index, upstream, norm_count, loss_sum, n_valid,
                    dlogits, nll, cnt);
    return MFT_OK;
  } catch (const mft::Error& e) {
    mft::set_last_error(e.what());
    return e.code;
  } catch (const std::exception& e) {
    mft::set_last_error(e.what());
    return MFT_EHIP;
  }
}
