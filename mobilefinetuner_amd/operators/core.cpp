// core.cpp — Tensor, autograd tape, operators, LM loss, Adam and memory hooks
// of the finetune_ops host library, on libmft_hip's C-ABI.
//
// Host code only: every computation is a libmft_hip kernel launch on the
// library's stream; this file moves pointers, shapes and gradients.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <fstream>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <sys/stat.h>

#include <unordered_map>
#include <unordered_set>

#include "finetune_ops/core/autograd_engine.h"
#include "finetune_ops/core/lm_loss.h"
#include "finetune_ops/core/memory_manager.h"
#include "finetune_ops/core/ops.h"
#include "finetune_ops/optim/adam.h"
#include "internal.h"

namespace ops {

namespace detail {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void mft_check(int rc, const char* what) {
  if (rc != 0) throw std::runtime_error(std::string(what) + ": " + mft_last_error());
}

mft_handle handle() {
  // One handle on the default stream: host copies (hipMemcpy) order with it.
  static mft_handle h = [] {
    mft_handle out = nullptr;
    mft_check(mft_create(&out, nullptr), "mft_create");
    return out;
  }();
  return h;
}

float read_scalar(const TensorPtr& t) {
  if (!t || t->numel() != 1) throw std::runtime_error("expected a one-element tensor");
  if (t->dtype() != kFloat32) throw std::runtime_error("expected a float32 tensor");
  return static_cast<const Tensor&>(*t).data<float>()[0];
}

}  // namespace detail

using detail::hip_check;
using detail::mft_check;

size_t dtype_size(DType t) {
  switch (t) {
    case kFloat32: return 4;
    case kInt32: return 4;
    case kFloat16: return 2;
  }
  throw std::runtime_error("unknown dtype");
}

// ---------------------------------------------------------------- Tensor --

void Tensor::init_shape(std::vector<int64_t> shape, DType dtype, Device device) {
  int64_t n = 1;
  for (int64_t d : shape) {
    if (d < 0) throw std::invalid_argument("Tensor: negative dimension");
    n *= d;
  }
  shape_ = std::move(shape);
  numel_ = n;
  dtype_ = dtype;
  device_ = device;
  pitch_ = shape_.empty() ? 1 : shape_.back();
}

// Device blocks of the tensors this library allocates come from a cache:
// a freed block is kept on a free list of its rounded size and handed to the
// next tensor of that size, instead of hipFree (which waits for the device)
// and hipMalloc on every temporary of a training step (input ids, masks,
// loss scalars, upstream gradients).  All of this library's work runs on the
// null stream, in order, so a block reused by a later tensor is only touched
// after the earlier tensor's queued work.  MemoryManager::clear_unused_memory
// and force_cleanup return the cached blocks to the device.
namespace {
struct DevCache {
  std::mutex mu;
  std::unordered_map<size_t, std::vector<void*>> free;  // rounded bytes → blocks
};
DevCache& dev_cache() {
  static DevCache* c = new DevCache();  // never destroyed: tensors may outlive static destruction
  return *c;
}
size_t round_block(size_t b) {
  if (b <= (size_t(1) << 20)) {
    size_t r = 256;
    while (r < b) r <<= 1;
    return r;
  }
  const size_t g = size_t(2) << 20;
  return (b + g - 1) / g * g;
}
void* dev_alloc(size_t bytes) {
  const size_t rb = round_block(bytes);
  {
    DevCache& c = dev_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.free.find(rb);
    if (it != c.free.end() && !it->second.empty()) {
      void* p = it->second.back();
      it->second.pop_back();
      return p;
    }
  }
  void* p = nullptr;
  hip_check(hipMalloc(&p, rb), "hipMalloc");
  return p;
}
void dev_release(void* p, size_t bytes) {
  DevCache& c = dev_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  c.free[round_block(bytes)].push_back(p);
}
void dev_cache_clear() {
  DevCache& c = dev_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  for (auto& e : c.free)
    for (void* p : e.second) (void)hipFree(p);
  c.free.clear();
}
}  // namespace

// Host data of small tensors (token ids, masks, labels, scalars) goes to
// the device through a ring of pinned staging slots with asynchronous copies
// on the null stream, so building a step's inputs does not wait for the
// device; a slot is reused once its previous copy has completed.
namespace {
struct StageRing {
  static constexpr int kSlots = 64;
  static constexpr size_t kSlotBytes = size_t(64) << 10;
  std::mutex mu;
  char* host = nullptr;
  hipEvent_t ev[kSlots] = {};
  bool used[kSlots] = {};
  int next = 0;
};
StageRing& stage_ring() {
  static StageRing* r = new StageRing();  // never destroyed (outlives static destruction)
  return *r;
}
// Copies `bytes` (≤ kSlotBytes) from host memory to dst asynchronously;
// false when the staging ring cannot be set up (the caller copies directly).
bool stage_upload(void* dst, const void* src, size_t bytes) {
  StageRing& r = stage_ring();
  if (bytes > StageRing::kSlotBytes) return false;
  std::lock_guard<std::mutex> lock(r.mu);
  if (!r.host) {
    if (hipHostMalloc(reinterpret_cast<void**>(&r.host), StageRing::kSlots * StageRing::kSlotBytes,
                      hipHostMallocDefault) != hipSuccess) {
      r.host = nullptr;
      return false;
    }
    for (auto& e : r.ev) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
  }
  const int i = r.next;
  r.next = (r.next + 1) % StageRing::kSlots;
  if (r.used[i]) hip_check(hipEventSynchronize(r.ev[i]), "hipEventSynchronize");
  char* slot = r.host + (size_t)i * StageRing::kSlotBytes;
  std::memcpy(slot, src, bytes);
  hip_check(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, nullptr), "hipMemcpyAsync H2D");
  hip_check(hipEventRecord(r.ev[i], nullptr), "hipEventRecord");
  r.used[i] = true;
  return true;
}
}  // namespace

Tensor::Tensor(std::vector<int64_t> shape, DType dtype, Device device) {
  init_shape(std::move(shape), dtype, device);
  const size_t bytes = (size_t)numel_ * dtype_size(dtype_);
  if (bytes) {
    dev_ = dev_alloc(bytes);
    owns_ = true;
    hip_check(hipMemsetAsync(dev_, 0, bytes, nullptr), "hipMemsetAsync");
  }
}

Tensor::Tensor(std::vector<int64_t> shape, const void* data, DType dtype, Device device) {
  init_shape(std::move(shape), dtype, device);
  const size_t bytes = (size_t)numel_ * dtype_size(dtype_);
  if (bytes) {
    if (!data) throw std::invalid_argument("Tensor: null data");
    if (device == kCPU && bytes <= kLazyBytes) {
      // scalars and other tiny host-built values (a loss, a backward seed,
      // an upstream gradient) stay on the host until a kernel needs them
      host_.assign(static_cast<const char*>(data), static_cast<const char*>(data) + bytes);
      host_state_ = 2;
      lazy_dev_ = true;
      owns_ = true;
      return;
    }
    dev_ = dev_alloc(bytes);
    owns_ = true;
    if (stage_upload(dev_, data, bytes)) {
      // small host-built tensors keep their host copy: the host checks of
      // ids and labels (check_ids, check_labels) then read no device memory
      host_.assign(static_cast<const char*>(data), static_cast<const char*>(data) + bytes);
      host_state_ = 1;
    } else {
      hip_check(hipMemcpy(dev_, data, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
  }
}

TensorPtr Tensor::view(std::vector<int64_t> shape, DType dtype, void* device_ptr, int64_t pitch,
                       std::shared_ptr<void> owner) {
  TensorPtr t(new Tensor());
  t->init_shape(std::move(shape), dtype, kGPU);
  if (!t->shape_.empty() && pitch < t->shape_.back()) throw std::invalid_argument("Tensor::view: pitch < row length");
  if (!t->shape_.empty()) t->pitch_ = pitch;
  t->dev_ = device_ptr;
  t->owns_ = false;
  t->owner_ = std::move(owner);
  return t;
}

Tensor::~Tensor() {
  if (owns_ && dev_) dev_release(dev_, (size_t)numel_ * dtype_size(dtype_));
}

struct MirrorGroup {
  char* dev = nullptr;
  size_t bytes = 0;
  // Host copy in pinned memory (allocated at the first host access): the
  // drivers' per-step gradient reads and writes move at DMA rate, and a copy
  // can be queued behind the kernels that produce the data.
  char* host = nullptr;
  void* host_dev = nullptr;     // `host` as kernels address it (null: copies only)
  hipEvent_t arrive = nullptr;  // end of the queued device→host copy (state 3)
  hipEvent_t depart = nullptr;  // end of the queued work that reads `host` (states 2 and 4)
  // 0 = stale, 1 = equal to the device, 2 = newer than the device,
  // 3 = a device→host copy is queued (equal to the device once `arrive` fires),
  // 4 = a host→device copy is queued: equal to the device, but the host copy
  //     is read by that copy until `depart` fires (host writes wait for it)
  int state = 0;
  // a queued kernel or copy reads `host` until `depart` fires (host writes wait)
  bool host_read = false;
  // host edits not yet on the device when zero_grad() requests arrived: they
  // go up before the fills unless every member is zeroed
  bool host_edits = false;
  int members = 0;  // views created in the group
  // zero_grad() requests not yet applied on the device: byte offset → bytes.
  // They run at the group's next device or host access, as one fill over the
  // whole range when every member asked (the drivers' zero_grad loop).
  std::map<size_t, size_t> zeros;
  ~MirrorGroup() {
    if (depart) (void)hipEventSynchronize(depart);  // a queued upload may still read `host`
    if (arrive) (void)hipEventDestroy(arrive);
    if (depart) (void)hipEventDestroy(depart);
    if (host) (void)hipHostFree(host);
  }
};

namespace {
void ensure_host(MirrorGroup& g) {
  if (g.host || g.bytes == 0) return;
  hip_check(hipHostMalloc(reinterpret_cast<void**>(&g.host), g.bytes, hipHostMallocDefault), "hipHostMalloc");
  std::memset(g.host, 0, g.bytes);
  if (hipHostGetDevicePointer(&g.host_dev, g.host, 0) != hipSuccess) {
    g.host_dev = nullptr;
    (void)hipGetLastError();
  }
  g.state = 0;
}

// `depart` marks the end of what the stream has queued so far that reads `host`
void mark_host_read(MirrorGroup& g) {
  if (!g.depart) hip_check(hipEventCreateWithFlags(&g.depart, hipEventDisableTiming), "hipEventCreate");
  hip_check(hipEventRecord(g.depart, nullptr), "hipEventRecord");
  g.host_read = true;
}

void flush_zeros(MirrorGroup& g) {
  if (g.zeros.empty()) return;
  if ((int)g.zeros.size() == g.members) {
    mft_check(mft_fill(detail::handle(), reinterpret_cast<float*>(g.dev), (int64_t)(g.bytes / 4), 0.f), "mft_fill");
  } else {
    if (g.host_edits) {  // the members not zeroed keep their host edits
      hip_check(hipMemcpyAsync(g.dev, g.host, g.bytes, hipMemcpyHostToDevice, nullptr), "hipMemcpyAsync H2D");
      mark_host_read(g);
    }
    for (const auto& z : g.zeros)
      mft_check(mft_fill(detail::handle(), reinterpret_cast<float*>(g.dev + z.first), (int64_t)(z.second / 4), 0.f),
                "mft_fill");
  }
  g.zeros.clear();
  g.host_edits = false;
  g.state = 0;
}
}  // namespace

namespace detail {
// Queues the copy of t's mirror group into its pinned host buffer behind the
// work already on the stream (the engine's backward), so a host read that
// follows waits for the kernels only, not for a copy started after them.
// Groupless tensors are left alone.
void prefetch_host(const TensorPtr& t) {
  if (!t || !t->mirror()) return;
  MirrorGroup& g = *t->mirror();
  flush_zeros(g);
  ensure_host(g);
  if (g.state != 0 || g.bytes == 0) return;  // already equal, newer on the host, or queued
  if (!g.arrive) hip_check(hipEventCreateWithFlags(&g.arrive, hipEventDisableTiming), "hipEventCreate");
  hip_check(hipMemcpyAsync(g.host, g.dev, g.bytes, hipMemcpyDeviceToHost, nullptr), "hipMemcpyAsync D2H");
  hip_check(hipEventRecord(g.arrive, nullptr), "hipEventRecord");
  g.state = 3;
}

}  // namespace detail

std::shared_ptr<MirrorGroup> Tensor::mirror_group(void* base, size_t bytes) {
  auto g = std::make_shared<MirrorGroup>();
  g->dev = static_cast<char*>(base);
  g->bytes = bytes;
  return g;
}

TensorPtr Tensor::view(std::vector<int64_t> shape, DType dtype, void* device_ptr, std::shared_ptr<void> owner,
                       std::shared_ptr<MirrorGroup> group) {
  const int64_t last = shape.empty() ? 1 : shape.back();
  TensorPtr t = view(std::move(shape), dtype, device_ptr, last, std::move(owner));
  if (group) {
    const char* p = static_cast<const char*>(device_ptr);
    if (p < group->dev || p + (size_t)t->numel_ * dtype_size(dtype) > group->dev + group->bytes)
      throw std::invalid_argument("Tensor::view: outside its mirror group");
    t->group_off_ = (size_t)(p - group->dev);
    ++group->members;
    t->group_ = std::move(group);
  }
  return t;
}

char* Tensor::host_ptr() const { return group_ ? group_->host + group_off_ : host_.data(); }

void Tensor::sync_host(bool will_write) const {
  if (group_) {
    MirrorGroup& g = *group_;
    flush_zeros(g);
    ensure_host(g);
    if (will_write && g.host_read) {
      hip_check(hipEventSynchronize(g.depart), "hipEventSynchronize");
      g.host_read = false;
    }
    if (g.state == 3 || (g.state == 4 && will_write)) {
      hip_check(hipEventSynchronize(g.state == 3 ? g.arrive : g.depart), "hipEventSynchronize");
      g.state = 1;
    }
    if (g.state == 0 && g.bytes > 0) {
      hip_check(hipMemcpy(g.host, g.dev, g.bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
      g.state = 1;
    }
    if (will_write) g.state = 2;
    return;
  }
  const size_t esz = dtype_size(dtype_);
  if (host_.size() != (size_t)numel_ * esz) {
    host_.assign((size_t)numel_ * esz, 0);
    host_state_ = 0;
  }
  if (host_state_ == 0 && numel_ > 0) {
    const int64_t row = shape_.empty() ? 1 : shape_.back();
    const int64_t rows = row ? numel_ / row : 0;
    if (pitch_ == row)
      hip_check(hipMemcpy(host_.data(), dev_, host_.size(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    else
      hip_check(hipMemcpy2D(host_.data(), row * esz, dev_, pitch_ * esz, row * esz, rows, hipMemcpyDeviceToHost),
                "hipMemcpy2D D2H");
    host_state_ = 1;
  }
  if (will_write) host_state_ = 2;
}

void Tensor::upload_if_dirty() const {
  if (lazy_dev_) {
    const size_t bytes = host_.size();
    dev_ = dev_alloc(bytes);
    lazy_dev_ = false;
    if (!stage_upload(dev_, host_.data(), bytes))
      hip_check(hipMemcpy(dev_, host_.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    host_state_ = 1;
    return;
  }
  if (group_) {
    MirrorGroup& g = *group_;
    flush_zeros(g);
    if (g.state == 2) {
      // queued behind the stream's work, ahead of the kernel that asked: the
      // pinned host copy stays untouched until `depart` (sync_host waits)
      hip_check(hipMemcpyAsync(g.dev, g.host, g.bytes, hipMemcpyHostToDevice, nullptr), "hipMemcpyAsync H2D");
      mark_host_read(g);
      g.state = 4;
    }
    return;
  }
  if (host_state_ != 2) return;
  const size_t esz = dtype_size(dtype_);
  const int64_t row = shape_.empty() ? 1 : shape_.back();
  const int64_t rows = row ? numel_ / row : 0;
  if (pitch_ == row)
    hip_check(hipMemcpy(dev_, host_.data(), host_.size(), hipMemcpyHostToDevice), "hipMemcpy H2D");
  else
    hip_check(hipMemcpy2D(dev_, pitch_ * esz, host_.data(), row * esz, row * esz, rows, hipMemcpyHostToDevice),
              "hipMemcpy2D H2D");
  host_state_ = 1;
}

void* Tensor::device_data() {
  upload_if_dirty();
  return dev_;
}

const void* Tensor::device_data() const {
  upload_if_dirty();
  return dev_;
}

bool Tensor::host_current() const {
  if (group_) return group_->state == 1 || group_->state == 2 || group_->state == 4;
  return host_state_ != 0 && host_.size() == (size_t)numel_ * dtype_size(dtype_);
}

void Tensor::mark_device_written() {
  // grouped views: callers take device_data() before a kernel writes, which
  // flushes any host edits of the group, so the whole mirror is now stale
  if (group_) group_->state = 0;
  else host_state_ = 0;
}

void Tensor::zero_grad() {
  if (!grad_) return;
  if (grad_->dtype() != kFloat32) throw std::runtime_error("zero_grad: float32 gradients only");
  if (!grad_->contiguous()) throw std::runtime_error("zero_grad: strided gradient");
  if (const auto& g = grad_->group_) {  // deferred: one fill for the whole group when every member asks
    // host edits of other members reach the device first (without applying
    // the zero requests already pending: those wait for the rest of the
    // group, so the drivers' zero_grad loop costs one fill)
    if (g->state == 2) g->host_edits = true;  // uploaded at the flush unless every member is zeroed
    g->zeros[grad_->group_off_] = (size_t)grad_->numel() * 4;
    g->state = 0;
    return;
  }
  mft_check(mft_fill(detail::handle(), static_cast<float*>(grad_->device_data()), grad_->numel(), 0.f), "mft_fill");
  grad_->mark_device_written();
}

void Tensor::backward() {
  if (numel_ != 1) throw std::runtime_error("backward(): the tensor must have one element (pass a gradient otherwise)");
  const float one = 1.f;
  backward(std::make_shared<Tensor>(std::vector<int64_t>{1}, &one, kFloat32, kCPU));
}

void Tensor::backward(const TensorPtr& grad_output) {
  autograd::Engine::instance().backward(shared_from_this(), grad_output);
}

TensorPtr zeros(const std::vector<int64_t>& shape, DType dtype) { return std::make_shared<Tensor>(shape, dtype, kGPU); }

TensorPtr from_host(const std::vector<int64_t>& shape, const void* data, DType dtype) {
  return std::make_shared<Tensor>(shape, data, dtype, kGPU);
}

// -------------------------------------------------------------- autograd --

namespace autograd {

Engine& Engine::instance() {
  static Engine e;
  return e;
}

void Engine::record(const TensorPtr& out, std::shared_ptr<Node> fn) {
  if (!enabled_) return;
  bool needs = false;
  for (const auto& in : fn->inputs) needs = needs || (in && (in->requires_grad() || in->grad_fn()));
  if (!needs) return;
  out->set_grad_fn(std::move(fn));
  out->set_requires_grad(true);
  if (recorded_.size() >= 4096) {  // forget outputs that no longer exist
    std::vector<std::weak_ptr<Tensor>> live;
    for (auto& w : recorded_)
      if (!w.expired()) live.push_back(w);
    recorded_.swap(live);
  }
  recorded_.push_back(out);
}

void Engine::clear_graph() {
  for (auto& w : recorded_)
    if (auto t = w.lock()) t->set_grad_fn(nullptr);
  recorded_.clear();
}

void accumulate_grad(const TensorPtr& t, const TensorPtr& g) {
  if (g->numel() != t->numel()) throw std::runtime_error("gradient size mismatch");
  if (!t->grad()) {
    auto z = std::make_shared<Tensor>(t->shape(), kFloat32, kGPU);
    t->set_grad(z);
  }
  const TensorPtr& dst = t->grad();
  if (!dst->contiguous() || !g->contiguous()) throw std::runtime_error("accumulate_grad: strided tensors");
  mft_check(mft_axpy(detail::handle(), 1.f, static_cast<const float*>(g->device_data()),
                     static_cast<float*>(dst->device_data()), g->numel()),
            "mft_axpy");
  dst->mark_device_written();
}

void Engine::backward(const TensorPtr& root, const TensorPtr& grad_output) {
  if (!root->grad_fn()) {
    if (root->requires_grad()) accumulate_grad(root, grad_output);
    return;
  }
  // Reverse topological order of the nodes reachable from the root.
  std::vector<Node*> order;
  std::unordered_set<Node*> seen;
  std::function<void(Node*)> visit = [&](Node* n) {
    if (!seen.insert(n).second) return;
    for (const auto& in : n->inputs)
      if (in && in->grad_fn()) visit(in->grad_fn().get());
    order.push_back(n);
  };
  visit(root->grad_fn().get());
  std::unordered_map<Node*, TensorPtr> pending;
  pending[root->grad_fn().get()] = grad_output;
  if (root->retains_grad()) accumulate_grad(root, grad_output);
  for (auto it = order.rbegin(); it != order.rend(); ++it) {
    Node* n = *it;
    auto pit = pending.find(n);
    if (pit == pending.end()) continue;
    TensorPtr g = pit->second;
    pending.erase(pit);
    std::vector<TensorPtr> gin = n->apply(g);
    for (size_t i = 0; i < n->inputs.size() && i < gin.size(); ++i) {
      const TensorPtr& in = n->inputs[i];
      const TensorPtr& gi = gin[i];
      if (!in || !gi) continue;
      if (in->grad_fn()) {
        Node* p = in->grad_fn().get();
        auto q = pending.find(p);
        if (q == pending.end()) {
          pending[p] = gi;
        } else {  // sum of the gradients reaching one output
          auto sum = std::make_shared<Tensor>(gi->shape(), kFloat32, kGPU);
          mft_check(mft_axpy(detail::handle(), 1.f, static_cast<const float*>(q->second->device_data()),
                             static_cast<float*>(sum->device_data()), sum->numel()), "mft_axpy");
          mft_check(mft_axpy(detail::handle(), 1.f, static_cast<const float*>(gi->device_data()),
                             static_cast<float*>(sum->device_data()), sum->numel()), "mft_axpy");
          q->second = sum;
        }
        if (in->retains_grad()) accumulate_grad(in, gi);
      } else if (in->requires_grad()) {
        accumulate_grad(in, gi);
      }
    }
  }
}

}  // namespace autograd

// ------------------------------------------------------------- operators --

namespace {

using autograd::Node;

const float* fptr(const TensorPtr& t) { return t ? static_cast<const float*>(t->device_data()) : nullptr; }

void require_f32(const TensorPtr& t, const char* what) {
  if (!t) throw std::invalid_argument(std::string(what) + ": null tensor");
  if (t->dtype() != kFloat32) throw std::invalid_argument(std::string(what) + ": float32 tensor required");
  if (!t->contiguous()) throw std::invalid_argument(std::string(what) + ": contiguous tensor required");
}

TensorPtr new_f32(const std::vector<int64_t>& shape) { return std::make_shared<Tensor>(shape, kFloat32, kGPU); }

// s·a computed on the host for a one-element float32 tensor whose host copy
// is current (a loss, a backward seed, the upstream gradient of a loss
// scale): no kernel, no copy, no wait.  The product is the one fp32 multiply
// the device's scale kernel performs.  Null otherwise.
TensorPtr host_scaled(const TensorPtr& a, float s) {
  if (a->numel() != 1 || a->dtype() != kFloat32 || !a->host_current()) return nullptr;
  const float v = static_cast<const Tensor&>(*a).data<float>()[0] * s;
  return std::make_shared<Tensor>(a->shape(), &v, kFloat32, kCPU);
}

struct MulNode : Node {
  float s;
  const char* name() const override { return "MulBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    if (auto h = host_scaled(g, s)) return {h};
    auto out = new_f32(g->shape());
    mft_check(mft_scale(detail::handle(), fptr(g), g->numel(), s, static_cast<float*>(out->device_data())), "mft_scale");
    return {out};
  }
};

struct AddNode : Node {
  const char* name() const override { return "AddBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override { return {g, g}; }
};

struct ReshapeNode : Node {
  std::vector<int64_t> in_shape;
  const char* name() const override { return "ReshapeBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    return {Tensor::view(in_shape, kFloat32, g->device_data(), in_shape.empty() ? 1 : in_shape.back(), g)};
  }
};

int64_t rows_of(const TensorPtr& x) { return x->shape().empty() ? 1 : x->numel() / x->shape().back(); }

struct LinearNode : Node {
  // inputs: x, A, B  (W, b frozen, saved below)
  TensorPtr W, xa;
  int w_dtype = MFT_F32;
  float scale = 0.f;
  int64_t M = 0, K = 0, N = 0;
  int r = 0;
  const char* name() const override { return "LoRALinearBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    require_f32(g, "linear backward");
    const TensorPtr& x = inputs[0];
    const TensorPtr A = inputs.size() > 1 ? inputs[1] : nullptr;
    const TensorPtr B = inputs.size() > 2 ? inputs[2] : nullptr;
    const bool need_dx = x->requires_grad() || x->grad_fn();
    TensorPtr dx = need_dx ? new_f32(x->shape()) : nullptr;
    TensorPtr dA = A ? new_f32(A->shape()) : nullptr;
    TensorPtr dB = B ? new_f32(B->shape()) : nullptr;
    mft_check(mft_lora_linear_bwd(detail::handle(), fptr(g), fptr(x), W->device_data(), w_dtype, fptr(A), fptr(B),
                                  fptr(xa), M, K, N, r, scale, dx ? static_cast<float*>(dx->device_data()) : nullptr,
                                  dA ? static_cast<float*>(dA->device_data()) : nullptr,
                                  dB ? static_cast<float*>(dB->device_data()) : nullptr, 0, 0),
              "mft_lora_linear_bwd");
    return {dx, dA, dB};
  }
};

struct AttnNode : Node {
  // inputs: q, k, v
  TensorPtr o, lse, kmask;
  int B = 0, S = 0, Hq = 0, Hkv = 0, hd = 0, window = 0;
  float scale = 0.f;
  const char* name() const override { return "CausalAttentionBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    require_f32(g, "attention backward");
    auto dq = new_f32(inputs[0]->shape()), dk = new_f32(inputs[1]->shape()), dv = new_f32(inputs[2]->shape());
    mft_check(mft_attn_bwd(detail::handle(), fptr(inputs[0]), (int64_t)Hq * hd, fptr(inputs[1]), (int64_t)Hkv * hd,
                           fptr(inputs[2]), (int64_t)Hkv * hd, fptr(o), (int64_t)Hq * hd, fptr(g), (int64_t)Hq * hd,
                           fptr(lse), B, Hq, Hkv, S, hd, scale, 1, window, fptr(kmask),
                           static_cast<float*>(dq->device_data()), (int64_t)Hq * hd,
                           static_cast<float*>(dk->device_data()), (int64_t)Hkv * hd,
                           static_cast<float*>(dv->device_data()), (int64_t)Hkv * hd),
              "mft_attn_bwd");
    return {dq, dk, dv};
  }
};

}  // namespace

TensorPtr mul(const TensorPtr& a, float s) {
  require_f32(a, "mul");
  TensorPtr out = host_scaled(a, s);
  if (!out) {
    out = new_f32(a->shape());
    mft_check(mft_scale(detail::handle(), fptr(a), a->numel(), s, static_cast<float*>(out->device_data())),
              "mft_scale");
  }
  auto n = std::make_shared<MulNode>();
  n->s = s;
  n->inputs = {a};
  autograd::Engine::instance().record(out, n);
  return out;
}

TensorPtr add(const TensorPtr& a, const TensorPtr& b) {
  require_f32(a, "add");
  require_f32(b, "add");
  if (a->shape() != b->shape()) throw std::invalid_argument("add: shape mismatch");
  auto out = new_f32(a->shape());
  float* o = static_cast<float*>(out->device_data());
  mft_check(mft_axpy(detail::handle(), 1.f, fptr(a), o, a->numel()), "mft_axpy");
  mft_check(mft_axpy(detail::handle(), 1.f, fptr(b), o, b->numel()), "mft_axpy");
  auto n = std::make_shared<AddNode>();
  n->inputs = {a, b};
  autograd::Engine::instance().record(out, n);
  return out;
}

TensorPtr lora_linear(const TensorPtr& x, const TensorPtr& W, const TensorPtr& b, const TensorPtr& A,
                      const TensorPtr& B, float scale) {
  require_f32(x, "linear input");
  if (!W || W->dim() != 2 || !W->contiguous()) throw std::invalid_argument("linear: W must be a contiguous [in, out] matrix");
  if (W->dtype() != kFloat32 && W->dtype() != kFloat16) throw std::invalid_argument("linear: W must be float32 or float16");
  if (W->requires_grad()) throw std::invalid_argument("linear: W is frozen on this path (no dW); call set_requires_grad(false)");
  if (b && b->requires_grad()) throw std::invalid_argument("linear: the bias is frozen on this path");
  const int64_t K = W->shape()[0], N = W->shape()[1];
  if (x->shape().empty() || x->shape().back() != K) throw std::invalid_argument("linear: x's last dimension must equal W's rows");
  if ((A == nullptr) != (B == nullptr)) throw std::invalid_argument("lora_linear: A and B must both be given");
  int r = 0;
  if (A) {
    require_f32(A, "lora A");
    require_f32(B, "lora B");
    r = (int)A->shape()[0];
    if (A->dim() != 2 || A->shape()[1] != K || B->dim() != 2 || B->shape()[0] != N || B->shape()[1] != r)
      throw std::invalid_argument("lora_linear: A must be [r, in] and B [out, r]");
  }
  if (b) {
    require_f32(b, "bias");
    if (b->numel() != N) throw std::invalid_argument("linear: bias must have out elements");
  }
  const int64_t M = rows_of(x);
  std::vector<int64_t> oshape = x->shape();
  oshape.back() = N;
  auto y = new_f32(oshape);
  TensorPtr xa = r ? new_f32({M, r}) : nullptr;
  const int wdt = W->dtype() == kFloat16 ? MFT_F16 : MFT_F32;
  mft_check(mft_lora_linear_fwd(detail::handle(), fptr(x), M, K, W->device_data(), wdt, N, fptr(b), fptr(A), fptr(B), r,
                                scale, static_cast<float*>(y->device_data()),
                                xa ? static_cast<float*>(xa->device_data()) : nullptr, nullptr),
            "mft_lora_linear_fwd");
  auto n = std::make_shared<LinearNode>();
  n->W = W;
  n->xa = xa;
  n->w_dtype = wdt;
  n->scale = scale;
  n->M = M;
  n->K = K;
  n->N = N;
  n->r = r;
  n->inputs = {x};
  if (A) {
    n->inputs.push_back(A);
    n->inputs.push_back(B);
  }
  autograd::Engine::instance().record(y, n);
  return y;
}

TensorPtr linear(const TensorPtr& x, const TensorPtr& W, const TensorPtr& b) {
  return lora_linear(x, W, b, nullptr, nullptr, 0.f);
}

TensorPtr causal_attention(const TensorPtr& q, const TensorPtr& k, const TensorPtr& v, float scale, int window,
                           const TensorPtr& key_mask) {
  require_f32(q, "attention q");
  require_f32(k, "attention k");
  require_f32(v, "attention v");
  if (q->dim() != 4 || k->dim() != 4 || v->dim() != 4 || k->shape() != v->shape())
    throw std::invalid_argument("causal_attention: q [B,S,Hq,hd], k/v [B,S,Hkv,hd]");
  const int B = (int)q->shape()[0], S = (int)q->shape()[1], Hq = (int)q->shape()[2], hd = (int)q->shape()[3];
  const int Hkv = (int)k->shape()[2];
  if (k->shape()[0] != B || k->shape()[1] != S || k->shape()[3] != hd || Hkv <= 0 || Hq % Hkv != 0)
    throw std::invalid_argument("causal_attention: q/k/v shapes disagree");
  if (key_mask) {
    require_f32(key_mask, "attention key mask");
    if (key_mask->numel() != (int64_t)B * S) throw std::invalid_argument("causal_attention: key mask must be [B, S]");
  }
  auto o = new_f32(q->shape());
  auto lse = new_f32({B, Hq, S});
  mft_check(mft_attn_fwd(detail::handle(), fptr(q), (int64_t)Hq * hd, fptr(k), (int64_t)Hkv * hd, fptr(v),
                         (int64_t)Hkv * hd, B, Hq, Hkv, S, hd, scale, 1, window, fptr(key_mask),
                         static_cast<float*>(o->device_data()), (int64_t)Hq * hd, static_cast<float*>(lse->device_data())),
            "mft_attn_fwd");
  auto n = std::make_shared<AttnNode>();
  n->o = o;
  n->lse = lse;
  n->kmask = key_mask;
  n->B = B;
  n->S = S;
  n->Hq = Hq;
  n->Hkv = Hkv;
  n->hd = hd;
  n->window = window;
  n->scale = scale;
  n->inputs = {q, k, v};
  autograd::Engine::instance().record(o, n);
  return o;
}

TensorPtr reshape(const TensorPtr& x, const std::vector<int64_t>& shape) {
  if (!x->contiguous()) throw std::invalid_argument("reshape: contiguous tensor required");
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  if (n != x->numel()) throw std::invalid_argument("reshape: element count differs");
  auto out = Tensor::view(shape, x->dtype(), x->device_data(), shape.empty() ? 1 : shape.back(), x);
  auto node = std::make_shared<ReshapeNode>();
  node->in_shape = x->shape();
  node->inputs = {x};
  autograd::Engine::instance().record(out, node);
  return out;
}

TensorPtr flatten(const TensorPtr& x, int start_dim, int end_dim) {
  const int nd = (int)x->dim();
  if (start_dim < 0) start_dim += nd;
  if (end_dim < 0) end_dim += nd;
  if (start_dim < 0 || end_dim >= nd || start_dim > end_dim) throw std::invalid_argument("flatten: bad dimensions");
  std::vector<int64_t> s;
  for (int i = 0; i < start_dim; ++i) s.push_back(x->shape()[i]);
  int64_t m = 1;
  for (int i = start_dim; i <= end_dim; ++i) m *= x->shape()[i];
  s.push_back(m);
  for (int i = end_dim + 1; i < nd; ++i) s.push_back(x->shape()[i]);
  return reshape(x, s);
}

// ------------------------------------------------------- layout / analysis --

namespace {

// Contiguous float32 input for the layout ops (views with a row pitch are
// gathered first).
TensorPtr dense_f32(const TensorPtr& x, const char* what) {
  if (!x || x->dtype() != kFloat32) throw std::invalid_argument(std::string(what) + ": float32 tensor required");
  if (x->contiguous()) return x;
  const int64_t rows = x->numel() / (x->shape().empty() ? 1 : x->shape().back());
  const int64_t shape[2] = {rows, x->shape().back()};
  const int64_t stride[2] = {x->pitch(), 1};
  auto out = new_f32(x->shape());
  mft_check(mft_strided_copy(detail::handle(), fptr(x), static_cast<float*>(out->device_data()), 2, shape, stride),
            "mft_strided_copy");
  return out;
}

int64_t norm_dim(int64_t d, int64_t nd, const char* what) {
  if (d < 0) d += nd;
  if (d < 0 || d >= nd) throw std::invalid_argument(std::string(what) + ": dimension out of range");
  return d;
}

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> st(shape.size(), 1);
  for (int64_t i = (int64_t)shape.size() - 2; i >= 0; --i) st[i] = st[i + 1] * shape[i + 1];
  return st;
}

TensorPtr gather(const TensorPtr& src, const std::vector<int64_t>& out_shape, const std::vector<int64_t>& strides,
                 const char* what) {
  if (out_shape.size() > 8) throw std::invalid_argument(std::string(what) + ": at most 8 dimensions");
  auto out = new_f32(out_shape);
  if (out->numel() == 0) return out;
  mft_check(mft_strided_copy(detail::handle(), fptr(src), static_cast<float*>(out->device_data()),
                             (int)out_shape.size(), out_shape.data(), strides.data()),
            "mft_strided_copy");
  return out;
}

}  // namespace

TensorPtr permute(const TensorPtr& x0, const std::vector<int64_t>& dims) {
  auto x = dense_f32(x0, "permute");
  const int64_t nd = x->dim();
  if ((int64_t)dims.size() != nd) throw std::invalid_argument("permute: one entry per dimension required");
  const auto in_st = contiguous_strides(x->shape());
  std::vector<int64_t> shape(nd), st(nd);
  std::vector<bool> seen(nd, false);
  for (int64_t i = 0; i < nd; ++i) {
    const int64_t d = norm_dim(dims[i], nd, "permute");
    if (seen[d]) throw std::invalid_argument("permute: repeated dimension");
    seen[d] = true;
    shape[i] = x->shape()[d];
    st[i] = in_st[d];
  }
  return gather(x, shape, st, "permute");
}

TensorPtr transpose(const TensorPtr& x, int64_t dim0, int64_t dim1) {
  const int64_t nd = x ? x->dim() : 0;
  std::vector<int64_t> dims(nd);
  for (int64_t i = 0; i < nd; ++i) dims[i] = i;
  std::swap(dims[norm_dim(dim0, nd, "transpose")], dims[norm_dim(dim1, nd, "transpose")]);
  return permute(x, dims);
}

TensorPtr repeat_kv_heads(const TensorPtr& x0, int n_rep) {
  auto x = dense_f32(x0, "repeat_kv_heads");
  if (x->dim() != 4 || n_rep < 1) throw std::invalid_argument("repeat_kv_heads: [B, H, S, D] and n_rep >= 1 required");
  const auto& s = x->shape();
  const auto in_st = contiguous_strides(s);
  // result viewed as [B, H, n_rep, S, D] with a zero stride on the repeat
  auto out = gather(x, {s[0], s[1], n_rep, s[2], s[3]}, {in_st[0], in_st[1], 0, in_st[2], in_st[3]},
                    "repeat_kv_heads");
  return reshape(out, {s[0], s[1] * n_rep, s[2], s[3]});
}

TensorPtr matmul(const TensorPtr& a0, const TensorPtr& b0) {
  auto a = dense_f32(a0, "matmul");
  auto b = dense_f32(b0, "matmul");
  if (a->dim() < 2 || b->dim() < 2) throw std::invalid_argument("matmul: operands need at least 2 dimensions");
  const int64_t M = a->shape()[a->dim() - 2], K = a->shape()[a->dim() - 1];
  const int64_t K2 = b->shape()[b->dim() - 2], N = b->shape()[b->dim() - 1];
  if (K != K2) throw std::invalid_argument("matmul: inner dimensions differ");
  const int64_t batch = a->numel() / std::max<int64_t>(1, M * K);
  const int64_t bbatch = b->numel() / std::max<int64_t>(1, K * N);
  if (bbatch != batch && !(b->dim() == 2))
    throw std::invalid_argument("matmul: leading dimensions of a and b must match (or b be 2-D)");
  std::vector<int64_t> shape(a->shape().begin(), a->shape().end() - 2);
  shape.push_back(M);
  shape.push_back(N);
  auto out = new_f32(shape);
  if (out->numel() == 0) return out;
  TensorPtr bb = b;
  if (b->dim() == 2 && batch > 1) {  // one shared right operand, repeated per batch entry
    bb = gather(b, {batch, K, N}, {0, N, 1}, "matmul");
  }
  mft_check(mft_batched_matmul(detail::handle(), fptr(a), fptr(bb), static_cast<float*>(out->device_data()),
                               (int)batch, (int)M, (int)K, (int)N),
            "mft_batched_matmul");
  return out;
}

// ----------------------------------------------------------------- loss --

namespace {

struct CeNode : Node {
  // inputs: logits
  TensorPtr labels;
  int ignore_index = -100;
  bool sum = false;
  int B = 0, S = 0;
  const char* name() const override { return "LmCrossEntropyBackward"; }
  std::vector<TensorPtr> apply(const TensorPtr& g) override {
    const float up = detail::read_scalar(g);
    const TensorPtr& logits = inputs[0];
    const int64_t V = logits->shape().back();
    auto dl = new_f32(logits->shape());
    auto scratch = new_f32({(int64_t)B * S});
    mft_check(mft_ce_fwd_bwd(detail::handle(), fptr(logits), static_cast<const int32_t*>(labels->device_data()), B, S, V,
                             ignore_index, up, sum ? 1 : 0, nullptr, nullptr, static_cast<float*>(dl->device_data()),
                             static_cast<float*>(scratch->device_data())),
              "mft_ce_fwd_bwd");
    return {dl};
  }
};

}  // namespace

namespace detail {

TensorPtr make_loss(double loss_sum, int64_t n_valid, bool sum) {
  const float v = sum ? (float)loss_sum : (n_valid > 0 ? (float)(loss_sum / (double)n_valid) : 0.f);
  return std::make_shared<Tensor>(std::vector<int64_t>{1}, &v, kFloat32, kCPU);
}

void check_ids(const TensorPtr& ids, int64_t vocab, const char* what) {
  const int32_t* p = static_cast<const Tensor&>(*ids).data<int32_t>();
  for (int64_t i = 0; i < ids->numel(); ++i)
    if (p[i] < 0 || (int64_t)p[i] >= vocab)
      throw std::invalid_argument(std::string(what) + ": token id " + std::to_string(p[i]) + " at position " +
                                  std::to_string(i) + " is outside [0, " + std::to_string(vocab) + ")");
}

void check_labels(const TensorPtr& labels, int64_t vocab, int ignore_index, const char* what) {
  const int32_t* p = static_cast<const Tensor&>(*labels).data<int32_t>();
  for (int64_t i = 0; i < labels->numel(); ++i)
    if (p[i] != ignore_index && (p[i] < 0 || (int64_t)p[i] >= vocab))
      throw std::invalid_argument(std::string(what) + ": label " + std::to_string(p[i]) + " at position " +
                                  std::to_string(i) + " is outside [0, " + std::to_string(vocab) +
                                  ") and is not ignore_index");
}

void make_parent_dirs(const std::string& path) {
  const size_t slash = path.find_last_of('/');
  if (slash == std::string::npos || slash == 0) return;
  const std::string dir = path.substr(0, slash);
  for (size_t i = 1; i <= dir.size(); ++i)
    if (i == dir.size() || dir[i] == '/') (void)::mkdir(dir.substr(0, i).c_str(), 0755);
}

void write_npy(const std::string& path, const void* data, const std::vector<int64_t>& shape, bool int32) {
  make_parent_dirs(path);
  std::string dict = std::string("{'descr': '") + (int32 ? "<i4" : "<f4") + "', 'fortran_order': False, 'shape': (";
  int64_t n = 1;
  for (size_t i = 0; i < shape.size(); ++i) {
    dict += std::to_string(shape[i]) + (shape.size() == 1 || i + 1 < shape.size() ? "," : "");
    if (i + 1 < shape.size()) dict += " ";
    n *= shape[i];
  }
  dict += "), }";
  // magic (6) + version (2) + header length (2) + header, padded with spaces
  // and a newline to a multiple of 64 bytes
  const size_t total = 10 + dict.size() + 1;
  dict += std::string((64 - total % 64) % 64, ' ') + "\n";
  std::ofstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("write_npy: cannot open " + path);
  const char magic[8] = {'\x93', 'N', 'U', 'M', 'P', 'Y', 1, 0};
  f.write(magic, 8);
  const uint16_t hl = (uint16_t)dict.size();
  const char hb[2] = {(char)(hl & 0xff), (char)(hl >> 8)};
  f.write(hb, 2);
  f.write(dict.data(), (std::streamsize)dict.size());
  f.write(static_cast<const char*>(data), (std::streamsize)(n * 4));
  if (!f) throw std::runtime_error("write_npy: write failed for " + path);
}

bool parse_reduction(const std::string& r) {
  if (r == "mean") return false;
  if (r == "sum") return true;
  throw std::invalid_argument("lm_cross_entropy: reduction must be \"mean\" or \"sum\"");
}

}  // namespace detail

TensorPtr lm_cross_entropy(const TensorPtr& logits, const TensorPtr& labels, int ignore_index,
                           const std::string& reduction) {
  const bool sum = detail::parse_reduction(reduction);
  if (!logits || logits->dtype() != kFloat32 || logits->dim() != 3)
    throw std::invalid_argument("lm_cross_entropy: logits must be float32 [B, S, V]");
  if (!labels || labels->dtype() != kInt32 || labels->numel() != logits->shape()[0] * logits->shape()[1])
    throw std::invalid_argument("lm_cross_entropy: labels must be int32 [B, S]");
  detail::check_labels(labels, logits->shape()[2], ignore_index, "lm_cross_entropy");
  // Logits produced by an engine-backed model go through the model's own
  // loss (its logits buffer turns into dlogits in place).
  if (auto hook = detail::model_loss_hook(logits)) return hook(labels, ignore_index, sum);
  if (!logits->contiguous()) throw std::invalid_argument("lm_cross_entropy: contiguous logits required");
  const int B = (int)logits->shape()[0], S = (int)logits->shape()[1];
  const int64_t V = logits->shape()[2];
  auto stats = std::make_shared<Tensor>(std::vector<int64_t>{4}, kFloat32, kGPU);  // double sum + int64 count
  auto scratch = new_f32({(int64_t)B * S});
  char* st = static_cast<char*>(stats->device_data());
  mft_check(mft_ce_fwd_bwd(detail::handle(), fptr(logits), static_cast<const int32_t*>(labels->device_data()), B, S, V,
                           ignore_index, 1.f, 0, reinterpret_cast<double*>(st), reinterpret_cast<int64_t*>(st + 8),
                           nullptr, static_cast<float*>(scratch->device_data())),
            "mft_ce_fwd_bwd");
  double ls = 0;
  int64_t nv = 0;
  hip_check(hipMemcpy(&ls, st, 8, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  hip_check(hipMemcpy(&nv, st + 8, 8, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  auto loss = detail::make_loss(ls, nv, sum);
  auto n = std::make_shared<CeNode>();
  n->labels = labels;
  n->ignore_index = ignore_index;
  n->sum = sum;
  n->B = B;
  n->S = S;
  n->inputs = {logits};
  autograd::Engine::instance().record(loss, n);
  return loss;
}

float perplexity_from_loss(float loss) { return std::exp(loss); }

// ------------------------------------------------------------------ Adam --

// Moment state of one parameter.  Keyed by the parameter's address, so the
// entry also remembers which tensor it belongs to: a parameter created after
// another was freed can reuse its address, and then gets fresh state.
struct Adam::State {
  std::weak_ptr<Tensor> owner;
  TensorPtr m, v;
};

struct Adam::GroupState {
  std::weak_ptr<MirrorGroup> group;
  TensorPtr m, v;  // one float per byte/4 of the group
};

Adam::Adam(const AdamConfig& cfg) : cfg_(cfg) {}
Adam::~Adam() = default;

void Adam::step(const std::vector<TensorPtr>& params, const std::vector<TensorPtr>& grads) {
  if (params.size() != grads.size()) throw std::invalid_argument("Adam::step: params and grads differ in length");
  ++t_;
  // Moment storage: a parameter inside a mirror group takes views into the
  // group's moment arena; others own theirs.
  std::vector<State*> sts(params.size(), nullptr);
  for (size_t i = 0; i < params.size(); ++i) {
    const TensorPtr& p = params[i];
    const TensorPtr& g = grads[i];
    if (!p || !g) continue;
    require_f32(p, "Adam parameter");
    require_f32(g, "Adam gradient");
    if (g->numel() != p->numel()) throw std::invalid_argument("Adam::step: gradient size differs from its parameter");
    auto& st = state_[p.get()];
    if (!st || st->owner.lock() != p || st->m->numel() != p->numel()) {
      st = std::make_unique<State>();
      st->owner = p;
      if (const auto& grp = p->mirror()) {
        auto& gs = gstate_[grp.get()];
        if (!gs || gs->group.lock() != grp) {
          gs = std::make_unique<GroupState>();
          gs->group = grp;
          gs->m = new_f32({(int64_t)(grp->bytes / 4)});
          gs->v = new_f32({(int64_t)(grp->bytes / 4)});
        }
        char* mb = static_cast<char*>(gs->m->device_data()) + p->mirror_offset();
        char* vb = static_cast<char*>(gs->v->device_data()) + p->mirror_offset();
        st->m = Tensor::view(p->shape(), kFloat32, mb, p->shape().empty() ? 1 : p->shape().back(), gs->m);
        st->v = Tensor::view(p->shape(), kFloat32, vb, p->shape().empty() ? 1 : p->shape().back(), gs->v);
      } else {
        st->m = new_f32(p->shape());
        st->v = new_f32(p->shape());
      }
    }
    sts[i] = st.get();
  }
  // Every member of one parameter group, each with its gradient at the same
  // offset of one gradient group (the LoRA parameters and gradients of a
  // model, as get_lora_parameters() and their grad() hand them out): one
  // update over the whole arenas (padding between tensors has zero
  // gradient and stays zero).
  const MirrorGroup* pg = params.empty() || !params[0] ? nullptr : params[0]->mirror().get();
  const MirrorGroup* gg = grads.empty() || !grads[0] ? nullptr : grads[0]->mirror().get();
  bool fused = pg && gg && pg->bytes == gg->bytes && (int)params.size() == pg->members;
  if (fused) {
    std::unordered_set<size_t> offs;
    for (size_t i = 0; i < params.size() && fused; ++i)
      fused = params[i] && grads[i] && params[i]->mirror().get() == pg && grads[i]->mirror().get() == gg &&
              params[i]->mirror_offset() == grads[i]->mirror_offset() &&
              offs.insert(params[i]->mirror_offset()).second;
  }
  if (fused) {
    GroupState& gs = *gstate_[pg];
    float* pd = static_cast<float*>(params[0]->device_data());  // flushes host edits of the parameters
    pd -= params[0]->mirror_offset() / 4;
    // Gradients edited on the host (the drivers' clip loop scales them in
    // place) are read by the update straight from the pinned host copy: no
    // upload, whose copy engine → kernel hand-off alone costs ≈50 µs.  The
    // device copy stays stale (host-newer state); the drivers' zero_grad()
    // that follows replaces it without an upload.
    MirrorGroup& gm = *grads[0]->mirror();
    const bool from_host = gm.state == 2 && gm.host_dev && gm.zeros.empty();
    float* gd = from_host ? static_cast<float*>(gm.host_dev)
                          : static_cast<float*>(grads[0]->device_data()) - grads[0]->mirror_offset() / 4;
    mft_check(mft_adam_step(detail::handle(), pd, gd, static_cast<float*>(gs.m->device_data()),
                            static_cast<float*>(gs.v->device_data()), (int64_t)(pg->bytes / 4), cfg_.learning_rate,
                            cfg_.beta1, cfg_.beta2, cfg_.epsilon, cfg_.weight_decay, t_, nullptr, 0),
              "mft_adam_step");
    if (from_host) mark_host_read(gm);
    params[0]->mark_device_written();
    return;
  }
  for (size_t i = 0; i < params.size(); ++i) {
    if (!sts[i]) continue;
    const TensorPtr& p = params[i];
    const TensorPtr& g = grads[i];
    mft_check(mft_adam_step(detail::handle(), static_cast<float*>(p->device_data()), static_cast<float*>(g->device_data()),
                            static_cast<float*>(sts[i]->m->device_data()), static_cast<float*>(sts[i]->v->device_data()),
                            p->numel(), cfg_.learning_rate, cfg_.beta1, cfg_.beta2, cfg_.epsilon, cfg_.weight_decay, t_,
                            nullptr, 0),
              "mft_adam_step");
    p->mark_device_written();
  }
}

// ---------------------------------------------------------------- memory --

MemoryManager& MemoryManager::instance() {
  static MemoryManager m;
  return m;
}

void MemoryManager::force_cleanup() { dev_cache_clear(); }
void MemoryManager::clear_unused_memory() { dev_cache_clear(); }
void MemoryManager::cleanup_dead_references() {}

void MemoryManager::print_memory_stats() const {
  size_t free_b = 0, total_b = 0;
  hip_check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
  std::printf("[MemoryManager] device: %.1f MiB used of %.1f MiB\n", (total_b - free_b) / 1048576.0,
              total_b / 1048576.0);
}

size_t MemoryMonitor::get_system_memory_usage() {
  std::ifstream f("/proc/self/statm");
  size_t pages = 0, resident = 0;
  if (f >> pages >> resident) return resident * 4096;
  return 0;
}

}  // namespace ops
