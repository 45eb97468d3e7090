// finetune_ops/core/tensor.h — the operators library's Tensor on the MI355X
// backend.
//
// Replaces the reference's operators/finetune_ops/core Tensor (absent from
// the published tree; its interface is fixed by the drivers' call sites):
//   make_shared<Tensor>(vector<int64_t>{B,S}, host_ptr, kInt32, kCPU)
//       (gpt2_medium_lora_finetune/src/mmlu/mmlu_runner.cpp:149-154,
//        gemma_3_270m_lora_finetune/src/eval_mmlu_gemma.cpp:200-209)
//   t->data<float>() as a host pointer, read and written in place
//       (gpt2_small_lora_finetune/src/main.cpp:354,389-405,476)
//   shape(), numel(), dtype(), grad(), zero_grad(), set_requires_grad(),
//   retain_grad(), backward()   (main.cpp:250,277,387,484,503-504;
//        gemma_3_270m_lora_finetune/src/main.cpp:84,503-504)
//
// Storage lives in HBM.  data<T>() returns a host mirror that is refreshed
// from the device when stale; after a non-const data<T>() the host copy is
// taken to be the newer one and is copied back before the next device use.
// So a driver's host loops over grads (the clip at main.cpp:384-409) keep
// working, and everything else stays on the GPU.  `Device` is recorded for
// source compatibility; every tensor is device-resident.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace ops {

enum DType { kFloat32 = 0, kInt32 = 1, kFloat16 = 2 };
enum Device { kCPU = 0, kGPU = 1 };

size_t dtype_size(DType t);

class Tensor;
using TensorPtr = std::shared_ptr<Tensor>;
// One host mirror shared by views that tile a device range (a model's LoRA
// parameter or gradient arena): the first host access copies the whole
// range once, and host edits go back in one copy before the next device use.
struct MirrorGroup;

namespace autograd {
class Node;
}

class Tensor : public std::enable_shared_from_this<Tensor> {
 public:
  // Zero-filled tensor.
  explicit Tensor(std::vector<int64_t> shape, DType dtype = kFloat32, Device device = kCPU);
  // Tensor holding a copy of `data` (host memory, row-major, numel elements).
  Tensor(std::vector<int64_t> shape, const void* data, DType dtype, Device device = kCPU);
  // View over device memory owned elsewhere (kept alive by `owner`); the
  // last dimension's rows are `pitch` elements apart (pitch >= last dim).
  static TensorPtr view(std::vector<int64_t> shape, DType dtype, void* device_ptr, int64_t pitch,
                        std::shared_ptr<void> owner);
  // A mirror group over device bytes [base, base + bytes), and a contiguous
  // view inside it whose host copy is the group's.
  static std::shared_ptr<MirrorGroup> mirror_group(void* base, size_t bytes);
  static TensorPtr view(std::vector<int64_t> shape, DType dtype, void* device_ptr, std::shared_ptr<void> owner,
                        std::shared_ptr<MirrorGroup> group);
  ~Tensor();
  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;

  const std::vector<int64_t>& shape() const { return shape_; }
  int64_t dim() const { return (int64_t)shape_.size(); }
  int64_t numel() const { return numel_; }
  DType dtype() const { return dtype_; }
  Device device() const { return device_; }
  bool empty() const { return numel_ == 0; }

  // Host view (row-major, contiguous).  The non-const form marks the host
  // copy as the newer one.
  template <class T>
  T* data() {
    sync_host(true);
    return reinterpret_cast<T*>(host_ptr());
  }
  template <class T>
  const T* data() const {
    sync_host(false);
    return reinterpret_cast<const T*>(host_ptr());
  }
  // Device pointer (pending host edits are copied back first).  The const
  // form does not mark the device copy as changed.
  void* device_data();
  const void* device_data() const;
  int64_t pitch() const { return pitch_; }
  bool contiguous() const { return shape_.empty() || pitch_ == shape_.back(); }
  // Called after a kernel wrote the device copy: the host mirror is stale.
  void mark_device_written();
  // The host copy is at least as new as the device copy: data() reads no
  // device memory (and waits for nothing).
  bool host_current() const;

  // ---- autograd ----
  bool requires_grad() const { return requires_grad_; }
  void set_requires_grad(bool r) { requires_grad_ = r; }
  TensorPtr grad() const { return grad_; }
  void set_grad(TensorPtr g) { grad_ = std::move(g); }
  void zero_grad();
  void retain_grad() { retain_grad_ = true; }
  bool retains_grad() const { return retain_grad_; }
  void backward();                               // scalar root, seed 1
  void backward(const TensorPtr& grad_output);   // seed given
  const std::shared_ptr<autograd::Node>& grad_fn() const { return grad_fn_; }
  void set_grad_fn(std::shared_ptr<autograd::Node> fn) { grad_fn_ = std::move(fn); }
  bool is_leaf() const { return grad_fn_ == nullptr; }

  // Device memory owner of a view (the model whose arena it points into).
  const std::shared_ptr<void>& owner() const { return owner_; }
  // Mirror group of a grouped view (null otherwise) and the view's byte
  // offset in it.
  const std::shared_ptr<MirrorGroup>& mirror() const { return group_; }
  size_t mirror_offset() const { return group_off_; }

 private:
  Tensor() = default;
  void init_shape(std::vector<int64_t> shape, DType dtype, Device device);
  void sync_host(bool will_write) const;
  void upload_if_dirty() const;
  char* host_ptr() const;

  std::vector<int64_t> shape_;
  int64_t numel_ = 0;
  DType dtype_ = kFloat32;
  Device device_ = kCPU;
  mutable void* dev_ = nullptr;
  bool owns_ = false;
  // host-built tensors of at most kLazyBytes: the device block is taken
  // (and the host values copied there) at the first device_data()
  static constexpr size_t kLazyBytes = 64;
  mutable bool lazy_dev_ = false;
  int64_t pitch_ = 0;
  std::shared_ptr<void> owner_;
  // host mirror: 0 = stale, 1 = equal to the device, 2 = newer than the device
  mutable std::vector<char> host_;
  mutable int host_state_ = 0;
  std::shared_ptr<MirrorGroup> group_;  // shared host mirror (grouped views)
  size_t group_off_ = 0;

  bool requires_grad_ = false;
  bool retain_grad_ = false;
  TensorPtr grad_;
  std::shared_ptr<autograd::Node> grad_fn_;
};

// Factories.
TensorPtr zeros(const std::vector<int64_t>& shape, DType dtype = kFloat32);
TensorPtr from_host(const std::vector<int64_t>& shape, const void* data, DType dtype);

}  // namespace ops
