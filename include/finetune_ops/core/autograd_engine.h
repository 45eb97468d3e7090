// finetune_ops/core/autograd_engine.h — the tape behind Tensor::backward().
//
// Replaces ops::autograd::Engine of the reference's operators library
// (absent), used as Engine::instance().set_enabled(bool) / clear_graph()
// (gpt2_small_lora_finetune/src/main.cpp:414-420) and implicitly by
// loss->backward() (main.cpp:484).  Each differentiable op records a Node
// holding its inputs; backward() visits the nodes reachable from the root in
// reverse topological order, hands each its output gradient, and
// accumulates leaf gradients (grads add up across backward() calls until
// zero_grad(), the driver's gradient accumulation, main.cpp:471-487).
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "finetune_ops/core/tensor.h"

namespace ops {
namespace autograd {

class Node {
 public:
  virtual ~Node() = default;
  virtual const char* name() const = 0;
  // Gradients of the inputs, in `inputs` order (nullptr = none); grad_out
  // is the gradient of this node's output.
  virtual std::vector<TensorPtr> apply(const TensorPtr& grad_out) = 0;
  std::vector<TensorPtr> inputs;
};

class Engine {
 public:
  static Engine& instance();
  void set_enabled(bool on) { enabled_ = on; }
  bool is_enabled() const { return enabled_; }
  // Drops the graph recorded so far: outputs created since keep their values
  // but no longer reach their inputs.
  void clear_graph();
  void backward(const TensorPtr& root, const TensorPtr& grad_output);
  // Records fn as the producer of out when any input needs a gradient.
  void record(const TensorPtr& out, std::shared_ptr<Node> fn);

 private:
  bool enabled_ = true;
  std::vector<std::weak_ptr<Tensor>> recorded_;
};

// Adds g into t's gradient (allocating it as zeros on first use).
void accumulate_grad(const TensorPtr& t, const TensorPtr& g);

}  // namespace autograd
}  // namespace ops
