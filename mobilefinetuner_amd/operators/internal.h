// internal.h — shared helpers of the finetune_ops host library (not installed).
#pragma once
#include <hip/hip_runtime.h>

#include <functional>
#include <memory>
#include <string>

#include "finetune_ops/core/tensor.h"
#include "mft_hip.h"

namespace ops {
namespace detail {

void hip_check(hipError_t e, const char* what);
void mft_check(int rc, const char* what);
mft_handle handle();
float read_scalar(const TensorPtr& t);
// Queues a device→host copy of t's mirror group behind the stream's work
// (the engine backward's gradients, read by the drivers' clip loop next).
void prefetch_host(const TensorPtr& t);
TensorPtr make_loss(double loss_sum, int64_t n_valid, bool sum);
bool parse_reduction(const std::string& r);

// Loss over logits that an engine-backed model produced (nullptr when the
// tensor is not such a logits view).
using ModelLoss = std::function<TensorPtr(const TensorPtr& labels, int ignore_index, bool sum)>;
ModelLoss model_loss_hook(const TensorPtr& logits);

// Host-side range checks of int32 index tensors (read through the host
// mirror; ids and labels come from the host): every token id in [0, vocab),
// every label in [0, vocab) or equal to ignore_index.  Throws
// std::invalid_argument naming the first offender.
void check_ids(const TensorPtr& ids, int64_t vocab, const char* what);
// Creates the parent directories of a file path (mkdir -p).
void make_parent_dirs(const std::string& path);
// Writes a row-major array as a NumPy .npy file (format 1.0, little
// endian): descr "<f4" or "<i4"; creates the parent directory.
void write_npy(const std::string& path, const void* data, const std::vector<int64_t>& shape, bool int32);
void check_labels(const TensorPtr& labels, int64_t vocab, int ignore_index, const char* what);

}  // namespace detail
}  // namespace ops
