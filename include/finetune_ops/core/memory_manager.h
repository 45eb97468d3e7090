// finetune_ops/core/memory_manager.h — memory housekeeping hooks.
//
// Replaces MemoryManager / MemoryMonitor of the reference (absent), which
// the drivers call between steps (gpt2_small_lora_finetune/src/main.cpp:
// 465,509-517,558).  On this backend tensors are device allocations freed
// when their last reference goes, so the cleanup calls synchronise and
// report; get_system_memory_usage() is the process's resident host memory.
#pragma once
#include <cstddef>

namespace ops {

class MemoryManager {
 public:
  static MemoryManager& instance();
  void force_cleanup();             // waits for queued device work
  void clear_unused_memory();       // same (nothing is cached)
  void cleanup_dead_references();   // nothing to do: references free on release
  void print_memory_stats() const;  // device bytes in use / total
};

class MemoryMonitor {
 public:
  static size_t get_system_memory_usage();  // resident set size in bytes
};

}  // namespace ops
