"""mobilefinetuner_amd — MI355X (gfx950) implementation of MobileFineTuner's
LoRA training hot path.

Layout:
  csrc/            HIP kernels (GEMM/LoRA, attention, cross-entropy, norms,
                   Adam), the C-ABI (capi.cpp) and the step engine
                   (engine.cpp); built into libmft_hip.so in this directory.
  _lib.py          ctypes declarations of the C-ABI.
  ops.py           thin Python wrappers that take torch device tensors and
                   call the C-ABI (used by the parity tests).
  engine.py        the training-step engine (GPT-2 / Qwen2 / Gemma3 LoRA).
  configs.py       the model/batch configurations of the benchmark.
"""
from ._lib import LIB_PATH, MFTError, lib  # noqa: F401

__all__ = ["LIB_PATH", "MFTError", "lib"]
