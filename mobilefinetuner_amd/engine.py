"""Python handle on the device-resident LoRA training step
(include/mft_engine.h).  All compute runs in libmft_hip.so; torch is used for
the device buffers of token ids / labels and the stream."""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import call, lib
from .configs import ModelConfig


def _dev(t, dt, what):
    """Device pointer of a contiguous tensor of dtype `dt` (None passes)."""
    if t is None:
        return None
    if not t.is_cuda or not t.is_contiguous() or t.dtype != dt:
        raise TypeError(f"{what}: contiguous {dt} device tensor required, got {t.dtype}")
    return C.c_void_p(t.data_ptr())


class Model:
    def __init__(self, cfg: ModelConfig, max_tokens: int, stream=None):
        self.cfg = cfg
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        self.stream = stream
        h = C.c_void_p()
        ccfg = cfg.to_ctypes()
        call("mft_model_create", C.byref(h), C.byref(ccfg), max_tokens, C.c_void_p(stream))
        self.h = h
        self.params = []
        n = lib().mft_model_num_params(h)
        for i in range(n):
            name = C.c_char_p()
            ndim = C.c_int()
            dims = (C.c_int64 * 2)()
            tr = C.c_int()
            f16 = C.c_int()
            data = C.c_void_p()
            grad = C.c_void_p()
            call("mft_model_param_info", h, i, C.byref(name), C.byref(ndim), dims, C.byref(tr),
                 C.byref(f16), C.byref(data), C.byref(grad))
            shape = tuple(dims[j] for j in range(ndim.value))
            self.params.append(dict(name=name.value.decode(), shape=shape, trainable=bool(tr.value),
                                    f16=bool(f16.value), data=data.value, grad=grad.value))
        self.by_name = {p["name"]: p for p in self.params}

    def close(self):
        if self.h:
            call("mft_model_destroy", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- parameter transfer (tests) ---
    def _handle(self):
        from .ops import handle
        return handle()

    def set_param(self, name: str, array) -> None:
        import numpy as np
        p = self.by_name[name]
        a = np.ascontiguousarray(array, dtype=np.uint16 if p["f16"] else np.float32)
        n = 1
        for s in p["shape"]:
            n *= s
        if a.size != n:
            raise ValueError(f"{name}: expected {n} elements, got {a.size}")
        call("mft_memcpy_h2d", self._handle(), C.c_void_p(p["data"]), a.ctypes.data_as(C.c_void_p),
             a.nbytes)
        if self.cfg.shard_budget > 0 and not p["trainable"]:
            call("mft_model_shard_reset", self.h)  # drop stale HBM copies of streamed tensors

    def get(self, name: str, grad: bool = False):
        import numpy as np
        p = self.by_name[name]
        dt = np.uint16 if (p["f16"] and not grad) else np.float32
        out = np.empty(p["shape"], dtype=dt)
        ptr = p["grad"] if grad else p["data"]
        call("mft_memcpy_d2h", self._handle(), out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr),
             out.nbytes)
        return out

    def init_params(self, seed: int, std: float = 0.02, a_std: float | None = None,
                    b_std: float = 0.02):
        if a_std is None:
            a_std = 1.0 / self.cfg.lora_r
        call("mft_model_init_params", self.h, seed, std, a_std, b_std)

    # --- step ---
    def fwd_bwd(self, ids, labels, mask=None, n_micro=1, seqs_per_micro=None, S=None,
                upstream=None):
        S = S or ids.shape[-1]
        nseq = ids.numel() // S
        seqs_per_micro = seqs_per_micro or nseq // n_micro
        if upstream is None:
            upstream = 1.0 / n_micro
        call("mft_model_fwd_bwd", self.h, _dev(ids, torch.int32, "ids"),
             _dev(mask, torch.float32, "mask"), _dev(labels, torch.int32, "labels"), n_micro,
             seqs_per_micro, S, upstream)

    def forward(self, ids, labels=None, mask=None, logits=None, n_micro=1, S=None):
        S = S or ids.shape[-1]
        nseq = ids.numel() // S
        call("mft_model_forward", self.h, _dev(ids, torch.int32, "ids"),
             _dev(mask, torch.float32, "mask"), _dev(labels, torch.int32, "labels"), n_micro,
             nseq // n_micro, S, _dev(logits, torch.float32, "logits"))

    def opt_step(self, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, clip=1.0):
        call("mft_model_opt_step", self.h, lr, b1, b2, eps, wd, clip)

    def train_step(self, ids, labels, mask=None, n_micro=1, seqs_per_micro=None, S=None,
                   upstream=None, lr=2e-4, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, clip=1.0,
                   graph=True):
        """Whole optimizer step (fwd+CE+bwd over all micro-batches, clip, Adam);
        graph=True replays a captured HIP graph after the first call."""
        S = S or ids.shape[-1]
        nseq = ids.numel() // S
        seqs_per_micro = seqs_per_micro or nseq // n_micro
        if upstream is None:
            upstream = 1.0 / n_micro
        call("mft_model_train_step", self.h, _dev(ids, torch.int32, "ids"),
             _dev(mask, torch.float32, "mask"), _dev(labels, torch.int32, "labels"), n_micro,
             seqs_per_micro, S, upstream, lr, b1, b2, eps, wd, clip, int(graph))

    def shard_stats(self):
        """(loads, hits, budget) of the shard store (zeros when not sharded)."""
        lo, hi, bu = C.c_int64(), C.c_int64(), C.c_int64()
        call("mft_model_shard_stats", self.h, C.byref(lo), C.byref(hi), C.byref(bu))
        return lo.value, hi.value, bu.value

    def set_training(self, on: bool):
        """Training forwards apply LoRA dropout; evaluation forwards do not."""
        call("mft_model_set_training", self.h, int(on))

    def read_stats(self):
        loss = C.c_float()
        n = C.c_int64()
        gn = C.c_float()
        call("mft_model_read_stats", self.h, C.byref(loss), C.byref(n), C.byref(gn))
        return loss.value, n.value, gn.value

    # --- alignment-dump debug mode (tests) ---
    def set_retain(self, layers):
        """Keep the activations and activation gradients of `layers` in later
        steps (mft_engine.h: mft_model_set_retain); [] turns it off."""
        mask = 0
        for l in layers:
            mask |= 1 << l
        call("mft_model_set_retain", self.h, C.c_uint64(mask))

    def _kept(self, fn, layer, name):
        import numpy as np
        p, rows, cols, ld = C.c_void_p(), C.c_int64(), C.c_int64(), C.c_int64()
        call(fn, self.h, layer, name.encode(), C.byref(p), C.byref(rows), C.byref(cols), C.byref(ld))
        torch.cuda.synchronize()
        n = (rows.value - 1) * ld.value + cols.value
        flat = np.empty(n, np.float32)
        call("mft_memcpy_d2h", self._handle(), flat.ctypes.data_as(C.c_void_p), p, flat.nbytes)
        return np.lib.stride_tricks.as_strided(flat, (rows.value, cols.value), (ld.value * 4, 4)).copy()

    def activation(self, layer, name):
        """A kept activation of the last forward as [rows, cols] (mft_model_activation)."""
        return self._kept("mft_model_activation", layer, name)

    def activation_grad(self, layer, name):
        """A retained activation gradient of the last backward (mft_model_activation_grad)."""
        return self._kept("mft_model_activation_grad", layer, name)

    # --- timing ---
    def set_timing(self, on: bool):
        call("mft_model_set_timing", self.h, int(on))

    def reset_timing(self):
        call("mft_model_reset_timing", self.h)

    def timing(self, cls: int):
        ms = C.c_double()
        work = C.c_double()
        n = C.c_int64()
        call("mft_model_timing", self.h, cls, C.byref(ms), C.byref(work), C.byref(n))
        return ms.value, work.value, n.value


CLS_LINEAR, CLS_LMHEAD, CLS_ATTN, CLS_CE, CLS_RANK = range(5)
