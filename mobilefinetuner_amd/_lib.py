"""ctypes bindings of libmft_hip.so (C-ABI declared in include/mft_hip.h and
include/mft_engine.h).

The library is the product path: nothing here falls back to a CPU or PyTorch
implementation.  If the shared object is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmft_hip.so")

c_f32p = C.c_void_p  # device pointers are passed as integers
_lib = None


class MFTError(RuntimeError):
    pass


class ModelCfg(C.Structure):
    """Mirror of mft_model_cfg (include/mft_engine.h)."""
    _fields_ = [
        ("arch", C.c_int), ("n_layer", C.c_int), ("d", C.c_int), ("n_head", C.c_int),
        ("n_kv_head", C.c_int), ("head_dim", C.c_int), ("d_ff", C.c_int), ("max_pos", C.c_int),
        ("vocab", C.c_int64), ("lora_r", C.c_int), ("lora_alpha", C.c_float),
        ("lora_mask", C.c_int), ("norm_eps", C.c_float), ("rope_theta", C.c_double),
        ("rope_local_theta", C.c_double), ("sliding_pattern", C.c_int),
        ("sliding_window", C.c_int), ("attn_scale", C.c_float), ("w_fp16", C.c_int),
        ("lora_dropout", C.c_float), ("dropout_seed", C.c_uint64), ("shard_budget", C.c_int64),
    ]


# name -> (restype, argtypes)
_P = C.c_void_p
_I = C.c_int
_L = C.c_int64
_F = C.c_float
_D = C.c_double
_SIGS = {
    "mft_create": (_I, [C.POINTER(_P), _P]),
    "mft_destroy": (_I, [_P]),
    "mft_set_stream": (_I, [_P, _P]),
    "mft_get_stream": (_P, [_P]),
    "mft_synchronize": (_I, [_P]),
    "mft_last_error": (C.c_char_p, []),
    "mft_version": (C.c_char_p, []),
    "mft_set_sync_check": (_I, [_I]),
    "mft_malloc": (_I, [C.POINTER(_P), C.c_size_t]),
    "mft_free": (_I, [_P]),
    "mft_memcpy_h2d": (_I, [_P, _P, _P, C.c_size_t]),
    "mft_memcpy_d2h": (_I, [_P, _P, _P, C.c_size_t]),
    "mft_memset": (_I, [_P, _P, _I, C.c_size_t]),
    "mft_lora_linear_fwd": (_I, [_P, _P, _L, _L, _P, _I, _L, _P, _P, _P, _I, _F, _P, _P, _P]),
    "mft_lora_linear_bwd": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _L, _L, _L, _I, _F, _P, _P, _P,
                                 _I, _I]),
    "mft_attn_fwd": (_I, [_P, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _L,
                          _P]),
    "mft_attn_bwd": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _L, _P, _L, _P, _I, _I, _I, _I, _I, _F,
                          _I, _I, _P, _P, _L, _P, _L, _P, _L]),
    "mft_ce_fwd_bwd": (_I, [_P, _P, _P, _I, _I, _L, _I, _F, _L, _P, _P, _P, _P]),
    "mft_ce_fwd_bwd_noalloc": (_I, [_P, _P, _P, _I, _I, _L, _I, _F, _L, _P, _P, _P, _P]),
    "mft_dequant_f16": (_I, [_P, _P, _P, _L]),
    "mft_quant_f16": (_I, [_P, _P, _P, _L]),
    "mft_adam_step": (_I, [_P, _P, _P, _P, _P, _L, _F, _F, _F, _F, _F, _I, _P, _I]),
    "mft_sumsq": (_I, [_P, _P, _L, _P]),
    "mft_clip_scale": (_I, [_P, _P, _F, _P, _P]),
    "mft_layernorm_fwd": (_I, [_P, _P, _P, _P, _L, _L, _F, _P, _P, _P]),
    "mft_layernorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _P, _I]),
    "mft_rmsnorm_fwd": (_I, [_P, _P, _P, _L, _L, _F, _I, _P, _P]),
    "mft_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _L, _L, _I, _P, _I]),
    "mft_glu_fwd": (_I, [_P, _P, _P, _L, _I, _P]),
    "mft_glu_bwd": (_I, [_P, _P, _P, _P, _L, _I, _P, _P]),
    "mft_rope": (_I, [_P, _P, _L, _I, _I, _I, _I, _D, _I]),
    "mft_strided_copy": (_I, [_P, _P, _P, _I, _P, _P]),
    "mft_batched_matmul": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "mft_embed": (_I, [_P, _P, _L, _I, _P, _L, _I, _P, _L, _F, _P, _P]),
    "mft_scale": (_I, [_P, _P, _L, _F, _P]),
    "mft_axpy": (_I, [_P, _F, _P, _P, _L]),
    "mft_fill": (_I, [_P, _P, _L, _F]),
    # engine
    "mft_model_create": (_I, [C.POINTER(_P), C.POINTER(ModelCfg), _L, _P]),
    "mft_model_destroy": (_I, [_P]),
    "mft_model_num_params": (_I, [_P]),
    "mft_model_param_info": (_I, [_P, _I, C.POINTER(C.c_char_p), C.POINTER(_I),
                                  C.POINTER(_L), C.POINTER(_I), C.POINTER(_I), C.POINTER(_P),
                                  C.POINTER(_P)]),
    "mft_model_init_params": (_I, [_P, C.c_uint64, _F, _F, _F]),
    "mft_model_fwd_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _F]),
    "mft_model_forward": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "mft_model_forward_train": (_I, [_P, _P, _P, _I, _I]),
    "mft_model_logits": (_I, [_P, C.POINTER(_P), C.POINTER(_L)]),
    "mft_model_ce": (_I, [_P, _P, _I, _I, _I, _F, _L, _I, _P, _P]),
    "mft_model_backward": (_I, [_P, _P, _I, _I]),
    "mft_model_opt_step": (_I, [_P, _F, _F, _F, _F, _F, _F]),
    "mft_model_train_step": (_I, [_P, _P, _P, _P, _I, _I, _I, _F, _F, _F, _F, _F, _F, _F, _I]),
    "mft_model_read_stats": (_I, [_P, C.POINTER(_F), C.POINTER(_L), C.POINTER(_F)]),
    "mft_model_activation": (_I, [_P, _I, C.c_char_p, C.POINTER(_P), C.POINTER(_L), C.POINTER(_L), C.POINTER(_L)]),
    "mft_model_activation_grad": (_I, [_P, _I, C.c_char_p, C.POINTER(_P), C.POINTER(_L), C.POINTER(_L),
                                       C.POINTER(_L)]),
    "mft_model_set_retain": (_I, [_P, C.c_uint64]),
    "mft_model_set_timing": (_I, [_P, _I]),
    "mft_model_set_training": (_I, [_P, _I]),
    "mft_model_shard_stats": (_I, [_P, C.POINTER(_L), C.POINTER(_L), C.POINTER(_L)]),
    "mft_model_shard_reset": (_I, [_P]),
    "mft_model_timing": (_I, [_P, _I, C.POINTER(_D), C.POINTER(_D), C.POINTER(_L)]),
    "mft_model_reset_timing": (_I, [_P]),
}


def lib():
    """Load libmft_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MFTError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950); there is no fallback path")
        L = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().mft_last_error().decode(errors="replace")
        raise MFTError(f"{what or 'mft call'} failed with status {status}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def exported_symbols() -> list[str]:
    return list(_SIGS)
