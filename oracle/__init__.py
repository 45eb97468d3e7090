"""CPU oracle — TEST INFRASTRUCTURE ONLY.

ctypes bindings of liboracle.so (oracle.h): the CPU restatement of the
reference's hot-path operators and training graphs.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package,
and only as the checker or as the timed CPU port; the product path never
does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = C.c_void_p
_I = C.c_int
_L = C.c_int64
_F = C.c_float
_D = C.c_double


class OrcCfg(C.Structure):
    _fields_ = [
        ("arch", _I), ("n_layer", _I), ("d", _I), ("n_head", _I), ("n_kv_head", _I),
        ("head_dim", _I), ("d_ff", _I), ("max_pos", _I), ("vocab", _L), ("lora_r", _I),
        ("lora_alpha", _F), ("lora_mask", _I), ("norm_eps", _F), ("rope_theta", _D),
        ("rope_local_theta", _D), ("sliding_pattern", _I), ("sliding_window", _I),
        ("attn_scale", _F), ("w_fp16", _I), ("lora_dropout", _F), ("dropout_seed", C.c_uint64),
    ]


_SIGS = {
    "orc_set_blas": (_I, [_I]),
    "orc_dropout_mask": (None, [C.c_uint64, C.c_uint32, C.c_uint32, _L, _F, _P]),
    "orc_blas_backend": (C.c_char_p, []),
    "orc_set_threads": (None, [_I]),
    "orc_get_threads": (_I, []),
    "orc_sgemm": (None, [_I, _I, _L, _L, _L, _F, _P, _L, _P, _L, _F, _P, _L]),
    "orc_lora_linear_fwd": (None, [_P, _L, _L, _P, _L, _P, _P, _P, _I, _F, _P, _P]),
    "orc_lora_linear_bwd": (None, [_P, _P, _P, _P, _P, _P, _L, _L, _L, _I, _F, _P, _P, _P, _I]),
    "orc_f16_to_f32": (None, [_P, _P, _L]),
    "orc_f32_to_f16": (None, [_P, _P, _L]),
    "orc_attn_fwd": (None, [_P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _L, _P]),
    "orc_attn_bwd": (None, [_P, _L, _P, _L, _P, _L, _P, _L, _P, _L, _P, _I, _I, _I, _I, _I, _F, _I,
                            _I, _P, _P, _L, _P, _L, _P, _L]),
    "orc_ce_fwd_bwd": (_L, [_P, _P, _I, _I, _L, _I, _F, _L, _P, _P, _P]),
    "orc_adam_step": (None, [_P, _P, _P, _P, _L, _F, _F, _F, _F, _F, _I]),
    "orc_sumsq": (_D, [_P, _L]),
    "orc_clip_scale": (_F, [_D, _F, _P]),
    "orc_layernorm_fwd": (None, [_P, _P, _P, _L, _L, _F, _P, _P, _P]),
    "orc_layernorm_bwd": (None, [_P, _P, _P, _P, _P, _L, _L, _P, _I]),
    "orc_rmsnorm_fwd": (None, [_P, _P, _L, _L, _F, _I, _P, _P]),
    "orc_rmsnorm_bwd": (None, [_P, _P, _P, _P, _L, _L, _I, _P, _I]),
    "orc_glu_fwd": (None, [_P, _P, _L, _I, _P]),
    "orc_glu_bwd": (None, [_P, _P, _P, _L, _I, _P, _P]),
    "orc_rope": (None, [_P, _L, _I, _I, _I, _I, _D, _I]),
    "orc_embed": (None, [_P, _L, _I, _P, _P, _P, _L, _F, _P]),
    "orc_model_create": (_P, [C.POINTER(OrcCfg)]),
    "orc_model_destroy": (None, [_P]),
    "orc_model_num_params": (_I, [_P]),
    "orc_model_param_info": (_L, [_P, _I, C.POINTER(C.c_char_p), C.POINTER(_I), C.POINTER(_L),
                                  C.POINTER(_I), C.POINTER(_I)]),
    "orc_model_param_data": (_P, [_P, _I]),
    "orc_model_param_grad": (_P, [_P, _I]),
    "orc_model_fwd_bwd": (_F, [_P, _P, _P, _P, _I, _I, _F]),
    "orc_model_forward": (_F, [_P, _P, _P, _P, _I, _I, _P]),
    "orc_model_opt_step": (_F, [_P, _F, _F, _F, _F, _F, _F]),
    "orc_model_set_retain": (None, [_P, C.c_uint64]),
    "orc_model_retained": (_P, [_P, _I, C.c_char_p, _I, C.POINTER(_L)]),
    "orc_attn_probs": (None, [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _F, _I, _I, _P,
                              _P, _P, _P, _P]),
}


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for n, (res, args) in _SIGS.items():
            f = getattr(L, n)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- op wrappers (numpy in, numpy out) ------------------------------------
def lora_linear_fwd(x, W, bias, A, B, scale):
    x, W = f32(x), f32(W)
    M, K = x.shape
    N = W.shape[1]
    r = 0 if A is None else A.shape[0]
    y = np.empty((M, N), np.float32)
    xa = np.empty((M, max(r, 1)), np.float32)
    lib().orc_lora_linear_fwd(ptr(x), M, K, ptr(W), N, ptr(None if bias is None else f32(bias)),
                              ptr(None if A is None else f32(A)), ptr(None if B is None else f32(B)),
                              r, scale, ptr(y), ptr(xa))
    return y, (xa if r else None)


def lora_linear_bwd(dy, x, W, A, B, xa, scale, need_dx=True):
    dy, x, W = f32(dy), f32(x), f32(W)
    M, N = dy.shape
    K = W.shape[0]
    r = 0 if A is None else A.shape[0]
    dx = np.empty((M, K), np.float32) if need_dx else None
    dA = np.zeros((r, K), np.float32) if r else None
    dB = np.zeros((N, r), np.float32) if r else None
    lib().orc_lora_linear_bwd(ptr(dy), ptr(x), ptr(W), ptr(None if A is None else f32(A)),
                              ptr(None if B is None else f32(B)), ptr(None if xa is None else f32(xa)),
                              M, K, N, r, scale, ptr(dx), ptr(dA), ptr(dB), 0)
    return dx, dA, dB


def f16_to_f32(bits_u16):
    b = np.ascontiguousarray(bits_u16, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_f16_to_f32(ptr(b), ptr(out), b.size)
    return out


def f32_to_f16(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16(ptr(x), ptr(out), x.size)
    return out


def attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, causal=True, window=0, kpad=None):
    """q [B*S, Hq*hd], k/v [B*S, Hkv*hd] contiguous."""
    q, k, v = f32(q), f32(k), f32(v)
    o = np.empty((B * S, Hq * hd), np.float32)
    lse = np.empty((B, Hq, S), np.float32)
    lib().orc_attn_fwd(ptr(q), Hq * hd, ptr(k), Hkv * hd, ptr(v), Hkv * hd, B, Hq, Hkv, S, hd,
                       scale, int(causal), window, ptr(None if kpad is None else f32(kpad)), ptr(o),
                       Hq * hd, ptr(lse))
    return o, lse


def attn_bwd(q, k, v, o, dout, lse, B, Hq, Hkv, S, hd, scale, causal=True, window=0, kpad=None):
    q, k, v, o, dout, lse = map(f32, (q, k, v, o, dout, lse))
    dq = np.empty((B * S, Hq * hd), np.float32)
    dk = np.empty((B * S, Hkv * hd), np.float32)
    dv = np.empty((B * S, Hkv * hd), np.float32)
    lib().orc_attn_bwd(ptr(q), Hq * hd, ptr(k), Hkv * hd, ptr(v), Hkv * hd, ptr(o), Hq * hd,
                       ptr(dout), Hq * hd, ptr(lse), B, Hq, Hkv, S, hd, scale, int(causal), window,
                       ptr(None if kpad is None else f32(kpad)), ptr(dq), Hq * hd, ptr(dk), Hkv * hd,
                       ptr(dv), Hkv * hd)
    return dq, dk, dv


def ce_fwd_bwd(logits, labels, B, S, ignore_index=-100, upstream=1.0, norm_count=0):
    lg = f32(logits)
    lb = np.ascontiguousarray(labels, dtype=np.int32)
    V = lg.shape[-1]
    ls = C.c_double()
    dl = np.empty_like(lg)
    nll = np.empty(B * S, np.float32)
    n = lib().orc_ce_fwd_bwd(ptr(lg), ptr(lb), B, S, V, ignore_index, upstream, norm_count,
                             C.byref(ls), ptr(dl), ptr(nll))
    return ls.value, n, dl, nll


def adam_step(p, g, m, v, lr, b1, b2, eps, wd, t):
    for a in (p, g, m, v):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    lib().orc_adam_step(ptr(p), ptr(g), ptr(m), ptr(v), p.size, lr, b1, b2, eps, wd, t)


def sumsq(g):
    return lib().orc_sumsq(ptr(f32(g)), g.size)


def clip_scale(ss, max_norm):
    norm = C.c_float()
    s = lib().orc_clip_scale(ss, max_norm, C.byref(norm))
    return s, norm.value


def layernorm_fwd(x, g, b, eps):
    x = f32(x)
    M, Cc = x.shape
    y = np.empty_like(x)
    mean = np.empty(M, np.float32)
    rstd = np.empty(M, np.float32)
    lib().orc_layernorm_fwd(ptr(x), ptr(f32(g)), ptr(f32(b)), M, Cc, eps, ptr(y), ptr(mean), ptr(rstd))
    return y, mean, rstd


def layernorm_bwd(dy, x, g, mean, rstd):
    x = f32(x)
    M, Cc = x.shape
    dx = np.empty_like(x)
    lib().orc_layernorm_bwd(ptr(f32(dy)), ptr(x), ptr(f32(g)), ptr(f32(mean)), ptr(f32(rstd)), M, Cc,
                            ptr(dx), 0)
    return dx


def rmsnorm_fwd(x, w, eps, unit_offset):
    x = f32(x)
    M, Cc = x.shape
    y = np.empty_like(x)
    rstd = np.empty(M, np.float32)
    lib().orc_rmsnorm_fwd(ptr(x), ptr(f32(w)), M, Cc, eps, int(unit_offset), ptr(y), ptr(rstd))
    return y, rstd


def rmsnorm_bwd(dy, x, w, rstd, unit_offset):
    x = f32(x)
    M, Cc = x.shape
    dx = np.empty_like(x)
    lib().orc_rmsnorm_bwd(ptr(f32(dy)), ptr(x), ptr(f32(w)), ptr(f32(rstd)), M, Cc, int(unit_offset),
                          ptr(dx), 0)
    return dx


def glu_fwd(gate, up, act):
    gate = f32(gate)
    out = np.empty_like(gate)
    lib().orc_glu_fwd(ptr(gate), ptr(None if up is None else f32(up)), gate.size, act, ptr(out))
    return out


def glu_bwd(dout, gate, up, act):
    gate = f32(gate)
    dg = np.empty_like(gate)
    du = np.empty_like(gate) if up is not None else None
    lib().orc_glu_bwd(ptr(f32(dout)), ptr(gate), ptr(None if up is None else f32(up)), gate.size, act,
                      ptr(dg), ptr(du))
    return dg, du


def rope(x, B, S, H, hd, theta, inverse=False):
    x = f32(x).copy()
    lib().orc_rope(ptr(x), H * hd, B, S, H, hd, theta, int(inverse))
    return x


def embed(ids, S, wte, wpe, scale, wte_f16=None):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    M = ids.size
    Cc = (wte if wte is not None else wte_f16).shape[1]
    h = np.empty((M, Cc), np.float32)
    lib().orc_embed(ptr(ids), M, S, ptr(None if wte is None else f32(wte)),
                    ptr(None if wte_f16 is None else np.ascontiguousarray(wte_f16, np.uint16)),
                    ptr(None if wpe is None else f32(wpe)), Cc, scale, ptr(h))
    return h


class OracleModel:
    """CPU restatement of the three LoRA training graphs."""

    def __init__(self, mcfg):
        c = OrcCfg(mcfg.arch, mcfg.n_layer, mcfg.d, mcfg.n_head, mcfg.n_kv_head, mcfg.head_dim,
                   mcfg.d_ff, mcfg.max_pos, mcfg.vocab, mcfg.lora_r, mcfg.lora_alpha,
                   mcfg.lora_mask, mcfg.norm_eps, mcfg.rope_theta, mcfg.rope_local_theta,
                   mcfg.sliding_pattern, mcfg.sliding_window, mcfg.attn_scale, mcfg.w_fp16,
                   mcfg.lora_dropout, mcfg.dropout_seed)
        self._c = c
        self.h = lib().orc_model_create(C.byref(c))
        self.params = []
        for i in range(lib().orc_model_num_params(self.h)):
            name = C.c_char_p()
            nd = C.c_int()
            dims = (C.c_int64 * 2)()
            tr = C.c_int()
            f16 = C.c_int()
            numel = lib().orc_model_param_info(self.h, i, C.byref(name), C.byref(nd), dims,
                                               C.byref(tr), C.byref(f16))
            shape = tuple(dims[j] for j in range(nd.value))
            self.params.append(dict(i=i, name=name.value.decode(), shape=shape, numel=numel,
                                    trainable=bool(tr.value), f16=bool(f16.value)))
        self.by_name = {p["name"]: p for p in self.params}

    def __del__(self):
        try:
            if self.h:
                lib().orc_model_destroy(self.h)
        except Exception:
            pass

    def _view(self, p, grad=False):
        addr = (lib().orc_model_param_grad if grad else lib().orc_model_param_data)(self.h, p["i"])
        dt = C.c_uint16 if (p["f16"] and not grad) else C.c_float
        buf = (dt * p["numel"]).from_address(addr)
        return np.ctypeslib.as_array(buf).reshape(p["shape"])

    def set_param(self, name, arr):
        p = self.by_name[name]
        v = self._view(p)
        v[...] = np.asarray(arr, dtype=v.dtype).reshape(p["shape"])

    def get(self, name, grad=False):
        return self._view(self.by_name[name], grad).copy()

    def fwd_bwd(self, ids, mask, labels, B, S, upstream):
        ids = np.ascontiguousarray(ids, np.int32)
        labels = np.ascontiguousarray(labels, np.int32)
        mask = None if mask is None else f32(mask)
        return lib().orc_model_fwd_bwd(self.h, ptr(ids), ptr(mask), ptr(labels), B, S, upstream)

    def forward(self, ids, mask, labels, B, S, want_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        labels = np.ascontiguousarray(labels, np.int32)
        mask = None if mask is None else f32(mask)
        lg = np.empty((B * S, self._c.vocab), np.float32) if want_logits else None
        loss = lib().orc_model_forward(self.h, ptr(ids), ptr(mask), ptr(labels), B, S, ptr(lg))
        return loss, lg

    def opt_step(self, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, clip=1.0):
        return lib().orc_model_opt_step(self.h, lr, b1, b2, eps, wd, clip)

    def set_retain(self, layers):
        """Keep the activations and activation gradients of `layers` in
        later steps (oracle.h: orc_model_set_retain)."""
        mask = 0
        for l in layers:
            mask |= 1 << l
        lib().orc_model_set_retain(self.h, mask)

    def retained(self, layer, name, grad=True):
        """A kept activation (grad=False) or activation gradient as a copy:
        [B*S, width], or [B, Hq, S, S] for "scores" / "probs"; None if absent."""
        n = C.c_int64()
        addr = lib().orc_model_retained(self.h, layer, name.encode(), 1 if grad else 0, C.byref(n))
        if not addr:
            return None
        return np.ctypeslib.as_array((C.c_float * n.value).from_address(addr)).copy()


def dropout_mask(seed, step, lid, shape, p):
    """The LoRA dropout mask (1/(1-p) where kept, 0 elsewhere) of stream
    `lid` in training forward `step` (oracle.h: orc_dropout_mask)."""
    out = np.empty(shape, np.float32)
    lib().orc_dropout_mask(seed, step, lid, out.size, p, ptr(out))
    return out
