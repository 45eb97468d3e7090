"""Python wrappers over the C-ABI kernels, taking torch device tensors.

torch supplies device memory and the current stream only; every computation
runs in libmft_hip.so.  Each wrapper mirrors one `operators` entry point of
the reference (see include/mft_hip.h for the reference citations).
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import call, lib

F32, F16 = 0, 1
_handles: dict = {}


def handle():
    """Handle bound to the current device and torch's current stream."""
    dev = torch.cuda.current_device()
    stream = torch.cuda.current_stream().cuda_stream
    h = _handles.get(dev)
    if h is None:
        hp = C.c_void_p()
        call("mft_create", C.byref(hp), C.c_void_p(stream))
        h = hp
        _handles[dev] = h
    else:
        call("mft_set_stream", h, C.c_void_p(stream))
    return h


def _p(t, dt=torch.float32):
    """Device pointer of a contiguous tensor whose dtype is `dt` (a dtype or a
    tuple of accepted dtypes): the C-ABI takes raw pointers, so the element
    type is checked here."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device tensor required")
    if not t.is_contiguous():
        raise ValueError("contiguous tensor required")
    if t.dtype not in (dt if isinstance(dt, tuple) else (dt,)):
        raise TypeError(f"tensor of dtype {dt} required, got {t.dtype}")
    return C.c_void_p(t.data_ptr())


_W = (torch.float32, torch.float16)
_U16 = (torch.int16, torch.uint16) if hasattr(torch, "uint16") else (torch.int16,)


def _wdtype(W):
    if W.dtype == torch.float32:
        return F32
    if W.dtype == torch.float16:
        return F16
    raise TypeError("W must be float32 or float16")


def lora_linear_fwd(x, W, bias, A, B, scale, resid=None):
    """y = x·W + bias + scale·(x·Aᵀ)·Bᵀ (+ resid); returns (y, xa)."""
    M, K = x.shape
    N = W.shape[1]
    r = A.shape[0] if A is not None else 0
    y = torch.empty(M, N, device=x.device, dtype=torch.float32)
    xa = torch.empty(M, max(r, 1), device=x.device, dtype=torch.float32) if r else None
    call("mft_lora_linear_fwd", handle(), _p(x), M, K, _p(W, _W), _wdtype(W), N, _p(bias), _p(A),
         _p(B), r, scale, _p(y), _p(xa), _p(resid))
    return y, xa


def lora_linear_bwd(dy, x, W, A, B, xa, scale, dA=None, dB=None, need_dx=True, accumulate=False,
                    dx=None, dx_accumulate=False):
    M, N = dy.shape
    K = W.shape[0]
    r = A.shape[0] if A is not None else 0
    if need_dx and dx is None:
        dx = torch.empty(M, K, device=dy.device, dtype=torch.float32)
    if r and dA is None:
        dA = torch.zeros_like(A)
    if r and dB is None:
        dB = torch.zeros_like(B)
    call("mft_lora_linear_bwd", handle(), _p(dy), _p(x), _p(W, _W), _wdtype(W), _p(A), _p(B), _p(xa),
         M, K, N, r, scale, _p(dx) if need_dx else None, _p(dA), _p(dB), int(accumulate),
         int(dx_accumulate))
    return dx, dA, dB


def _check_f32(*ts):
    for t in ts:
        if not t.is_cuda or t.dtype != torch.float32:
            raise TypeError("float32 device tensors required")


def _rs(t, H, hd):
    return t.stride(-3) if t.dim() == 4 else H * hd


def attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, causal=True, window=0, kpad=None, q_rs=None,
             k_rs=None, v_rs=None):
    """q/k/v are flat device buffers viewed as [B,S,H,hd] with row strides."""
    q_rs = q_rs or Hq * hd
    k_rs = k_rs or Hkv * hd
    v_rs = v_rs or Hkv * hd
    o = torch.empty(B * S, Hq * hd, device=q.device, dtype=torch.float32)
    lse = torch.empty(B, Hq, S, device=q.device, dtype=torch.float32)
    _check_f32(q, k, v)
    call("mft_attn_fwd", handle(), C.c_void_p(q.data_ptr()), q_rs, C.c_void_p(k.data_ptr()), k_rs,
         C.c_void_p(v.data_ptr()), v_rs, B, Hq, Hkv, S, hd, scale, int(causal), window, _p(kpad),
         _p(o), Hq * hd, _p(lse))
    return o, lse


def attn_bwd(q, k, v, o, dout, lse, B, Hq, Hkv, S, hd, scale, causal=True, window=0, kpad=None,
             q_rs=None, k_rs=None, v_rs=None):
    q_rs = q_rs or Hq * hd
    k_rs = k_rs or Hkv * hd
    v_rs = v_rs or Hkv * hd
    dq = torch.empty(B * S, Hq * hd, device=q.device, dtype=torch.float32)
    dk = torch.empty(B * S, Hkv * hd, device=q.device, dtype=torch.float32)
    dv = torch.empty(B * S, Hkv * hd, device=q.device, dtype=torch.float32)
    _check_f32(q, k, v)
    call("mft_attn_bwd", handle(), C.c_void_p(q.data_ptr()), q_rs, C.c_void_p(k.data_ptr()), k_rs,
         C.c_void_p(v.data_ptr()), v_rs, _p(o), Hq * hd, _p(dout), Hq * hd, _p(lse), B, Hq, Hkv, S,
         hd, scale, int(causal), window, _p(kpad), _p(dq), Hq * hd, _p(dk), Hkv * hd, _p(dv),
         Hkv * hd)
    return dq, dk, dv


def ce_fwd_bwd(logits, labels, B, S, ignore_index=-100, upstream=1.0, norm_count=0,
               in_place=False, want_grad=True):
    """Returns (loss_sum float64 tensor[1], n_valid int64 tensor[1], dlogits, row_nll)."""
    V = logits.shape[-1]
    loss = torch.zeros(1, device=logits.device, dtype=torch.float64)
    cnt = torch.zeros(1, device=logits.device, dtype=torch.int64)
    nll = torch.empty(B * S, device=logits.device, dtype=torch.float32)
    dl = None
    if want_grad:
        dl = logits if in_place else torch.empty_like(logits)
    call("mft_ce_fwd_bwd", handle(), _p(logits), _p(labels, torch.int32), B, S, V, ignore_index,
         upstream, norm_count, _p(loss, torch.float64), _p(cnt, torch.int64), _p(dl), _p(nll))
    return loss, cnt, dl, nll


def dequant_f16(src_u16):
    dst = torch.empty(src_u16.shape, device=src_u16.device, dtype=torch.float32)
    return dequant_f16_into(src_u16, dst)


def dequant_f16_into(src_u16, dst):
    if dst.numel() != src_u16.numel():
        raise ValueError("dst must hold as many elements as src")
    call("mft_dequant_f16", handle(), _p(src_u16, _U16 + (torch.float16,)), _p(dst), src_u16.numel())
    return dst


def quant_f16(src):
    dst = torch.empty(src.shape, device=src.device, dtype=torch.int16)
    call("mft_quant_f16", handle(), _p(src), _p(dst, torch.int16), src.numel())
    return dst


def adam_step(p, g, m, v, lr, b1, b2, eps, wd, t, clip_scale=None, zero_grad=False):
    call("mft_adam_step", handle(), _p(p), _p(g), _p(m), _p(v), p.numel(), lr, b1, b2, eps, wd, t,
         _p(clip_scale), int(zero_grad))


def sumsq(g, out=None):
    if out is None:
        out = torch.zeros(1, device=g.device, dtype=torch.float64)
    call("mft_sumsq", handle(), _p(g), g.numel(), _p(out, torch.float64))
    return out


def clip_scale(ss, max_norm):
    out = torch.empty(2, device=ss.device, dtype=torch.float32)
    call("mft_clip_scale", handle(), _p(ss, torch.float64), max_norm, C.c_void_p(out.data_ptr()),
         C.c_void_p(out.data_ptr() + 4))
    return out


def layernorm_fwd(x, g, b, eps):
    M, Cc = x.shape
    y = torch.empty_like(x)
    mean = torch.empty(M, device=x.device, dtype=torch.float32)
    rstd = torch.empty(M, device=x.device, dtype=torch.float32)
    call("mft_layernorm_fwd", handle(), _p(x), _p(g), _p(b), M, Cc, eps, _p(y), _p(mean), _p(rstd))
    return y, mean, rstd


def layernorm_bwd(dy, x, g, mean, rstd, dx=None, accumulate=False):
    M, Cc = x.shape
    if dx is None:
        dx = torch.empty_like(x)
    call("mft_layernorm_bwd", handle(), _p(dy), _p(x), _p(g), _p(mean), _p(rstd), M, Cc, _p(dx),
         int(accumulate))
    return dx


def rmsnorm_fwd(x, w, eps, unit_offset):
    M, Cc = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(M, device=x.device, dtype=torch.float32)
    call("mft_rmsnorm_fwd", handle(), _p(x), _p(w), M, Cc, eps, int(unit_offset), _p(y), _p(rstd))
    return y, rstd


def rmsnorm_bwd(dy, x, w, rstd, unit_offset, dx=None, accumulate=False):
    M, Cc = x.shape
    if dx is None:
        dx = torch.empty_like(x)
    call("mft_rmsnorm_bwd", handle(), _p(dy), _p(x), _p(w), _p(rstd), M, Cc, int(unit_offset),
         _p(dx), int(accumulate))
    return dx


def glu_fwd(gate, up, act):
    out = torch.empty_like(gate)
    call("mft_glu_fwd", handle(), _p(gate), _p(up), gate.numel(), act, _p(out))
    return out


def glu_bwd(dout, gate, up, act):
    dgate = torch.empty_like(gate)
    dup = torch.empty_like(gate) if up is not None else None
    call("mft_glu_bwd", handle(), _p(dout), _p(gate), _p(up), gate.numel(), act, _p(dgate), _p(dup))
    return dgate, dup


def rope_(x, B, S, H, hd, theta, inverse=False, rs=None):
    call("mft_rope", handle(), _p(x), rs or H * hd, B, S, H, hd, float(theta), int(inverse))
    return x


def embed(ids, S, wte, wpe, scale, out=None, bad=None):
    """h = wte[ids]·scale (+ wpe[pos]).  An id outside [0, vocab) gives a zero
    row and sets bad[0] = 1 (bad: optional int32 device tensor)."""
    M = ids.numel()
    V, Cc = wte.shape
    if out is None:
        out = torch.empty(M, Cc, device=ids.device, dtype=torch.float32)
    call("mft_embed", handle(), _p(ids, torch.int32), M, S, _p(wte, _W), V, _wdtype(wte),
         _p(wpe), Cc, scale, _p(out), _p(bad, torch.int32))
    return out


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("C", "torch", "call", "lib")]
