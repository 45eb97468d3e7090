"""Pins the CPU oracle's operators (oracle/oracle_ops.c) against independent
formulations: fp64 torch autograd of the forward definition and torch
library routines (layer_norm, gelu, silu, cross_entropy,
scaled_dot_product_attention, Adam), central finite differences, closed forms
and exhaustive fp16 enumeration.  CPU only."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from conftest import rel_err

RNG = np.random.default_rng(1234)


def T(a, **kw):
    """fp64 torch tensor of a numpy array (references run in double)."""
    return torch.tensor(np.asarray(a, dtype=np.float64), **kw)


def rn(*shape, std=1.0):
    return (RNG.standard_normal(shape) * std).astype(np.float32)


# ---------------------------------------------------------------- LoRA linear
@pytest.mark.parametrize("M,K,N,r", [(7, 12, 20, 1), (33, 48, 40, 8), (64, 64, 96, 4)])
def test_lora_linear_fwd_merged_weight(M, K, N, r):
    x, W, b, A, B = rn(M, K), rn(K, N, std=0.1), rn(N), rn(r, K), rn(N, r, std=0.1)
    s = 16.0 / r
    y, xa = O.lora_linear_fwd(x, W, b, A, B, s)
    # merged-weight form W' = W + s·AᵀBᵀ (LoraInjector::merge_all equivalence)
    Wm = W.astype(np.float64) + s * A.T.astype(np.float64) @ B.T.astype(np.float64)
    ref = x.astype(np.float64) @ Wm + b
    assert rel_err(y, ref) < 1e-6
    assert rel_err(xa, x.astype(np.float64) @ A.T.astype(np.float64)) < 1e-6


def test_lora_linear_zero_B_is_plain_linear():
    x, W, b, A = rn(9, 16), rn(16, 24), rn(24), rn(4, 16)
    y, _ = O.lora_linear_fwd(x, W, b, A, np.zeros((24, 4), np.float32), 2.0)
    assert rel_err(y, x.astype(np.float64) @ W + b) < 1e-6
    dy = rn(9, 24)
    _, dA, dB = O.lora_linear_bwd(dy, x, W, A, np.zeros((24, 4), np.float32), x @ A.T, 2.0)
    assert np.abs(dA).max() == 0.0


@pytest.mark.parametrize("M,K,N,r", [(5, 12, 20, 2), (31, 40, 24, 8)])
def test_lora_linear_bwd_autograd(M, K, N, r):
    x, W, b, A, B = rn(M, K), rn(K, N, std=0.2), rn(N), rn(r, K), rn(N, r)
    s = 32.0 / r
    dy = rn(M, N)
    y, xa = O.lora_linear_fwd(x, W, b, A, B, s)
    dx, dA, dB = O.lora_linear_bwd(dy, x, W, A, B, xa, s)
    tx, tA, tB = (T(v, requires_grad=True) for v in (x, A, B))
    ty = tx @ T(W) + T(b) + s * (tx @ tA.T) @ tB.T
    ty.backward(T(dy))
    assert rel_err(dx, tx.grad.numpy()) < 1e-6
    assert rel_err(dA, tA.grad.numpy()) < 1e-6
    assert rel_err(dB, tB.grad.numpy()) < 1e-6


def test_lora_linear_bwd_finite_difference():
    M, K, N, r = 3, 5, 4, 2
    x, W, A, B = (rn(M, K).astype(np.float64), rn(K, N).astype(np.float64),
                  rn(r, K).astype(np.float64), rn(N, r).astype(np.float64))
    s, dy = 1.5, rn(M, N).astype(np.float64)

    def loss(x_, A_, B_):
        return float(np.sum(dy * (x_ @ W + s * (x_ @ A_.T) @ B_.T)))

    _, xa = O.lora_linear_fwd(x, W, None, A, B, s)
    dx, dA, dB = O.lora_linear_bwd(dy, x, W, A, B, xa, s)
    eps = 1e-4
    for arr, grad, which in ((x, dx, 0), (A, dA, 1), (B, dB, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [x.copy(), A.copy(), B.copy()]
            args[which][idx] += eps
            lp = loss(*args)
            args[which][idx] -= 2 * eps
            lm = loss(*args)
            num[idx] = (lp - lm) / (2 * eps)
        assert rel_err(grad, num) < 1e-4


# ---------------------------------------------------------------- attention
def torch_attn(q, k, v, B, Hq, Hkv, S, hd, scale, causal=True, window=0, kpad=None):
    """Textbook: repeat KV heads (repeat_kv_heads), materialised scores."""
    tq = q.reshape(B, S, Hq, hd).permute(0, 2, 1, 3)
    tk = k.reshape(B, S, Hkv, hd).permute(0, 2, 1, 3).repeat_interleave(Hq // Hkv, dim=1)
    tv = v.reshape(B, S, Hkv, hd).permute(0, 2, 1, 3).repeat_interleave(Hq // Hkv, dim=1)
    sc = (tq @ tk.transpose(-2, -1)) * scale
    i = torch.arange(S)[:, None]
    j = torch.arange(S)[None, :]
    vis = torch.ones(S, S, dtype=torch.bool)
    if causal:
        vis &= j <= i
    if window:
        vis &= (i - j) < window
    vis = vis[None, None].expand(B, Hq, S, S)
    if kpad is not None:
        vis = vis & (torch.tensor(kpad) > 0.5)[:, None, None, :]
    sc = sc.masked_fill(~vis, float("-inf"))
    p = torch.softmax(sc, -1)
    p = torch.nan_to_num(p, nan=0.0)
    o = p @ tv
    return o.permute(0, 2, 1, 3).reshape(B * S, Hq * hd)


@pytest.mark.parametrize("B,Hq,Hkv,S,hd,window", [(2, 4, 4, 9, 8, 0), (1, 6, 2, 13, 16, 0),
                                                   (2, 4, 1, 17, 8, 5)])
def test_attention_fwd_bwd_vs_autograd(B, Hq, Hkv, S, hd, window):
    q, k, v = rn(B * S, Hq * hd), rn(B * S, Hkv * hd), rn(B * S, Hkv * hd)
    scale = hd ** -0.5
    kpad = np.ones((B, S), np.float32)
    if B > 1:
        kpad[1, -3:] = 0
    o, lse = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, True, window, kpad)
    tq, tk, tv = (T(a, requires_grad=True) for a in (q, k, v))
    to = torch_attn(tq, tk, tv, B, Hq, Hkv, S, hd, scale, True, window, kpad)
    assert rel_err(o, to.detach().numpy()) < 1e-6
    g = rn(B * S, Hq * hd)
    to.backward(T(g))
    dq, dk, dv = O.attn_bwd(q, k, v, o, g, lse, B, Hq, Hkv, S, hd, scale, True, window, kpad)
    assert rel_err(dq, tq.grad.numpy()) < 1e-5
    assert rel_err(dk, tk.grad.numpy()) < 1e-5
    assert rel_err(dv, tv.grad.numpy()) < 1e-5


def test_attention_matches_sdpa_and_invariants():
    B, H, S, hd = 2, 3, 11, 16
    q, k, v = rn(B * S, H * hd), rn(B * S, H * hd), rn(B * S, H * hd)
    o, lse = O.attn_fwd(q, k, v, B, H, H, S, hd, hd ** -0.5)
    tq, tk, tv = (T(a).reshape(B, S, H, hd).permute(0, 2, 1, 3) for a in (q, k, v))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    assert rel_err(o, ref.permute(0, 2, 1, 3).reshape(B * S, H * hd).numpy()) < 1e-6
    # row 0 attends only to key 0 → O = V[0], lse = scale·q0·k0
    assert np.allclose(o.reshape(B, S, H, hd)[:, 0], v.reshape(B, S, H, hd)[:, 0], atol=1e-6)
    qk = (q.reshape(B, S, H, hd)[:, 0] * k.reshape(B, S, H, hd)[:, 0]).sum(-1) * hd ** -0.5
    assert np.allclose(lse[:, :, 0], qk, atol=1e-5)


def test_attention_gqa_equals_repeated_mha():
    B, Hq, Hkv, S, hd = 1, 8, 2, 10, 8
    q, k, v = rn(B * S, Hq * hd), rn(B * S, Hkv * hd), rn(B * S, Hkv * hd)
    o1, _ = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, 0.3)
    kr = np.repeat(k.reshape(B * S, Hkv, hd), Hq // Hkv, axis=1).reshape(B * S, Hq * hd)
    vr = np.repeat(v.reshape(B * S, Hkv, hd), Hq // Hkv, axis=1).reshape(B * S, Hq * hd)
    o2, _ = O.attn_fwd(q, kr, vr, B, Hq, Hq, S, hd, 0.3)
    assert np.array_equal(o1, o2)


# ---------------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("B,S,V", [(2, 7, 50), (3, 5, 1031)])
def test_ce_vs_torch_cross_entropy(B, S, V):
    logits = rn(B * S, V, std=3.0)
    labels = RNG.integers(0, V, size=(B, S)).astype(np.int32)
    labels[0, 2] = -100
    labels[-1, -1] = -100
    up = 0.5
    ls, n, dl, nll = O.ce_fwd_bwd(logits, labels, B, S, -100, up)
    tl = T(logits, requires_grad=True)
    shift = tl.reshape(B, S, V)[:, :-1].reshape(-1, V)
    tgt = torch.tensor(labels[:, 1:].reshape(-1).astype(np.int64))
    loss = torch.nn.functional.cross_entropy(shift, tgt, ignore_index=-100, reduction="mean")
    (loss * up).backward()
    valid = int((labels[:, 1:] != -100).sum())
    assert n == valid
    assert abs(ls / n - loss.item()) < 1e-6 * max(1.0, abs(loss.item()))
    assert rel_err(dl, tl.grad.numpy()) < 1e-6
    assert np.all(nll.reshape(B, S)[:, -1] == 0)


def test_ce_closed_forms():
    B, S, V = 2, 6, 37
    ls, n, dl, _ = O.ce_fwd_bwd(np.zeros((B * S, V), np.float32),
                                np.ones((B, S), np.int32), B, S)
    assert abs(ls / n - math.log(V)) < 1e-6
    logits = rn(B * S, V, std=4.0)
    _, _, dl, _ = O.ce_fwd_bwd(logits, RNG.integers(0, V, (B, S)).astype(np.int32), B, S)
    assert np.abs(dl.sum(-1)).max() < 1e-6        # Σ_v dlogits = 0 per row
    assert np.abs(dl.reshape(B, S, V)[:, -1]).max() == 0   # last position has no target


# ---------------------------------------------------------------- fp16
def test_ce_out_of_range_label_equals_ignored():
    """A label outside [0, V) (other than ignore_index) contributes nothing and
    is not counted: identical to the same label set to ignore_index (the
    reference indexes such a label unchecked, so this is the defined rule)."""
    rng = np.random.default_rng(3)
    B, S, V = 2, 7, 50
    lg = rng.standard_normal((B * S, V)).astype(np.float32)
    lab = rng.integers(0, V, (B, S)).astype(np.int32)
    bad = lab.copy()
    bad[0, 2], bad[1, 5] = V, -7
    ign = lab.copy()
    ign[0, 2], ign[1, 5] = -100, -100
    a = O.ce_fwd_bwd(lg, bad, B, S, -100, 1.0)
    b = O.ce_fwd_bwd(lg, ign, B, S, -100, 1.0)
    # the loss sum is an OpenMP reduction (order varies run to run): fp64-close
    assert abs(a[0] - b[0]) <= 1e-12 * abs(b[0]) and a[1] == b[1] == B * (S - 1) - 2
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])


def test_f16_exhaustive_widening():
    bits = np.arange(65536, dtype=np.uint16)
    out = O.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_nearest_even():
    x = np.concatenate([rn(200000, std=0.02), rn(1000, std=1e-6), rn(1000, std=3e4),
                        np.array([0.0, -0.0, 65504, 65520, 65519.99, 1e-8, 5.96e-8, 2.98e-8,
                                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    out = O.f32_to_f16(x)
    assert np.array_equal(out, x.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- Adam / clip
def test_adam_matches_torch_adam():
    n = 1000
    p = rn(n)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    tp = torch.nn.Parameter(torch.tensor(p, dtype=torch.float32))
    opt = torch.optim.Adam([tp], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    for t in range(1, 6):
        g = rn(n)
        O.adam_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.0, t)
        tp.grad = torch.tensor(g, dtype=torch.float32)
        opt.step()
    assert rel_err(p, tp.detach().numpy()) < 1e-6


@pytest.mark.parametrize("wd", [0.01, 0.1])
def test_adam_weight_decay_matches_torch_adamw(wd):
    """Weight decay is decoupled: the reference's PyTorch mirrors train with
    torch.optim.AdamW (pytorch_alignment/gpt2_lora_finetune.py:313)."""
    n = 1000
    p = rn(n)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    tp = torch.nn.Parameter(torch.tensor(p, dtype=torch.float32))
    opt = torch.optim.AdamW([tp], lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    for t in range(1, 6):
        g = rn(n)
        O.adam_step(p, g, m, v, 1e-2, 0.9, 0.999, 1e-8, wd, t)
        tp.grad = torch.tensor(g, dtype=torch.float32)
        opt.step()
    assert rel_err(p, tp.detach().numpy()) < 1e-6
    # a coupled (L2-in-gradient) decay would differ far beyond that
    p2 = rn(n)
    p2c = p2.copy()
    g = rn(n)
    O.adam_step(p2, g, np.zeros(n, np.float32), np.zeros(n, np.float32), 1e-2, 0.9, 0.999, 1e-8, wd, 1)
    gc = g + wd * p2c
    coupled = p2c - 1e-2 * gc / (np.abs(gc) + 1e-8)
    assert rel_err(p2, coupled) > 1e-4


def test_adam_first_step_closed_form():
    p = rn(100)
    p0 = p.copy()
    g = rn(100)
    O.adam_step(p, g, np.zeros(100, np.float32), np.zeros(100, np.float32), 0.01, 0.9, 0.999,
                1e-8, 0.0, 1)
    ref = p0 - 0.01 * g / (np.abs(g) + 1e-8)
    assert np.abs(p - ref).max() < 1e-6


def test_sumsq_and_clip():
    g = rn(12345)
    ss = O.sumsq(g)
    assert abs(ss - float(np.sum(g.astype(np.float64) ** 2))) < 1e-9 * ss
    s, nrm = O.clip_scale(ss, 1.0)
    assert abs(s - 1.0 / (math.sqrt(ss) + 1e-6)) < 1e-6 and nrm == 1.0
    s2, nrm2 = O.clip_scale(0.25, 1.0)
    assert s2 == 1.0 and abs(nrm2 - 0.5) < 1e-7


# ---------------------------------------------------------------- norms / activations
def test_layernorm_vs_torch():
    x, g, b = rn(13, 40, std=2.0), rn(40), rn(40)
    y, mean, rstd = O.layernorm_fwd(x, g, b, 1e-5)
    tx = T(x, requires_grad=True)
    ty = torch.nn.functional.layer_norm(tx, (40,), T(g), T(b), 1e-5)
    assert rel_err(y, ty.detach().numpy()) < 1e-6
    dy = rn(13, 40)
    ty.backward(T(dy))
    assert rel_err(O.layernorm_bwd(dy, x, g, mean, rstd), tx.grad.numpy()) < 1e-5


@pytest.mark.parametrize("unit", [0, 1])
def test_rmsnorm_vs_autograd(unit):
    x, w = rn(11, 64, std=2.0), rn(64, std=0.3)
    y, rstd = O.rmsnorm_fwd(x, w, 1e-6, unit)
    tx = T(x, requires_grad=True)
    tw = T(w) + (1.0 if unit else 0.0)
    ty = tx * torch.rsqrt(tx.pow(2).mean(-1, keepdim=True) + 1e-6) * tw
    assert rel_err(y, ty.detach().numpy()) < 1e-6
    dy = rn(11, 64)
    ty.backward(T(dy))
    assert rel_err(O.rmsnorm_bwd(dy, x, w, rstd, unit), tx.grad.numpy()) < 1e-5


@pytest.mark.parametrize("act", [0, 1])
def test_glu_vs_torch(act):
    gate, up, dout = rn(500, std=3), rn(500), rn(500)
    tg = T(gate, requires_grad=True)
    tu = T(up, requires_grad=True)
    a = (torch.nn.functional.gelu(tg, approximate="tanh") if act == 0
         else torch.nn.functional.silu(tg))
    out = a * tu
    assert rel_err(O.glu_fwd(gate, up, act), out.detach().numpy()) < 1e-6
    out.backward(T(dout))
    dg, du = O.glu_bwd(dout, gate, up, act)
    assert rel_err(dg, tg.grad.numpy()) < 1e-5
    assert rel_err(du, tu.grad.numpy()) < 1e-6
    # GPT-2 MLP: plain activation when up is absent
    assert rel_err(O.glu_fwd(gate, None, 0),
                   torch.nn.functional.gelu(T(gate), approximate="tanh").numpy()) < 1e-6


def test_rope_vs_hf_apply_rotary():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    B, S, H, hd, theta = 2, 9, 3, 16, 10000.0
    x = rn(B * S, H * hd)
    out = O.rope(x, B, S, H, hd, theta)
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    freqs = torch.arange(S, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat([freqs, freqs], -1)
    cos, sin = emb.cos()[None], emb.sin()[None]
    tx = T(x).reshape(B, S, H, hd).permute(0, 2, 1, 3)
    ref, _ = apply_rotary_pos_emb(tx, tx, cos, sin)
    assert rel_err(out, ref.permute(0, 2, 1, 3).reshape(B * S, H * hd).numpy()) < 1e-6
    back = O.rope(out, B, S, H, hd, theta, inverse=True)   # inverse = transpose rotation
    assert rel_err(back, x) < 1e-6


def test_embed_gather():
    V, Cc, S = 50, 8, 4
    wte, wpe = rn(V, Cc), rn(S, Cc)
    ids = RNG.integers(0, V, (3, S)).astype(np.int32)
    h = O.embed(ids, S, wte, wpe, 1.0)
    ref = wte[ids.reshape(-1)] + np.tile(wpe, (3, 1))
    assert np.allclose(h, ref, atol=0)
    h2 = O.embed(ids, S, wte, None, math.sqrt(Cc))
    assert np.allclose(h2, wte[ids.reshape(-1)] * np.float32(math.sqrt(Cc)), atol=1e-6)
