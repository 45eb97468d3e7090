"""Pins the oracle's retained intermediates (oracle.h: orc_model_set_retain;
the Gemma driver's alignment dump, gemma_3_270m_lora_finetune/src/main.cpp:
547-657) against HF transformers' retain_grad() on the same intermediates
(tests/golden/hf_gemma_retained.npz, written by make_hf_retain_golden.py),
and the closed-form attention scores/probabilities against the oracle's own
attention kernels.  CPU only."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import rel_err
from test_oracle_models import CASES, init_values

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_gemma_retained.npz")
NAMES = ["x", "norm1", "q_proj", "k_proj", "v", "q_normed", "k_normed", "q", "k", "scores", "probs", "attn",
         "o_proj", "mid", "norm2", "gate", "up", "gate_act", "act", "down_proj", "out"]


@pytest.fixture(scope="module")
def golden_and_oracle():
    z = np.load(GOLDEN)
    mc = CASES["gemma3"]
    om = O.OracleModel(mc)
    vals = init_values(om, seed=int(z["seed"]))
    for name, v in vals.items():  # the golden was made from these exact parameters
        assert abs(float(np.sum(v.astype(np.float64) ** 2)) - float(z[f"ss/{name}"])) < 1e-9 * (
            1 + float(z[f"ss/{name}"])), name
    ids, labels = z["ids"], z["labels"]
    B, S = ids.shape
    layers = [int(l) for l in z["layers"]]
    om.set_retain(layers)
    loss = om.fwd_bwd(ids, np.ones((B, S), np.float32), labels, B, S, 1.0)
    assert abs(loss - float(z["loss"])) < 2e-5 * abs(float(z["loss"]))
    return z, om, layers


@pytest.mark.parametrize("name", NAMES)
def test_retained_gradients_match_hf_retain_grad(golden_and_oracle, name):
    z, om, layers = golden_and_oracle
    for li in layers:
        ref = z[f"{li}/{name}"].ravel()
        got = om.retained(li, name, grad=True)
        assert got is not None, (li, name)
        assert rel_err(got, ref) < 1e-4, (li, name, rel_err(got, ref))


def test_retained_embedding_gradient_and_probabilities(golden_and_oracle):
    z, om, layers = golden_and_oracle
    assert rel_err(om.retained(-1, "embed", grad=True), z["-1/embed"].ravel()) < 1e-4
    # layer 0's input gradient is the embedding's
    assert np.array_equal(om.retained(-1, "embed", grad=True), om.retained(0, "x", grad=True))
    for li in layers:
        assert rel_err(om.retained(li, "probs", grad=False), z[f"{li}/probs_act"].ravel()) < 1e-5


def test_closed_form_attention_gradients_agree_with_attention_backward():
    """dQ = scale·dS·K and dV = Pᵀ·dO (GQA: summed over the group) from the
    closed-form scores/probabilities reproduce orc_attn_bwd's dQ and dV, and
    P reproduces orc_attn_fwd's output — two independent code paths; a wrong
    mask, scale or delta in either shows here.  Sliding window and a padded
    key included."""
    rng = np.random.default_rng(3)
    B, Hq, Hkv, S, hd, win = 2, 4, 2, 9, 8, 4
    scale = 0.3
    q, k, v, dout = (rng.standard_normal((B * S, n * hd)).astype(np.float32) for n in (Hq, Hkv, Hkv, Hq))
    kpad = np.ones((B, S), np.float32)
    kpad[1, 2] = 0
    o, lse = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, True, win, kpad)
    dq, dk, dv = O.attn_bwd(q, k, v, o, dout, lse, B, Hq, Hkv, S, hd, scale, True, win, kpad)
    ns = B * Hq * S * S
    sc, pr, dp, ds = (np.empty(ns, np.float32) for _ in range(4))
    O.lib().orc_attn_probs(O.ptr(q), Hq * hd, O.ptr(k), Hkv * hd, O.ptr(v), Hkv * hd, O.ptr(dout), Hq * hd,
                           B, Hq, Hkv, S, hd, scale, 1, win, O.ptr(kpad), O.ptr(sc), O.ptr(pr), O.ptr(dp), O.ptr(ds))
    P, dS = pr.reshape(B, Hq, S, S).astype(np.float64), ds.reshape(B, Hq, S, S).astype(np.float64)
    qh = q.reshape(B, S, Hq, hd).transpose(0, 2, 1, 3).astype(np.float64)
    kh = np.repeat(k.reshape(B, S, Hkv, hd).transpose(0, 2, 1, 3), Hq // Hkv, axis=1).astype(np.float64)
    vh = np.repeat(v.reshape(B, S, Hkv, hd).transpose(0, 2, 1, 3), Hq // Hkv, axis=1).astype(np.float64)
    gh = dout.reshape(B, S, Hq, hd).transpose(0, 2, 1, 3).astype(np.float64)
    tok = lambda t: t.transpose(0, 2, 1, 3).reshape(B * S, -1)  # noqa: E731
    assert rel_err(tok(P @ vh), o) < 1e-5
    assert rel_err(tok(scale * dS @ kh), dq) < 1e-5
    dv_heads = np.swapaxes(P, -1, -2) @ gh  # [B, Hq, S, hd]
    dv_kv = dv_heads.reshape(B, Hkv, Hq // Hkv, S, hd).sum(axis=2)
    assert rel_err(tok(dv_kv), dv) < 1e-5
    dk_heads = scale * np.swapaxes(dS, -1, -2) @ qh
    assert rel_err(tok(dk_heads.reshape(B, Hkv, Hq // Hkv, S, hd).sum(axis=2)), dk) < 1e-5
    masked = sc.reshape(B, Hq, S, S) < -1e38
    assert np.all(P[masked] == 0) and np.all(dS[masked] == 0) and masked[1, :, :, 2].all()
