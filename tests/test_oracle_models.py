"""Pins the oracle's GPT-2 / Qwen2 / Gemma3 LoRA training graphs
(oracle/oracle_model.c) against HF transformers model classes built from
local config objects (no download), run in fp64, with LoRA added as
x·W + b + s·(x·Aᵀ)·Bᵀ around the targeted projections (PEFT semantics).
Compared: per-step loss, every LoRA gradient, and the parameters after one
clip + Adam step.  CPU only."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import rel_err
from mobilefinetuner_amd.configs import gemma3, gpt2, qwen2

RNG = np.random.default_rng(7)


class LoraWrap(torch.nn.Module):
    def __init__(self, base, A, B, s):
        super().__init__()
        self.base = base
        self.A = torch.nn.Parameter(torch.tensor(A, dtype=torch.float64))
        self.B = torch.nn.Parameter(torch.tensor(B, dtype=torch.float64))
        self.s = s

    def forward(self, x):
        return self.base(x) + self.s * (x @ self.A.T) @ self.B.T


def init_values(om, seed=0, norm_std=0.1):
    rng = np.random.default_rng(seed)
    vals = {}
    for p in om.params:
        n = p["name"]
        if n.endswith("lora_A"):
            v = rng.standard_normal(p["shape"]) / 8.0
        elif "norm" in n or "ln_" in n:
            v = rng.standard_normal(p["shape"]) * norm_std + (1.0 if ("ln_" in n and n.endswith("weight")) else 0.0)
        else:
            v = rng.standard_normal(p["shape"]) * 0.02 * (5.0 if n.endswith("lora_B") else 1.0)
        v = v.astype(np.float32)
        if p["f16"]:
            v16 = v.astype(np.float16)
            om.set_param(n, v16.view(np.uint16))
            vals[n] = v16.astype(np.float32)
        else:
            om.set_param(n, v)
            vals[n] = v
    return vals


def hf_model(mc):
    import transformers as T
    if mc.arch == 0:
        cfg = T.GPT2Config(vocab_size=mc.vocab, n_positions=mc.max_pos, n_embd=mc.d,
                           n_layer=mc.n_layer, n_head=mc.n_head, activation_function="gelu_new",
                           resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0,
                           layer_norm_epsilon=mc.norm_eps, tie_word_embeddings=True)
        model = T.GPT2LMHeadModel(cfg)
    elif mc.arch == 1:
        cfg = T.Qwen2Config(vocab_size=mc.vocab, hidden_size=mc.d, intermediate_size=mc.d_ff,
                            num_hidden_layers=mc.n_layer, num_attention_heads=mc.n_head,
                            num_key_value_heads=mc.n_kv_head, max_position_embeddings=mc.max_pos,
                            rope_theta=mc.rope_theta, rms_norm_eps=mc.norm_eps,
                            tie_word_embeddings=True, attention_dropout=0.0)
        model = T.Qwen2ForCausalLM(cfg)
    else:
        from transformers.models.gemma3 import Gemma3ForCausalLM, Gemma3TextConfig
        cfg = Gemma3TextConfig(vocab_size=mc.vocab, hidden_size=mc.d, intermediate_size=mc.d_ff,
                               num_hidden_layers=mc.n_layer, num_attention_heads=mc.n_head,
                               num_key_value_heads=mc.n_kv_head, head_dim=mc.head_dim,
                               query_pre_attn_scalar=round(mc.attn_scale ** -2),
                               sliding_window=mc.sliding_window, rope_theta=mc.rope_theta,
                               rope_local_base_freq=mc.rope_local_theta, rms_norm_eps=mc.norm_eps,
                               hidden_activation="gelu_pytorch_tanh", max_position_embeddings=mc.max_pos,
                               final_logit_softcapping=None, attn_logit_softcapping=None,
                               tie_word_embeddings=True, attention_dropout=0.0)
        model = Gemma3ForCausalLM(cfg)
    model.config._attn_implementation = "eager"
    return model.double().eval()


def load_hf(model, mc, vals):
    prefix = "transformer." if mc.arch == 0 else "model."
    sd = model.state_dict()
    lora = {}
    with torch.no_grad():
        for name, v in vals.items():
            if "lora_" in name:
                lora[name] = v
                continue
            key = prefix + name + (".weight" if name in ("wte", "wpe") else "")
            t = torch.tensor(v, dtype=torch.float64)
            if mc.arch != 0 and name.endswith("proj.weight"):
                t = t.T  # HF nn.Linear keeps [out, in]; the reference layout is [in, out]
            assert sd[key].shape == t.shape, key
            sd[key].copy_(t)
    s = mc.lora_alpha / mc.lora_r
    wraps = {}
    for name in {n.rsplit(".", 1)[0] for n in lora}:
        mod_path = prefix + name
        parent = model.get_submodule(mod_path.rsplit(".", 1)[0])
        leaf = mod_path.rsplit(".", 1)[1]
        w = LoraWrap(getattr(parent, leaf), lora[name + ".lora_A"], lora[name + ".lora_B"], s)
        setattr(parent, leaf, w)
        wraps[name] = w
    return wraps


CASES = {
    "gpt2": gpt2(2, 64, 4, vocab=101, max_pos=32, name="gpt2-tiny"),
    "gpt2-mlp-lora": gpt2(2, 32, 2, vocab=67, max_pos=16, name="gpt2-tiny-all", lora_mask=0b1111),
    "qwen2": qwen2(2, 64, 4, 2, 16, 96, vocab=97, name="qwen-tiny", max_pos=64),
    "gemma3": gemma3(6, 64, 4, 1, 16, 96, vocab=89, name="gemma-tiny", sliding_window=5,
                     query_pre_attn_scalar=16),
}


@pytest.mark.parametrize("case", list(CASES))
def test_model_step_vs_hf(case):
    mc = CASES[case]
    B, S = 2, 12
    om = O.OracleModel(mc)
    vals = init_values(om, seed=3)
    # ids from a per-case generator: the result must not depend on test order
    rng = np.random.default_rng(sorted(CASES).index(case) + 11)
    ids = rng.integers(0, mc.vocab, (B, S)).astype(np.int32)
    labels = ids.copy()
    labels[1, 4] = -100
    mask = np.ones((B, S), np.float32)
    loss = om.fwd_bwd(ids, mask, labels, B, S, 1.0)

    model = hf_model(mc)
    wraps = load_hf(model, mc, vals)
    out = model(input_ids=torch.tensor(ids, dtype=torch.long),
                labels=torch.tensor(labels, dtype=torch.long))
    assert abs(loss - out.loss.item()) < 2e-5 * abs(out.loss.item()), (loss, out.loss.item())
    out.loss.backward()
    for name, w in wraps.items():
        assert rel_err(om.get(name + ".lora_A", grad=True), w.A.grad.numpy()) < 1e-4, name
        assert rel_err(om.get(name + ".lora_B", grad=True), w.B.grad.numpy()) < 1e-4, name

    # one clip + Adam step (clip_and_get_grad_norm then Adam::step)
    lr, clip = 1e-3, 0.05
    params = [p for w in wraps.values() for p in (w.A, w.B)]
    tot = torch.sqrt(sum((p.grad ** 2).sum() for p in params))
    norm = om.opt_step(lr, clip=clip)
    assert abs(norm - min(tot.item(), clip)) < 1e-5 * max(1.0, tot.item())
    if tot > clip:
        for p in params:
            p.grad *= clip / (tot + 1e-6)
    grads = {id(p): p.grad.detach().clone() for p in params}
    opt = torch.optim.Adam(params, lr=lr, betas=(0.9, 0.999), eps=1e-8)
    opt.step()
    for name, w in wraps.items():
        for t, p in (("lora_A", w.A), ("lora_B", w.B)):
            # Adam's first step is ~lr*sign(g); an element whose fp64 gradient
            # is below the fp32 gradient's rounding noise (1e-6 of the tensor's
            # largest) has no defined sign in fp32, so it is left out.
            g = grads[id(p)].numpy()
            ok = np.abs(g) > 1e-6 * np.abs(g).max()
            assert ok.mean() > 0.99, (name, t)
            assert rel_err(om.get(name + "." + t)[ok], p.detach().numpy()[ok]) < 2e-5, (name, t)
        assert np.abs(om.get(name + ".lora_A", grad=True)).max() == 0  # zero_grad


def test_grad_accum_loss_scaling_equals_grad_scaling():
    """Loss scaling by 1/accum (gpt2 main.cpp:480-485) and host grad scaling
    (qwen wikitext_main.cpp:147-157) give the same accumulated gradient."""
    mc = CASES["qwen2"]
    B, S = 1, 10
    ids = RNG.integers(0, mc.vocab, (2, B, S)).astype(np.int32)
    a = O.OracleModel(mc)
    init_values(a, seed=5)
    b = O.OracleModel(mc)
    init_values(b, seed=5)
    for i in range(2):
        a.fwd_bwd(ids[i], None, ids[i], B, S, 0.5)
        b.fwd_bwd(ids[i], None, ids[i], B, S, 1.0)
    n = "layers.0.self_attn.q_proj.lora_B"
    assert rel_err(a.get(n, grad=True), 0.5 * b.get(n, grad=True)) < 1e-6


def test_fp16_storage_model_equals_dequantised_fp32():
    """Config-5 semantics: fp16-stored frozen weights behave exactly like the
    fp32 model whose weights are those fp16 values widened."""
    base = gemma3(2, 32, 2, 1, 16, 48, vocab=61, name="g16", sliding_window=4,
                  query_pre_attn_scalar=16)
    f16 = gemma3(2, 32, 2, 1, 16, 48, vocab=61, name="g16", sliding_window=4,
                 query_pre_attn_scalar=16, w_fp16=1)
    a = O.OracleModel(f16)
    vals = init_values(a, seed=11)
    b = O.OracleModel(base)
    for n, v in vals.items():
        b.set_param(n, v)
    ids = RNG.integers(0, 61, (2, 8)).astype(np.int32)
    la = a.fwd_bwd(ids, None, ids, 2, 8, 1.0)
    lb = b.fwd_bwd(ids, None, ids, 2, 8, 1.0)
    assert la == lb
    n = "layers.1.mlp.down_proj.lora_A"
    assert np.array_equal(a.get(n, grad=True), b.get(n, grad=True))


def test_blas_backed_oracle_equals_exact_loops():
    """The CPU-baseline configuration (GEMMs in a dlopen'd CBLAS, threads on
    libgomp) computes the same step as the fp64-accumulating loops, also with
    torch (and its OpenMP runtime) already loaded in the process."""
    import sys
    assert "torch" in sys.modules
    mc = gpt2(2, 256, 4, vocab=5003, max_pos=64, name="gpt2-blas")
    res = []
    for blas in (0, 1):
        O.lib().orc_set_blas(blas)
        om = O.OracleModel(mc)
        init_values(om, seed=21)
        ids = np.random.default_rng(2).integers(0, mc.vocab, (2, 64)).astype(np.int32)
        loss = om.fwd_bwd(ids, None, ids, 2, 64, 1.0)
        res.append((loss, om.get("h.0.attn.c_attn.lora_A", grad=True)))
    O.lib().orc_set_blas(0)
    if O.lib().orc_blas_backend() is None:
        pytest.skip("no CBLAS available")
    assert abs(res[0][0] - res[1][0]) < 1e-5 * res[0][0]
    assert rel_err(res[1][1], res[0][1]) < 1e-4


class LoraDropWrap(LoraWrap):
    """PEFT's lora_B(lora_A(dropout(x)))·s with a given dropout mask
    (1/(1-p) where kept) over the token rows of x."""

    def __init__(self, base, A, B, s, mask):
        super().__init__(base, A, B, s)
        self.mask = torch.tensor(mask, dtype=torch.float64)

    def forward(self, x):
        xd = x * self.mask.reshape(x.shape)
        return self.base(x) + self.s * (xd @ self.A.T) @ self.B.T


def _lid(mc, name):
    """The dropout stream id of a LoRA linear: layer·8 + target index."""
    parts = name.split(".")
    layer = int(parts[1])
    tail = ".".join(parts[2:])
    names = (["attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"] if mc.arch == 0 else
             ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
              "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"])
    return layer * 8 + names.index(tail)


def test_dropout_mask_statistics_and_determinism():
    """The mask holds exactly 0 or 1/(1-p), keeps a Binomial(n, 1-p) share of
    elements (within 5 sigma), is a pure function of (seed, step, stream) and
    differs between steps and streams; p = 0 keeps everything."""
    n, p = 200_000, 0.1
    m = O.dropout_mask(9, 1, 3, (n,), p)
    keep = m > 0
    assert np.all((m == 0) | (m == np.float32(1 / (1 - p))))
    assert abs(keep.mean() - (1 - p)) < 5 * np.sqrt(p * (1 - p) / n)
    assert np.array_equal(m, O.dropout_mask(9, 1, 3, (n,), p))
    for other in (O.dropout_mask(9, 2, 3, (n,), p), O.dropout_mask(9, 1, 4, (n,), p),
                  O.dropout_mask(10, 1, 3, (n,), p)):
        agree = ((other > 0) == keep).mean()
        assert agree < 1 - p * (1 - p)  # independent masks agree on p²+(1-p)² of elements
    assert np.all(O.dropout_mask(9, 1, 3, (1000,), 0.0) == 1.0)


@pytest.mark.parametrize("case", ["gpt2-mlp-lora", "qwen2"])
def test_model_step_with_lora_dropout_vs_hf(case):
    """LoRA dropout (training forward, p = 0.2): the oracle's loss and every
    LoRA gradient against HF models whose LoRA branch reads x·mask, the mask
    of each linear taken from the oracle's stream (step 1 of the run).  A
    second oracle forward in evaluation mode applies no dropout."""
    import dataclasses
    mc = dataclasses.replace(CASES[case], lora_dropout=0.2, dropout_seed=77)
    B, S = 2, 12
    om = O.OracleModel(mc)
    vals = init_values(om, seed=4)
    ids = np.random.default_rng(31).integers(0, mc.vocab, (B, S)).astype(np.int32)
    loss = om.fwd_bwd(ids, None, ids, B, S, 1.0)
    model = hf_model(mc)
    wraps = load_hf(model, dataclasses.replace(mc, lora_dropout=0.0), vals)
    prefix = "transformer." if mc.arch == 0 else "model."
    for name, w in list(wraps.items()):
        K = w.A.shape[1]
        mask = O.dropout_mask(77, 1, _lid(mc, name), (B * S, K), 0.2)
        dw = LoraDropWrap(w.base, w.A.detach().numpy(), w.B.detach().numpy(), w.s, mask)
        mod_path = prefix + name
        parent = model.get_submodule(mod_path.rsplit(".", 1)[0])
        setattr(parent, mod_path.rsplit(".", 1)[1], dw)
        wraps[name] = dw
    out = model(input_ids=torch.tensor(ids, dtype=torch.long), labels=torch.tensor(ids, dtype=torch.long))
    assert abs(loss - out.loss.item()) < 2e-5 * abs(out.loss.item()), (loss, out.loss.item())
    out.loss.backward()
    for name, w in wraps.items():
        assert rel_err(om.get(name + ".lora_A", grad=True), w.A.grad.numpy()) < 1e-4, name
        assert rel_err(om.get(name + ".lora_B", grad=True), w.B.grad.numpy()) < 1e-4, name
    # evaluation forward: no dropout, same loss as a model built without it
    plain = O.OracleModel(dataclasses.replace(mc, lora_dropout=0.0))
    for n, v in vals.items():
        plain.set_param(n, v)
    assert om.forward(ids, None, ids, B, S)[0] == plain.forward(ids, None, ids, B, S)[0]
