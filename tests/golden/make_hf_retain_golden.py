"""Writes tests/golden/hf_gemma_retained.npz: the activation gradients that
the Gemma driver's alignment dump reads (retain_grad() on every
intermediate, gemma_3_270m_lora_finetune/src/main.cpp:547-657), computed by
HF transformers' Gemma3ForCausalLM (third-party library, not reference
code) built from a local config in float64 with LoRA around all seven
projections, for layers 0 (sliding window) and 5 (global) of the tiny
Gemma3 case of tests/test_oracle_models.py.

Gradients are kept with retain_grad(): module outputs and inputs through
forward hooks; the post-RoPE q/k through a wrapper of the module's
apply_rotary_pos_emb; the pre-softmax scores through a wrapper of softmax;
the probabilities from output_attentions.  Keys "<layer>/<name>" use the
oracle's names (oracle.h: orc_model_set_retain), token-major
[B·S, width] or [B, H, S, S]; "-1/embed" is the embedding output's
gradient, "<layer>/probs_act" the probabilities themselves.
Regenerate with:  python tests/golden/make_hf_retain_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402
from test_oracle_models import CASES, hf_model, init_values, load_hf  # noqa: E402

B, S = 2, 12
SEED = 5
LAYERS = (0, 5)


def main():
    import transformers.models.gemma3.modeling_gemma3 as G

    mc = CASES["gemma3"]
    om = O.OracleModel(mc)
    vals = init_values(om, seed=SEED)
    rng = np.random.default_rng(41)
    ids = rng.integers(0, mc.vocab, (B, S)).astype(np.int32)
    labels = ids.copy()
    labels[0, 7] = -100
    model = hf_model(mc)
    load_hf(model, mc, vals)

    kept = {}  # (layer, name) -> tensor whose .grad is wanted
    tok = lambda t: t.reshape(B * S, -1)  # noqa: E731  [B, S, C] -> [B·S, C]
    head = lambda t: t.transpose(1, 2).reshape(B * S, -1)  # noqa: E731  [B, H, S, hd] -> [B·S, H·hd]

    def keep(layer, name, t, how=tok):
        t.retain_grad()
        kept[(layer, name)] = (t, how)

    hooks = []
    layers = model.model.layers
    hooks.append(model.model.embed_tokens.register_forward_hook(lambda m, a, o: keep(-1, "embed", o)))
    current = {"layer": None}
    for li in LAYERS:
        L = layers[li]
        at, mlp = L.self_attn, L.mlp

        def pre_layer(m, a, kw, li=li):
            current["layer"] = li
            keep(li, "x", a[0] if a else kw["hidden_states"])

        def post_layer(m, a, o, li=li):
            keep(li, "out", o[0] if isinstance(o, tuple) else o)
            current["layer"] = None

        hooks.append(L.register_forward_pre_hook(pre_layer, with_kwargs=True))
        hooks.append(L.register_forward_hook(post_layer))
        for mod, name in ((L.input_layernorm, "norm1"), (at.q_proj, "q_proj"), (at.k_proj, "k_proj"),
                          (at.v_proj, "v"), (at.o_proj, "o_proj"), (L.pre_feedforward_layernorm, "norm2"),
                          (mlp.gate_proj, "gate"), (mlp.up_proj, "up"), (mlp.act_fn, "gate_act"),
                          (mlp.down_proj, "down_proj")):
            hooks.append(mod.register_forward_hook(lambda m, a, o, li=li, name=name: keep(li, name, o)))
        hooks.append(at.q_norm.register_forward_hook(lambda m, a, o, li=li: keep(li, "q_normed", o, head)))
        hooks.append(at.k_norm.register_forward_hook(lambda m, a, o, li=li: keep(li, "k_normed", o, head)))
        hooks.append(at.o_proj.register_forward_pre_hook(lambda m, a, li=li: keep(li, "attn", a[0])))
        hooks.append(L.pre_feedforward_layernorm.register_forward_pre_hook(
            lambda m, a, li=li: keep(li, "mid", a[0])))
        hooks.append(mlp.down_proj.register_forward_pre_hook(lambda m, a, li=li: keep(li, "act", a[0])))

    rope0, softmax0 = G.apply_rotary_pos_emb, torch.nn.functional.softmax

    def rope(q, k, cos, sin, *a, **kw):
        qo, ko = rope0(q, k, cos, sin, *a, **kw)
        if current["layer"] is not None:
            keep(current["layer"], "q", qo, head)
            keep(current["layer"], "k", ko, head)
        return qo, ko

    def softmax(x, *a, **kw):
        if current["layer"] is not None and x.dim() == 4:
            keep(current["layer"], "scores", x, lambda t: t)
        return softmax0(x, *a, **kw)

    G.apply_rotary_pos_emb, torch.nn.functional.softmax = rope, softmax
    try:
        res = model(input_ids=torch.tensor(ids, dtype=torch.long), labels=torch.tensor(labels, dtype=torch.long),
                    output_attentions=True)
    finally:
        G.apply_rotary_pos_emb, torch.nn.functional.softmax = rope0, softmax0
        for h in hooks:
            h.remove()
    probs = {li: res.attentions[li] for li in LAYERS}
    for li in LAYERS:
        probs[li].retain_grad()
    res.loss.backward()

    out = {"seed": np.array(SEED), "ids": ids, "labels": labels, "loss": np.array(res.loss.item()),
           "layers": np.array(LAYERS)}
    for name, v in vals.items():
        out[f"ss/{name}"] = np.array(float(np.sum(v.astype(np.float64) ** 2)))
    for (li, name), (t, how) in kept.items():
        out[f"{li}/{name}"] = how(t.grad.detach()).numpy().astype(np.float32)
    for li in LAYERS:
        out[f"{li}/probs"] = probs[li].grad.detach().numpy().astype(np.float32)
        out[f"{li}/probs_act"] = probs[li].detach().numpy().astype(np.float32)
    path = os.path.join(HERE, "hf_gemma_retained.npz")
    np.savez_compressed(path + ".tmp.npz", **out)
    os.replace(path + ".tmp.npz", path)
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main()
