"""Writes tests/golden/hf_lora_step.npz: per-case inputs and expected outputs
of one LoRA training micro-step computed by HF transformers model classes
(GPT2LMHeadModel, Qwen2ForCausalLM, Gemma3ForCausalLM) built from local
config objects (no download) in float64, with LoRA as x·W + b + s·(x·Aᵀ)·Bᵀ
around the targeted projections.  transformers is a third-party library, not
reference code: these vectors pin the oracle's model graphs (HF semantics
the reference's drivers load checkpoints for) without needing transformers
at test time.

Stored per case: the parameter seed and a per-tensor sum-of-squares
fingerprint of the parameters it generates (tests/test_oracle_models.py
init_values), ids, labels (with one ignored target), the loss and every LoRA
gradient.  Regenerate with:  python tests/golden/make_hf_golden.py
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
SEED = 3


def main():
    out = {}
    for ci, (case, mc) in enumerate(sorted(CASES.items())):
        om = O.OracleModel(mc)
        vals = init_values(om, seed=SEED)
        rng = np.random.default_rng(100 + ci)
        ids = rng.integers(0, mc.vocab, (B, S)).astype(np.int32)
        labels = ids.copy()
        labels[1, 4] = -100
        model = hf_model(mc)
        wraps = load_hf(model, mc, vals)
        res = model(input_ids=torch.tensor(ids, dtype=torch.long), labels=torch.tensor(labels, dtype=torch.long))
        res.loss.backward()
        out[f"{case}/seed"] = np.array(SEED)
        out[f"{case}/ids"] = ids
        out[f"{case}/labels"] = labels
        out[f"{case}/loss"] = np.array(res.loss.item())
        for name, v in vals.items():
            out[f"{case}/ss/{name}"] = np.array(float(np.sum(v.astype(np.float64) ** 2)))
        for name, w in wraps.items():
            out[f"{case}/grad/{name}.lora_A"] = w.A.grad.numpy().astype(np.float32)
            out[f"{case}/grad/{name}.lora_B"] = w.B.grad.numpy().astype(np.float32)
        print(case, "loss", res.loss.item(), "lora tensors", 2 * len(wraps))
    np.savez_compressed(os.path.join(HERE, "hf_lora_step.npz"), **out)


if __name__ == "__main__":
    main()
