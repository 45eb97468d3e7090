"""Pins the oracle's model graphs against committed golden vectors
(tests/golden/hf_lora_step.npz, written by tests/golden/make_hf_golden.py
from HF transformers model classes in float64): loss and every LoRA gradient
of one micro-step for GPT-2 (attention targets and all four targets), Qwen2
(GQA, q/k/v biases) and Gemma3 (sliding window, QK-norm, GeGLU).  Needs no
transformers at test time.  CPU only."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import rel_err
from test_oracle_models import CASES, init_values

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_lora_step.npz")


def load():
    z = np.load(GOLDEN, allow_pickle=False)
    cases = {}
    for k in z.files:
        case, rest = k.split("/", 1)
        cases.setdefault(case, {})[rest] = z[k]
    return cases


GOLD = load()


def test_golden_covers_every_model_case():
    assert set(GOLD) == set(CASES)


@pytest.mark.parametrize("case", sorted(CASES))
def test_oracle_matches_hf_golden(case):
    g = GOLD[case]
    mc = CASES[case]
    om = O.OracleModel(mc)
    vals = init_values(om, seed=int(g["seed"]))
    # the parameters regenerate exactly (guards against a changed generator)
    for name, v in vals.items():
        ss = float(np.sum(v.astype(np.float64) ** 2))
        assert abs(ss - float(g["ss/" + name])) <= 1e-9 * max(1.0, ss), name
    ids, labels = g["ids"], g["labels"]
    B, S = ids.shape
    loss = om.fwd_bwd(ids, np.ones((B, S), np.float32), labels, B, S, 1.0)
    assert abs(loss - float(g["loss"])) < 2e-5 * abs(float(g["loss"])), (loss, float(g["loss"]))
    grads = [k for k in g if k.startswith("grad/")]
    assert grads
    for k in grads:
        name = k[len("grad/"):]
        assert rel_err(om.get(name, grad=True), g[k]) < 1e-4, name
