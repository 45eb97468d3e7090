"""Shared test helpers: seeded parameter values for the model graphs."""
import numpy as np


def param_values(params, seed=0, norm_std=0.1, w_std=0.02):
    """Seeded values for a parameter list (dicts with name/shape/f16).
    LoRA A ~ N(0, 1/8), LoRA B ~ N(0, 0.1) (non-zero branch), weights and
    biases N(0, w_std), norm weights perturbed around their identity value.
    fp16-stored tensors are returned as uint16 bit patterns (RNE)."""
    rng = np.random.default_rng(seed)
    vals = {}
    for p in params:
        n = p["name"]
        if n.endswith("lora_A"):
            v = rng.standard_normal(p["shape"]) / 8.0
        elif n.endswith("lora_B"):
            v = rng.standard_normal(p["shape"]) * 0.1
        elif "norm" in n or "ln_" in n:
            base = 1.0 if ("ln_" in n and n.endswith("weight")) else 0.0
            v = rng.standard_normal(p["shape"]) * norm_std + base
        else:
            v = rng.standard_normal(p["shape"]) * w_std
        v = v.astype(np.float32)
        if p["f16"]:
            v = v.astype(np.float16).view(np.uint16)
        vals[n] = v
    return vals
