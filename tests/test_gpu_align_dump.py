"""The Gemma driver's alignment dump on the GPU engine
(gemma_3_270m_lora_finetune/src/main.cpp:547-657): with retention on, one
step keeps every named activation and activation gradient of the chosen
layers, and the attention scores / probabilities with their gradients.  All
compared with the oracle's retained intermediates (oracle.h:
orc_model_set_retain, pinned against HF retain_grad() by
tests/test_oracle_retained.py) on the same parameters and batch, at the fp32
bar — for the merged q|k|v / gate|up GEMMs, separate q/k/v GEMMs, and the
fp16-stored-W path (oracle fed the same fp16 values)."""
import numpy as np
import pytest

import oracle as O
from conftest import rel_err
from helpers import param_values
from mobilefinetuner_amd.configs import gemma3

pytestmark = pytest.mark.gpu
TOL = 1e-4

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from mobilefinetuner_amd.engine import Model  # noqa: E402

NAMES = ["x", "norm1", "q_proj", "k_proj", "v", "q_normed", "k_normed", "q", "k", "attn", "o_proj", "mid",
         "norm2", "gate", "up", "gate_act", "act", "down_proj", "out", "scores", "probs"]
CASES = {
    # merged LoRA on all seven projections: fused q|k|v and gate|up GEMMs; padding mask
    "gemma3-fused": (gemma3(6, 128, 2, 1, 256, 256, vocab=1009, name="gemma-t", sliding_window=24,
                            query_pre_attn_scalar=256), 2, 40, [0, 5], True),
    # LoRA on q and v: separate q, k, v GEMMs
    "gemma3-qv": (gemma3(2, 128, 2, 1, 256, 256, vocab=509, name="gemma-qv", sliding_window=24,
                         query_pre_attn_scalar=256, lora_mask=0b0000101), 2, 32, [0, 1], False),
    # fp16-stored W: the rank-r panel path on the fp16 matrix cores
    "gemma3-fp16w": (gemma3(2, 128, 4, 2, 64, 320, vocab=611, name="gemma-t16", w_fp16=1, sliding_window=512,
                            query_pre_attn_scalar=64), 2, 32, [1], False),
}


@pytest.mark.parametrize("case", list(CASES))
def test_retained_intermediates_match_oracle(case):
    mc, B, S, layers, pad = CASES[case]
    print(f"align dump {case} B={B} S={S} layers={layers}", flush=True)
    O.lib().orc_set_blas(0)
    om = O.OracleModel(mc)
    eng = Model(mc, B * S)
    for n, v in param_values(om.params, seed=4).items():
        om.set_param(n, v)
        eng.set_param(n, v)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, mc.vocab, (B, S)).astype(np.int32)
    labels = ids.copy()
    labels[0, 3] = -100
    mask = np.ones((B, S), np.float32)
    if pad:
        mask[1, -6:] = 0.0
        labels[1, -6:] = -100
    om.set_retain(layers)
    eng.set_retain(layers)
    lo = om.fwd_bwd(ids, mask, labels, B, S, 1.0)
    eng.fwd_bwd(torch.from_numpy(ids).cuda(), torch.from_numpy(labels).cuda(), torch.from_numpy(mask).cuda())
    le, _, _ = eng.read_stats()
    assert abs(le - lo) < TOL * abs(lo), (le, lo)
    for li in layers:
        for name in NAMES:
            for grad in (False, True):
                ref = om.retained(li, name, grad=grad)
                got = (eng.activation_grad if grad else eng.activation)(li, name).ravel()
                assert ref is not None and got.size == ref.size, (li, name, grad)
                if name == "scores" and not grad:  # masked entries: −FLT_MAX in both
                    masked = ref < -1e38
                    assert np.array_equal(got < -1e38, masked), (li, name)
                    ref, got = ref[~masked], got[~masked]
                err = rel_err(got, ref)
                print(f"  l{li} {name:10s} {'grad' if grad else 'act '} {err:.2e}", flush=True)
                assert err < TOL, (li, name, grad, err)
    if 0 in layers:  # the embedding's gradient = layer 0's input gradient
        assert rel_err(eng.activation_grad(-1, "embed").ravel(), om.retained(-1, "embed", grad=True)) < TOL
    # retention off: later steps keep the training path's results
    eng.set_retain([])
    lo2 = om.fwd_bwd(ids, mask, labels, B, S, 1.0)
    eng.fwd_bwd(torch.from_numpy(ids).cuda(), torch.from_numpy(labels).cuda(), torch.from_numpy(mask).cuda())
    assert abs(eng.read_stats()[0] - lo2) < TOL * abs(lo2)
    eng.close()


def test_retention_is_refused_for_other_architectures():
    from mobilefinetuner_amd.configs import gpt2
    eng = Model(gpt2(1, 64, 2, vocab=97, max_pos=16, name="g"), 16)
    with pytest.raises(Exception, match="Gemma3"):
        eng.set_retain([0])
    eng.close()
