"""Shard store (ParameterSharder's require() streaming, README.md:302-329):
frozen linear weights and the token embedding live in pinned host memory and
stream into an HBM pool of a fixed budget, least recently used evicted, the
next tensor prefetched on a copy stream.  A budget below the model's weight
bytes must give steps bit-identical to the same model with every weight
resident; a budget below the largest tensor is rejected
(scripts/benchmark/test_sharding_aggressive.sh:58-65)."""
import dataclasses

import numpy as np
import pytest

import oracle as O
from conftest import rel_err
from helpers import param_values
from mobilefinetuner_amd.configs import gemma3, gpt2, qwen2

pytestmark = pytest.mark.gpu
TOL = 1e-4

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from mobilefinetuner_amd.engine import Model  # noqa: E402

# fp16-stored weights: the rank-r panel path.  A model whose weights all stay
# in HBM runs q|k|v and gate|up as segmented launches (one launch for the
# three / two projections); the shard store launches each projection on its
# own (one streamed weight at a time), so bit-for-bit comparisons pit the
# streamed model against a store whose budget holds every weight (resident
# after the first use: the same kernels on the same values).
F16 = gemma3(3, 128, 2, 1, 256, 320, vocab=611, name="gemma-s16", w_fp16=1, sliding_window=24,
             query_pre_attn_scalar=256)


def streamed(model):
    """Byte sizes of the tensors the shard store streams (linear weights and
    the token embedding)."""
    out = []
    for p in model.params:
        if p["trainable"] or len(p["shape"]) != 2 or p["name"] == "wpe":
            continue
        n = int(np.prod(p["shape"]))
        out.append(n * (2 if p["f16"] else 4))
    return out


def steps(eng, ids, S, n, lr=1e-3):
    losses = []
    for i in range(n):
        eng.train_step(ids[i], ids[i], S=S, lr=lr, clip=1.0, graph=True)
        losses.append(eng.read_stats())
    return losses


def test_streamed_steps_equal_resident_steps_bit_for_bit():
    B, S = 2, 32
    print("shard store: gemma3 fp16 W, budget 1.3x the largest tensor", flush=True)
    hbm = Model(F16, B * S)  # every weight in HBM, no store
    sizes = streamed(hbm)
    budget = int(max(sizes) * 1.3)
    assert budget < sum(sizes)
    ref = Model(dataclasses.replace(F16, shard_budget=2 * sum(sizes)), B * S)  # the store, everything fits
    sh = Model(dataclasses.replace(F16, shard_budget=budget), B * S)
    vals = param_values(hbm.params, seed=3)
    for n, v in vals.items():
        hbm.set_param(n, v)
        ref.set_param(n, v)
        sh.set_param(n, v)
    rng = np.random.default_rng(4)
    ids = [torch.from_numpy(rng.integers(0, F16.vocab, (B * S,)).astype(np.int32)).cuda() for _ in range(3)]
    la = steps(ref, ids, S, 3)
    lb = steps(sh, ids, S, 3)
    lh = steps(hbm, ids, S, 3)
    assert la == lb, (la, lb)
    for p in ref.params:
        if p["trainable"]:
            assert np.array_equal(ref.get(p["name"]), sh.get(p["name"])), p["name"]
            # the store-free model's segmented launches sum in another order
            assert rel_err(hbm.get(p["name"]), sh.get(p["name"])) < 1e-5, p["name"]
    for (x, _, _), (y, _, _) in zip(lh, lb):
        assert abs(x - y) <= 1e-5 * abs(y), (lh, lb)
    loads_ref, _, _ = ref.shard_stats()
    assert loads_ref == len(sizes), loads_ref  # the roomy store loaded each weight once
    loads, hits, bud = sh.shard_stats()
    # every tensor is used at least twice per step; with room for about one
    # tensor most uses have to stream
    assert bud == budget & ~255 and loads > 2 * len(sizes), (loads, hits, bud)
    assert hbm.shard_stats() == (0, 0, 0)
    hbm.close()
    ref.close()
    sh.close()


def test_budget_holding_every_tensor_streams_each_once():
    B, S = 2, 32
    probe = Model(F16, B * S)
    sizes = streamed(probe)
    probe.close()
    eng = Model(dataclasses.replace(F16, shard_budget=sum(s + 256 for s in sizes)), B * S)
    eng.init_params(5)
    ids = [torch.from_numpy(np.random.default_rng(i).integers(0, F16.vocab, (B * S,)).astype(np.int32)).cuda()
           for i in range(3)]
    steps(eng, ids, S, 1)
    loads1, hits1, _ = eng.shard_stats()
    steps(eng, ids[1:], S, 2)
    loads3, hits3, _ = eng.shard_stats()
    assert loads1 == len(sizes) and loads3 == loads1 and hits3 > hits1, (loads1, loads3, hits1, hits3)
    eng.close()


def test_streamed_fp32_gpt2_step_matches_oracle():
    """fp32 weights streamed (a sharded model takes the rank-r panel path,
    not the merged W_eff): loss and LoRA gradients against the oracle."""
    mc = gpt2(2, 256, 4, vocab=1000, max_pos=128, name="gpt2-shard", lora_mask=0b1111)
    B, S = 2, 48
    probe = Model(mc, B * S)
    sizes = streamed(probe)
    probe.close()
    mc = dataclasses.replace(mc, shard_budget=int(max(sizes) * 1.5))
    print("shard store: gpt2 fp32, budget", mc.shard_budget, flush=True)
    O.lib().orc_set_blas(0)
    om = O.OracleModel(mc)
    eng = Model(mc, B * S)
    for n, v in param_values(om.params, seed=6).items():
        om.set_param(n, v)
        eng.set_param(n, v)
    rng = np.random.default_rng(7)
    for step in range(2):
        ids = rng.integers(0, mc.vocab, (B, S)).astype(np.int32)
        lo = om.fwd_bwd(ids, None, ids, B, S, 1.0)
        dev = torch.from_numpy(ids.reshape(-1)).cuda()
        eng.fwd_bwd(dev, dev, S=S)
        torch.cuda.synchronize()
        for p in om.params:
            if p["trainable"]:
                ge, go = eng.get(p["name"], grad=True), om.get(p["name"], grad=True)
                assert rel_err(ge, go) < TOL, (step, p["name"], rel_err(ge, go))
        om.opt_step(1e-3, clip=1.0)
        eng.opt_step(1e-3, clip=1.0)
        le = eng.read_stats()[0]
        assert abs(le - lo) < TOL * abs(lo), (step, le, lo)
        for p in om.params:
            if p["trainable"]:
                om.set_param(p["name"], eng.get(p["name"]))
    eng.close()


def test_budget_below_largest_tensor_is_rejected():
    mc = qwen2(1, 128, 2, 1, 64, 256, vocab=997, name="qwen-shard")
    probe = Model(mc, 64)
    largest = max(streamed(probe))
    probe.close()
    with pytest.raises(RuntimeError, match="below the largest streamed tensor"):
        Model(dataclasses.replace(mc, shard_budget=largest // 2), 64)
