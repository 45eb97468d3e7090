"""Parity of the finetune_ops C++ API (Tensor / autograd / models / Adam on
the GPU) against the CPU oracle, through the driver-style program
tests/cpp/test_operators.cpp (built by __graft_entry__.build())."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "bin", "test_operators")


@pytest.mark.gpu
def test_cpp_operator_api_matches_oracle():
    assert os.path.exists(EXE), "tests/cpp/bin/test_operators missing: run __graft_entry__.build()"
    print("running", EXE, flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=300)
    print(r.stdout[-6000:])
    print(r.stderr[-2000:])
    fails = [ln for ln in r.stdout.splitlines() if ln.startswith("FAIL")]
    assert r.returncode == 0 and not fails, "\n".join(fails) or r.stderr[-2000:]
    # every family and the op chain actually ran
    for tag in ("ops chain dA", "gpt2 step1", "qwen2 step1", "qwen2-dropout step1", "gemma3 step1", "gemma3-fp16w step1",
                "gpt2 checkpoint logits equal", "qwen2 checkpoint logits equal",
                "gemma trainer step3 loss", "gemma trainer LoRA params after 3 steps",
                "resume adapters restored bit for bit", "resumed LoRA params after 2 more steps",
                "gemma retain_grad dlogits", "layout matmul", "gemma trainer embedding dump values",
                "align grad attn_scores_l0", "align grad q_rotary_out_l2", "align grad hidden_states_emb",
                "align analytical dq_l0", "align analytical dv_l2", "gpt2 partial zero_grad keeps host edits"):
        assert any(tag in ln for ln in r.stdout.splitlines()), tag
