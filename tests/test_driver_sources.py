"""The reference drivers' own sources compile, unmodified, against this
build's operators headers (include/finetune_ops): the GPT-2 small / medium,
Qwen2.5 (WikiText) and Gemma-3 270M / 1B training programs.  Their data
layer and tokenizers are outside this build; tests/driver_stubs declares the
names those drivers use from them (WikiText2Dataset, WT2Config, the BPE and
Gemma tokenizers) and nothing else.  g++ -fsyntax-only, CPU only; skipped
where the reference tree is not present."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
DRIVERS = [
    "gpt2_small_lora_finetune/src/main.cpp",
    "gpt2_medium_lora_finetune/src/main.cpp",
    "qwen_lora_finetune/src/wikitext_main.cpp",
    "gemma_3_270m_lora_finetune/src/main.cpp",
    "gemma_3_1b_pt_lora_finetune/src/main.cpp",
]


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
@pytest.mark.parametrize("src", DRIVERS)
def test_reference_driver_compiles_against_headers(src):
    path = os.path.join(REF, src)
    if not os.path.exists(path):
        pytest.skip(f"{src} not in the reference tree")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        "-I", os.path.join(ROOT, "tests", "driver_stubs"), path],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
