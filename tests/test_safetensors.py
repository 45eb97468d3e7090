"""Safetensors I/O of the operators library (host layer, no GPU).

The `safetensors` package writes the inputs and reads our outputs, so the
reader, the writer and their agreement on the format are checked against an
independent implementation; the key mappers are checked against the
state_dict keys and layouts of HF's GPT2LMHeadModel, Qwen2ForCausalLM and
Gemma3ForCausalLM built from tiny local configs (no download).  The drivers'
load calls are gpt2_small_lora_finetune/src/main.cpp:207-219 (transpose off),
qwen_lora_finetune/src/wikitext_main.cpp:67-74 (transpose on) and
gemma_3_270m_lora_finetune/src/main.cpp:332-340 (the default, on).
"""
import os
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file
from safetensors.torch import save_file

from test_oracle_models import CASES, hf_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin", "test_safetensors")

pytestmark = pytest.mark.skipif(not os.path.exists(BIN), reason="tests/cpp not built (run __graft_entry__.build())")


def run(*args, ok=True):
    r = subprocess.run([BIN, *map(str, args)], capture_output=True, text=True, timeout=120)
    if ok:
        assert r.returncode == 0, r.stdout + r.stderr
    return r


def test_roundtrip_dtypes_and_transpose(tmp_path):
    g = torch.Generator().manual_seed(7)
    src = {
        "a.f32": torch.randn(5, 7, generator=g),
        "b.f16": torch.randn(3, 4, generator=g).half(),
        "c.bf16": torch.randn(6, 2, generator=g).bfloat16(),
        "d.vec": torch.randn(9, generator=g),
        "e.cube": torch.randn(2, 3, 4, generator=g),
        "f.empty": torch.zeros(0, 3),
        "g.special": torch.tensor([[0.0, -0.0, float("inf")], [float("-inf"), 6.1e-5, 65504.0]]).half(),
    }
    meta = {"format": "pt", "note": 'quote " backslash \\ tab \t'}
    fin = tmp_path / "in.safetensors"
    save_file(src, str(fin), metadata=meta)
    for transpose in (0, 1):
        fout = tmp_path / f"out{transpose}.safetensors"
        run("convert", fin, fout, transpose)
        out = load_file(str(fout))
        assert set(out) == set(src)
        for k, t in src.items():
            want = t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()
            if transpose and want.ndim == 2:
                want = want.T
            got = out[k]
            assert got.dtype == (np.float16 if t.dtype == torch.float16 else np.float32), k
            assert got.shape == want.shape, k
            np.testing.assert_array_equal(got.view(np.uint8), np.ascontiguousarray(want).view(np.uint8), err_msg=k)
        with open(fout, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            assert (8 + n) % 8 == 0  # data section 8-byte aligned
        from safetensors import safe_open
        with safe_open(str(fout), "np") as f:
            assert f.metadata() == meta


def _write_raw(path, header: bytes, data: bytes):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header)))
        f.write(header)
        f.write(data)


@pytest.mark.parametrize("header,data,msg", [
    (b'{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', b"\0" * 8, "do not match"),
    (b'{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 4, "do not match"),
    (b'{"x":{"dtype":"Q7","shape":[2],"data_offsets":[0,8]}}', b"\0" * 8, "unknown dtype"),
    (b'{"x":{"dtype":"F32","shape":[-2],"data_offsets":[0,8]}}', b"\0" * 8, "shape"),
    (b'{"x":{"dtype":"F32","shape":[2]}}', b"\0" * 8, "malformed"),
    (b'{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}', b"\0" * 8, "expected"),
    (b'[1,2]', b"", "not an object"),
])
def test_malformed_headers_rejected(tmp_path, header, data, msg):
    p = tmp_path / "bad.safetensors"
    _write_raw(p, header, data)
    r = run("header", p, ok=False)
    assert r.returncode == 1 and msg in r.stdout, r.stdout


def test_truncated_and_missing(tmp_path):
    p = tmp_path / "short.safetensors"
    p.write_bytes(b"\x10\0\0")
    r = run("header", p, ok=False)
    assert r.returncode == 1 and "too short" in r.stdout
    p2 = tmp_path / "len.safetensors"
    p2.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    r = run("header", p2, ok=False)
    assert r.returncode == 1 and "bad header length" in r.stdout
    r = run("header", tmp_path / "absent.safetensors", ok=False)
    assert r.returncode == 1 and "cannot open" in r.stdout


def _hf_state(case):
    model = hf_model(CASES[case])
    sd = {k: v.float().contiguous().clone() for k, v in model.state_dict().items()
          if k != "lm_head.weight" and not k.endswith((".attn.bias", ".attn.masked_bias"))}
    return sd


@pytest.mark.parametrize("case,arch,transpose,prefix", [
    ("gpt2", "gpt2", 0, "transformer."),
    ("qwen2", "qwen", 1, ""),
    ("gemma3", "gemma", 1, ""),
])
def test_mapping_matches_hf_layout(tmp_path, case, arch, transpose, prefix):
    """Every HF parameter is mapped exactly once and loads, after the
    drivers' transpose choice, in the [in, out] layout the models take."""
    mc = CASES[case]
    sd = _hf_state(case)
    fin = tmp_path / "model.safetensors"
    save_file(sd, str(fin))
    lines = run("mapping", arch, mc.n_layer).stdout.strip().splitlines()
    mapping = dict(line.split("\t") for line in lines)
    hf_keys = {prefix + v for v in mapping.values()}
    assert hf_keys == set(sd), sorted(hf_keys ^ set(sd))
    fout = tmp_path / "mapped.safetensors"
    run("load_mapped", arch, mc.n_layer, fin, fout, transpose)
    out = load_file(str(fout))
    assert set(out) == set(mapping)
    for internal, hf in mapping.items():
        want = sd[prefix + hf].numpy()
        if transpose and want.ndim == 2 and "embed" not in internal:
            want = want.T  # nn.Linear [out, in] → [in, out]
        np.testing.assert_array_equal(out[internal], want, err_msg=internal)
