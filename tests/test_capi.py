"""CPU checks of the drop-in boundary: libmft_hip.so loads and exports every
function declared in include/*.h, the ctypes declarations match, and host-side
argument validation rejects bad shapes before any kernel launch (no GPU
needed for these error paths)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "mobilefinetuner_amd", "libmft_hip.so")


def declared_functions():
    names = []
    for hdr in ("mft_hip.h", "mft_engine.h"):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(mft_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "mobilefinetuner_amd", "csrc")],
                       check=True)
    return C.CDLL(LIB)


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_declarations_cover_header():
    from mobilefinetuner_amd._lib import exported_symbols
    assert set(declared_functions()) == set(exported_symbols())


def test_version_and_error_string(lib):
    lib.mft_version.restype = C.c_char_p
    assert b"gfx950" in lib.mft_version()
    lib.mft_last_error.restype = C.c_char_p
    assert isinstance(lib.mft_last_error(), bytes)


def test_null_handle_rejected_without_gpu(lib):
    lib.mft_last_error.restype = C.c_char_p
    rc = lib.mft_synchronize(None)
    assert rc == 1  # MFT_EINVAL
    assert b"null handle" in lib.mft_last_error()


def test_bad_model_config_rejected_without_gpu():
    from mobilefinetuner_amd import _lib
    from mobilefinetuner_amd.configs import gpt2
    L = _lib.lib()
    cfg = gpt2(2, 100, 3).to_ctypes()   # 3 heads × 33 != 100: invalid GPT-2 shape
    h = C.c_void_p()
    rc = L.mft_model_create(C.byref(h), C.byref(cfg), 128, None)
    assert rc == 1
    assert b"n_head*head_dim" in L.mft_last_error()


class _FakeDev:
    """Stands in for a contiguous device tensor (no GPU in this process)."""

    def __init__(self, dtype):
        import torch
        self.dtype = dtype
        self.is_cuda = True
        self._torch = torch

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return 4096


def test_ops_pointer_helper_checks_dtype():
    """The C-ABI takes raw pointers, so the Python wrappers check element types:
    a float64 tensor handed to a float32 argument is an error, not a misread."""
    import torch

    from mobilefinetuner_amd import ops
    assert ops._p(_FakeDev(torch.float32)).value == 4096
    with pytest.raises(TypeError):
        ops._p(_FakeDev(torch.float64))
    with pytest.raises(TypeError):
        ops._p(_FakeDev(torch.float32), torch.int32)
    assert ops._p(_FakeDev(torch.float16), (torch.float32, torch.float16)).value == 4096
    assert ops._p(None) is None


OPS_LIB = os.path.join(ROOT, "mobilefinetuner_amd", "libfinetune_ops.so")
OPS_HDRS = os.path.join(ROOT, "include", "finetune_ops")


def test_operator_headers_compile_standalone(tmp_path):
    """Every finetune_ops header compiles on its own with the host compiler
    (the reference drivers include them individually)."""
    hdrs = sorted(os.path.relpath(os.path.join(d, f), os.path.join(ROOT, "include"))
                  for d, _, fs in os.walk(OPS_HDRS) for f in fs if f.endswith(".h"))
    assert len(hdrs) >= 10
    for h in hdrs:
        src = tmp_path / "inc.cpp"
        src.write_text(f'#include "{h}"\nint main() {{ return 0; }}\n')
        r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                            "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
        assert r.returncode == 0, (h, r.stderr)


def test_operator_library_loads_and_exports_api():
    """libfinetune_ops.so (built by build()) loads without a GPU and exports
    the operator API the drivers link against."""
    if not os.path.exists(OPS_LIB):
        pytest.skip("libfinetune_ops.so not built (run __graft_entry__.build())")
    C.CDLL(os.path.join(ROOT, "mobilefinetuner_amd", "libmft_hip.so"), mode=C.RTLD_GLOBAL)
    C.CDLL(OPS_LIB)
    r = subprocess.run(["nm", "-DC", "--defined-only", OPS_LIB], capture_output=True, text=True, check=True)
    for sym in ("ops::lm_cross_entropy(", "ops::mul(", "ops::lora_linear(", "ops::causal_attention(",
                "ops::Adam::step(", "ops::GPT2Model::GPT2Model(", "ops::QwenModel::init_lora(",
                "ops::GemmaLoraInjector::inject(", "ops::LoraInjector::inject(", "ops::EngineModel::forward(",
                "ops::autograd::Engine::instance(", "ops::Tensor::backward(", "ops::perplexity_from_loss(",
                "ops::MemoryMonitor::get_system_memory_usage(", "ops::GPT2Config::from_pretrained("):
        assert sym in r.stdout, sym


def test_config_readers_parse_hf_config_json(tmp_path):
    """GPT2Config / QwenConfig / GemmaTextConfig::from_pretrained read the
    numeric fields of HF config.json files (no GPU call involved)."""
    if not os.path.exists(OPS_LIB):
        pytest.skip("libfinetune_ops.so not built (run __graft_entry__.build())")
    (tmp_path / "gpt2.json").write_text('{"n_embd": 1024, "n_layer": 24, "n_head": 16, "vocab_size": 50257,'
                                        ' "n_positions": 1024, "layer_norm_epsilon": 1e-05, "n_inner": null}')
    (tmp_path / "qwen.json").write_text('{"hidden_size": 896, "num_hidden_layers": 24, "num_attention_heads": 14,'
                                        ' "num_key_value_heads": 2, "intermediate_size": 4864,'
                                        ' "vocab_size": 151936, "rope_theta": 1000000.0, "rms_norm_eps": 1e-06}')
    (tmp_path / "config.json").write_text('{"hidden_size": 640, "num_hidden_layers": 18, "head_dim": 256,'
                                          ' "num_key_value_heads": 1, "sliding_window": 512,'
                                          ' "rope_local_base_freq": 10000.0, "query_pre_attn_scalar": 256}')
    src = tmp_path / "cfg.cpp"
    src.write_text(r'''
#include <cstdio>
#include "finetune_ops/graph/gpt2_model.h"
#include "finetune_ops/graph/qwen_model.h"
#include "finetune_ops/graph/gemma_model.h"
int main(int, char** argv) {
  std::string d = argv[1];
  auto g = ops::GPT2Config::from_pretrained(d + "/gpt2.json");
  auto q = ops::QwenConfig::from_pretrained(d + "/qwen.json");
  auto m = ops::GemmaTextConfig::from_pretrained(d);
  std::printf("%d %d %d %d %d %g | %d %d %d %g | %d %d %d %d %g\n", g.n_embd, g.n_layer, g.n_head, g.vocab_size,
              g.n_inner, g.layer_norm_epsilon, q.hidden_size, q.num_key_value_heads, q.intermediate_size,
              q.rope_theta, m.hidden_size, m.num_hidden_layers, m.head_dim, m.sliding_window,
              m.query_pre_attn_scalar);
  return 0;
}
''')
    exe = tmp_path / "cfg"
    subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
                    "-L", os.path.dirname(OPS_LIB), "-lfinetune_ops", "-lmft_hip",
                    "-Wl,-rpath," + os.path.dirname(OPS_LIB)], check=True)
    out = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, check=True).stdout.split()
    assert out == ["1024", "24", "16", "50257", "0", "1e-05", "|", "896", "2", "4864", "1e+06", "|",
                   "640", "18", "256", "512", "256"]
