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
