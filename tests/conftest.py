import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU check")


def rel_err(a, b):
    """‖a−b‖₂ / ‖b‖₂ (the tolerance metric of the benchmark)."""
    import numpy as np
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b.ravel())
    num = np.linalg.norm((a - b).ravel())
    return num / den if den > 0 else num


@pytest.fixture
def rel():
    return rel_err


@pytest.fixture(autouse=True)
def _torch_default_dtype_untouched():
    """Process-wide torch state set by one test module would leak into every
    module collected after it (a float64 default dtype once turned dtype-less
    allocations float64): fail the test that changes it."""
    torch = sys.modules.get("torch")
    before = torch.get_default_dtype() if torch is not None else None
    yield
    torch = sys.modules.get("torch")
    if torch is not None and before is not None:
        assert torch.get_default_dtype() == before, "test changed torch's default dtype"
    if torch is not None:
        assert torch.get_default_dtype() == torch.float32, "torch default dtype is not float32"
