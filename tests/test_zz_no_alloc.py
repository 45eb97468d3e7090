"""mft_ce_fwd_bwd_noalloc (the cross-entropy entry point whose scratch is a
fixed device array inside the library) against mft_ce_fwd_bwd, through the
C-ABI: two calls in a row, the second on a smaller input, must give
bit-identical loss sums, counts, row NLLs and dlogits (same kernels, same
reduction order).  Sizes beyond the array's maximum are rejected on the host
before any launch."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from mobilefinetuner_amd._lib import MFTError, call, lib  # noqa: E402
from mobilefinetuner_amd.ops import handle  # noqa: E402

MAX_ROWS = 1 << 16


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _run(name, logits, labels, B, S, up, keep_nll):
    V = logits.shape[-1]
    loss = torch.zeros(1, device="cuda", dtype=torch.float64)
    cnt = torch.zeros(1, device="cuda", dtype=torch.int64)
    dl = torch.empty_like(logits)
    nll = torch.empty(B * S, device="cuda", dtype=torch.float32) if keep_nll else None
    call(name, handle(), _ptr(logits), _ptr(labels), B, S, V, -100, up, 0, _ptr(loss), _ptr(cnt),
         _ptr(dl), _ptr(nll))
    torch.cuda.synchronize()
    return loss, cnt, dl, nll


@pytest.mark.parametrize("keep_nll", [False, True])
def test_noalloc_ce_equals_allocating_entry_point(keep_nll):
    rng = np.random.default_rng(31)
    # each call smaller than the one before it in its pair: stale scratch must
    # not leak into it; the last pair runs the maximum row count (65536, the
    # separately counted targets) and then a count-in-row-workgroup batch
    for B, S, V, up in ((4, 128, 50257, 1.0), (2, 33, 3001, 0.5), (16, 4096, 64, 1.0), (2, 1000, 77, 0.5)):
        print(f"ce noalloc B={B} S={S} V={V} keep_nll={keep_nll}", flush=True)
        logits = torch.from_numpy((rng.standard_normal((B * S, V)) * 2).astype(np.float32)).cuda()
        lab = rng.integers(0, V, (B, S)).astype(np.int32)
        lab[0, 3] = -100
        labels = torch.from_numpy(lab).cuda()
        ref = _run("mft_ce_fwd_bwd", logits, labels, B, S, up, True)
        got = _run("mft_ce_fwd_bwd_noalloc", logits, labels, B, S, up, keep_nll)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
        assert int(got[1].item()) == B * (S - 1) - 1
        assert torch.equal(got[2], ref[2])
        if keep_nll:
            assert torch.equal(got[3], ref[3])


def test_noalloc_ce_rejects_beyond_maximum():
    logits = torch.zeros(1, 8, device="cuda")
    labels = torch.zeros(1, device="cuda", dtype=torch.int32)
    with pytest.raises(MFTError, match="no-allocation maximum"):
        call("mft_ce_fwd_bwd_noalloc", handle(), _ptr(logits), _ptr(labels), 2, MAX_ROWS, 8, -100,
             1.0, 0, None, None, None, None)
    assert lib() is not None
