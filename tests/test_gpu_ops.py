"""GPU parity of every C-ABI kernel entry point against the CPU oracle on the
same seeded inputs.  Tolerances (relative L2 error ‖y−y_ref‖/‖y_ref‖):
fp32 path ≤ 1e-4; fp16-stored-W path ≤ 2e-3 (the benchmark's bars) —
fp16 W is widened exactly, so those cases are also held to 1e-4 against an
oracle fed the same fp16 values; integer/bit work is bit-exact."""
import math

import numpy as np
import pytest

import oracle as O
from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-4
TOL_F16W = 2e-3

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from mobilefinetuner_amd import ops  # noqa: E402

DEV = "cuda"
RNG = np.random.default_rng(2024)


def rn(*shape, std=1.0):
    return (RNG.standard_normal(shape) * std).astype(np.float32)


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def h(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.fixture(autouse=True, scope="module")
def _exact_oracle():
    O.lib().orc_set_blas(0)  # fp64-accumulating reference loops
    yield


# ------------------------------------------------------------------ LoRA linear
LIN_SHAPES = [
    (77, 132, 200, 8, True),     # ragged M/N, K not a multiple of 16
    (512, 768, 2304, 8, True),   # GPT-2 small c_attn
    (512, 768, 768, 8, True),    # GPT-2 small attn c_proj (split-K path)
    (64, 3072, 768, 4, False),   # few tiles, deep K (split-K)
    (256, 1024, 4096, 16, True), # rank 16, 64 tiles of 64x64 (the 128x128 kernel needs >= 1024 tiles)
    (33, 20, 50, 0, True),       # plain frozen linear (no LoRA)
]


@pytest.mark.parametrize("M,K,N,r,bias", LIN_SHAPES)
def test_lora_linear_fwd(M, K, N, r, bias):
    print(f"lora_linear_fwd M={M} K={K} N={N} r={r}", flush=True)
    x, W, b = rn(M, K), rn(K, N, std=0.05), rn(N) if bias else None
    A, B = (rn(r, K, std=1 / 8), rn(N, r, std=0.02)) if r else (None, None)
    s = 16.0 / max(r, 1)
    y_ref, xa_ref = O.lora_linear_fwd(x, W, b, A, B, s)
    y, xa = ops.lora_linear_fwd(g(x), g(W), g(b) if bias else None, g(A) if r else None,
                                g(B) if r else None, s)
    assert rel_err(h(y), y_ref) < TOL
    if r:
        assert rel_err(h(xa), xa_ref) < TOL


def test_lora_linear_fwd_fused_residual():
    M, K, N, r = 96, 256, 256, 8
    x, W, b, A, B, res = rn(M, K), rn(K, N, std=0.05), rn(N), rn(r, K), rn(N, r), rn(M, N)
    y_ref, _ = O.lora_linear_fwd(x, W, b, A, B, 2.0)
    y, _ = ops.lora_linear_fwd(g(x), g(W), g(b), g(A), g(B), 2.0, resid=g(res))
    assert rel_err(h(y), y_ref + res) < TOL


@pytest.mark.parametrize("M,K,N,r", [(77, 132, 200, 8), (512, 768, 2304, 8), (512, 3072, 768, 8),
                                     (1024, 896, 128, 8), (64, 1024, 1024, 4)])
def test_lora_linear_bwd(M, K, N, r):
    print(f"lora_linear_bwd M={M} K={K} N={N} r={r}", flush=True)
    x, W, A, B, dy = rn(M, K), rn(K, N, std=0.05), rn(r, K, std=1 / 8), rn(N, r, std=0.02), rn(M, N)
    s = 2.0
    _, xa = O.lora_linear_fwd(x, W, None, A, B, s)
    dx_ref, dA_ref, dB_ref = O.lora_linear_bwd(dy, x, W, A, B, xa, s)
    dx, dA, dB = ops.lora_linear_bwd(g(dy), g(x), g(W), g(A), g(B), g(xa), s)
    assert rel_err(h(dx), dx_ref) < TOL
    assert rel_err(h(dA), dA_ref) < TOL
    assert rel_err(h(dB), dB_ref) < TOL
    # accumulate semantics: a second call adds
    ops.lora_linear_bwd(g(dy), g(x), g(W), g(A), g(B), g(xa), s, dA=dA, dB=dB, need_dx=False,
                        accumulate=True)
    assert rel_err(h(dA), 2 * dA_ref) < TOL


@pytest.mark.parametrize("M,K,N", [(128, 1152, 1024), (200, 640, 2048)])
def test_lora_linear_fp16_weight(M, K, N):
    """W stored as fp16 and widened in the GEMM's tile load (config 5)."""
    r = 8
    x, A, B, dy = rn(M, K), rn(r, K, std=1 / 8), rn(N, r, std=0.02), rn(M, N)
    W32 = rn(K, N, std=0.02)
    W16 = W32.astype(np.float16)
    Wf = W16.astype(np.float32)
    y_ref, xa_ref = O.lora_linear_fwd(x, Wf, None, A, B, 4.0)
    y, xa = ops.lora_linear_fwd(g(x), g(W16), None, g(A), g(B), 4.0)
    assert rel_err(h(y), y_ref) < TOL  # exact widening: held to the fp32 bar
    # against the unrounded fp32 weights: the fp16-W bar
    assert rel_err(h(y), O.lora_linear_fwd(x, W32, None, A, B, 4.0)[0]) < TOL_F16W
    dx_ref, dA_ref, dB_ref = O.lora_linear_bwd(dy, x, Wf, A, B, xa_ref, 4.0)
    dx, dA, dB = ops.lora_linear_bwd(g(dy), g(x), g(W16), g(A), g(B), xa, 4.0)
    assert rel_err(h(dx), dx_ref) < TOL
    assert rel_err(h(dA), dA_ref) < TOL
    assert rel_err(h(dB), dB_ref) < TOL


def row_rel_err(a, b):
    """Largest per-row relative error (rows of any magnitude count alike)."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    num = np.linalg.norm(a64 - b64, axis=1)
    den = np.linalg.norm(b64, axis=1)
    return float(np.max(np.where(den > 0, num / np.maximum(den, 1e-300), num)))


F16_MMA_SHAPES = [
    (128, 1152, 1024),  # Gemma-3 1B q projection / dX of o
    (77, 96, 200),      # ragged M and N, three 32-deep panels (odd count)
    (256, 6912, 1152),  # down projection: split-K
    (64, 256, 2304),
]


@pytest.mark.parametrize("M,K,N", F16_MMA_SHAPES)
def test_lora_linear_fp16_matrix_cores_rows_of_any_scale(M, K, N):
    """fp16 W on the fp16 matrix cores: x (forward) and dY (dX) are split
    per row into fp16 hi/lo planes with a power-of-two row scale.  Rows span
    1e-30 .. 1e8 (gradients are tiny, activations are not) and one row is
    zero, so a missing or wrong row scale shows as a row far off; every row is
    held to 2e-5 relative against the oracle (double accumulation) on the same
    fp16 values: the pair keeps 22 significand bits, and fp32 accumulation
    over K = 6912 alone is a few 1e-6."""
    print(f"fp16 matrix-core linear M={M} K={K} N={N}", flush=True)
    r = 8
    rng = np.random.default_rng(M + K + N)
    mags = 10.0 ** rng.uniform(-30, 8, size=(M, 1))
    mags[M // 2] = 0.0
    x = (rn(M, K) * mags).astype(np.float32)
    dy = (rn(M, N) * mags[::-1]).astype(np.float32)
    A, B = rn(r, K, std=1 / 8), rn(N, r, std=0.02)
    Wf = rn(K, N, std=0.02).astype(np.float16).astype(np.float32)
    W16 = Wf.astype(np.float16)
    y_ref, xa_ref = O.lora_linear_fwd(x, Wf, None, A, B, 4.0)
    y, xa = ops.lora_linear_fwd(g(x), g(W16), None, g(A), g(B), 4.0)
    assert row_rel_err(h(y), y_ref) < 2e-5
    assert np.all(h(y)[M // 2] == 0.0)
    dx_ref, _, _ = O.lora_linear_bwd(dy, x, Wf, A, B, xa_ref, 4.0)
    dx, _, _ = ops.lora_linear_bwd(g(dy), g(x), g(W16), g(A), g(B), xa, 4.0)
    assert row_rel_err(h(dx), dx_ref) < 2e-5


def test_lora_linear_fp16_k_tail_takes_widened_path():
    """K = 132 is not a whole number of 32-deep panels: the fp16-W linear
    runs the fp32 kernels with W widened in the tile load instead, same bar."""
    M, K, N, r = 50, 132, 96, 4
    x, A, B = rn(M, K), rn(r, K, std=1 / 8), rn(N, r, std=0.02)
    W16 = rn(K, N, std=0.02).astype(np.float16)
    y_ref, _ = O.lora_linear_fwd(x, W16.astype(np.float32), None, A, B, 2.0)
    y, _ = ops.lora_linear_fwd(g(x), g(W16), None, g(A), g(B), 2.0)
    assert rel_err(h(y), y_ref) < TOL


def test_lm_head_fp16_vocab_gemms():
    """Gemma-3 1B's LM head with the tied embedding E [V, d] stored as fp16
    (config 5): logits = h·Eᵀ runs the 128×128 kernel with an [N, K] fp16
    operand widened in the tile load (8192 tiles at M = 512, V = 262144), and
    dH = dlogits·E reduces over the whole vocabulary (K = 262144, split 16
    ways).  Both against the oracle (BLAS-backed GEMMs) on the same fp16
    values, at the fp32 bar."""
    M, d, V = 512, 1152, 262144
    print(f"lm head fp16 M={M} d={d} V={V}", flush=True)
    E16 = rn(V, d, std=0.02).astype(np.float16)
    Ef = E16.astype(np.float32)
    hf = rn(M, d)
    dlg = rn(M, V, std=1e-4)
    O.lib().orc_set_blas(1)
    try:
        logits_ref = O.lora_linear_bwd(hf, None, Ef, None, None, None, 1.0)[0]
        dh_ref = O.lora_linear_fwd(dlg, Ef, None, None, None, 1.0)[0]
    finally:
        O.lib().orc_set_blas(0)
    gE = g(E16)
    logits = ops.lora_linear_bwd(g(hf), None, gE, None, None, None, 1.0)[0]
    assert rel_err(h(logits), logits_ref) < TOL
    del logits
    dh = ops.lora_linear_fwd(g(dlg), gE, None, None, None, 1.0)[0]
    assert rel_err(h(dh), dh_ref) < TOL


PIPE_SHAPES = [
    (512, 1024, 4096, False),  # 64x64 tiles, 32 whole panels
    (512, 1024, 1024, False),  # 32x64 tiles
    (200, 96, 300, False),     # three panels (odd count), ragged M and N
    (512, 4096, 1024, False),  # split-K: whole panels in every split
    (128, 1152, 1024, True),   # fp16 W widened in the pipelined tile load
]


@pytest.mark.parametrize("M,K,N,f16", PIPE_SHAPES)
def test_plain_linear_pipelined(M, K, N, f16):
    """Linears without a rank-r panel whose K splits into whole 32-deep panels:
    dX (W as the [N,K] operand of dY·Wᵀ) runs the three-stage pipelined GEMM,
    the forward (W as [K,N]) the two-stage one; both against the oracle,
    including an odd panel count, split-K and fp16 W."""
    print(f"pipelined gemm M={M} K={K} N={N} f16={f16}", flush=True)
    x, dy, b = rn(M, K), rn(M, N), rn(N)
    W = rn(K, N, std=0.03)
    Wd = W.astype(np.float16) if f16 else W
    Wf = Wd.astype(np.float32)
    y_ref, _ = O.lora_linear_fwd(x, Wf, b, None, None, 1.0)
    y, _ = ops.lora_linear_fwd(g(x), g(Wd), g(b), None, None, 1.0)
    assert rel_err(h(y), y_ref) < TOL
    dx_ref, _, _ = O.lora_linear_bwd(dy, x, Wf, None, None, None, 1.0)
    dx, _, _ = ops.lora_linear_bwd(g(dy), g(x), g(Wd), None, None, None, 1.0)
    assert rel_err(h(dx), dx_ref) < TOL


def test_lm_head_shapes_odd_vocab():
    """LM-head-shaped product with an odd output width (V = 5003); the
    reduction over an odd V (dH = dlogits·E) runs inside the engine on a
    padded logits pitch and is covered by the model tests (odd vocabularies)."""
    M, d, V = 96, 256, 5003
    x, E = rn(M, d), rn(V, d, std=0.02)
    y_ref, _ = O.lora_linear_fwd(x, E.T.copy(), None, None, None, 1.0)
    y, _ = ops.lora_linear_fwd(g(x), g(E.T.copy()), None, None, None, 1.0)
    assert rel_err(h(y), y_ref) < TOL


def test_lora_linear_rejects_unaligned_pitch():
    """Host-side validation: a row pitch that breaks 16-byte alignment is an
    error, not a silent misread."""
    dl = g(rn(8, 5003))
    with pytest.raises(Exception, match="lda"):
        ops.lora_linear_bwd(dl, g(rn(8, 64)), g(rn(64, 5003)), None, None, None, 1.0)


# ------------------------------------------------------------------ attention
ATTN = [
    (4, 12, 12, 128, 64, 0, False),   # GPT-2 small
    (2, 14, 2, 160, 64, 0, True),     # Qwen-style GQA 7:1, padding mask
    (2, 4, 1, 96, 256, 0, False),     # Gemma hd=256, GQA 4:1
    (1, 4, 1, 200, 256, 64, False),   # Gemma sliding window
    (2, 4, 1, 144, 256, 0, True),     # hd=256 short-sequence forward: padding mask, GQA 4:1
    (1, 4, 2, 77, 128, 0, True),      # hd=128, ragged S
    (2, 4, 2, 200, 64, 48, True),     # short-sequence kernels: sliding window, padding, GQA
    # grids large enough for the 4- and 2-wave workgroup variants
    (8, 16, 4, 256, 64, 0, False),    # 4 waves / workgroup, GQA 4:1
    (4, 8, 2, 500, 128, 0, True),     # 2 waves / workgroup, ragged S, padding mask
    (4, 8, 2, 512, 256, 128, False),  # 2 waves / workgroup, hd=256 sliding window
    # hd=256 at S <= 256: the short backward (head dimension split over the waves)
    (4, 4, 1, 256, 256, 0, False),    # Gemma-3 270M attention shape
    (1, 2, 2, 33, 256, 0, True),      # one query head per KV head (no partial rows), ragged S, padding
    (2, 8, 2, 256, 256, 32, False),   # two KV heads of four query heads each, sliding window 32
]


@pytest.mark.parametrize("B,Hq,Hkv,S,hd,window,pad", ATTN)
def test_attention_fwd_bwd(B, Hq, Hkv, S, hd, window, pad):
    print(f"attention B={B} Hq={Hq} Hkv={Hkv} S={S} hd={hd} win={window}", flush=True)
    q, k, v = rn(B * S, Hq * hd), rn(B * S, Hkv * hd), rn(B * S, Hkv * hd)
    scale = hd ** -0.5
    kpad = None
    if pad:
        kpad = np.ones((B, S), np.float32)
        kpad[-1, S - S // 4:] = 0
        kpad[0, :3] = 0  # leading padded keys: queries 0-2 of sequence 0 see nothing
    o_ref, lse_ref = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, True, window, kpad)
    o, lse = ops.attn_fwd(g(q), g(k), g(v), B, Hq, Hkv, S, hd, scale, True, window,
                          g(kpad) if pad else None)
    assert rel_err(h(o), o_ref) < TOL
    fin = np.isfinite(lse_ref)
    assert rel_err(h(lse)[fin], lse_ref[fin]) < TOL
    dout = rn(B * S, Hq * hd)
    dq_ref, dk_ref, dv_ref = O.attn_bwd(q, k, v, o_ref, dout, lse_ref, B, Hq, Hkv, S, hd, scale,
                                        True, window, kpad)
    dq, dk, dv = ops.attn_bwd(g(q), g(k), g(v), o, g(dout), lse, B, Hq, Hkv, S, hd, scale, True,
                              window, g(kpad) if pad else None)
    assert rel_err(h(dq), dq_ref) < TOL
    assert rel_err(h(dk), dk_ref) < TOL
    assert rel_err(h(dv), dv_ref) < TOL


def test_attention_hd256_short_non_causal():
    """Non-causal attention at head_dim 256 and S <= 256 (every query tile of
    the short backward sees every key tile), GQA 4:1, padding mask."""
    B, Hq, Hkv, S, hd = 2, 4, 1, 80, 256
    q, k, v, dout = rn(B * S, Hq * hd), rn(B * S, Hkv * hd), rn(B * S, Hkv * hd), rn(B * S, Hq * hd)
    kpad = np.ones((B, S), np.float32)
    kpad[1, S - 9:] = 0
    scale = hd ** -0.5
    o_ref, lse_ref = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, False, 0, kpad)
    o, lse = ops.attn_fwd(g(q), g(k), g(v), B, Hq, Hkv, S, hd, scale, False, 0, g(kpad))
    assert rel_err(h(o), o_ref) < TOL
    dq_ref, dk_ref, dv_ref = O.attn_bwd(q, k, v, o_ref, dout, lse_ref, B, Hq, Hkv, S, hd, scale, False, 0, kpad)
    dq, dk, dv = ops.attn_bwd(g(q), g(k), g(v), o, g(dout), lse, B, Hq, Hkv, S, hd, scale, False, 0, g(kpad))
    assert rel_err(h(dq), dq_ref) < TOL
    assert rel_err(h(dk), dk_ref) < TOL
    assert rel_err(h(dv), dv_ref) < TOL


SPLIT_CASES = [
    (1, 14, 2, 1024, 64, 0, False),   # Qwen2.5-0.5B shape: the default plan splits it
    (2, 4, 1, 300, 256, 128, True),   # hd=256, sliding window, padding, ragged
    (1, 4, 2, 333, 128, 0, True),     # hd=128, ragged S, padding
]
_SPLIT_REF = {}


def _split_case(i):
    """Inputs and oracle outputs of SPLIT_CASES[i], computed once per session."""
    if i not in _SPLIT_REF:
        B, Hq, Hkv, S, hd, window, pad = SPLIT_CASES[i]
        rng = np.random.default_rng(100 + i)
        q, k, v, dout = (rng.standard_normal((B * S, n * hd)).astype(np.float32)
                         for n in (Hq, Hkv, Hkv, Hq))
        kpad = None
        if pad:
            kpad = np.ones((B, S), np.float32)
            kpad[-1, S - S // 4:] = 0
            kpad[0, :3] = 0  # leading padded keys: early queries see nothing
        scale = hd ** -0.5
        o, lse = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, scale, True, window, kpad)
        grads = O.attn_bwd(q, k, v, o, dout, lse, B, Hq, Hkv, S, hd, scale, True, window, kpad)
        _SPLIT_REF[i] = (q, k, v, dout, kpad, o, lse, grads)
    return _SPLIT_REF[i]


@pytest.mark.parametrize("per", ["0", "1", "2", "3"])
def test_attention_split(monkeypatch, per):
    """Forward split into key chunks and backward split into query (dK/dV) and
    key (dQ) chunks of `per` loop blocks, merged by the combine / partial-sum
    kernels, against the oracle; 0 = unsplit.  Results must not depend on the
    chunking beyond fp32 rounding."""
    monkeypatch.setenv("MFT_ATTN_KBPC", per)
    monkeypatch.setenv("MFT_ATTN_BWD_BPC", per)
    for i, (B, Hq, Hkv, S, hd, window, pad) in enumerate(SPLIT_CASES):
        print(f"attention split per={per} B={B} Hq={Hq} S={S} hd={hd} win={window}", flush=True)
        q, k, v, dout, kpad, o_ref, lse_ref, (dq_ref, dk_ref, dv_ref) = _split_case(i)
        kp = g(kpad) if pad else None
        scale = hd ** -0.5
        o, lse = ops.attn_fwd(g(q), g(k), g(v), B, Hq, Hkv, S, hd, scale, True, window, kp)
        assert rel_err(h(o), o_ref) < TOL
        fin = np.isfinite(lse_ref)
        assert np.array_equal(np.isfinite(h(lse)), fin)
        assert rel_err(h(lse)[fin], lse_ref[fin]) < TOL
        dq, dk, dv = ops.attn_bwd(g(q), g(k), g(v), o, g(dout), lse, B, Hq, Hkv, S, hd, scale, True,
                                  window, kp)
        assert rel_err(h(dq), dq_ref) < TOL
        assert rel_err(h(dk), dk_ref) < TOL
        assert rel_err(h(dv), dv_ref) < TOL


@pytest.mark.parametrize("mode", ["0", "1"])
def test_attention_short_and_blocked_kernels(monkeypatch, mode):
    """Each kernel family on the other's shapes: the short-sequence kernels
    (one workgroup per 16-row tile, waves splitting the inner loop) forced
    at S = 1024 and 333, the blocked kernels forced at GPT-2's S = 128."""
    monkeypatch.setenv("MFT_ATTN_SHORT", mode)
    cases = [(4, 12, 12, 128, 64, 0, False, None)] if mode == "0" else [
        (None,) * 7 + (0,), (None,) * 7 + (2,)]
    for case in cases:
        if case[-1] is not None:
            B, Hq, Hkv, S, hd, window, pad = SPLIT_CASES[case[-1]]
            q, k, v, dout, kpad, o_ref, lse_ref, (dq_ref, dk_ref, dv_ref) = _split_case(case[-1])
        else:
            B, Hq, Hkv, S, hd, window, pad = case[:7]
            q, k, v, dout = rn(B * S, Hq * hd), rn(B * S, Hkv * hd), rn(B * S, Hkv * hd), rn(B * S, Hq * hd)
            kpad = None
            o_ref, lse_ref = O.attn_fwd(q, k, v, B, Hq, Hkv, S, hd, hd ** -0.5, True, window, kpad)
            dq_ref, dk_ref, dv_ref = O.attn_bwd(q, k, v, o_ref, dout, lse_ref, B, Hq, Hkv, S, hd,
                                                hd ** -0.5, True, window, kpad)
        print(f"attention MFT_ATTN_SHORT={mode} B={B} Hq={Hq} Hkv={Hkv} S={S} hd={hd}", flush=True)
        kp = g(kpad) if kpad is not None else None
        scale = hd ** -0.5
        o, lse = ops.attn_fwd(g(q), g(k), g(v), B, Hq, Hkv, S, hd, scale, True, window, kp)
        assert rel_err(h(o), o_ref) < TOL
        fin = np.isfinite(lse_ref)
        assert rel_err(h(lse)[fin], lse_ref[fin]) < TOL
        dq, dk, dv = ops.attn_bwd(g(q), g(k), g(v), o, g(dout), lse, B, Hq, Hkv, S, hd, scale, True,
                                  window, kp)
        assert rel_err(h(dq), dq_ref) < TOL
        assert rel_err(h(dk), dk_ref) < TOL
        assert rel_err(h(dv), dv_ref) < TOL


def test_attention_strided_qkv_view():
    """q/k/v as views into one fused [M, 3d] QKV buffer (GPT-2 c_attn output)."""
    B, H, S, hd = 2, 4, 64, 64
    d = H * hd
    qkv = rn(B * S, 3 * d)
    q, k, v = qkv[:, :d].copy(), qkv[:, d:2 * d].copy(), qkv[:, 2 * d:].copy()
    o_ref, _ = O.attn_fwd(q, k, v, B, H, H, S, hd, 0.125)
    t = g(qkv)
    o, _ = ops.attn_fwd(t, t[:, d:], t[:, 2 * d:], B, H, H, S, hd, 0.125, q_rs=3 * d, k_rs=3 * d,
                        v_rs=3 * d)
    assert rel_err(h(o), o_ref) < TOL


# ------------------------------------------------------------------ cross-entropy
# (2, 2100, 600): beyond 4096 rows the target count is formed by a launch of
# its own instead of inside every row workgroup
@pytest.mark.parametrize("B,S,V", [(2, 64, 50257), (1, 33, 151936), (2, 16, 262144), (3, 7, 97), (2, 2100, 600)])
def test_cross_entropy(B, S, V):
    print(f"ce B={B} S={S} V={V}", flush=True)
    logits = rn(B * S, V, std=2.0)
    labels = RNG.integers(0, V, (B, S)).astype(np.int32)
    labels[0, 3] = -100
    up = 0.5
    ls_ref, n_ref, dl_ref, nll_ref = O.ce_fwd_bwd(logits, labels, B, S, -100, up)
    t = g(logits)
    ls, n, dl, nll = ops.ce_fwd_bwd(t, g(labels), B, S, -100, up, in_place=True)
    assert int(h(n)[0]) == n_ref
    assert abs(float(h(ls)[0]) - ls_ref) < TOL * abs(ls_ref)
    assert rel_err(h(nll), nll_ref) < TOL
    assert rel_err(h(dl), dl_ref) < TOL


def test_cross_entropy_out_of_range_labels_count_as_ignored():
    """A label outside [0, V) other than ignore_index is excluded from both the
    loss and the normaliser (the count kernel and the row kernel apply the same
    test), exactly as the oracle does."""
    B, S, V = 2, 9, 3001
    logits = rn(B * S, V, std=2.0)
    labels = RNG.integers(0, V, (B, S)).astype(np.int32)
    labels[0, 2], labels[0, 5], labels[1, 4], labels[1, 7] = V, -5, V + 1000, -100
    ls_ref, n_ref, dl_ref, nll_ref = O.ce_fwd_bwd(logits, labels, B, S, -100, 1.0)
    assert n_ref == B * (S - 1) - 4
    ls, n, dl, nll = ops.ce_fwd_bwd(g(logits), g(labels), B, S, -100, 1.0)
    assert int(h(n)[0]) == n_ref
    assert abs(float(h(ls)[0]) - ls_ref) < TOL * abs(ls_ref)
    assert rel_err(h(dl), dl_ref) < TOL
    assert np.abs(h(dl).reshape(B, S, V)[0, 1]).max() == 0.0  # row predicting label V


def test_cross_entropy_all_ignored_row_zero_grad():
    B, S, V = 1, 5, 1000
    logits = rn(B * S, V)
    labels = np.full((B, S), -100, np.int32)
    ls, n, dl, _ = ops.ce_fwd_bwd(g(logits), g(labels), B, S)
    assert int(h(n)[0]) == 0 and float(h(ls)[0]) == 0.0
    assert np.abs(h(dl)).max() == 0.0


# ------------------------------------------------------------------ fp16
def test_dequant_f16_exhaustive_bit_exact():
    bits = np.arange(65536, dtype=np.uint16)
    out = h(ops.dequant_f16(g(bits.view(np.int16))))
    ref = O.f16_to_f32(bits)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_quant_f16_round_nearest_even_bit_exact():
    x = np.concatenate([rn(100000, std=0.02), rn(1000, std=1e-6), rn(100, std=3e4)])
    out = h(ops.quant_f16(g(x))).view(np.uint16)
    assert np.array_equal(out, O.f32_to_f16(x))


def test_dequant_large_and_unaligned():
    n = (1 << 22) + 3
    bits = RNG.integers(0, 0x7C00, n).astype(np.uint16)
    out = h(ops.dequant_f16(g(bits.view(np.int16))))
    assert np.array_equal(out, O.f16_to_f32(bits))
    out2 = h(ops.dequant_f16(g(bits.view(np.int16))[1:]))
    assert np.array_equal(out2, O.f16_to_f32(bits[1:]))


# ------------------------------------------------------------------ Adam / clip
def test_adam_sumsq_clip():
    n = 100003
    p, gr = rn(n), rn(n, std=0.1)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    tp, tg, tm, tv = g(p), g(gr), g(m), g(v)
    ss = ops.sumsq(tg)
    ss_ref = O.sumsq(gr)
    assert abs(float(h(ss)[0]) - ss_ref) < 1e-12 * ss_ref
    sc = ops.clip_scale(ss, 1.0)
    s_ref, n_ref = O.clip_scale(ss_ref, 1.0)
    assert abs(float(h(sc)[0]) - s_ref) < 1e-7 and abs(float(h(sc)[1]) - n_ref) < 1e-6
    gref = (gr * np.float32(s_ref)).astype(np.float32)
    for t in (1, 2, 3):
        ops.adam_step(tp, tg, tm, tv, 2e-4, 0.9, 0.999, 1e-8, 0.0, t, clip_scale=sc)
        O.adam_step(p, gref, m, v, 2e-4, 0.9, 0.999, 1e-8, 0.0, t)
    assert rel_err(h(tp), p) < 1e-6
    assert rel_err(h(tm), m) < 1e-6
    ops.adam_step(tp, tg, tm, tv, 2e-4, 0.9, 0.999, 1e-8, 0.0, 4, zero_grad=True)
    assert np.abs(h(tg)).max() == 0


def test_adam_weight_decay():
    n = 4099
    p, gr = rn(n), rn(n, std=0.1)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    tp, tg, tm, tv = g(p), g(gr), g(m), g(v)
    for t in (1, 2, 3):
        ops.adam_step(tp, tg, tm, tv, 1e-2, 0.9, 0.999, 1e-8, 0.05, t)
        O.adam_step(p, gr, m, v, 1e-2, 0.9, 0.999, 1e-8, 0.05, t)
    assert rel_err(h(tp), p) < 1e-6
    assert rel_err(h(tv), v) < 1e-6


# ------------------------------------------------------------------ support ops
@pytest.mark.parametrize("C", [1024, 3072])
def test_layernorm(C):
    x, gm, b, dy = rn(300, C, std=2), rn(C), rn(C), rn(300, C)
    y_ref, mu, rs = O.layernorm_fwd(x, gm, b, 1e-5)
    y, tmu, trs = ops.layernorm_fwd(g(x), g(gm), g(b), 1e-5)
    assert rel_err(h(y), y_ref) < TOL
    assert rel_err(h(ops.layernorm_bwd(g(dy), g(x), g(gm), tmu, trs)),
                   O.layernorm_bwd(dy, x, gm, mu, rs)) < TOL


# Row groups of 4 waves (896, 640, 4000: one to four chunks per thread), 2
# waves (384, with an odd row count so the last workgroup holds a row past
# the end) and 1 wave (256).
@pytest.mark.parametrize("C,unit", [(896, 0), (640, 1), (256, 1), (384, 0), (4000, 1)])
def test_rmsnorm(C, unit):
    x, w, dy = rn(501, C, std=2), rn(C, std=0.3), rn(501, C)
    y_ref, rs = O.rmsnorm_fwd(x, w, 1e-6, unit)
    y, trs = ops.rmsnorm_fwd(g(x), g(w), 1e-6, unit)
    assert rel_err(h(y), y_ref) < TOL
    assert rel_err(h(ops.rmsnorm_bwd(g(dy), g(x), g(w), trs, unit)),
                   O.rmsnorm_bwd(dy, x, w, rs, unit)) < TOL


@pytest.mark.parametrize("n", [300007, 300008])  # odd: the scalar kernels; a multiple of 4: the 128-bit ones
@pytest.mark.parametrize("act,gated", [(0, False), (0, True), (1, True)])
def test_glu(act, gated, n):
    gate, up, dout = rn(n, std=3), rn(n) if gated else None, rn(n)
    out = ops.glu_fwd(g(gate), g(up) if gated else None, act)
    assert rel_err(h(out), O.glu_fwd(gate, up, act)) < TOL
    dg, du = ops.glu_bwd(g(dout), g(gate), g(up) if gated else None, act)
    dg_ref, du_ref = O.glu_bwd(dout, gate, up, act)
    assert rel_err(h(dg), dg_ref) < TOL
    if gated:
        assert rel_err(h(du), du_ref) < TOL


@pytest.mark.parametrize("S,H,hd,theta", [(1024, 14, 64, 1e6), (256, 4, 256, 1e4)])
def test_rope(S, H, hd, theta):
    B = 2
    x = rn(B * S, H * hd)
    t = g(x)
    ops.rope_(t, B, S, H, hd, theta)
    assert rel_err(h(t), O.rope(x, B, S, H, hd, theta)) < TOL
    ops.rope_(t, B, S, H, hd, theta, inverse=True)
    assert rel_err(h(t), x) < TOL


def test_embed():
    V, C, S = 50257, 768, 128
    wte, wpe = rn(V, C, std=0.02), rn(1024, C, std=0.02)
    ids = RNG.integers(0, V, (4, S)).astype(np.int32)
    # NaN-filled output: a row the kernel never wrote stays NaN
    out = torch.full((4 * S, C), float("nan"), device=DEV)
    gi, gw, gp = g(ids), g(wte), g(wpe)
    ops.embed(gi, S, gw, gp, 1.0, out=out)
    got, ref = h(out), O.embed(ids, S, wte, wpe, 1.0)
    exact = np.all(got == ref, axis=1)
    assert exact.all(), (f"{exact.sum()}/{len(exact)} rows exact, "
                         f"{np.isnan(got).all(axis=1).sum()} rows unwritten")
    w16 = wte.astype(np.float16)
    out16 = ops.embed(g(ids), S, g(w16), None, math.sqrt(640))
    ref16 = O.embed(ids, S, None, None, math.sqrt(640), wte_f16=w16.view(np.uint16))
    assert np.array_equal(h(out16), ref16)


def test_embed_out_of_range_ids_give_zero_rows_and_flag():
    """Ids outside [0, vocab) read nothing: their rows are zeros and the
    device flag is set; the other rows are exact."""
    V, C, S = 1000, 64, 8
    wte = rn(V, C)
    ids = RNG.integers(0, V, (2, S)).astype(np.int32)
    bad_rows = [(0, 1), (0, 6), (1, 3)]
    ids[0, 1], ids[0, 6], ids[1, 3] = -100, V, V + 12345
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = h(ops.embed(g(ids), S, g(wte), None, 1.0, bad=bad)).reshape(2, S, C)
    assert int(h(bad)[0]) == 1
    for b in range(2):
        for s in range(S):
            if (b, s) in bad_rows:
                assert np.all(out[b, s] == 0.0)
            else:
                assert np.array_equal(out[b, s], wte[ids[b, s]])
    ok = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.embed(g(np.clip(ids, 0, V - 1)), S, g(wte), None, 1.0, bad=ok)
    assert int(h(ok)[0]) == 0


def test_outputs_float32_whatever_the_default_dtype():
    """Wrapper-allocated outputs are float32 even when torch's default dtype is
    not (the kernels write fp32 through raw pointers)."""
    ids = RNG.integers(0, 300, (2, 16)).astype(np.int32)
    wte, x = rn(300, 64), rn(32, 64)
    gm, b = rn(64), rn(64)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        out = ops.embed(g(ids), 16, g(wte), None, 1.0)
        y, mean, rstd = ops.layernorm_fwd(g(x), g(gm), g(b), 1e-5)
        ry, rr = ops.rmsnorm_fwd(g(x), g(gm), 1e-6, 0)
    finally:
        torch.set_default_dtype(old)
    assert all(t.dtype == torch.float32 for t in (out, y, mean, rstd, ry, rr))
    assert np.array_equal(h(out), O.embed(ids, 16, wte, None, 1.0))
    assert rel_err(h(y), O.layernorm_fwd(x, gm, b, 1e-5)[0]) < TOL
    with pytest.raises(TypeError):
        ops.embed(g(ids.astype(np.int64)), 16, g(wte), None, 1.0)


def test_split_k_gemm_repeatable():
    """Split-K partials are summed in split order: repeated calls give
    bit-identical results, equal to the oracle."""
    M, K, N = 256, 4096, 512          # 32 tiles of 64×64 → split 8
    x, W = rn(M, K), rn(K, N, std=0.02)
    y_ref, _ = O.lora_linear_fwd(x, W, None, None, None, 1.0)
    outs = [h(ops.lora_linear_fwd(g(x), g(W), None, None, None, 1.0)[0]) for _ in range(3)]
    assert rel_err(outs[0], y_ref) < TOL
    assert all(np.array_equal(o, outs[0]) for o in outs[1:])
