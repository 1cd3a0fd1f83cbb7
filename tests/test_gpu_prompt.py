"""Long contexts and the prompt path of the GPU forward, against the oracle's
restatement of tools/vq-runtime/src/model.rs:441-591 (oracle/forward.py).

The small model of test_gpu_forward.py with a 256-position cache and a
40-position sliding window, run over 210 tokens:

  - the decode step (sparkmv_model_forward) at every position, checked at
    positions on both sides of 16 (the attention chunk), of 40 (the window
    edge, after which a sliding layer's chunks start mid-window) and of 192
    (twelve chunks: past it the full layer's combine runs its four-chunk
    loop), with every KV row; then one verify block of 8 at position 210;
  - the prompt path (sparkmv_model_forward_batch, vq-model-gpu.cu:858-953):
    chunks of 100 (the prefill GEMM), 10 (the batched GEMV) and 100 tokens
    without logits, then decode steps on the cache the chunks wrote.

Bars: decode steps and chunks of at most 16 tokens keep the decode
arithmetic, 1e-5 with f32 activations. Longer chunks run the prefill GEMM,
where x enters the matrix cores as f16, as in the reference's own prompt
path: f32 activations then meet 5e-3 (each matvec input rounded to f16's
11 bits), bf16 activations the decode tests' 2e-2.
"""
import numpy as np
import pytest

import forward as fw
from test_gpu_forward import CFG, build, rel_l2

pytestmark = pytest.mark.gpu

LONG = dict(CFG, max_ctx=256, sliding_window=40)
NTOK = 210
CHECK_POS = [0, 1, 15, 16, 17, 39, 40, 41, 56, 57, 191, 192, 193, 208, 209]


def tokens(n, seed=5):
    return [int(t) for t in np.random.default_rng(seed).integers(0, LONG["vocab"], n)]


def kv_rows(model, dev, li, n, kvd):
    """The first n rows of layer li's K and V cache, copied device to device."""
    import ctypes
    import torch
    hip = ctypes.CDLL("libamdhip64.so")
    out = []
    for ptr in model.kv(li):
        buf = torch.empty((n, kvd), dtype=torch.float32, device=dev)
        assert hip.hipMemcpy(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(ptr), ctypes.c_size_t(n * kvd * 4),
                             ctypes.c_int(3)) == 0
        out.append(buf.cpu().numpy())
    return out


def check_kv(model, oracle, dev, n, bar, label, cfg=None):
    cfg = cfg or LONG
    kvd = cfg["kv_heads"] * cfg["head_dim"]
    worst = 0.0
    for li in range(cfg["layers"]):
        for got, want in zip(kv_rows(model, dev, li, n, kvd), (oracle.kv_k[li], oracle.kv_v[li])):
            worst = max(worst, rel_l2(got, want[:n]))
    print(f"{label}: KV rows 0..{n - 1} worst relL2 {worst:.2e}")
    assert worst <= bar


@pytest.mark.parametrize("head_kind", ["q8_0", "vq"])
def test_long_context_decode_and_verify(sm, ref, dev, head_kind):
    import torch
    model, oracle = build(sm, ref, dev, head_kind, sm.X_F32, LONG)
    toks = tokens(NTOK + 8)
    logits = torch.full((LONG["vocab"],), float("nan"), device=dev)
    worst = 0.0
    for pos in range(NTOK):
        model.forward(toks[pos], pos, logits)
        want = oracle.forward(toks[pos], pos)
        if pos in CHECK_POS:
            torch.cuda.synchronize()
            err = rel_l2(logits.cpu().numpy(), want)
            worst = max(worst, err)
            print(f"head {head_kind} pos {pos}: logits relL2 {err:.2e}")
            assert err <= 1e-5, pos
    torch.cuda.synchronize()
    check_kv(model, oracle, dev, NTOK, 1e-5, f"head {head_kind} decode")
    block = toks[NTOK:NTOK + 8]
    out = torch.full((8, LONG["vocab"]), float("nan"), device=dev)
    model.verify(block, NTOK, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, t in enumerate(block):
        err = rel_l2(got[i], oracle.forward(t, NTOK + i))
        print(f"head {head_kind} verify row {i} (pos {NTOK + i}): relL2 {err:.2e}")
        assert err <= 1e-5
    print(f"head {head_kind}: worst decode relL2 {worst:.2e}")


@pytest.mark.parametrize("head_kind,xd", [("q8_0", "f32"), ("vq", "f32"), ("q8_0", "bf16")])
def test_forward_batch_against_oracle(sm, ref, dev, head_kind, xd):
    import torch
    x_dtype = sm.X_F32 if xd == "f32" else sm.X_BF16
    bar = 5e-3 if xd == "f32" else 2e-2
    model, oracle = build(sm, ref, dev, head_kind, x_dtype, LONG)
    model.reserve(128)
    toks = tokens(NTOK + 2, seed=9)
    logits = torch.full((LONG["vocab"],), float("nan"), device=dev)
    want = None
    for p in range(100):
        want = oracle.forward(toks[p], p)
    model.forward_batch(toks[:100], 0, logits)
    torch.cuda.synchronize()
    err = rel_l2(logits.cpu().numpy(), want)
    print(f"head {head_kind} x {xd}: chunk 0..99 (prefill GEMM), last logits relL2 {err:.2e}")
    assert err <= bar
    for p in range(100, 110):
        want = oracle.forward(toks[p], p)
    model.forward_batch(toks[100:110], 100, logits)
    torch.cuda.synchronize()
    err = rel_l2(logits.cpu().numpy(), want)
    print(f"head {head_kind} x {xd}: chunk 100..109 (batched GEMV), last logits relL2 {err:.2e}")
    assert err <= bar
    for p in range(110, NTOK):
        oracle.forward(toks[p], p)
    model.forward_batch(toks[110:NTOK], 110)      # no logits, as between prompt chunks
    assert len(model) == NTOK
    for p in (NTOK, NTOK + 1):
        model.forward(toks[p], p, logits)
        torch.cuda.synchronize()
        err = rel_l2(logits.cpu().numpy(), oracle.forward(toks[p], p))
        print(f"head {head_kind} x {xd}: decode at {p} after the chunks, relL2 {err:.2e}")
        assert err <= bar
    if xd == "f32":
        check_kv(model, oracle, dev, NTOK + 2, bar, f"head {head_kind} prompt")


@pytest.mark.parametrize("xd", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kvh", [(4, 1), (8, 2)], ids=["kv1", "kv2"])
def test_forward_batch_mfma_attention(sm, ref, dev, heads, kvh, xd):
    """Heads of 256 with 4 query heads per kv head (the reference model's
    shape) take the matrix-core prompt attention (16 tokens per workgroup,
    K and V through LDS 16 positions at a time). Chunks of 100 and 37
    tokens cross the 40-position window and tile boundaries mid-block; the
    last logits, the decode steps after and every KV row (each layer's rows
    depend on every token's attention output in the layers below) meet the
    prompt bar against the oracle: 5e-3 with f32 activations, 2e-2 with
    bf16 ones (the attention then writes only its bf16 output, the path the
    real model and the 512-token bench take)."""
    import torch
    cfg = dict(LONG, head_dim=256, heads=heads, kv_heads=kvh)
    model, oracle = build(sm, ref, dev, "q8_0", sm.X_F32 if xd == "f32" else sm.X_BF16, cfg)
    model.reserve(128)
    toks = tokens(139, seed=17)
    logits = torch.full((cfg["vocab"],), float("nan"), device=dev)
    bar = 5e-3 if xd == "f32" else 2e-2
    for lo, hi in ((0, 100), (100, 137)):
        want = None
        for p in range(lo, hi):
            want = oracle.forward(toks[p], p)
        model.forward_batch(toks[lo:hi], lo, logits)
        torch.cuda.synchronize()
        err = rel_l2(logits.cpu().numpy(), want)
        print(f"heads {heads}/{kvh}: chunk {lo}..{hi - 1}, last logits relL2 {err:.2e}")
        assert err <= bar
    for p in (137, 138):
        model.forward(toks[p], p, logits)
        torch.cuda.synchronize()
        err = rel_l2(logits.cpu().numpy(), oracle.forward(toks[p], p))
        print(f"heads {heads}/{kvh} x {xd}: decode at {p}, relL2 {err:.2e}")
        assert err <= bar
    check_kv(model, oracle, dev, 139, bar, f"heads {heads}/{kvh} x {xd} prompt", cfg)


def test_forward_batch_short_chunk_is_exact(sm, ref, dev):
    """A chunk of 12 tokens (at most 16: every matvec on the batched GEMV)
    keeps the decode arithmetic: 1e-5 with f32 activations for the last
    logits and every KV row, the attention of each token over the chunk's
    own earlier positions included."""
    import torch
    model, oracle = build(sm, ref, dev, "q8_0", sm.X_F32, LONG)
    toks = tokens(12, seed=13)
    want = None
    for p, t in enumerate(toks):
        want = oracle.forward(t, p)
    logits = torch.full((LONG["vocab"],), float("nan"), device=dev)
    model.forward_batch(toks, 0, logits)
    torch.cuda.synchronize()
    err = rel_l2(logits.cpu().numpy(), want)
    print(f"12-token chunk: last logits relL2 {err:.2e}")
    assert err <= 1e-5
    check_kv(model, oracle, dev, 12, 1e-5, "12-token chunk")


@pytest.mark.parametrize("heads,kvh", [(4, 1), (8, 2)], ids=["kv1", "kv2"])
def test_forward_batch_mfma_attention_is_exact(sm, ref, dev, heads, kvh):
    """The matrix-core prompt attention alone, held to the decode bar: 30
    decode steps, then a chunk of 12 tokens at position 30 (the batched GEMV
    keeps every matvec exact in f32), whose last two tokens' 40-position
    windows start past 0, then two decode steps. Its products and sums are
    f32 like the decode attention's, only summed in another order, so the
    last logits and every KV row meet 1e-5."""
    import torch
    cfg = dict(LONG, head_dim=256, heads=heads, kv_heads=kvh)
    model, oracle = build(sm, ref, dev, "q8_0", sm.X_F32, cfg)
    toks = tokens(44, seed=19)
    logits = torch.full((cfg["vocab"],), float("nan"), device=dev)
    for p in range(30):
        model.forward(toks[p], p, logits)
        oracle.forward(toks[p], p)
    want = None
    for p in range(30, 42):
        want = oracle.forward(toks[p], p)
    model.forward_batch(toks[30:42], 30, logits)
    torch.cuda.synchronize()
    err = rel_l2(logits.cpu().numpy(), want)
    print(f"heads {heads}/{kvh}: 12-token chunk at 30, last logits relL2 {err:.2e}")
    assert err <= 1e-5
    for p in (42, 43):
        model.forward(toks[p], p, logits)
        torch.cuda.synchronize()
        err = rel_l2(logits.cpu().numpy(), oracle.forward(toks[p], p))
        print(f"heads {heads}/{kvh}: decode at {p}, relL2 {err:.2e}")
        assert err <= 1e-5
    check_kv(model, oracle, dev, 44, 1e-5, f"heads {heads}/{kvh} chunk at 30", cfg)


def test_forward_batch_refusals(sm, ref, dev):
    import torch
    model, _ = build(sm, ref, dev, "q8_0", sm.X_F32, LONG)
    logits = torch.zeros(LONG["vocab"], device=dev)
    with pytest.raises(sm.SparkmvError):
        model.forward_batch([1] * 513, 0, logits)
    assert "1..512 tokens" in sm.last_error()
    with pytest.raises(sm.SparkmvError):
        model.forward_batch([1] * 20, LONG["max_ctx"] - 10, logits)
    assert "exceed" in sm.last_error()
    with pytest.raises(sm.SparkmvError):
        model.forward_batch([1, LONG["vocab"]], 0, logits)
    assert "outside the vocabulary" in sm.last_error()
    for bad in (0, 513):
        with pytest.raises(sm.SparkmvError):
            model.reserve(bad)
    assert len(model) == 0


def poison_kv(model, dev):
    """Every K and V byte 0xFF (a NaN in f32): what a cache that reuses freed
    memory may hold before its rows are written."""
    import ctypes
    import torch
    hip = ctypes.CDLL("libamdhip64.so")
    n = LONG["max_ctx"] * LONG["kv_heads"] * LONG["head_dim"] * 4
    for li in range(LONG["layers"]):
        for ptr in model.kv(li):
            assert hip.hipMemset(ctypes.c_void_p(ptr), ctypes.c_int(0xFF), ctypes.c_size_t(n)) == 0
    assert hip.hipDeviceSynchronize() == 0
    torch.cuda.synchronize(dev)


@pytest.mark.parametrize("path", ["decode", "verify", "chunks"])
def test_unwritten_cache_rows_are_not_read(sm, ref, dev, path):
    """The attention reads whole 16-row chunks of the cache and skips the
    rows past the position: with NaN in every row not yet written, each
    path still meets its bar (decode and verify 1e-5, a 12-token chunk
    1e-5, a 100-token chunk 5e-3)."""
    import torch
    model, oracle = build(sm, ref, dev, "q8_0", sm.X_F32, LONG)
    poison_kv(model, dev)
    toks = tokens(120, seed=17)
    V = LONG["vocab"]
    if path == "decode":
        logits = torch.full((V,), float("nan"), device=dev)
        for pos in range(18):
            model.forward(toks[pos], pos, logits)
            torch.cuda.synchronize()
            err = rel_l2(logits.cpu().numpy(), oracle.forward(toks[pos], pos))
            assert err <= 1e-5, pos
    elif path == "verify":
        out = torch.full((8, V), float("nan"), device=dev)
        model.verify(toks[:8], 0, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for i in range(8):
            assert rel_l2(got[i], oracle.forward(toks[i], i)) <= 1e-5, i
    else:
        logits = torch.full((V,), float("nan"), device=dev)
        for n0, n1, bar in ((0, 12, 1e-5), (12, 112, 5e-3)):
            want = None
            for p in range(n0, n1):
                want = oracle.forward(toks[p], p)
            model.forward_batch(toks[n0:n1], n0, logits)
            torch.cuda.synchronize()
            err = rel_l2(logits.cpu().numpy(), want)
            print(f"chunk {n0}..{n1 - 1} over a NaN cache: relL2 {err:.2e}")
            assert err <= bar
