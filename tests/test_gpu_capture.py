"""Layer-input capture, the embedding row and argmax on the GPU model
(sparkmv_model_enable_capture / _captured / _embed_row, sparkmv_argmax),
against the oracle's restatement of tools/vq-runtime/src/model.rs:322-354,
:466-471 and :594-605.

The small model of test_gpu_prompt.py (256-position cache, 40-position
window) captures two layers, listed out of order. Rows come from every path:
eager decode steps, replays of the captured decode graph, a verify block of
8 and a prompt chunk of 30 tokens (the prefill GEMM). Then a rollback, and
decode steps that overwrite the dropped rows.

Bars: rows from the decode arithmetic (decode, replay, verify) meet 1e-5
with f32 activations. The prompt chunk's matvecs take x as f16, so its rows
meet 5e-3 (the prompt tests' bar). The refusals carry the GPU runtime's
messages (vq-model-gpu.cu:707-736).
"""
import numpy as np
import pytest

from test_gpu_forward import build, rel_l2
from test_gpu_prompt import LONG, tokens

pytestmark = pytest.mark.gpu


def test_capture_refusals(sm, ref, dev):
    model, _ = build(sm, ref, dev, "q8_0", sm.X_F32, LONG)
    for layers, msg in (([], "0 layers requested, the limit is 8"), (list(range(9)), "9 layers requested"),
                        ([3], "capture: layer 3 is outside 0..3"), ([1, -1], "layer -1 is outside"),
                        ([0, 2, 0], "capture: layer 0 is listed twice")):
        with pytest.raises(sm.SparkmvError):
            model.enable_capture(layers)
        assert msg in sm.last_error(), (layers, sm.last_error())
    model.enable_capture([1])
    with pytest.raises(sm.SparkmvError):
        model.enable_capture([0])
    assert "capture: already enabled" in sm.last_error()
    with pytest.raises(sm.SparkmvError):
        model.captured(1)
    assert "capture slot 1 is outside 0..0" in sm.last_error()


@pytest.mark.parametrize("head_kind", ["q8_0", "vq"])
def test_capture_every_path_and_rollback(sm, ref, dev, head_kind):
    import torch
    model, oracle = build(sm, ref, dev, head_kind, sm.X_F32, LONG)
    layers = [2, 0]                       # slot 0 = layer 2, slot 1 = layer 0
    model.enable_capture(layers)
    oracle.enable_capture(layers)
    toks = tokens(80, seed=23)
    V = LONG["vocab"]
    logits = torch.zeros(V, device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for p in range(20):                # eager decode steps
            model.forward(toks[p], p, logits, stream)
        model.capture(logits, stream)      # the graph records the copies
        for p in range(20, 25):
            model.replay(toks[p], p, stream)
    torch.cuda.synchronize()
    out = torch.zeros((8, V), device=dev)
    model.verify(toks[25:33], 25, out)     # a verify block
    model.reserve(64)
    model.forward_batch(toks[33:63], 33)   # a prompt chunk on the prefill GEMM
    torch.cuda.synchronize()
    for p in range(63):
        oracle.forward(toks[p], p)
    assert len(model) == 63
    for k, li in enumerate(layers):
        got = model.captured(k).cpu().numpy()
        assert got.shape == (63, LONG["hidden"])
        want = oracle.capture[li][:63]
        e_exact, e_prompt = rel_l2(got[:33], want[:33]), rel_l2(got[33:], want[33:])
        print(f"head {head_kind} layer {li}: rows 0..32 relL2 {e_exact:.2e}, rows 33..62 {e_prompt:.2e}")
        assert e_exact <= 1e-5 and e_prompt <= 5e-3
    # a rollback drops rows with the KV rows; later steps write them again
    model.rollback(10)
    assert model.captured(0).shape[0] == 10
    alt = tokens(3, seed=29)
    for i, t in enumerate(alt):
        model.forward(t, 10 + i, logits)
        oracle.forward(t, 10 + i)
    torch.cuda.synchronize()
    for k, li in enumerate(layers):
        got = model.captured(k).cpu().numpy()
        assert got.shape[0] == 13
        assert rel_l2(got, oracle.capture[li][:13]) <= 1e-5
    model.reset()
    assert len(model) == 0 and model.captured(1).shape[0] == 0


@pytest.mark.parametrize("head_kind", ["q8_0", "vq"])
def test_embed_row_is_the_decoded_row(sm, ref, dev, head_kind):
    """embed_row (model.rs:352-354) equals the oracle's decoded row bit for
    bit: each Q8_0 weight is d * q exactly, each VQ weight the reference
    decode's one rounding."""
    model, oracle = build(sm, ref, dev, head_kind, sm.X_F32, LONG)
    for t in (0, 7, LONG["vocab"] - 1):
        got = model.embed_row(t).cpu().numpy()
        want = oracle.embed[t].astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), t
    with pytest.raises(sm.SparkmvError):
        model.embed_row(LONG["vocab"])
    assert "outside the vocabulary" in sm.last_error()


def test_argmax_matches_model_argmax(sm, dev):
    """Model::argmax (model.rs:594-605): the first of equal maxima, NaN never
    chosen, 0 when nothing exceeds -inf; checked against the same scan in
    numpy at the head's width and at widths that are not multiples of 1024."""
    import torch

    def scan(v):
        best, bi = -np.inf, 0
        for i, x in enumerate(v):
            if x > best:
                best, bi = x, i
        return bi

    rng = np.random.default_rng(31)
    cases = []
    v = rng.standard_normal(151936).astype(np.float32)
    v[[5000, 70000, 150000]] = 9.0          # three equal maxima: the first wins
    v[rng.integers(0, v.size, 50)] = np.nan
    cases.append(v)
    w = rng.standard_normal(1337).astype(np.float32)
    w[1336] = 50.0                           # the maximum in the last partial stride
    cases.append(w)
    cases.append(np.full(77, -np.inf, np.float32))
    cases.append(np.full(5, np.nan, np.float32))
    cases.append(np.array([-3.0], np.float32))
    u = np.zeros(4096, np.float32)
    u[[1025, 3]] = 1.0                       # a tie across threads: index 3, not 1025
    cases.append(u)
    for c in cases:
        got = int(sm.argmax(torch.from_numpy(c).to(dev)).item())
        assert got == scan(c), (c.size, got, scan(c))
    with pytest.raises(sm.SparkmvError):
        sm.argmax(torch.zeros(0, device=dev))
