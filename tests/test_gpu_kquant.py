"""GPU parity of the ggml Q6_K / Q8_0 path through the C-ABI against the oracle.

Decoded weights bit-exact; GEMV within 1e-3 relative L2 of the oracle's
f64 matvec (held to 1e-5 here, the f32 accumulation's actual error)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIGHT = 1e-5


def rel_l2(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / max(np.linalg.norm(want), 1e-300))


def _blocks(sm, kind, seed, rows, cols):
    return sm.synth_q6k(seed, rows, cols) if kind == "q6_k" else sm.synth_q8_0(seed, rows, cols)


def _dequant_ref(ref, kind, blocks, rows, cols):
    return ref.q6k_dequant(blocks, rows, cols) if kind == "q6_k" else ref.q8_0_dequant(blocks, rows, cols)


# q6_k also at the Q6_K trunk's launch shapes: q + k + v + head gate stacked by
# rows (6160 x 2560), gate + up stacked (20480 x 2560) and o (2560 x 4096)
SHAPES = {"q6_k": [(2560, 10240), (13, 512), (4, 256), (64, 2560), (6160, 2560), (20480, 2560), (2560, 4096)],
          "q8_0": [(1024, 2560), (3, 32), (5, 96), (64, 2560), (7, 4096), (5, 512), (40, 1536)]}


@pytest.mark.parametrize("kind,shape", [(k, s) for k in SHAPES for s in SHAPES[k]])
@pytest.mark.parametrize("offset", [0, 2], ids=["aligned", "offset2"])
def test_kquant_gemv_and_dequant(sm, ref, dev, kind, shape, offset):
    """offset 2 places the blocks 2 bytes past a 4-byte boundary, which flips
    every block's alignment and makes the buffer's final block end flush."""
    import torch
    rows, cols = shape
    blocks = _blocks(sm, kind, rows * 3 + cols, rows, cols)
    W = _dequant_ref(ref, kind, blocks, rows, cols)
    dbuf = torch.zeros(blocks.nbytes + offset, dtype=torch.uint8, device=dev)
    dbuf[offset:] = torch.from_numpy(blocks).to(dev)
    db = dbuf[offset:]
    out = torch.full((rows, cols), float("nan"), device=dev)
    sm.kquant_dequant(kind, db, rows, cols, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), W.view(np.uint32))
    for ncol in (1, 4):
        xb = sm.synth_bf16(ncol + cols, ncol * cols).reshape(ncol, cols)
        xf = sm.bf16_to_f32(xb).reshape(ncol, cols)
        xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
        y = torch.full((ncol, rows), float("nan"), device=dev)
        sm.kquant_gemv(kind, db, rows, cols, xt, y, ncols=ncol)
        torch.cuda.synchronize()
        want = xf.astype(np.float64) @ W.astype(np.float64).T
        err = rel_l2(y.cpu().numpy(), want)
        print(f"{kind} {rows}x{cols} ncol {ncol} offset {offset}: relL2 {err:.2e}")
        assert err <= TIGHT
    # f32 activations, accumulating into y
    xf = np.random.default_rng(4).standard_normal(cols).astype(np.float32)
    y0 = np.random.default_rng(5).standard_normal(rows).astype(np.float32)
    y = torch.from_numpy(y0.copy()).to(dev)
    sm.kquant_gemv(kind, db, rows, cols, torch.from_numpy(xf).to(dev), y, accumulate=True)
    torch.cuda.synchronize()
    want = y0.astype(np.float64) + W.astype(np.float64) @ xf.astype(np.float64)
    assert rel_l2(y.cpu().numpy(), want) <= TIGHT


def test_kquant_matches_runtime_dot(sm, ref, dev):
    """Against the runtime's own decode-then-dot path (model.rs:209-234)."""
    import torch
    rows, cols = 256, 2560
    blocks = sm.synth_q8_0(9, rows, cols)
    x = sm.bf16_to_f32(sm.synth_bf16(10, cols))
    yr = ref.q8_0_matvec(blocks, rows, cols, x)
    y = torch.zeros(rows, device=dev)
    sm.kquant_gemv("q8_0", torch.from_numpy(blocks).to(dev), rows, cols, torch.from_numpy(x).to(dev), y)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), yr) <= TIGHT


@pytest.mark.parametrize("kind", ["q8_0", "q6_k"])
def test_kquant_columns_equal_single_launches(sm, dev, kind):
    """A speculative verify's head columns must be exactly the logits a
    one-column launch gives: the reference found that any other arithmetic
    for the 8-row verify head changes accepted tokens
    (Spark-X2.6-4B-Base-handoff.md:299-302). Bit-exact, per column."""
    import torch
    rows, cols, ncol = 1000, 2560, 8
    blocks = torch.from_numpy(_blocks(sm, kind, 31, rows, cols)).to(dev)
    xb = sm.synth_bf16(32, ncol * cols).reshape(ncol, cols)
    xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    y8 = torch.full((ncol, rows), float("nan"), device=dev)
    sm.kquant_gemv(kind, blocks, rows, cols, xt, y8, ncols=ncol)
    for n in range(ncol):
        y1 = torch.full((1, rows), float("nan"), device=dev)
        sm.kquant_gemv(kind, blocks, rows, cols, xt[n:n + 1].contiguous(), y1)
        torch.cuda.synchronize()
        assert np.array_equal(y8[n].cpu().numpy().view(np.uint32), y1[0].cpu().numpy().view(np.uint32)), n


def test_q8_0_sixteen_columns(sm, ref, dev):
    """16 columns of 4096 (147 KB of x in LDS), against the oracle and
    bit-equal to a one-column launch."""
    import torch
    rows, cols, ncol = 64, 4096, 16
    blocks = sm.synth_q8_0(41, rows, cols)
    W = ref.q8_0_dequant(blocks, rows, cols).astype(np.float64)
    db = torch.from_numpy(blocks).to(dev)
    xb = sm.synth_bf16(42, ncol * cols).reshape(ncol, cols)
    xf = sm.bf16_to_f32(xb).reshape(ncol, cols)
    xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    y = torch.full((ncol, rows), float("nan"), device=dev)
    sm.kquant_gemv("q8_0", db, rows, cols, xt, y, ncols=ncol)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), xf.astype(np.float64) @ W.T) <= TIGHT
    # x of 16 columns does not fit beside the row slots: the launch goes in
    # column groups, and every column still equals a one-column launch
    for n in range(ncol):
        y1 = torch.full((1, rows), float("nan"), device=dev)
        sm.kquant_gemv("q8_0", db, rows, cols, xt[n:n + 1].contiguous(), y1)
        torch.cuda.synchronize()
        assert np.array_equal(y[n].cpu().numpy().view(np.uint32), y1[0].cpu().numpy().view(np.uint32)), n


@pytest.mark.parametrize("ncol,xdt", [(3, "bf16"), (5, "f32")])
def test_q8_0_columns_equal_single_launches(sm, ref, dev, ncol, xdt):
    """Fewer columns than the kernel's width (3 of 16 B-operand rows), and f32
    x (its hi and lo halves, two matrix-core products per block): every
    column bit-equal to a one-column launch and within 1e-5 of the oracle.
    Rows not a multiple of 16 leave the last tile partial."""
    import torch
    rows, cols = 300, 2560
    blocks = sm.synth_q8_0(51, rows, cols)
    W = ref.q8_0_dequant(blocks, rows, cols).astype(np.float64)
    db = torch.from_numpy(blocks).to(dev)
    if xdt == "bf16":
        xb = sm.synth_bf16(52, ncol * cols).reshape(ncol, cols)
        xf = sm.bf16_to_f32(xb).reshape(ncol, cols)
        xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    else:
        xf = np.random.default_rng(53).standard_normal((ncol, cols)).astype(np.float32)
        xt = torch.from_numpy(xf).to(dev)
    y = torch.full((ncol, rows), float("nan"), device=dev)
    sm.kquant_gemv("q8_0", db, rows, cols, xt, y, ncols=ncol)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), xf.astype(np.float64) @ W.T) <= TIGHT
    for n in range(ncol):
        y1 = torch.full((1, rows), float("nan"), device=dev)
        sm.kquant_gemv("q8_0", db, rows, cols, xt[n:n + 1].contiguous(), y1)
        torch.cuda.synchronize()
        assert np.array_equal(y[n].cpu().numpy().view(np.uint32), y1[0].cpu().numpy().view(np.uint32)), n


def test_kquant_errors(sm, dev):
    import torch
    L = sm.lib()
    b = torch.zeros(210, dtype=torch.uint8, device=dev)
    x = torch.zeros(256, device=dev)
    y = torch.zeros(1, device=dev)
    assert L.sparkmv_q6k_gemv(b.data_ptr(), 1, 200, x.data_ptr(), 1, 256, 1, y.data_ptr(), 1, 0, None) == -1
    assert "multiple of 256" in sm.last_error()
    assert L.sparkmv_q8_0_gemv(b.data_ptr() + 1, 1, 32, x.data_ptr(), 1, 32, 1, y.data_ptr(), 1, 0, None) == -1
    assert "aligned" in sm.last_error()
    assert L.sparkmv_q8_0_gemv(b.data_ptr(), 1, 32, x.data_ptr(), 7, 32, 1, y.data_ptr(), 1, 0, None) == -1
