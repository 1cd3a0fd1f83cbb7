"""GPU tests of the per-token plan (sparkmv_plan_*): a recorded chain of VQ
and k-quant launches, run eagerly and replayed as one HIP graph.

The eager run must match the oracle. Every graph replay must equal the eager
run bit for bit (the same kernels on the same inputs). Between replays the
outputs are cleared by other device work and the host synchronizes, so a
replay that skipped or reordered a node would show."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIGHT = 1e-5
HIDDEN, FFN = 512, 1024


def rel_l2(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / max(np.linalg.norm(want), 1e-300))


def _chain(sm, ref, dev, ncol):
    """A scaled-down layer and head: q+k+v sharing x, o, gate+up sharing x,
    down, then a Q8_0 and a Q6_K matrix. Returns the plan, the outputs (with
    their row counts) and what the oracle says they hold."""
    import torch
    xs = {}
    for c in (HIDDEN, FFN):
        xb = sm.synth_bf16(c + ncol, ncol * c).reshape(ncol, c)
        xs[c] = (torch.from_numpy(xb.view(np.int16).copy()).to(dev), sm.bf16_to_f32(xb).reshape(ncol, c))
    plan = sm.Plan()
    outs = []
    groups = [[(256, HIDDEN), (64, HIDDEN), (64, HIDDEN)], [(HIDDEN, FFN)], [(FFN, HIDDEN), (FFN, HIDDEN)],
              [(HIDDEN, FFN)]]
    seed = 40
    for grp in groups:
        cols = grp[0][1]
        width = max(r for r, _ in grp)
        mats, ys, Ws = [], [], []
        for rows, _ in grp:
            data = sm.synth_container(seed, rows, cols)
            seed += 1
            mats.append(sm.DeviceContainer(data, dev))
            Ws.append(ref.decode(data).astype(np.float64))
            ys.append(torch.full((ncol, width), float("nan"), device=dev))
        plan.add_vq(mats, xs[cols][0], ys, ncols=ncol)
        for y, W, (rows, _) in zip(ys, Ws, grp):
            outs.append((y, rows, xs[cols][1].astype(np.float64) @ W.T))
    for kind, rows, cols in (("q8_0", 1000, HIDDEN), ("q6_k", HIDDEN, FFN)):
        host = sm.synth_q8_0(seed, rows, cols) if kind == "q8_0" else sm.synth_q6k(seed, rows, cols)
        seed += 1
        W = (ref.q8_0_dequant if kind == "q8_0" else ref.q6k_dequant)(host, rows, cols).astype(np.float64)
        blocks = torch.from_numpy(host).to(dev)
        y = torch.full((ncol, rows), float("nan"), device=dev)
        plan.add_kquant(kind, blocks, rows, cols, xs[cols][0], y, ncols=ncol)
        plan.keep.append(blocks)
        outs.append((y, rows, xs[cols][1].astype(np.float64) @ W.T))
    plan.keep.append(xs)
    return plan, outs


@pytest.mark.parametrize("ncol", [1, 8])
def test_plan_eager_then_graph_replays(sm, ref, dev, ncol):
    import torch
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        plan, outs = _chain(sm, ref, dev, ncol)
        assert len(plan) == 6
        plan.run(stream)
        torch.cuda.synchronize()
        eager = []
        for y, rows, want in outs:
            got = y[:, :rows].cpu().numpy().copy()
            assert rel_l2(got, want) <= TIGHT
            eager.append(got)
        plan.capture(stream)
        for rep in range(3):
            for y, _, _ in outs:
                y.zero_()
            torch.cuda.synchronize()
            plan.launch(stream)
            torch.cuda.synchronize()
            for (y, rows, _), e in zip(outs, eager):
                got = y[:, :rows].cpu().numpy()
                assert np.array_equal(got.view(np.uint32), e.view(np.uint32)), rep


def test_plan_times_every_op(sm, ref, dev):
    import torch
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        plan, outs = _chain(sm, ref, dev, 1)
        plan.run(stream)
        t = plan.time_ops(stream, iters=3)
        torch.cuda.synchronize()
    assert t.shape == (len(plan),) and np.all(t > 0) and np.all(t < 10.0)
    # the timing pass runs the same kernels: outputs still hold the chain's result
    for y, rows, want in outs:
        assert rel_l2(y[:, :rows].cpu().numpy(), want) <= TIGHT


def test_plan_errors_and_empty_plan(sm, dev):
    import torch
    plan = sm.Plan()
    assert len(plan) == 0
    stream = torch.cuda.Stream(device=dev)
    plan.run(stream)
    L = sm.lib()
    x = torch.zeros(8, dtype=torch.int16, device=dev)
    y = torch.zeros(4, device=dev)
    assert L.sparkmv_plan_add_kquant(plan.h, 5, x.data_ptr(), 4, 32, x.data_ptr(), 0, 32, 1, y.data_ptr(), 4, 0) == -1
    assert "kind" in sm.last_error()
    assert L.sparkmv_plan_capture(plan.h, None) == -1
    assert "null stream" in sm.last_error()


@pytest.mark.parametrize("rows", [2560, 2200, 2222])
@pytest.mark.parametrize("acc", [False, True], ids=["overwrite", "accumulate"])
def test_plan_shared_tiles_repeat_exactly(sm, ref, dev, rows, acc):
    """Eight columns over 10240 columns with x read from global memory: a
    single matrix whose whole tiles would leave most CUs idle takes shared
    tiles in a plan (two workgroups meet through the plan's zeroed words).
    Row counts of 2560 (the verify set's down), 2200 and 2222 (a ragged last
    tile) put (tile, chunk) units over the workgroups so that some tiles
    straddle two of them; below about 2048 rows the search keeps whole
    tiles. Three runs from the same start
    (eager, then a captured graph replayed twice) give identical bits, the
    words returning to zero each time; each matches the oracle's decode
    times x in f64, plus y0 when accumulating; and the same op launched
    without a plan (no words: whole tiles only) agrees to within the f32
    sums' reordering."""
    import torch
    cols, N = 10240, 8
    h = sm.synth_container(0x5100 + rows, rows, cols)
    M = sm.DeviceContainer(h, dev)
    xb = sm.synth_bf16(0x5101, N * cols).reshape(N, cols)
    xf = sm.bf16_to_f32(xb).reshape(N, cols).astype(np.float64)
    x = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    y0 = np.random.default_rng(rows).standard_normal((N, rows)).astype(np.float32)
    y0t = torch.from_numpy(y0).to(dev)
    y = y0t.clone()
    plan = sm.Plan()
    plan.add_vq([M], x, [y], ncols=N, accumulate=acc)
    stream = torch.cuda.Stream(device=dev)
    outs = []
    with torch.cuda.stream(stream):
        y.copy_(y0t)
        plan.run(stream)
        torch.cuda.synchronize()
        outs.append(y.clone())
        plan.capture(stream)
        for _ in range(2):
            y.copy_(y0t)
            torch.cuda.synchronize()
            plan.launch(stream)
            torch.cuda.synchronize()
            outs.append(y.clone())
    for k, o in enumerate(outs[1:], 1):
        assert torch.equal(o, outs[0]), f"run {k} differs from run 0"
    want = xf @ ref.decode(h).astype(np.float64).T + (y0.astype(np.float64) if acc else 0.0)
    err = rel_l2(outs[0].cpu().numpy(), want)
    y2 = y0t.clone()
    M.gemv(x, y2, ncols=N, accumulate=acc)
    torch.cuda.synchronize()
    err2 = rel_l2(outs[0].cpu().numpy(), y2.cpu().numpy())
    print(f"rows {rows} accumulate {acc}: relL2 vs oracle {err:.2e}, vs the launch without words {err2:.2e}")
    assert err <= TIGHT and err2 <= TIGHT
    # the plan took shared tiles: its sums differ from whole tiles' in order
    assert not torch.equal(outs[0], y2), "shared tiles were not used"
