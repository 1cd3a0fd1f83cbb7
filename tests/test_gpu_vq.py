"""GPU parity of the VQ path through the C-ABI against the oracle.

Tolerances: decoded weights bit-exact; GEMV outputs within 1e-3 relative L2
of the f64 matvec of the oracle's decoded matrix (the stated bar). The MFMA
path's products are exact, so the tests also hold it to 1e-5 to catch
regressions long before the bar.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BAR = 1e-3
TIGHT = 1e-5


def rel_l2(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / max(np.linalg.norm(want), 1e-300))


def _x(sm, seed, ncol, cols, f32):
    import torch
    xb = sm.synth_bf16(seed, ncol * cols).reshape(ncol, cols)
    xf = sm.bf16_to_f32(xb).reshape(ncol, cols)
    if f32:   # an f32 activation that is not bf16-representable
        xf = (xf * np.float32(1.0 + 2.0 ** -12)).astype(np.float32)
        return torch.from_numpy(xf.copy()).cuda(), xf
    return torch.from_numpy(xb.view(np.int16).copy()).cuda(), xf


GEOMS = [
    # rows, cols, dim, nc, stages, v3
    (64, 256, 4, 4096, 2, 1),
    (37, 256, 4, 4096, 2, 1),
    (16, 2560, 4, 4096, 2, 1),
    (100, 384, 4, 8192, 2, 1),
    (48, 192, 4, 1024, 2, 1),
    (24, 64, 4, 256, 2, 0),
    (16, 128, 8, 4096, 1, 1),
    (5, 12, 4, 4096, 2, 1),
    (40, 128, 4, 3000, 1, 1),
]


@pytest.mark.parametrize("geom", GEOMS, ids=[f"{g[0]}x{g[1]}_d{g[2]}_nc{g[3]}_s{g[4]}_v{g[5]}" for g in GEOMS])
@pytest.mark.parametrize("f32", [False, True], ids=["bf16x", "f32x"])
def test_gemv_all_variants(sm, ref, dev, geom, f32):
    import torch
    rows, cols, dim, nc, ns, v3 = geom
    data = sm.synth_container(rows * 7 + cols, rows, cols, dim, nc, ns, v3)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    for ncol in (1, 3, 8):
        xt, xf = _x(sm, 5 + ncol, ncol, cols, f32)
        want = xf.astype(np.float64) @ W.T          # [ncol, rows]
        for variant in (0, 1, 2, 3):
            if not sm.lib().sparkmv_vq_gemv_ready(dim, nc, rows, cols, v3, variant):
                continue
            y = torch.full((ncol, rows), float("nan"), device=dev)
            dc.gemv(xt, y, ncols=ncol, accumulate=False, variant=variant)
            got = y.cpu().numpy()
            err = rel_l2(got, want)
            print(f"rows {rows} cols {cols} nc {nc} ncol {ncol} variant {variant} f32 {f32}: relL2 {err:.2e}")
            assert err <= BAR
            assert err <= TIGHT


def test_accumulate_adds_into_y(sm, ref, dev):
    import torch
    rows, cols = 96, 512
    data = sm.synth_container(3, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, 8, 1, cols, False)
    y0 = np.random.default_rng(0).standard_normal((1, rows)).astype(np.float32)
    y = torch.from_numpy(y0.copy()).to(dev)
    dc.gemv(xt, y, accumulate=True)
    want = y0.astype(np.float64) + xf.astype(np.float64) @ W.T
    assert rel_l2(y.cpu().numpy(), want) <= TIGHT


def test_batched_columns_equal_single_columns(sm, dev):
    """Decode-once N=8 gives each column what an N=1 call gives it."""
    import torch
    rows, cols = 256, 2560
    dc = sm.DeviceContainer(sm.synth_container(21, rows, cols))
    xt, _ = _x(sm, 9, 8, cols, False)
    y8 = torch.zeros(8, rows, device=dev)
    dc.gemv(xt, y8, ncols=8)
    for n in range(8):
        y1 = torch.zeros(1, rows, device=dev)
        dc.gemv(xt[n:n + 1], y1, ncols=1)
        a, b = y8[n].cpu().numpy(), y1[0].cpu().numpy()
        assert rel_l2(a, b) <= 1e-6, n


@pytest.mark.parametrize("rows,cols,ncol,nc", [(96, 10240, 8, 4096), (40, 10240, 16, 4096), (33, 2560, 8, 4096),
                                               (64, 4096, 8, 4096), (48, 4096, 8, 8192), (24, 8192, 3, 4096)])
def test_verify_columns_against_oracle(sm, ref, dev, rows, cols, ncol, nc):
    """Speculative-verify shapes: N columns decoded once. When x holds 48 KB
    or more (N = 8 at 4096 and 10240 columns, 3 columns of 8192) each lane
    reads its activations from global memory with its index words; smaller x
    (N = 8 at 2560 columns) is staged in LDS. 13-bit indices and an odd
    column count included; every column must match the oracle and the N=1
    result."""
    import torch
    data = sm.synth_container(rows + ncol, rows, cols, 4, nc, 2, 1)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, cols + ncol, ncol, cols, False)
    y = torch.full((ncol, rows), float("nan"), device=dev)
    dc.gemv(xt, y, ncols=ncol)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = xf.astype(np.float64) @ W.T
    err = rel_l2(got, want)
    print(f"{rows}x{cols} N={ncol}: relL2 {err:.2e}")
    assert err <= TIGHT
    for n in (0, ncol - 1):
        y1 = torch.zeros(1, rows, device=dev)
        dc.gemv(xt[n:n + 1], y1, ncols=1)
        torch.cuda.synchronize()
        assert rel_l2(got[n], y1[0].cpu().numpy()) <= 1e-6, n


def test_verify_multi_matrix_x_from_global(sm, ref, dev):
    """Several matrices sharing x in one launch with 8 columns of 4096 (x read
    from global memory), ragged row counts, then accumulating into y."""
    import torch
    cols, ncol = 4096, 8
    shapes = [160, 40, 40, 16]
    datas = [sm.synth_container(300 + i, r, cols) for i, r in enumerate(shapes)]
    mats = [sm.DeviceContainer(d) for d in datas]
    Ws = [ref.decode(d).astype(np.float64) for d in datas]
    xt, xf = _x(sm, 9, ncol, cols, False)
    ys = [torch.full((ncol, max(shapes)), float("nan"), device=dev) for _ in shapes]
    sm.gemv_multi(mats, xt, ys, ncols=ncol)
    torch.cuda.synchronize()
    got = [y[:, :r].cpu().numpy().copy() for y, r in zip(ys, shapes)]
    for W, g in zip(Ws, got):
        assert rel_l2(g, xf.astype(np.float64) @ W.T) <= TIGHT
    sm.gemv_multi(mats, xt, ys, ncols=ncol, accumulate=True)
    torch.cuda.synchronize()
    for W, y, r in zip(Ws, ys, shapes):
        assert rel_l2(y[:, :r].cpu().numpy(), 2 * (xf.astype(np.float64) @ W.T)) <= TIGHT


def test_reference_abi_per_stage(sm, ref, dev):
    """vqg_gemv_launch per stage payload, f32 x, y accumulating across stages:
    the reference runtime's calling pattern (vq-model-gpu.cu:651-660)."""
    import torch
    rows, cols = 80, 640
    data = sm.synth_container(31, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    x = np.sin(np.arange(cols, dtype=np.float32) * 0.001).astype(np.float32)   # the reference gate's x
    xd = torch.from_numpy(x).to(dev)
    L = sm.lib()
    for variant in (0, 1, 2, 3):
        y = torch.zeros(rows, device=dev)
        for p in dc.stage_ptrs:
            sm.check(L.vqg_gemv_launch(p, 4, 4096, rows, cols, 1, xd.data_ptr(), y.data_ptr(), variant), "launch")
        torch.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), W @ x.astype(np.float64)) <= TIGHT
        ms = ctypes.c_double()
        y.zero_()
        sm.check(L.vqg_gemv_t(dc.stage_ptrs[0], 4, 4096, rows, cols, 1, xd.data_ptr(), y.data_ptr(), variant, 128, 3,
                              ctypes.byref(ms)), "timed")
        assert ms.value > 0


@pytest.mark.parametrize("threads", [32, 96, 160, 1024])
def test_reference_abi_warp_widths(sm, ref, dev, threads):
    """The reference takes any multiple of 32 up to 1024 as the launch width
    of variants 1-3 (decode-gpu.cu:815-818); here a width rounds up to whole
    64-lane waves and never changes the result."""
    import torch
    rows, cols = 72, 512
    data = sm.synth_container(33, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    x = np.cos(np.arange(cols, dtype=np.float32) * 0.003).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    L = sm.lib()
    for variant in (1, 2, 3):
        y = torch.zeros(rows, device=dev)
        for p in dc.stage_ptrs:
            sm.check(L.vqg_gemv_launch_t(p, 4, 4096, rows, cols, 1, xd.data_ptr(), y.data_ptr(), variant, threads),
                     "launch")
        torch.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), W @ x.astype(np.float64)) <= TIGHT, (variant, threads)


@pytest.mark.parametrize("dim,nc,v3", [(8, 4096, 1), (8, 8192, 0), (4, 16384, 0)])
def test_reference_variants_beyond_dim4(sm, ref, dev, dim, nc, v3):
    """Every variant the reference's readiness rules call ready runs and
    matches the oracle: the block path (3) for a dim-8 DQV3 stream, the
    shared-codebook kernel (0, via vqg_gemv_t) with a 128 KB codebook, and
    the dim-4 path (2) on a DQVQ stream."""
    import torch
    rows, cols = 40, 1024
    data = sm.synth_container(34 + dim, rows, cols, dim=dim, nc=nc, nstages=1, v3=v3)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    x = np.sin(np.arange(cols, dtype=np.float32) * 0.002).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    L = sm.lib()
    ran = []
    for variant in (0, 1, 2, 3):
        if not L.vqg_gemv_ready(dim, nc, rows, cols, v3, variant):
            continue
        y = torch.zeros(rows, device=dev)
        ms = ctypes.c_double()
        sm.check(L.vqg_gemv_t(dc.stage_ptrs[0], dim, nc, rows, cols, v3, xd.data_ptr(), y.data_ptr(), variant, 128, 1,
                              ctypes.byref(ms)), f"variant {variant}")
        torch.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), W @ x.astype(np.float64)) <= TIGHT, variant
        ran.append(variant)
    assert 0 in ran and 1 in ran


def test_reference_abi_errors(sm, dev):
    import torch
    L = sm.lib()
    dc = sm.DeviceContainer(sm.synth_container(2, 32, 128))
    x = torch.zeros(128, device=dev)
    y = torch.zeros(32, device=dev)
    p = dc.stage_ptrs[0]
    assert L.vqg_gemv_launch(p, 4, 16384, 32, 128, 1, x.data_ptr(), y.data_ptr(), 0) == -1
    assert "13 index bits" in sm.last_error()
    assert L.vqg_gemv_launch(p, 4, 4096, 0, 128, 1, x.data_ptr(), y.data_ptr(), 0) == -1
    assert L.vqg_gemv_launch(p, 4, 4096, 32, 128, 1, x.data_ptr(), y.data_ptr(), 9) == -1
    assert L.vqg_gemv_launch_t(p, 4, 4096, 32, 128, 1, x.data_ptr(), y.data_ptr(), 3, 100) == -1
    assert "warp multiple" in sm.last_error()
    assert L.vqg_gemv_launch(p, 4, 1024, 32, 128, 1, x.data_ptr(), y.data_ptr(), 3) == -1
    assert "block kernel" in sm.last_error()
    assert L.vqg_row_dequant(p, 4, 4096, 32, 128, 1, 32, y.data_ptr()) == -1
    torch.cuda.synchronize()


@pytest.mark.parametrize("geom", GEOMS, ids=[f"{g[0]}x{g[1]}_d{g[2]}_nc{g[3]}_s{g[4]}_v{g[5]}" for g in GEOMS])
def test_dequant_bit_exact(sm, ref, dev, geom):
    import torch
    rows, cols, dim, nc, ns, v3 = geom
    data = sm.synth_container(rows + 11 * cols, rows, cols, dim, nc, ns, v3)
    want = ref.decode(data)
    dc = sm.DeviceContainer(data)
    out = torch.full((rows, cols), float("nan"), device=dev)
    dc.dequant(out, accumulate=False)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the reference entry points: stage by stage into zeros, and single rows
    L = sm.lib()
    out.zero_()
    ms = ctypes.c_double()
    for p in dc.stage_ptrs:
        sm.check(L.vqg_dequant(p, dim, nc, rows, cols, v3, out.data_ptr(), 1, ctypes.byref(ms)), "vqg_dequant")
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    row = torch.zeros(cols, device=dev)
    r = rows // 2
    for p in dc.stage_ptrs:
        sm.check(L.vqg_row_dequant(p, dim, nc, rows, cols, v3, r, row.data_ptr()), "row dequant")
    torch.cuda.synchronize()
    assert np.array_equal(row.cpu().numpy().view(np.uint32), want[r].view(np.uint32))


def test_golden_fixtures_on_gpu(sm, dev):
    """The reference decoder's own dumps, reproduced by the GPU dequant."""
    import glob
    import os
    import torch
    from conftest import GOLDEN
    for path in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        with np.load(path, allow_pickle=False) as z:
            data, want = z["container"], z["decoded"]
        dc = sm.DeviceContainer(data)
        out = torch.zeros(want.shape, device=dev)
        dc.dequant(out)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), path


def test_multi_matrix_launch(sm, ref, dev):
    """q, k, v and the head gate of one layer (scaled down) in one launch,
    with one and with two activation columns (one ldy for every matrix)."""
    import torch
    cols = 512
    shapes = [256, 64, 64, 16]
    datas = [sm.synth_container(100 + i, r, cols) for i, r in enumerate(shapes)]
    mats = [sm.DeviceContainer(d) for d in datas]
    Ws = [ref.decode(d).astype(np.float64) for d in datas]
    for ncol in (1, 2):
        xt, xf = _x(sm, 4 + ncol, ncol, cols, False)
        ys = [torch.full((ncol, max(shapes)), float("nan"), device=dev) for _ in shapes]
        sm.gemv_multi(mats, xt, ys, ncols=ncol)
        torch.cuda.synchronize()
        for W, y, r in zip(Ws, ys, shapes):
            got = y[:, :r].cpu().numpy()
            assert rel_l2(got, xf.astype(np.float64) @ W.T) <= TIGHT


@pytest.mark.parametrize("ntok", [1, 37, 130])
def test_prefill_token_major(sm, ref, dev, ntok):
    import torch
    rows, cols = 64, 256
    data = sm.synth_container(55, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, 12, ntok, cols, False)
    y = torch.full((ntok, rows), float("nan"), device=dev)
    dc.prefill(xt, y)
    assert rel_l2(y.cpu().numpy(), xf.astype(np.float64) @ W.T) <= BAR


@pytest.mark.parametrize("rows,cols,ntok,nc,f32", [(320, 2560, 200, 4096, False), (130, 1024, 512, 4096, False),
                                                    (64, 512, 77, 8192, False), (96, 640, 130, 4096, True),
                                                    (256, 10240, 64, 4096, False), (10240, 256, 1024, 4096, False),
                                                    (10200, 256, 1000, 8192, True)])
def test_prefill_mfma_against_oracle(sm, ref, dev, rows, cols, ntok, nc, f32):
    """The matrix-core prefill: ragged row and token tiles (130 rows end
    inside a four-row store), f32 x, the long 10240-column rows of down_proj
    (256 x 10240 x 64 tokens splits K sixteen ways: one row tile, one token
    tile), and an 8192-entry two-stage codebook, whose LDS only the weight-
    tile kernel holds (64 x 512 and 10200 x 256).

    Both two-stage modes run. With the stages apart (sparkmv_prefill_fold
    0), a 4096-entry codebook and bf16 x, each stage's exact codewords meet x
    (exact in f16) with f32 accumulation: the GEMV's 1e-5. The default folds
    each weight g0 c0 + g1 c1 to f16 (so does the weight-tile kernel, in
    both modes), and f32 x rounds to f16 as the reference's prefill rounds
    it: those meet the GEMM gate, 1e-3."""
    import torch
    data = sm.synth_container(rows * 3 + ntok, rows, cols, 4, nc, 2, 1)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, ntok + 5, ntok, cols, f32)
    want = xf.astype(np.float64) @ W.T
    for fold in (True, False):
        with sm.prefill_mode(fold):
            y = torch.full((ntok, rows), float("nan"), device=dev)
            dc.prefill(xt, y)
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            err = rel_l2(got, want)
            bar = BAR if fold or f32 or nc > 4096 else TIGHT
            print(f"prefill {rows}x{cols} ntok {ntok} nc {nc} f32 {f32} fold {fold}: relL2 {err:.2e} (bar {bar:.0e})")
            assert err <= bar
            # accumulate adds into y
            y2 = torch.from_numpy(got.copy()).to(dev)
            dc.prefill(xt, y2, accumulate=True)
            torch.cuda.synchronize()
            assert rel_l2(y2.cpu().numpy(), 2 * want) <= bar
    assert sm.prefill_fold() is True


@pytest.mark.parametrize("rows,cols,ntok", [(1024, 2560, 256), (512, 10240, 130)])
def test_prefill_fold_error_bound(sm, ref, dev, rows, cols, ntok):
    """The two-stage switch (sparkmv_prefill_fold): stages apart meet the
    GEMV's 1e-5 against the oracle's exact decode; folded into one f16
    weight (the default) they add that weight's rounding, bounded by the
    GEMM gate 1e-3 against both the oracle and the exact path, and not zero
    (the switch took effect). The setting is process-wide and restored."""
    import torch
    data = sm.synth_container(0x7F00 + cols, rows, cols, 4, 4096, 2, 1)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, 0x7F10 + cols, ntok, cols, False)
    want = xf.astype(np.float64) @ W.T
    assert sm.prefill_fold() is True
    ys = {}
    for fold in (False, True):
        prev = sm.prefill_fold(fold)
        try:
            y = torch.full((ntok, rows), float("nan"), device=dev)
            dc.prefill(xt, y)
            torch.cuda.synchronize()
            ys[fold] = y.cpu().numpy()
        finally:
            sm.prefill_fold(prev)
    assert sm.prefill_fold() is True
    e_exact, e_fold = rel_l2(ys[False], want), rel_l2(ys[True], want)
    e_between = rel_l2(ys[True], ys[False])
    print(f"prefill {rows}x{cols} ntok {ntok}: stages apart {e_exact:.2e}, folded {e_fold:.2e}, "
          f"folded vs apart {e_between:.2e}")
    assert e_exact <= TIGHT
    assert e_fold <= BAR and e_between <= BAR
    assert e_between > 0.0


def test_prefill_full_size_down_split_k(sm, ref, dev):
    """down_proj at its real size, 2560 x 10240 against 512 bf16 tokens: the
    2560 rows give 10 x 4 row and token tiles, so K splits five ways and a
    reduction adds the slices in split order. Two runs are bit-identical (the
    split order fixes the sums), and the result meets the GEMM gate against
    the oracle's decode and an f64 product."""
    import torch
    rows, cols, ntok = 2560, 10240, 512
    data = sm.synth_container(0x9F01, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, 0x9F11, ntok, cols, False)
    ys = []
    for _ in range(2):
        y = torch.full((ntok, rows), float("nan"), device=dev)
        dc.prefill(xt, y)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))
    err = rel_l2(ys[0], xf.astype(np.float64) @ W.T)
    print(f"prefill {rows}x{cols} ntok {ntok}: relL2 {err:.2e}")
    assert err <= BAR


def test_prefill_refusals(sm, dev):
    """Calls the prefill refuses before any launch, with real device buffers
    so that a check that wrongly passed could not touch bad memory."""
    import torch
    rows, cols, ntok = 64, 256, 8
    dc = sm.DeviceContainer(sm.synth_container(57, rows, cols))
    x = torch.zeros(ntok, cols, dtype=torch.int16, device=dev)
    y = torch.zeros(ntok, rows, device=dev)
    pp, keep = dc._stages()
    L, h = sm.lib(), dc.host

    def call(nst=h.nstages, xp=x.data_ptr(), xd=sm.X_BF16, ldx=cols, n=ntok, yp=y.data_ptr(), ldy=rows):
        return L.sparkmv_vq_prefill(pp, nst, h.dim, h.nc, rows, cols, h.v3, xp, xd, ldx, n, yp, ldy, 0, None)

    assert call() == 0
    torch.cuda.synchronize()
    for kw, msg in [({"n": 0}, "at least one token"), ({"ldx": cols - 8}, "ldx/ldy"), ({"ldy": rows - 4}, "ldx/ldy"),
                    ({"xd": 7}, "x dtype"), ({"xp": None}, "null pointer"), ({"yp": None}, "null pointer")]:
        assert call(**kw) == -1, kw
        assert msg in sm.last_error(), (kw, sm.last_error())


def test_prefill_reference_layout(sm, ref, dev):
    import torch
    rows, cols, ntok = 48, 128, 20
    data = sm.synth_container(56, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    x = np.random.default_rng(1).standard_normal((ntok, cols)).astype(np.float32)
    xT = torch.from_numpy(np.ascontiguousarray(x.T)).to(dev)
    y = torch.zeros(ntok, rows, device=dev)
    L = sm.lib()
    for p in dc.stage_ptrs:
        sm.check(L.vqg_prefill_launch(p, 4, 4096, rows, cols, 1, xT.data_ptr(), ntok, y.data_ptr(), 0), "prefill")
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), x.astype(np.float64) @ W.T) <= BAR


@pytest.mark.parametrize("rows,cols,ntok,nc,variant,tile", [(320, 2560, 200, 4096, 2, (128, 64)),
                                                          (130, 1024, 512, 8192, 1, (64, 64)),
                                                          (10240, 256, 1024, 8192, 2, (128, 64)),
                                                          (64, 512, 36, 4096, 0, None),
                                                          (48, 640, 37, 4096, 2, (256, 64)),
                                                          (96, 256, 12, 4096, 3, None)])
def test_prefill_reference_layout_variants(sm, ref, dev, rows, cols, ntok, nc, variant, tile):
    """The reference's prefill ABI (xT [cols][ntok] f32, y [ntok][rows]
    accumulating, one stage per call, as vq-model-gpu.cu:838-851 drives it).
    Tiled variants with ntok a multiple of 4 run the matrix cores on K-major
    x; 37 tokens and the legacy variant run one thread per output. The bar
    is the GEMM gate's 1e-3 relative L2 (weights enter the MFMA as f16)."""
    import torch
    data = sm.synth_container(rows + ntok + variant, rows, cols, 4, nc, 2, 1)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    x = np.random.default_rng(ntok).standard_normal((ntok, cols)).astype(np.float32)
    xT = torch.from_numpy(np.ascontiguousarray(x.T)).to(dev)
    base = np.random.default_rng(rows).standard_normal((ntok, rows)).astype(np.float32)
    y = torch.from_numpy(base.copy()).to(dev)
    L = sm.lib()
    for p in dc.stage_ptrs:
        if tile is None:
            rc = L.vqg_prefill_launch(p, 4, nc, rows, cols, 1, xT.data_ptr(), ntok, y.data_ptr(), variant)
        else:
            rc = L.vqg_prefill_launch_tile(p, 4, nc, rows, cols, 1, xT.data_ptr(), ntok, y.data_ptr(),
                                           tile[0], tile[1], variant)
        sm.check(rc, "prefill")
    torch.cuda.synchronize()
    want = x.astype(np.float64) @ W.T
    err = rel_l2(y.cpu().numpy() - base, want)
    print(f"reference-layout prefill {rows}x{cols} ntok {ntok} nc {nc} variant {variant}: relL2 {err:.2e}")
    assert err <= BAR


def test_full_size_ffn_up(sm, ref, dev):
    """10240 x 2560, dim 4, nc 4096, 2 stages, bf16 x: the single-GEMV workload
    at its real size, against the oracle's decode and an f64 matvec."""
    import torch
    rows, cols = 10240, 2560
    data = sm.synth_container(2024, rows, cols)
    W = ref.decode(data)
    dc = sm.DeviceContainer(data)
    xt, xf = _x(sm, 77, 1, cols, False)
    y = torch.zeros(1, rows, device=dev)
    dc.gemv(xt, y)
    y64 = ref.matvec_f64(W, xf[0])
    err = rel_l2(y.cpu().numpy()[0], y64)
    print(f"10240x2560 relL2 vs f64 {err:.3e}")
    assert err <= TIGHT
    yr = ref.matvec(W, xf[0])          # the runtime's own f32 dot (model.rs:209-234)
    assert rel_l2(y.cpu().numpy()[0], yr) <= TIGHT
    out = torch.zeros(rows, cols, device=dev)
    dc.dequant(out)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), W.view(np.uint32))


TRUNK_F32 = [
    # (matrix rows, ...), cols: the decode layer's launches with f32 x
    ((4096, 1024, 1024, 16), 2560),   # q + k + v + head gate, one launch
    ((2560,), 4096),                  # o
    ((10240, 10240), 2560),           # gate + up, one launch
    ((10240,), 2560),                 # gate alone
    ((2560,), 10240),                 # down
]


@pytest.mark.parametrize("shapes,cols", TRUNK_F32, ids=["qkvg", "o", "gate_up", "gate", "down"])
def test_f32_x_at_trunk_shapes(sm, ref, dev, shapes, cols):
    """f32 activations (the reference's arithmetic: x split into f16 hi + lo,
    two MFMAs per step) at the decode layer's real launch shapes, whose
    one-column shapes run the straight-line units of 2, 5 and 10 macro
    steps; every row against the oracle's decode times x in f64, within
    1e-5, with y filled with NaN first so every row must be written."""
    import torch
    datas = [sm.synth_container(0xF320 + 7 * i + cols, r, cols) for i, r in enumerate(shapes)]
    mats = [sm.DeviceContainer(d, dev) for d in datas]
    xt, xf = _x(sm, 0xF32 + cols, 1, cols, True)
    ys = [torch.full((1, max(shapes)), float("nan"), device=dev) for _ in shapes]
    print(f"f32 x: rows {shapes} x {cols}", flush=True)
    sm.gemv_multi(mats, xt, ys)
    torch.cuda.synchronize()
    for d, y, r in zip(datas, ys, shapes):
        W = ref.decode(d).astype(np.float64)
        err = rel_l2(y[0, :r].cpu().numpy(), W @ xf[0].astype(np.float64))
        print(f"  {r} rows: relL2 {err:.2e}")
        assert err <= TIGHT, (r, err)
