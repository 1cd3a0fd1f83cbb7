"""Activations outside f16's range through every GEMV path that converts x to
f16 for the matrix cores or the dot2 units.

The reference's decode arithmetic keeps x in f32 (tools/vq-format/src/
lib.rs:215-227; tools/vq/gpu/decode-gpu.cu:228-260), so x far above 65504 or
far below 2^-14 must give the same answer as x of ordinary size. Two checks
per path:

- Scaling bf16 x by a power of two scales y by the same power bit for bit.
  The in-range run is exact in f16 (x is N(0,1) bf16 with |x| < 2^-14 set
  to zero), and so is a rescaled one, so any term lost or rounded
  differently in the rescale breaks the equality. (f32 x is split into
  hi + lo f16, whose lo part sits on f16's subnormal grid in one run and
  not in the other, so f32 x is held to the bar only.)
- y matches the f64 product of the oracle's decoded matrix at the GEMV bar
  (1e-5 relative L2), including x with one huge element per column and
  columns of very different size.

A non-finite x must give non-finite y exactly where the f64 product does,
and leave the other columns of the launch at the bar.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIGHT = 1e-5


def rel_l2(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / max(np.linalg.norm(want), 1e-300))


def base_x(sm, seed, ncol, cols):
    """bf16 N(0,1) activations [ncol, cols] as f32, with |x| < 2^-14 zeroed."""
    xf = sm.bf16_to_f32(sm.synth_bf16(seed, ncol * cols)).reshape(ncol, cols).copy()
    xf[np.abs(xf) < 2.0 ** -14] = 0.0
    return xf


def to_dev(xf, dev, f32):
    """f32 values that bf16 holds exactly -> a device tensor of bf16 bits (or f32)."""
    import torch
    if f32:
        return torch.from_numpy(np.ascontiguousarray(xf, np.float32)).to(dev)
    bits = np.ascontiguousarray(xf, np.float32).view(np.uint32)
    assert not np.any(bits & 0xFFFF), "value not representable in bf16"
    return torch.from_numpy((bits >> 16).astype(np.uint16).view(np.int16)).to(dev)


def run_vq(sm, dev, dc, xf, rows, f32):
    import torch
    ncol = xf.shape[0]
    y = torch.full((ncol, rows), float("nan"), device=dev)
    dc.gemv(to_dev(xf, dev, f32), y, ncols=ncol)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def run_kq(sm, dev, kind, db, rows, cols, xf, f32):
    import torch
    ncol = xf.shape[0]
    y = torch.full((ncol, rows), float("nan"), device=dev)
    sm.kquant_gemv(kind, db, rows, cols, to_dev(xf, dev, f32), y, ncols=ncol)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def per_col_err(got, xf, W):
    want = xf.astype(np.float64) @ W.T
    return max(rel_l2(got[n], want[n]) for n in range(got.shape[0]))


# rows, cols, columns, f32 x, shifts; the paths: one column staged in one
# pass; f32 x (ring kernel, hi + lo f16); several columns staged in LDS;
# several columns read from global memory per step (which checks the range
# per unit and per column after the fact, and runs a unit again scaled).
VQ_CASES = [
    (256, 2560, 1, False, (20, -30, 100)),
    (64, 256, 1, True, (20, -30)),
    (33, 2560, 8, False, (20, -30)),
    (64, 4096, 8, False, (20, 12, -30, -100)),
]


@pytest.mark.parametrize("rows,cols,ncol,f32,shifts", VQ_CASES,
                         ids=["one-column", "f32-x", "staged-columns", "x-from-global"])
def test_vq_gemv_power_of_two_scaling(sm, ref, dev, rows, cols, ncol, f32, shifts):
    data = sm.synth_container(rows + 17 * ncol, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xf = base_x(sm, 71 + ncol, ncol, cols)
    if f32:
        xf = xf * np.float32(1.0 + 2.0 ** -12)
    y0 = run_vq(sm, dev, dc, xf, rows, f32)
    assert per_col_err(y0, xf, W) <= TIGHT
    for s in shifts:
        xs = np.ldexp(xf, s).astype(np.float32)
        ys = run_vq(sm, dev, dc, xs, rows, f32)
        err = per_col_err(ys, xs, W)
        same = np.array_equal(ys, np.ldexp(y0, s).astype(np.float32))
        print(f"vq {rows}x{cols} N={ncol} f32={f32} x*2^{s}: relL2 {err:.2e}, bit-exact scaling {same}")
        assert err <= TIGHT
        assert same or f32


@pytest.mark.parametrize("rows,cols,ncol,f32", [(256, 2560, 1, False), (64, 256, 1, True), (33, 2560, 8, False),
                                                (64, 4096, 8, False)],
                         ids=["one-column", "f32-x", "staged-columns", "x-from-global"])
def test_vq_gemv_spikes_and_mixed_columns(sm, ref, dev, rows, cols, ncol, f32):
    """One element per column of 2^18 (1 + 2^-7) among N(0,1), and with several
    columns, column 0 alone 2^20 times larger than the others."""
    data = sm.synth_container(rows + 5, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xf = base_x(sm, 91, ncol, cols)
    xf[:, 7] = 264192.0
    got = run_vq(sm, dev, dc, xf, rows, f32)
    err = per_col_err(got, xf, W)
    print(f"vq spike {rows}x{cols} N={ncol}: relL2 {err:.2e}")
    assert err <= TIGHT
    if ncol > 1:
        xm = base_x(sm, 92, ncol, cols)
        xm[0] = np.ldexp(xm[0], 20)
        got = run_vq(sm, dev, dc, xm, rows, f32)
        err = per_col_err(got, xm, W)
        print(f"vq mixed columns {rows}x{cols} N={ncol}: relL2 {err:.2e}")
        assert err <= TIGHT


def test_vq_gemv_small_columns_from_global(sm, ref, dev):
    """x read from global memory (8 columns of 4096): columns of very small
    values beside ordinary ones. Column 1 holds N(0,1) * 2^-20 with ALL its
    values kept, down to bf16's smallest normals, and column 2 N(0,1) * 2^-40
    (below f16's smallest subnormal). Converted to f16 as they are, such
    columns would lose their values below 2^-14 (2^-24 apart at best); each
    column is brought into range by a power of two of its own, so every
    column meets the bar and the ordinary columns are unchanged."""
    rows, cols, ncol = 64, 4096, 8
    data = sm.synth_container(rows + 29, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xf = base_x(sm, 93, ncol, cols)
    y_plain = run_vq(sm, dev, dc, xf, rows, False)
    full = sm.bf16_to_f32(sm.synth_bf16(94, 2 * cols)).reshape(2, cols)
    xs = xf.copy()
    xs[1] = np.ldexp(full[0], -20)
    xs[2] = np.ldexp(full[1], -40)
    got = run_vq(sm, dev, dc, xs, rows, False)
    want = xs.astype(np.float64) @ W.T
    errs = [rel_l2(got[n], want[n]) for n in range(ncol)]
    print("small columns from global memory, relL2 per column:", [f"{e:.1e}" for e in errs])
    assert max(errs) <= TIGHT
    keep = [n for n in range(ncol) if n not in (1, 2)]
    assert np.array_equal(got[keep], y_plain[keep])


@pytest.mark.parametrize("rows,cols,ncol", [(256, 2560, 1), (64, 4096, 8)], ids=["one-column", "x-from-global"])
def test_vq_gemv_non_finite_x(sm, ref, dev, rows, cols, ncol):
    data = sm.synth_container(rows + 3, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xf = base_x(sm, 93, ncol, cols)
    xf[0, 5] = np.inf
    got = run_vq(sm, dev, dc, xf, rows, False)
    with np.errstate(invalid="ignore"):
        want = xf.astype(np.float64) @ W.T
    assert not np.isfinite(got[0]).any()
    assert np.array_equal(np.isfinite(got), np.isfinite(want))
    if ncol > 1:
        assert per_col_err(got[1:], xf[1:], W) <= TIGHT


def run_vq_plan(sm, dev, dc, xf, rows):
    """One several-column op in a plan (the plan gives it exchange words, so
    a matrix whose x is too large to stage whole splits its tiles by K chunk
    and stages each chunk's x)."""
    import torch
    ncol = xf.shape[0]
    x = to_dev(xf, dev, False)
    y = torch.full((ncol, rows), float("nan"), device=dev)
    plan = sm.Plan()
    plan.add_vq([dc], x, [y], ncols=ncol)
    plan.run(torch.cuda.current_stream())
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_vq_plan_chunk_split_range(sm, ref, dev):
    """Chunk-split tiles (the verify set's down shape, 2560 x 10240 at N = 8,
    in a plan): every workgroup checks the range of the x chunk it staged and
    rescales it by a power of two of its own, and the chunk sums are brought
    back before they meet. Scaling x by 2^20 and 2^-30 scales y bit for bit;
    one element of 2^18 (1 + 2^-7) per column, and column 0 alone 2^20 times
    larger, meet the bar; an infinity gives non-finite y exactly where the
    f64 product does and leaves the other columns at the bar."""
    rows, cols, ncol = 2560, 10240, 8
    data = sm.synth_container(0x6C01, rows, cols)
    W = ref.decode(data).astype(np.float64)
    dc = sm.DeviceContainer(data)
    xf = base_x(sm, 0x6C02, ncol, cols)
    y0 = run_vq_plan(sm, dev, dc, xf, rows)
    assert per_col_err(y0, xf, W) <= TIGHT
    for sh in (20, -30):
        xs = np.ldexp(xf, sh).astype(np.float32)
        ys = run_vq_plan(sm, dev, dc, xs, rows)
        err = per_col_err(ys, xs, W)
        same = np.array_equal(ys, np.ldexp(y0, sh).astype(np.float32))
        print(f"chunk-split x*2^{sh}: relL2 {err:.2e}, bit-exact scaling {same}")
        assert err <= TIGHT and same
    xp = xf.copy()
    xp[:, 7] = 264192.0
    err = per_col_err(run_vq_plan(sm, dev, dc, xp, rows), xp, W)
    xm = base_x(sm, 0x6C03, ncol, cols)
    xm[0] = np.ldexp(xm[0], 20)
    err_m = per_col_err(run_vq_plan(sm, dev, dc, xm, rows), xm, W)
    print(f"chunk-split spike relL2 {err:.2e}, mixed columns {err_m:.2e}")
    assert err <= TIGHT and err_m <= TIGHT
    xn = xf.copy()
    xn[0, 5000] = np.inf
    got = run_vq_plan(sm, dev, dc, xn, rows)
    with np.errstate(invalid="ignore"):
        want = xn.astype(np.float64) @ W.T
    assert not np.isfinite(got[0]).any()
    assert np.array_equal(np.isfinite(got), np.isfinite(want))
    assert per_col_err(got[1:], xn[1:], W) <= TIGHT


# kind, rows, cols, columns, f32 x: Q8_0 one column and four rows per lane;
# Q6_K staged rows (even superblocks per row), the wide form (odd, at most
# 12288 columns) and the plain one (odd, wider).
KQ_CASES = [
    ("q8_0", 300, 2560, 1, False),
    ("q8_0", 300, 2560, 8, False),
    ("q8_0", 300, 2560, 1, True),
    ("q6_k", 40, 2560, 1, False),
    ("q6_k", 40, 2560, 4, False),
    ("q6_k", 40, 2304, 1, False),
    ("q6_k", 24, 12544, 1, False),
]


def kq_weights(sm, ref, kind, rows, cols, seed):
    import torch
    if kind == "q8_0":
        blocks = sm.synth_q8_0(seed, rows, cols)
        W = ref.q8_0_dequant(blocks, rows, cols)
    else:
        blocks = sm.synth_q6k(seed, rows, cols)
        W = ref.q6k_dequant(blocks, rows, cols)
    return torch.from_numpy(blocks.copy()).cuda(), W.astype(np.float64)


@pytest.mark.parametrize("kind,rows,cols,ncol,f32", KQ_CASES,
                         ids=["q8_0", "q8_0-8col", "q8_0-f32", "q6k-staged", "q6k-staged-4col", "q6k-wide", "q6k-plain"])
def test_kquant_gemv_power_of_two_scaling(sm, ref, dev, kind, rows, cols, ncol, f32):
    db, W = kq_weights(sm, ref, kind, rows, cols, rows + cols + ncol)
    xf = base_x(sm, 81 + ncol, ncol, cols)
    if f32:
        xf = xf * np.float32(1.0 + 2.0 ** -12)
    y0 = run_kq(sm, dev, kind, db, rows, cols, xf, f32)
    assert per_col_err(y0, xf, W) <= TIGHT
    for s in (20, -20, 100):
        xs = np.ldexp(xf, s).astype(np.float32)
        ys = run_kq(sm, dev, kind, db, rows, cols, xs, f32)
        err = per_col_err(ys, xs, W)
        same = np.array_equal(ys, np.ldexp(y0, s).astype(np.float32))
        print(f"{kind} {rows}x{cols} N={ncol} f32={f32} x*2^{s}: relL2 {err:.2e}, bit-exact scaling {same}")
        assert err <= TIGHT
        assert same or f32


@pytest.mark.parametrize("kind,rows,cols,ncol", [("q8_0", 300, 2560, 8), ("q6_k", 40, 2560, 4)],
                         ids=["q8_0-8col", "q6k-staged-4col"])
def test_kquant_gemv_spikes_mixed_and_non_finite(sm, ref, dev, kind, rows, cols, ncol):
    db, W = kq_weights(sm, ref, kind, rows, cols, 7)
    xf = base_x(sm, 95, ncol, cols)
    xf[:, 7] = 264192.0
    assert per_col_err(run_kq(sm, dev, kind, db, rows, cols, xf, False), xf, W) <= TIGHT
    xm = base_x(sm, 96, ncol, cols)
    xm[0] = np.ldexp(xm[0], 20)
    assert per_col_err(run_kq(sm, dev, kind, db, rows, cols, xm, False), xm, W) <= TIGHT
    xn = base_x(sm, 97, ncol, cols)
    xn[0, 5] = np.inf
    got = run_kq(sm, dev, kind, db, rows, cols, xn, False)
    with np.errstate(invalid="ignore"):
        want = xn.astype(np.float64) @ W.T
    assert not np.isfinite(got[0]).any()
    assert np.array_equal(np.isfinite(got), np.isfinite(want))
    assert per_col_err(got[1:], xn[1:], W) <= TIGHT
