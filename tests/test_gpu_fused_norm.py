"""rms_norm fused into the matvec launch that reads it (sparkmv_vq_gemv_norm,
the decode forward's q+k+v+g and gate+up launches), at the reference
model's real shapes.

Each workgroup stages x = bf16(rms_norm(h) * w) itself from the f32 residual
h (model.rs:236-245: squares summed in f64, 1 / sqrt rounded once to f32,
(h * inv) * w in f32, then bf16 as the bf16 activations are stored). Checks:

  - x as the kernel staged it (x_out) against the oracle's rms_norm rounded to
    bf16: a value may differ by one bf16 step where the f64 sums, added in
    another order, round inv to a neighbouring f32 (at most a handful);
  - y against the oracle's bit-exact decode times that x in f64 (1e-5), and
    bit for bit against the unfused launch (sparkmv_vq_gemv_multi) on the same
    bf16 x: the fused kernel changes the staging only;
  - a norm weight 2^20 times larger takes the kernel's range rescale (x past
    f16's range) and scales y by exactly 2^20;
  - calls the fused kernel does not take are refused with a message.
"""
import numpy as np
import pytest

import chain_check as cc
import forward as fw

pytestmark = pytest.mark.gpu

TIGHT = 1e-5
HID, QD, KVD, NHEAD, FFN = 2560, 4096, 1024, 16, 10240


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def run(sm, dev, mats, h, w, rows):
    import torch
    ys = [torch.full((r,), float("nan"), device=dev) for r in rows]
    xo = torch.zeros(HID, dtype=torch.int16, device=dev)
    sm.gemv_norm(mats, torch.from_numpy(h).to(dev), torch.from_numpy(w).to(dev), ys, eps=1e-6, x_out=xo)
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys], xo


@pytest.mark.parametrize("group", ["q+k+v+g", "gate+up"])
def test_fused_norm_against_oracle(sm, ref, dev, group):
    import torch
    shapes = [(QD, HID), (KVD, HID), (KVD, HID), (NHEAD, HID)] if group == "q+k+v+g" else [(FFN, HID), (FFN, HID)]
    hosts = [sm.synth_container(0x4E00 + 7 * i + len(shapes), r, c) for i, (r, c) in enumerate(shapes)]
    mats = [sm.DeviceContainer(h, dev) for h in hosts]
    rows = [r for r, _ in shapes]
    # |x| well above 2^-14 everywhere, so x stays exact in f16 under the
    # rescale and the 2^20 check can be bit for bit
    rng = np.random.default_rng(len(shapes))
    n = rng.standard_normal(HID)
    h = (3.0 * np.sign(n) * (0.25 + np.abs(n))).astype(np.float32)
    w = np.clip(1.0 + 0.2 * rng.standard_normal(HID), 0.2, None).astype(np.float32)
    ys, xo = run(sm, dev, mats, h, w, rows)
    x16 = xo.cpu().numpy().view(np.uint16)
    want16 = cc.bf16_bits(fw.rms_norm(h, w, 1e-6))
    mismatch = int(np.sum(x16 != want16))
    print(f"{group}: staged x differs from the oracle's bf16(rms_norm) in {mismatch} of {HID} values")
    assert mismatch <= 4
    x = cc.bf16_f32(x16)
    for i, (hh, y) in enumerate(zip(hosts, ys)):
        err = rel_l2(y, ref.matvec_f64(ref.decode(hh), x))
        print(f"{group} matrix {i} {shapes[i]}: relL2 {err:.2e}")
        assert err <= TIGHT
    # the same x through the unfused launch: identical bits
    yu = [torch.full((r,), float("nan"), device=dev) for r in rows]
    sm.gemv_multi(mats, xo.view(1, -1), [y.view(1, -1) for y in yu])
    torch.cuda.synchronize()
    for a, b in zip(ys, yu):
        assert np.array_equal(a.view(np.uint32), b.cpu().numpy().view(np.uint32))
    # a norm weight 2^20 larger: x past f16's range, rescaled in the kernel
    ys2, _ = run(sm, dev, mats, h, np.ldexp(w, 20).astype(np.float32), rows)
    for a, b in zip(ys, ys2):
        assert np.array_equal(np.ldexp(a, 20).astype(np.float32).view(np.uint32), b.view(np.uint32))


def test_fused_norm_refusals(sm, dev):
    import torch
    m = sm.DeviceContainer(sm.synth_container(0x4E50, 64, 200), dev)
    h = torch.ones(200, device=dev)
    y = torch.zeros(64, device=dev)
    with pytest.raises(sm.SparkmvError):
        sm.gemv_norm([m], h, h, [y])
    assert "does not take this call" in sm.last_error()
    m2 = sm.DeviceContainer(sm.synth_container(0x4E51, 64, 256), dev)
    h2 = torch.ones(256, device=dev)
    with pytest.raises(sm.SparkmvError):
        sm.gemv_norm([m2], h2, h2, [y], eps=0.0)
    assert "eps" in sm.last_error()
