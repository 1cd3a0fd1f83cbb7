"""Weights loaded from artifact files straight into the matvec kernels: Q8_0
and Q6_K tensors from a GGUF file, a VQ container from a manifest directory
(the loaders of tools/dspark/src/gguf.rs and tools/vq-runtime/src/
vq_source.rs), each GEMV checked against the oracle's decode and an f64
product at the GEMV bar."""
import numpy as np
import pytest

from test_artifacts import write_gguf

pytestmark = pytest.mark.gpu

TIGHT = 1e-5


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def test_gguf_kquant_weights_through_the_gemv(sm, ref, dev, tmp_path):
    import torch
    q8 = sm.synth_q8_0(21, 300, 2560)
    q6 = sm.synth_q6k(22, 40, 2560)
    path = tmp_path / "w.gguf"
    write_gguf(path, [("general.architecture", 8, "spark")],
               [("token_embd.weight", [2560, 300], 8, q8.tobytes()), ("blk.0.ffn_down.weight", [2560, 40], 14,
                                                                     q6.tobytes())])
    xb = sm.synth_bf16(23, 2560)
    xf = sm.bf16_to_f32(xb)
    xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    with sm.Gguf(path) as g:
        for name in ("token_embd.weight", "blk.0.ffn_down.weight"):
            kind, rows, cols, blocks = g.kquant(name)
            W = ref.q8_0_dequant(blocks, rows, cols) if kind == 8 else ref.q6k_dequant(blocks, rows, cols)
            db = torch.from_numpy(blocks.copy()).to(dev)
            y = torch.full((rows,), float("nan"), device=dev)
            sm.kquant_gemv("q8_0" if kind == 8 else "q6_k", db, rows, cols, xt, y)
            torch.cuda.synchronize()
            err = rel_l2(y.cpu().numpy(), W.astype(np.float64) @ xf.astype(np.float64))
            print(f"gguf {name} ({'Q8_0' if kind == 8 else 'Q6_K'} {rows}x{cols}): relL2 {err:.2e}")
            assert err <= TIGHT


def test_manifest_container_through_the_gemv(sm, ref, dev, tmp_path):
    import torch
    cont = sm.synth_container(31, 256, 2560)
    (tmp_path / "blk.0.mlp.up_proj.weight.bin").write_bytes(cont.tobytes())
    (tmp_path / "manifest.txt").write_text(f"blk.0.mlp.up_proj.weight 256 2560 2 {cont.nbytes} 3.0\n")
    d = sm.VqDir(tmp_path)
    dc = sm.DeviceContainer(d.read("blk.0.mlp.up_proj.weight"), dev)
    W = ref.decode(cont).astype(np.float64)
    xb = sm.synth_bf16(32, 2560)
    xf = sm.bf16_to_f32(xb)
    y = torch.full((1, 256), float("nan"), device=dev)
    dc.gemv(torch.from_numpy(xb.view(np.int16).copy()).to(dev).reshape(1, 2560), y)
    torch.cuda.synchronize()
    err = rel_l2(y.cpu().numpy()[0], W @ xf.astype(np.float64))
    print(f"manifest container 256x2560: relL2 {err:.2e}")
    assert err <= TIGHT


def test_tuned_profile_round_trip(sm, ref, dev, tmp_path):
    """tools/vq-tune's sweep on this device (gemv variants and widths, prefill
    tiles, each gated at 1e-4 against the reference candidate) over a small
    manifest directory, written as a VQPROF 1 profile with the directory's
    fingerprint and the device name; the profile is trusted only for that
    directory and device, and a plan that applies it computes the GEMV at
    the bar with the tuned kernels."""
    import torch
    conts = {"blk.0.mlp.up_proj.weight": sm.synth_container(41, 512, 2560),
             "blk.0.mlp.down_proj.weight": sm.synth_container(42, 256, 1024)}
    lines = []
    for name, c in conts.items():
        (tmp_path / f"{name}.bin").write_bytes(c.tobytes())
        h = sm.Container(c)
        lines.append(f"{name} {h.rows} {h.cols} {h.nstages} {c.nbytes} 1.0")
    (tmp_path / "manifest.txt").write_text("\n".join(lines) + "\n")
    mats = [sm.DeviceContainer(c, dev) for c in conts.values()]
    entries, rejected = sm.tune(mats, iters=3, tokens=128)
    assert sorted(e.kind for e in entries) == [0, 0, 1, 1]
    assert not rejected, rejected
    fp = sm.profile_fingerprint(tmp_path)
    gpu = sm.device_name()
    path = tmp_path / "vq-tune.profile"
    sm.profile_write(path, fp, gpu, "hip", entries)
    pf = sm.Profile(path)
    assert pf.trusted(fp, gpu) and not pf.trusted(fp ^ 1, gpu) and not pf.trusted(fp, gpu + "x")
    plan = sm.Plan()
    ys, xs, Ws = [], [], []
    for i, (m, c) in enumerate(zip(mats, conts.values())):
        e = pf.find(0, m.host.dim, m.host.nc, m.rows, m.cols, m.host.v3)
        p = pf.find(1, m.host.dim, m.host.nc, m.rows, m.cols, m.host.v3)
        print(f"{m.rows}x{m.cols}: gemv variant {e.variant} threads {e.threads} {e.rate:.0f} GB/s; "
              f"prefill variant {p.variant} tile {p.bn}x{p.bk} {p.rate:.0f} tok/s")
        assert e.variant in (0, 1, 2, 3) and p.variant in (1, 2, 3)
        xb = sm.synth_bf16(43 + i, m.cols)
        x = torch.from_numpy(xb.view(np.int16).copy()).to(dev).reshape(1, m.cols)
        y = torch.full((1, m.rows), float("nan"), device=dev)
        plan.add_vq([m], x, [y])
        ys.append(y); xs.append(xb); Ws.append(ref.decode(c).astype(np.float64))
    assert plan.apply_profile(pf, fp, gpu) == 2
    plan.run()
    torch.cuda.synchronize()
    for y, xb, W in zip(ys, xs, Ws):
        assert rel_l2(y.cpu().numpy()[0], W @ sm.bf16_to_f32(xb).astype(np.float64)) <= TIGHT
