"""GPU tests of applying a tuning profile (sparkmv_plan_apply_profile,
sparkmv_model_apply_profile), as the reference's loader applies one
(tools/vq/gpu/vq-model-gpu.cu:300-324): a runnable entry changes the kernel
that runs, a stale or non-ready entry is refused with the heuristic kept,
and a profile measured for another device changes nothing."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIGHT = 1e-5


def rel_l2(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / max(np.linalg.norm(want), 1e-300))


def _entry(sm, g, variant, threads):
    dim, nc, rows, cols, v3 = g
    return sm.ProfileEntry(kind=0, dim=dim, nc=nc, rows=rows, cols=cols, v3=v3, variant=variant, threads=threads,
                           rate=1.0)


def test_plan_profile_applies_refuses_and_keeps(sm, ref, dev, tmp_path):
    import torch
    # A: tuned to the reference's generic warp kernel (variant 1) at width 96;
    # B: a 10-bit stream tuned to the block kernel (variant 3: not ready here);
    # C: a width that is not a warp multiple. D: no entry at all.
    geoms = {"A": (4, 4096, 80, 640, 1), "B": (4, 1024, 48, 256, 1), "C": (4, 4096, 64, 512, 1),
             "D": (4, 4096, 96, 384, 1)}
    entries = [_entry(sm, geoms["A"], 1, 96), _entry(sm, geoms["B"], 3, 256), _entry(sm, geoms["C"], 2, 100)]
    gpu = sm.device_name()
    path = tmp_path / "p.profile"
    sm.profile_write(path, 7, gpu, "hip", entries)
    pf = sm.Profile(path)

    def build():
        plan, outs = sm.Plan(), {}
        for i, (k, (dim, nc, rows, cols, v3)) in enumerate(geoms.items()):
            c = sm.synth_container(60 + i, rows, cols, dim, nc, 2, v3)
            m = sm.DeviceContainer(c, dev)
            xb = sm.synth_bf16(70 + i, cols)
            x = torch.from_numpy(xb.view(np.int16).copy()).to(dev).reshape(1, cols)
            y = torch.full((1, rows), float("nan"), device=dev)
            plan.add_vq([m], x, [y])
            outs[k] = (y, ref.decode(c).astype(np.float64) @ sm.bf16_to_f32(xb).astype(np.float64))
        return plan, outs

    base, bouts = build()
    base.run()
    tuned, touts = build()
    assert tuned.apply_profile(pf, 8, gpu) == 0                    # another artifact: nothing changes
    assert "another artifact or device" in sm.last_error()
    assert tuned.apply_profile(pf, 7, gpu + " (other)") == 0       # another device: nothing changes
    assert all(tuned.op_kernel(i) == (0, 0) for i in range(4))
    assert tuned.apply_profile(pf, 7, gpu) == 1
    assert "2 entries are not runnable" in sm.last_error(), sm.last_error()
    kernels = {k: tuned.op_kernel(i) for i, k in enumerate(geoms)}
    assert kernels == {"A": (1, 128), "B": (0, 0), "C": (0, 0), "D": (0, 0)}, kernels
    tuned.run()
    torch.cuda.synchronize()
    for k in geoms:
        assert rel_l2(touts[k][0].cpu().numpy()[0], touts[k][1]) <= TIGHT, k
        same = torch.equal(touts[k][0], bouts[k][0])
        # the tuned op ran another kernel (f32 wave sums instead of MFMA
        # partials), so its bits differ; the others ran the heuristic's kernel
        assert same == (k != "A"), (k, same)


def test_model_profile(sm, ref, dev, tmp_path):
    """A model takes a trusted profile per geometry: the out projection tuned
    to the generic kernel runs it (the logits change in their last bits and
    stay at the oracle's bar), the refused entries keep the heuristic."""
    import torch
    import test_gpu_forward as tf
    m, orc = tf.build(sm, ref, dev, "q8_0", sm.X_F32)
    cfg = tf.CFG
    hid, qd = cfg["hidden"], cfg["heads"] * cfg["head_dim"]
    logits0 = torch.zeros(cfg["vocab"], device=dev)
    m.forward(3, 0, logits0)
    torch.cuda.synchronize()
    entries = [_entry(sm, (4, 4096, hid, qd, 1), 1, 256), _entry(sm, (4, 4096, cfg["intermediate"], hid, 1), 2, 33)]
    gpu = sm.device_name()
    path = tmp_path / "m.profile"
    sm.profile_write(path, 11, gpu, "hip", entries)
    pf = sm.Profile(path)
    assert m.apply_profile(pf, 11, gpu) == 1
    assert m.matvec_kernel(hid, qd) == (1, 256)
    assert m.matvec_kernel(cfg["intermediate"], hid) == (0, 0)
    m.rollback(0)
    logits = torch.zeros(cfg["vocab"], device=dev)
    m.forward(3, 0, logits)
    torch.cuda.synchronize()
    want = orc.forward(3, 0)
    assert rel_l2(logits.cpu().numpy(), want) <= 1e-5
    assert not torch.equal(logits, logits0)
