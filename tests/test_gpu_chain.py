"""GPU tests of the decode chain (sparkmv_chain_*, sparkmv.DecodeChain): the
per-token matvec chain as one persistent launch, every op reading the
published words of the ops it depends on.

Each op is checked from what the GPU actually read (oracle/chain_check.py):
the staged input recorded by the chain equals the reference's transform of
the previous op's output (rms_norm, bf16 rounding, gelu * up), and every
matvec equals the oracle's bit-exact decode times that input in f64 within
1e-5 relative L2 (f32 accumulation; the products are exact). A second launch
must reproduce the first bit for bit: the launch reads its epoch base from
device memory, and the sums are added in a fixed order."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIGHT = 1e-5


def make_layers(sm, dev, nlayers, hid, qd, kvd, gd, ffn, nc=4096, seed0=0x5A00):
    shapes = {"q": (qd, hid), "k": (kvd, hid), "v": (kvd, hid), "g": (gd, hid), "o": (hid, qd),
              "gate": (ffn, hid), "up": (ffn, hid), "down": (hid, ffn)}
    host, devl = [], []
    for l in range(nlayers):
        hl = {n: sm.synth_container(seed0 + 16 * l + i, r, c, nc=nc) for i, (n, (r, c)) in enumerate(shapes.items())}
        host.append(hl)
        devl.append({n: sm.DeviceContainer(b, dev) for n, b in hl.items()})
    return host, devl


def build(sm, dev, nlayers, hid, qd, kvd, gd, ffn, head_rows, nc=4096, waves=None, record=True):
    import torch
    host, devl = make_layers(sm, dev, nlayers, hid, qd, kvd, gd, ffn, nc=nc)
    head = sm.synth_q8_0(0x4EAD, head_rows, hid)
    h0 = torch.from_numpy(sm.bf16_to_f32(sm.synth_bf16(0xE0, hid))).to(dev)
    dc = sm.DecodeChain(devl, torch.from_numpy(head).to(dev), head_rows, h0, record_inputs=record)
    if waves:
        dc.chain.tune(waves, 2, 16)
    return dc, host, head


def check(cc, dc, host, head, layers):
    import torch
    torch.cuda.synchronize()
    dc.chain.status()
    res = cc.check_decode_chain(dc, host, head, layers, xouts=dc.xouts)
    for k in ("q+k+v+g", "o", "gate+up", "down", "head"):
        assert res[k] <= TIGHT, (k, res)
    # rebuilt inputs: rms_norm sums may round their last bit differently
    # (f64 sums in another order), so a handful of values may differ by one
    # bf16 step; the bf16 copies and the final norm are exact functions
    assert res["q16_mismatch"] == 0, res
    assert res["x_mismatch"] <= 4, res
    assert res["act_mismatch"] <= 4, res
    assert res["hn_mismatch"] <= 2, res
    # the o and down ops read the earlier ops' bf16 outputs as they are
    for l in layers:
        assert torch.equal(dc.xouts[4 * l + 1], dc.q16[l])
        assert torch.equal(dc.xouts[4 * l + 3], dc.act[l])
    return res


@pytest.mark.parametrize("waves", [16, 12, 8])
def test_chain_small_against_oracle(sm, dev, waves):
    import chain_check as cc
    import torch
    dc, host, head = build(sm, dev, 3, 512, 1024, 256, 16, 1024, 300, waves=waves)
    dc.launch()
    res = check(cc, dc, host, head, range(3))
    first = [t.clone() for t in (dc.h, dc.act, dc.logits)]
    dc.launch()
    torch.cuda.synchronize()
    dc.chain.status()
    for a, b in zip(first, (dc.h, dc.act, dc.logits)):
        assert torch.equal(a, b), "a second launch differs"
    print(f"waves {waves}: {res}")


def test_chain_odd_rows_and_small_codebook(sm, dev):
    """Row counts that are not a multiple of 16 (ragged last tiles), a
    3000-entry codebook (12-bit indices, not a power of two), and a
    matrix of one partial tile."""
    import chain_check as cc
    dc, host, head = build(sm, dev, 2, 384, 640, 136, 6, 1152, 77, nc=3000)
    dc.launch()
    check(cc, dc, host, head, range(2))


def test_chain_shapes_of_the_real_layer(sm, dev):
    """One layer at the reference model's real shapes (hidden 2560, q 4096,
    k and v 1024, 16-row head gate, FFN 10240): the shapes the chain's
    search picks for the decode set, every row checked."""
    import chain_check as cc
    dc, host, head = build(sm, dev, 1, 2560, 4096, 1024, 16, 10240, 4096)
    dc.launch()
    res = check(cc, dc, host, head, range(1))
    shapes = [dc.chain.op_shape(i) for i in range(len(dc.chain))]
    print("shapes (S, C, unit):", shapes, res)


def _x16(sm, seed, n):
    """bf16 activations: device int16 [n], host f32 [n]"""
    import torch
    xb = sm.synth_bf16(seed, n)
    return torch.from_numpy(xb.view(np.int16).copy()).cuda(), sm.bf16_to_f32(xb)


def test_chain_addend_from_two_ops_back_after_an_op_that_does_not_wait(sm, ref, dev):
    """Ops A, B (wait=0), C (wait=1, y_add = A's y): C must add exactly what A
    wrote, although B, between them, did not wait for anything. Every read of
    a chain output waits for that output's own words, so nothing depends on
    the ops in between. Checked against the oracle's decode times x in f64,
    and the same on a second launch."""
    import torch
    import chain_check as cc
    r, c = 640, 512
    ha, hb, hc = (sm.synth_container(0x7A0 + k, rr, c) for k, rr in ((0, r), (1, c), (2, r)))
    A, B, C = (sm.DeviceContainer(h, dev) for h in (ha, hb, hc))
    x0, x0h = _x16(sm, 0x7A5, c)
    yA, yB, yC = torch.zeros(r, device=dev), torch.zeros(c, device=dev), torch.zeros(r, device=dev)
    yB16 = torch.zeros(c, dtype=torch.int16, device=dev)
    ch = sm.Chain()
    ch.add_vq([A], x0, sm.X_MODE_BF16, ys=[yA], label="A")
    ch.add_vq([B], x0, sm.X_MODE_BF16, ys=[yB], ys_bf16=[yB16], wait=False, label="B")
    ch.add_vq([C], yB16, sm.X_MODE_BF16, ys=[yC], y_add=[yA], wait=True, label="C")
    for launch in range(2):
        ch.launch()
        torch.cuda.synchronize()
        ch.status()
        wa = ref.matvec_f64(ref.decode(ha), x0h)
        wb = ref.matvec_f64(ref.decode(hb), x0h)
        assert cc.rel_l2(yA.cpu().numpy(), wa) <= TIGHT
        assert cc.rel_l2(yB.cpu().numpy(), wb) <= TIGHT
        b16 = yB16.cpu().numpy().view(np.uint16)
        assert np.array_equal(b16, cc.bf16_bits(yB.cpu().numpy())), launch
        want = yA.cpu().numpy().astype(np.float64) + ref.matvec_f64(ref.decode(hc), cc.bf16_f32(b16))
        got = yC.cpu().numpy()
        assert float(np.linalg.norm(got - want) / np.linalg.norm(want)) <= TIGHT, launch


def test_chain_refuses_partial_and_conflicting_buffers(sm, dev):
    """An input that only overlaps an earlier op's output, and an output over
    an earlier op's external input, are refused when the chain is built (no
    order holds between such accesses inside one launch)."""
    import torch
    r, c = 256, 256
    h = sm.synth_container(0x7B0, r, c)
    M = sm.DeviceContainer(h, dev)
    x0, _ = _x16(sm, 0x7B1, c)
    big = torch.zeros(2 * r, dtype=torch.int16, device=dev)
    y = torch.zeros(r, device=dev)
    ch = sm.Chain()
    ch.add_vq([M], x0, sm.X_MODE_BF16, ys=[y], ys_bf16=[big[:r]])
    ch.add_vq([M], big[8:8 + c], sm.X_MODE_BF16, ys=[torch.zeros(r, device=dev)])
    with pytest.raises(sm.SparkmvError, match="part of op 0"):
        ch.launch()
    ch2 = sm.Chain()
    ch2.add_vq([M], x0, sm.X_MODE_BF16, ys=[y])
    ch2.add_vq([M], x0, sm.X_MODE_BF16, ys=[torch.zeros(r, device=dev)], ys_bf16=[x0])
    with pytest.raises(sm.SparkmvError, match="external input"):
        ch2.launch()


def test_chain_real_shapes_repeat_and_trace(sm, dev):
    """Two layers at the real shapes, launched three times: every launch's
    outputs are bit-identical (the epoch base advances in device memory), and
    a phase trace of a launch is ordered (op start <= x arrived <= x staged <=
    units done <= epilogue issued in every workgroup)."""
    import torch
    dc, host, head = build(sm, dev, 2, 2560, 4096, 1024, 16, 10240, 512, record=False)
    dc.launch()
    torch.cuda.synchronize()
    dc.chain.status()
    first = [t.clone() for t in (dc.h, dc.hm, dc.act, dc.q16, dc.logits)]
    buf = dc.chain.trace(True)
    for _ in range(2):
        dc.launch()
        torch.cuda.synchronize()
        dc.chain.status()
        for a, b in zip(first, (dc.h, dc.hm, dc.act, dc.q16, dc.logits)):
            assert torch.equal(a, b), "a repeated launch differs"
    dc.chain.trace(False)
    tr = buf.cpu().numpy().astype(np.int64)
    t = (tr[:, :, :7] - tr[0, 0, 0] + (1 << 31)) % (1 << 32) - (1 << 31)   # signed ticks from workgroup 0's start
    # the clock reads are not ordered against each other by the compiler
    # within a few instructions: allow 2 ticks (20 ns)
    for a, b in ((0, 1), (1, 2), (2, 3), (3, 4), (4, 5), (5, 6)):
        bad = np.argwhere(t[:, :, b] < t[:, :, a] - 2)
        assert bad.size == 0, (a, b, bad[:4].tolist(), t[bad[0][0], bad[0][1]].tolist())
    # ops follow one another in every workgroup
    assert np.all(t[:, 1:, 0] >= t[:, :-1, 6] - 2)
