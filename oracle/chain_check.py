"""Oracle checks of a decode chain's outputs (sparkmv.DecodeChain).

Test infrastructure only: tests/ and bench.py's output check compare against
it; the product library never imports it.

Every op of the chain is checked from what the GPU actually read: the
inputs are rebuilt from the chain's own intermediate buffers with the
reference's transforms (rms_norm model.rs:236-245, gelu model.rs:253-258,
bf16 rounding to nearest even as the activations are stored), and each
matvec is compared with the oracle's bit-exact decode of the container
(lib.rs:197-211) times that input in f64 — the reference's own gate method
(tools/vq/gpu/decode-gpu.c:469-484). The Q8_0 head is compared on every row
with the closed-form dequant (ggml block layout, 34 B per 32 weights) and the
runtime's f32 dot (model.rs:209-234).
"""
import numpy as np

import forward as fw
import sparkref as ref

F32 = np.float32


bf16_bits = fw.bf16_bits   # f32 -> bf16 bits, round to nearest even; NaN -> quiet NaN


def bf16_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def rel_l2(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


def norm_bf16(h, eps):
    """bf16(rms_norm(h)) with weight 1, as the chain's staging computes it."""
    return bf16_bits(fw.rms_norm(np.asarray(h, F32), np.ones(h.size, F32), eps))


def gelu_mul_bf16(gate, up):
    return bf16_bits((fw.gelu(gate) * np.asarray(up, F32)).astype(F32))


def _u16(t):
    return t.detach().cpu().numpy().view(np.uint16)


def _f32(t):
    return t.detach().cpu().numpy().astype(F32)


def check_decode_chain(dc, host_layers, head_blocks, layers, xouts=None):
    """Check layers `layers` of a DecodeChain and every row of its head.

    host_layers[l][name] are the containers' host bytes (DECODE_MATS names).
    xouts, when given, is the list of per-op staged-x tensors (x_out), and
    the rebuilt inputs are also compared with them. Returns a dict: per op
    kind the largest relative L2 error of the matvec, and per rebuilt input
    the number of bf16 values that differ from the GPU's."""
    out = {"q+k+v+g": 0.0, "o": 0.0, "gate+up": 0.0, "down": 0.0, "head": 0.0,
           "x_mismatch": 0, "act_mismatch": 0, "q16_mismatch": 0, "hn_mismatch": 0}
    eps = dc.eps

    def mv(name, l, x):
        W = ref.decode(host_layers[l][name])
        return ref.matvec_f64(W, np.asarray(x, F32))

    for l in layers:
        h = _f32(dc.h[l])
        hm = _f32(dc.hm[l])
        h1 = _f32(dc.h[l + 1])
        xa = norm_bf16(h, eps)
        if xouts is not None:
            out["x_mismatch"] += int(np.sum(_u16(xouts[4 * l]) != xa))
        xa_f = bf16_f32(xa)
        for name, buf in (("q", dc.q), ("k", dc.k), ("v", dc.v), ("g", dc.g)):
            out["q+k+v+g"] = max(out["q+k+v+g"], rel_l2(_f32(buf[l]), mv(name, l, xa_f)))
        q16 = _u16(dc.q16[l])
        out["q16_mismatch"] += int(np.sum(q16 != bf16_bits(_f32(dc.q[l]))))
        y = mv("o", l, bf16_f32(q16))
        out["o"] = max(out["o"], float(np.linalg.norm(hm - (h.astype(np.float64) + y)) / max(np.linalg.norm(y), 1e-30)))
        xc = norm_bf16(hm, eps)
        if xouts is not None:
            out["x_mismatch"] += int(np.sum(_u16(xouts[4 * l + 2]) != xc))
        xc_f = bf16_f32(xc)
        gate, up = _f32(dc.gate[l]), _f32(dc.up[l])
        out["gate+up"] = max(out["gate+up"], rel_l2(gate, mv("gate", l, xc_f)), rel_l2(up, mv("up", l, xc_f)))
        act = _u16(dc.act[l])
        out["act_mismatch"] += int(np.sum(act != gelu_mul_bf16(gate, up)))
        y = mv("down", l, bf16_f32(act))
        out["down"] = max(out["down"],
                          float(np.linalg.norm(h1 - (hm.astype(np.float64) + y)) / max(np.linalg.norm(y), 1e-30)))
    hL = _f32(dc.h[dc.L])
    hn = _u16(dc.hn)
    out["hn_mismatch"] = int(np.sum(hn != norm_bf16(hL, eps)))
    want = ref.q8_0_matvec(np.asarray(head_blocks), dc.head_rows, dc.hidden, bf16_f32(hn))
    out["head"] = rel_l2(_f32(dc.logits), want)
    return out


def worst_matvec(res):
    return max(res[k] for k in ("q+k+v+g", "o", "gate+up", "down", "head"))



def check_decode_set(ds, layer_mats, layers):
    """The decode-set plan's outputs (bench.py's DecodeSet): every row and
    column of the kept layers' matvecs against the oracle's decode times x in
    f64, and every head row against the oracle's closed-form Q8_0 dequant
    and the runtime's f32 dot (model.rs:209-234). Returns the
    largest relative L2 error per launch group (q+k+v+g, o, gate+up, down,
    head), over all columns."""
    res = {}
    group_names = {}
    for i, (name, _, _, grp) in enumerate(layer_mats):
        group_names.setdefault(grp, []).append(name)
    for l in layers:
        for i, y in ds.ys[l]:
            name, rows, cols, grp = layer_mats[i]
            W = ref.decode(ds.hosts[l][i]).astype(np.float64)
            X = ds.xs[cols][1].astype(np.float64)
            want = X @ W.T                       # [ncol, rows]
            got = _f32(y)[:, :rows]
            key = "+".join(group_names[grp])
            res[key] = max(res.get(key, 0.0), rel_l2(got, want))
    x = ds.xs[layer_mats[0][2]][1]
    got = _f32(ds.logits)
    worst = 0.0
    for n in range(ds.ncol):
        want = ref.q8_0_matvec(ds.head, ds.head_rows, x.shape[1], x[n])
        worst = max(worst, rel_l2(got[n], want))
    res["head"] = worst
    return res


def check_kquant_set(groups, xs, head_blocks, head_rows, logits):
    """The Q6_K decode set's outputs (bench.py --workload decode-set-q6k):
    groups is a list of (key, Q6_K blocks of the stacked rows, rows, cols, y
    tensor); each y against the oracle's closed-form Q6_K dequant (ggml
    layout, 210 B per 256 weights) times x in f64, and every head row
    against the closed-form Q8_0 dot. xs[cols] is the f32 value of the bf16
    x each launch read. Returns the largest relative L2 error per key and
    for the head."""
    res = {}
    for key, blocks, rows, cols, y in groups:
        W = ref.q6k_dequant(blocks, rows, cols)
        want = ref.matvec_f64(W, np.asarray(xs[cols], F32))
        res[key] = max(res.get(key, 0.0), rel_l2(_f32(y)[:rows], want))
    x = np.asarray(xs[head_blocks.size // (head_rows * 34) * 32], F32)
    res["head"] = rel_l2(_f32(logits), ref.q8_0_matvec(np.asarray(head_blocks), head_rows, x.size, x))
    return res
