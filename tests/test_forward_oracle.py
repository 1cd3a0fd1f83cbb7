"""The forward oracle (oracle/forward.py, a numpy restatement of
tools/vq-runtime/src/model.rs:441-591) pinned against an independent f64
formulation built from torch's library routines: F.rms_norm, a rotation
written as complex multiplication, F.scaled_dot_product_attention with the
key/value heads repeated, F.gelu(approximate="none"), torch.sigmoid.

A plausible slip in the restatement changes the logits far beyond f32
rounding and fails here: the kv-head mapping (h * kv_heads / heads, not
h % kv_heads), the rotation's pairing (i, i + half), the rotated prefix
head_dim * partial, the sliding window's first position, the norm's weight
(w, not 1 + w), the gate's placement after the softmax.
"""
import math

import numpy as np
import pytest

import forward as fw

CFG = dict(hidden=96, layers=3, heads=4, kv_heads=2, head_dim=24, intermediate=160, vocab=50, eps=1e-6,
           sliding_window=3, rope_full_theta=5.0e6, rope_full_partial=0.25, rope_slide_theta=1.0e4,
           rope_slide_partial=1.0, max_ctx=16)
FULL = [False, True, False]


def weights(seed, cfg=CFG, full=FULL):
    rng = np.random.default_rng(seed)
    hd, heads, kvh = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    qd, kvd, hid, inter = heads * hd, kvh * hd, cfg["hidden"], cfg["intermediate"]

    def mat(r, c):
        return (rng.standard_normal((r, c)) / math.sqrt(c)).astype(np.float32)

    layers = []
    for li in range(cfg["layers"]):
        layers.append(dict(in_norm=(1 + 0.2 * rng.standard_normal(hid)).astype(np.float32),
                           post_norm=(1 + 0.2 * rng.standard_normal(hid)).astype(np.float32),
                           qkv=mat(qd + 2 * kvd, hid), attn_gate=mat(heads, hid), out=mat(hid, qd),
                           gate=mat(inter, hid), up=mat(inter, hid), down=mat(hid, inter), full=full[li]))
    embed = rng.standard_normal((cfg["vocab"], hid)).astype(np.float32)
    norm = (1 + 0.2 * rng.standard_normal(hid)).astype(np.float32)
    return layers, embed, norm


def torch_forward(cfg, layers, embed, norm, tokens, bf16=(), slip=None):
    """The same model from torch's own routines, in f64; logits per step.
    bf16: the matvec inputs to round through torch.bfloat16 ("in_norm",
    "attn", "post_norm", "act", "final"); slip: a deliberate mistake, for
    the test that shows the formulation tells it apart."""
    import torch
    import torch.nn.functional as F
    dt = torch.float64

    def R(name, x):
        return x.to(torch.float32).to(torch.bfloat16).to(dt) if name in bf16 else x
    T = lambda a: torch.tensor(np.asarray(a, np.float64), dtype=dt)
    hd, heads, kvh, hid = cfg["head_dim"], cfg["heads"], cfg["kv_heads"], cfg["hidden"]
    qd, kvd = heads * hd, kvh * hd
    E, Nf = T(embed), T(norm)
    Ls = [{k: (T(v) if k != "full" else v) for k, v in L.items()} for L in layers]
    K = [[] for _ in layers]
    V = [[] for _ in layers]
    out = []
    for pos, tok in enumerate(tokens):
        h = E[tok].clone()
        for li, L in enumerate(Ls):
            full = L["full"]
            theta = cfg["rope_full_theta"] if full else cfg["rope_slide_theta"]
            partial = cfg["rope_full_partial"] if full else cfg["rope_slide_partial"]
            dim = fw.rope_dim(hd, partial)
            half = dim // 2
            xn = R("in_norm", F.rms_norm(h, (hid,), weight=L["in_norm"], eps=cfg["eps"]))
            qkv = L["qkv"] @ xn
            g = torch.sigmoid(L["attn_gate"] @ xn)
            q = qkv[:qd].reshape(heads, hd).clone()
            k = qkv[qd:qd + kvd].reshape(kvh, hd).clone()
            v = qkv[qd + kvd:].reshape(kvh, hd).clone()
            ang = pos * torch.pow(torch.tensor(float(theta), dtype=dt), -2.0 * torch.arange(half, dtype=dt) / dim)
            rot = torch.polar(torch.ones(half, dtype=dt), ang)
            for t in (q, k):
                z = torch.complex(t[:, :half], t[:, half:2 * half]) * rot
                t[:, :half] = z.real
                t[:, half:2 * half] = z.imag
            K[li].append(k)
            V[li].append(v)
            start = 0 if full else max(pos + 1 - cfg["sliding_window"], 0)
            Ks = torch.stack(K[li][start:], 0).repeat_interleave(heads // kvh, dim=1).transpose(0, 1)
            Vs = torch.stack(V[li][start:], 0).repeat_interleave(heads // kvh, dim=1).transpose(0, 1)
            o = F.scaled_dot_product_attention(q[:, None, :], Ks.contiguous(), Vs.contiguous())[:, 0, :]
            h = h + L["out"] @ R("attn", (o * g[:, None]).reshape(-1))
            if slip == "round_residual":
                h = R("in_norm", h)
            xn = R("post_norm", F.rms_norm(h, (hid,), weight=L["post_norm"], eps=cfg["eps"]))
            h = h + L["down"] @ R("act", F.gelu(L["gate"] @ xn, approximate="none") * (L["up"] @ xn))
        out.append((E @ R("final", F.rms_norm(h, (hid,), weight=Nf, eps=cfg["eps"]))).numpy())
    return out


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_forward_oracle_against_torch_routines():
    layers, embed, norm = weights(1)
    tokens = [3, 17, 41, 8, 8, 29, 0]          # past the 3-position window
    f = fw.Forward(CFG, layers, embed, norm)
    got = [f.forward(t, p) for p, t in enumerate(tokens)]
    want = torch_forward(CFG, layers, embed, norm, tokens)
    for p, (g, w) in enumerate(zip(got, want)):
        err = rel_l2(g, w)
        print(f"pos {p}: relL2 {err:.2e}")
        assert err <= 2e-5


@pytest.mark.parametrize("slip", ["kv_mod", "window", "norm_1pw", "rope_interleaved"])
def test_torch_formulation_tells_slips_apart(slip):
    """Each slip, planted in a copy of the oracle, moves the logits far past
    the tolerance above, so the agreement is not an accident of the data."""
    layers, embed, norm = weights(2)
    tokens = [3, 17, 41, 8, 29]
    want = torch_forward(CFG, layers, embed, norm, tokens)

    class Slipped(fw.Forward):
        pass

    saved = (fw.rms_norm, fw.apply_rope)
    cfg = dict(CFG)
    try:
        if slip == "norm_1pw":
            fw.rms_norm = lambda x, w, eps: saved[0](x, (1 + w).astype(np.float32), eps)
        elif slip == "rope_interleaved":
            def inter(x, cos, sin, dim):
                a, b = x[0:dim:2].copy(), x[1:dim:2].copy()
                x[0:dim:2] = a * cos - b * sin
                x[1:dim:2] = b * cos + a * sin
            fw.apply_rope = inter
        elif slip == "window":
            cfg["sliding_window"] = CFG["sliding_window"] + 1
        f = Slipped(cfg, layers, embed, norm)
        if slip == "kv_mod":
            heads, kvh = CFG["heads"], CFG["kv_heads"]
            # heads 0..3 -> kv 0,1,0,1 instead of 0,0,1,1: swap the kv heads of heads 1 and 2 by
            # swapping the q heads' rows of every layer's qkv matrix
            for L in f.layers:
                hd = CFG["head_dim"]
                L = L
                q = L["qkv"].copy()
                q[hd:2 * hd], q[2 * hd:3 * hd] = L["qkv"][2 * hd:3 * hd], L["qkv"][hd:2 * hd]
                L["qkv"] = q
                gt = L["attn_gate"].copy()
                gt[[1, 2]] = gt[[2, 1]]
                L["attn_gate"] = gt
                o = L["out"].copy()
                o[:, hd:2 * hd], o[:, 2 * hd:3 * hd] = L["out"][:, 2 * hd:3 * hd], L["out"][:, hd:2 * hd]
                L["out"] = o
        got = [f.forward(t, p) for p, t in enumerate(tokens)]
    finally:
        fw.rms_norm, fw.apply_rope = saved
    worst = max(rel_l2(g, w) for g, w in zip(got, want))
    print(f"{slip}: worst relL2 {worst:.2e}")
    assert worst > 1e-3


def test_helpers_against_closed_forms():
    import torch
    import torch.nn.functional as F
    x = np.linspace(-6, 6, 97).astype(np.float32)
    g = F.gelu(torch.tensor(x, dtype=torch.float64), approximate="none").numpy()
    assert np.max(np.abs(fw.gelu(x) - g)) <= 2e-6
    assert np.max(np.abs(fw.sigmoid(x) - torch.sigmoid(torch.tensor(x, dtype=torch.float64)).numpy())) <= 2e-7
    # position 0 rotates by nothing; a rotation keeps each pair's length
    v = np.random.default_rng(3).standard_normal(24).astype(np.float32)
    dim, c, s = fw.rope_table(0, 24, 1e4, 1.0)
    w = v.copy()
    fw.apply_rope(w, c, s, dim)
    assert np.array_equal(w, v)
    dim, c, s = fw.rope_table(7, 24, 1e4, 1.0)
    w = v.copy()
    fw.apply_rope(w, c, s, dim)
    h = dim // 2
    assert np.allclose(w[:h] ** 2 + w[h:dim] ** 2, v[:h] ** 2 + v[h:dim] ** 2, rtol=1e-5)
    # partial rotary: 24 * 0.25 = 6 rotated, the rest untouched
    dim, c, s = fw.rope_table(5, 24, 5e6, 0.25)
    assert dim == 6
    w = v.copy()
    fw.apply_rope(w, c, s, dim)
    assert np.array_equal(w[6:], v[6:])
    # rms_norm of a constant vector is the weight times its sign
    assert np.allclose(fw.rms_norm(np.full(8, -3.0, np.float32), np.arange(8, dtype=np.float32), 0.0),
                       -np.arange(8, dtype=np.float32), rtol=1e-6)


def test_single_position_attention_is_gated_value():
    """At position 0 every head's softmax is one weight on one value: the
    attention output is V[0] times the head's gate, whatever q and K are."""
    layers, embed, norm = weights(4)
    cfg = dict(CFG, layers=1)
    f = fw.Forward(cfg, layers[:1], embed, norm)
    f.forward(5, 0)
    L = layers[0]
    xn = fw.rms_norm(embed[5], L["in_norm"], cfg["eps"])
    qkv = L["qkv"] @ xn
    hd, heads, kvh = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    v = qkv[heads * hd + kvh * hd:]
    assert np.array_equal(f.kv_v[0][0], v.astype(np.float32))


BF16_POINTS = ("in_norm", "attn", "post_norm", "act", "final")


def test_bf16_oracle_against_torch_routines():
    """The oracle's bf16 mode (every matvec input rounded to bf16, nothing
    else) against the torch f64 formulation with the same five inputs cast
    through torch.bfloat16. The two round values computed in f32 and in
    f64, so an element near a rounding boundary may land on the other bf16
    neighbour; the bar allows a few such (5e-4), while each wrong placement
    below moves the logits by more than four times the bar."""
    layers, embed, norm = weights(2)
    tokens = [3, 17, 41, 8, 8, 29, 0]
    f = fw.Forward(CFG, layers, embed, norm, x_bf16=True)
    got = [f.forward(t, p) for p, t in enumerate(tokens)]
    want = torch_forward(CFG, layers, embed, norm, tokens, bf16=BF16_POINTS)
    worst = max(rel_l2(g, w) for g, w in zip(got, want))
    print(f"bf16 oracle vs torch bf16 formulation: worst relL2 {worst:.2e}")
    assert worst <= 5e-4
    wrong = {"no rounding": torch_forward(CFG, layers, embed, norm, tokens),
             "attn not rounded": torch_forward(CFG, layers, embed, norm, tokens,
                                               bf16=tuple(p for p in BF16_POINTS if p != "attn")),
             "act not rounded": torch_forward(CFG, layers, embed, norm, tokens,
                                              bf16=tuple(p for p in BF16_POINTS if p != "act")),
             "residual rounded too": torch_forward(CFG, layers, embed, norm, tokens, bf16=BF16_POINTS,
                                                   slip="round_residual")}
    for name, w in wrong.items():
        d = max(rel_l2(g, ww) for g, ww in zip(got, w))
        print(f"  {name}: relL2 {d:.2e}")
        assert d > 2e-3, name
