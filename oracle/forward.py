"""CPU restatement of the reference's decode forward, in numpy.

Test infrastructure only: tests/ compare the GPU forward against it
(sparkmv_model_forward); the product library never imports it.

It follows tools/vq-runtime/src/model.rs:441-591 (Model::forward) in f32
with the same helpers:

  rms_norm      model.rs:236-245  sum of squares in f64, inv rounded to f32
  sigmoid       model.rs:248-250
  gelu          model.rs:253-258  x/2 (1 + erf(x / sqrt 2)), erf in f64
  rope table    model.rs:416-428  f32 powf / cos / sin over head_dim * partial
  apply_rope    model.rs:430-438  pairs (i, i + half)
  attention     model.rs:505-557  GQA head h -> kv head h * kv_heads / heads,
                                  window [pos + 1 - sliding_window, pos] on
                                  sliding layers, sigmoid gate per head
  MLP           model.rs:566-581
  tied head     model.rs:583-590

The matrices are given as f32 arrays (the oracle's bit-exact decode of the
VQ containers or Q8_0 blocks). Sums run in numpy's order, not the Rust
dot's 8-lane order, so results agree to f32 rounding, not bit for bit.

With x_bf16 the restatement also rounds, to bf16 (nearest, ties to even),
exactly the values a matvec reads when the GPU forward runs on bf16
activations: the normed input of qkv and the head gate, the gated attention
output (the out matvec's input), the normed input of gate and up, gelu(gate)
* up (down's input) and the final norm (the head's input). The residual,
the KV cache, the gate and every sum stay f32, as on the GPU. This mode is
this build's arithmetic, not the reference's (which is f32 throughout).
"""
import math

import numpy as np
from scipy.special import erf

F32 = np.float32


def bf16_bits(x):
    """f32 -> bf16 bits, round to nearest even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint32)
    return r.astype(np.uint16)


def bf16_round(x):
    """x rounded to bf16 (nearest, ties to even), as f32 values."""
    x = np.asarray(x, F32)
    return (bf16_bits(x.ravel()).astype(np.uint32) << 16).view(F32).reshape(x.shape)


def rms_norm(x, w, eps):
    """model.rs:236-245."""
    ss = float(np.sum(x.astype(np.float64) ** 2))
    inv = F32(1.0 / math.sqrt(ss / x.size + float(F32(eps))))
    return ((x * inv) * w).astype(F32)


def sigmoid(x):
    """model.rs:248-250."""
    x = np.asarray(x, F32)
    return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)


def gelu(x):
    """model.rs:253-258: erf of x / sqrt(2) in f64, the rest in f32."""
    x = np.asarray(x, F32)
    e = erf(x.astype(np.float64) * (1.0 / math.sqrt(2.0))).astype(F32)
    return (F32(0.5) * x * (F32(1.0) + e)).astype(F32)


def rope_dim(head_dim, partial):
    """The rotated prefix of a head: (head_dim * partial) as usize, at most head_dim (model.rs:419)."""
    return min(int(F32(head_dim) * F32(partial)), head_dim)


def rope_table(pos, head_dim, theta, partial):
    """model.rs:416-428: cos and sin of pos * theta^(-2i/dim), i < dim/2, in f32."""
    dim = rope_dim(head_dim, partial)
    half = dim // 2
    i = np.arange(half)
    freq = (F32(1.0) / np.power(F32(theta), (2 * i).astype(F32) / F32(dim))).astype(F32)
    a = (F32(pos) * freq).astype(F32)
    return dim, np.cos(a).astype(F32), np.sin(a).astype(F32)


def apply_rope(x, cos, sin, dim):
    """model.rs:430-438, in place on one head's slice."""
    half = dim // 2
    a = x[:half].copy()
    b = x[half:2 * half].copy()
    x[:half] = a * cos - b * sin
    x[half:2 * half] = b * cos + a * sin


class Forward:
    """One model's decode state: cfg as sparkmv_model_cfg's fields (dict),
    layers a list of dicts of f32 arrays (in_norm, post_norm, qkv, attn_gate,
    out, gate, up, down) plus full (bool), embed [vocab, hidden] f32, norm
    [hidden] f32; x_bf16 rounds every matvec's input to bf16."""

    def __init__(self, cfg, layers, embed, norm, x_bf16=False):
        self.c = cfg
        self.q = bf16_round if x_bf16 else (lambda v: v)   # a matvec's input
        self.layers = layers
        self.embed = embed
        self.norm = norm
        kvd = cfg["kv_heads"] * cfg["head_dim"]
        self.kv_k = [np.zeros((cfg["max_ctx"], kvd), F32) for _ in layers]
        self.kv_v = [np.zeros((cfg["max_ctx"], kvd), F32) for _ in layers]
        self.capture = {}   # layer -> [max_ctx, hidden] rows of its input

    def enable_capture(self, layer_ids):
        """model.rs:322-348: every forward position then records the residual
        entering each listed layer (model.rs:466-471)."""
        self.capture = {li: np.zeros((self.c["max_ctx"], self.c["hidden"]), F32) for li in layer_ids}

    def forward(self, token, pos):
        """model.rs:441-591: the logits of token at pos."""
        c = self.c
        hd, heads, kvh_n = c["head_dim"], c["heads"], c["kv_heads"]
        qd, kvd = heads * hd, kvh_n * hd
        scale = F32(1.0) / F32(math.sqrt(F32(hd)))
        h = self.embed[token].astype(F32).copy()
        for li, L in enumerate(self.layers):
            if li in self.capture:
                self.capture[li][pos] = h
            full = bool(L["full"])
            theta = c["rope_full_theta"] if full else c["rope_slide_theta"]
            partial = c["rope_full_partial"] if full else c["rope_slide_partial"]
            dim, cos, sin = rope_table(pos, hd, theta, partial)
            xn = self.q(rms_norm(h, L["in_norm"], c["eps"]))
            qkv = (L["qkv"] @ xn).astype(F32)
            gate = (L["attn_gate"] @ xn).astype(F32)
            for hh in range(heads):
                apply_rope(qkv[hh * hd:(hh + 1) * hd], cos, sin, dim)
            for hh in range(kvh_n):
                o = qd + hh * hd
                apply_rope(qkv[o:o + hd], cos, sin, dim)
            self.kv_k[li][pos] = qkv[qd:qd + kvd]
            self.kv_v[li][pos] = qkv[qd + kvd:qd + 2 * kvd]
            start = 0 if full else max(pos + 1 - c["sliding_window"], 0)
            K = self.kv_k[li][start:pos + 1]
            V = self.kv_v[li][start:pos + 1]
            attn = np.zeros(qd, F32)
            g = sigmoid(gate)
            for hh in range(heads):
                kv = hh * kvh_n // heads
                q = qkv[hh * hd:(hh + 1) * hd]
                sc = (K[:, kv * hd:(kv + 1) * hd] @ q).astype(F32) * scale
                e = np.exp(sc - sc.max()).astype(F32)
                p = (e * (F32(1.0) / F32(e.sum(dtype=F32)))).astype(F32)
                attn[hh * hd:(hh + 1) * hd] = (p @ V[:, kv * hd:(kv + 1) * hd]).astype(F32) * g[hh]
            h = (h + (L["out"] @ self.q(attn)).astype(F32)).astype(F32)
            xn = self.q(rms_norm(h, L["post_norm"], c["eps"]))
            act = (gelu((L["gate"] @ xn).astype(F32)) * (L["up"] @ xn).astype(F32)).astype(F32)
            h = (h + (L["down"] @ self.q(act)).astype(F32)).astype(F32)
        xn = self.q(rms_norm(h, self.norm, c["eps"]))
        return (self.embed @ xn).astype(F32)
