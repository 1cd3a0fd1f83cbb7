"""Pins the oracle (oracle/sparkref.c) before anything is checked against it.

Sources of truth used here, none of them the oracle's own formulas:
  * golden fixtures: matrices dumped by the reference's C decoder
    (tools/vq/decode.c) and its refusals, written by tests/golden/make_golden.py;
  * numpy's IEEE half -> single conversion, exhaustively;
  * numpy float32 sequential accumulation (np.add.accumulate) for the
    fused dot_row order;
  * hand-computed known answers for the 8-lane dot and for the Q6_K / Q8_0
    block layouts (the reference holds no code for those: its k-quant
    kernels come from ggml, which it does not vendor);
  * brute force on tiny inputs (pack known indices, read them back).
"""
import glob
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN

CASES = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(CASES) >= 8


def test_f16_exhaustive(ref):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([ref.f16(int(v)) for v in h], dtype=np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), np.nonzero(~same)[0][:10]


@pytest.mark.parametrize("path", CASES, ids=[os.path.basename(c)[:-4] for c in CASES])
def test_decode_matches_reference_decoder(ref, path):
    g = load(path)
    got = ref.decode(g["container"])
    assert got.shape == g["decoded"].shape
    assert np.array_equal(got.view(np.uint32), g["decoded"].view(np.uint32)), "decode differs from tools/vq/decode.c"


@pytest.mark.parametrize("path", CASES, ids=[os.path.basename(c)[:-4] for c in CASES])
def test_refusals(ref, path):
    """Every damaged variant the reference's C decoder refused is refused; the
    Rust reader (lib.rs:277-296) is stricter on a stage whose header
    disagrees with the container, and the oracle follows the Rust reader."""
    g = load(path)
    data = g["container"]
    variants = {
        "truncated": data[:-1],
        "payload_count": _flip(data, 24, 0x01),
        "stage_dim": _put16(data, 36, 2 * int(g["geometry"][3])),
        "magic": _put8(data, 0, ord("X")),
        "nc16384": _put16(_put16(data, 6, 16384), 38, 16384),
    }
    for name, refused in zip(g["damaged_names"], g["damaged_refused"]):
        ok, msg, _ = ref.container_check(variants[str(name)])
        assert not ok, f"{name} accepted"
        if str(name) == "nc16384":
            assert "13 index bits" in msg
        if not bool(refused):
            assert str(name) == "stage_dim"


def _flip(d, o, m):
    e = d.copy()
    e[o] ^= m
    return e


def _put8(d, o, v):
    e = d.copy()
    e[o] = v
    return e


def _put16(d, o, v):
    e = d.copy()
    e[o:o + 2] = np.frombuffer(np.uint16(v).tobytes(), np.uint8)
    return e


@pytest.mark.parametrize("v3,nc,rows,cols,dim", [(1, 4096, 3, 40, 4), (1, 8192, 2, 72, 4), (1, 1024, 4, 28, 4),
                                                 (1, 300, 2, 20, 2), (0, 256, 3, 16, 4), (0, 512, 5, 12, 4),
                                                 (0, 1000, 2, 36, 4)])
def test_pack_then_index_roundtrip(ref, v3, nc, rows, cols, dim):
    rng = np.random.default_rng(nc + rows)
    idx = rng.integers(0, nc, size=rows * (cols // dim), dtype=np.uint32)
    cb = rng.integers(0, 0x7bff, size=nc * dim).astype(np.uint16)
    gains = np.full(rows, 0x3C00, dtype=np.uint16)
    p = ref.pack(v3, cb, idx, gains, rows, cols, dim, nc)
    assert p.nbytes == ref.stage_bytes(v3, rows, cols, dim, nc)
    assert np.array_equal(ref.stage_indices(p).ravel(), idx)


def test_v3_stage_bytes_examples(ref):
    # 10240 x 2560, dim 4, nc 4096: 24 + 32768 + 20480 + 10240 * 960
    assert ref.stage_bytes(1, 10240, 2560, 4, 4096) == 9883672
    # nc 8192 carries a 1-bit plane of ceil(640 / 8) bytes per row
    assert ref.stage_bytes(1, 16, 2560, 4, 8192) == 24 + 65536 + 32 + 16 * (960 + 80)
    # DQVQ, 9-bit, guard byte
    assert ref.stage_bytes(0, 3, 16, 4, 512) == 16 + 512 * 8 + 6 + (12 * 9 + 7) // 8 + 1


def test_dot_short_is_sequential(ref):
    a = np.array([1e8, 1, -1e8, 1, 1], dtype=np.float32)
    assert ref.dot(a, np.ones(5, np.float32)) == 2.0


def test_dot_eight_lanes_then_pairwise(ref):
    # lane 0 holds 1e8 and -1e8 (cancel), lanes 1..7 hold 1: 8-lane sum is 7,
    # a sequential sum would lose every 1 against 1e8 and give 0.
    a = np.zeros(16, np.float32)
    a[0], a[8] = 1e8, -1e8
    a[1:8] = 1
    assert ref.dot(a, np.ones(16, np.float32)) == 7.0
    # the scalar tail is added in order after the lanes combine: 7 + 1e8 rounds
    # to 1e8 + 8 (f32 spacing 8 there), minus 1e8 is 8, plus 3 is 11
    b = np.concatenate([a, np.array([1e8, -1e8, 3], np.float32)])
    assert ref.dot(b, np.ones(19, np.float32)) == 11.0


def test_dot_exact_integers(ref):
    rng = np.random.default_rng(5)
    for n in (1, 7, 8, 9, 64, 1003):
        a = rng.integers(-50, 50, n).astype(np.float32)
        b = rng.integers(-50, 50, n).astype(np.float32)
        assert ref.dot(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def test_dot_row_is_sequential_f32(ref):
    """One stage with unit gains: dot_row must equal numpy's sequential float32
    accumulation of W[r, k] * x[k] (lib.rs:215-227)."""
    rows, cols, nc = 6, 128, 256
    rng = np.random.default_rng(9)
    cbf = (rng.standard_normal(nc * 4) * 0.02).astype(np.float16)
    idx = rng.integers(0, nc, rows * cols // 4, dtype=np.uint32)
    stage = ref.pack(1, cbf.view(np.uint16), idx, np.full(rows, 0x3C00, np.uint16), rows, cols, 4, nc)
    cont = _container(stage, rows, cols, 4, nc, 1)
    x = rng.standard_normal(cols).astype(np.float32)
    y = ref.gemv_fused(cont, x, 1)
    W = cbf.astype(np.float32).reshape(nc, 4)[idx].reshape(rows, cols)
    for r in range(rows):
        want = np.add.accumulate((W[r] * x).astype(np.float32), dtype=np.float32)[-1]
        assert y[r] == want


def _container(stage, rows, cols, dim, nc, ns):
    hdr = np.zeros(32, np.uint8)
    hdr[:4] = np.frombuffer(b"RQVQ", np.uint8)
    hdr[4:6] = np.frombuffer(np.uint16(dim).tobytes(), np.uint8)
    hdr[6:8] = np.frombuffer(np.uint16(nc).tobytes(), np.uint8)
    hdr[8:10] = np.frombuffer(np.uint16(ns).tobytes(), np.uint8)
    hdr[12:16] = np.frombuffer(np.uint32(rows).tobytes(), np.uint8)
    hdr[16:20] = np.frombuffer(np.uint32(cols).tobytes(), np.uint8)
    hdr[24:32] = np.frombuffer(np.uint64(stage.nbytes * ns).tobytes(), np.uint8)
    return np.concatenate([hdr] + [stage] * ns)


@pytest.mark.parametrize("path", CASES[:3], ids=[os.path.basename(c)[:-4] for c in CASES[:3]])
def test_matvec_close_to_f64(ref, path):
    g = load(path)
    W = g["decoded"]
    x = np.random.default_rng(3).standard_normal(W.shape[1]).astype(np.float32)
    y = ref.matvec(W, x)
    y64 = W.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(ref.matvec_f64(W, x), y64, rtol=1e-12, atol=1e-12)
    assert np.linalg.norm(y - y64) <= 1e-6 * np.linalg.norm(y64)
    yf = ref.gemv_fused(g["container"], x)
    assert np.linalg.norm(yf - y64) <= 1e-5 * np.linalg.norm(y64)


def test_q8_0_known_answer(ref):
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(0x3400).tobytes(), np.uint8)   # d = 0.25
    qs = np.array([-128, -1, 0, 1, 127, 5] + [0] * 26, dtype=np.int8)
    blk[2:] = qs.view(np.uint8)
    neg = blk.copy()
    neg[0:2] = np.frombuffer(np.uint16(0xC000).tobytes(), np.uint8)   # d = -2
    w = ref.q8_0_dequant(np.concatenate([blk, neg]), 1, 64)[0]
    assert list(w[:6]) == [-32.0, -0.25, 0.0, 0.25, 31.75, 1.25]
    assert list(w[32:38]) == [256.0, 2.0, -0.0, -2.0, -254.0, -10.0]
    assert not w[6:32].any()


def _q6k_block(d_bits, scales):
    blk = np.zeros(210, np.uint8)
    blk[192:208] = np.array(scales, np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    return blk


def test_q6k_known_answer_uniform(ref):
    w = ref.q6k_dequant(_q6k_block(0x3C00, [1] * 16), 1, 256)[0]       # d = 1, q = 0 -> -32
    assert (w == -32.0).all()


def test_q6k_known_answer_layout(ref):
    """Hand-worked block: d = 0.5, scales[s] = s - 8, and six bytes set."""
    blk = _q6k_block(0x3800, [s - 8 for s in range(16)])
    blk[5], blk[37] = 0x3A, 0xC7           # ql, half 0
    blk[128 + 5] = 0xE4                    # qh, half 0, l = 5
    blk[64 + 40] = 0x5F                    # ql, half 1, l = 8, odd quarters
    blk[128 + 32 + 8] = 0x48               # qh, half 1, l = 8
    w = ref.q6k_dequant(blk, 1, 256)[0]
    want = np.zeros(256, np.float32)
    # every weight with q = 0 is 0.5 * scale * -32 = -16 * scale
    base_scale = {(0, 0, 0): -8, (0, 1, 0): -6, (0, 2, 0): -4, (0, 3, 0): -2,
                  (0, 0, 1): -7, (0, 1, 1): -5, (0, 2, 1): -3, (0, 3, 1): -1,
                  (1, 0, 0): 0, (1, 1, 0): 2, (1, 2, 0): 4, (1, 3, 0): 6,
                  (1, 0, 1): 1, (1, 1, 1): 3, (1, 2, 1): 5, (1, 3, 1): 7}
    for (h, k, half16), sc in base_scale.items():
        lo = 128 * h + 32 * k + 16 * half16
        want[lo:lo + 16] = -16.0 * sc
    # hand-decoded exceptions
    want[5], want[37], want[69], want[101] = 88.0, 27.0, -6.0, -28.0
    want[168], want[232] = 15.0, -33.0
    assert np.array_equal(w, want), np.nonzero(w != want)[0]


def test_q6k_matvec_close_to_f64(ref):
    rng = np.random.default_rng(2)
    rows, cols = 8, 512
    blocks = rng.integers(0, 256, rows * (cols // 256) * 210).astype(np.uint8)
    for b in range(rows * 2):   # keep d small and finite
        blocks[b * 210 + 208:b * 210 + 210] = np.frombuffer(np.float16(rng.uniform(1e-4, 1e-3)).tobytes(), np.uint8)
    W = ref.q6k_dequant(blocks, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = ref.q6k_matvec(blocks, rows, cols, x)
    y64 = W.astype(np.float64) @ x
    assert np.linalg.norm(y - y64) <= 1e-6 * np.linalg.norm(y64)


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref", "decode")),
                    reason="reference decoder not built (reference tree absent)")
def test_live_reference_decoder(ref, sm, tmp_path):
    """Where the reference tree exists, also decode a fresh container live."""
    data = sm.synth_container(99, 21, 192, 4, 4096, 2, 1)
    src, out = tmp_path / "c.bin", tmp_path / "w.f32"
    data.tofile(src)
    subprocess.run([ref.REF_DECODE, "dump", str(src), str(out)], check=True, stdout=subprocess.DEVNULL)
    want = np.fromfile(out, np.float32).reshape(21, 192)
    assert np.array_equal(ref.decode(data).view(np.uint32), want.view(np.uint32))


def _torch_bf16_bits(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def test_bf16_bits_matches_torch_rounding():
    """The oracle's f32 -> bf16 rounding (chain_check.bf16_bits: round to
    nearest, ties to even; NaN stays NaN) against torch's conversion, which
    rounds the same way. Covers random values over the whole exponent range,
    exact ties with an even and with an odd kept bit (both signs), values one
    ulp either side of a tie, subnormals, the largest finite values (which
    round to infinity), zeros and infinities, bit for bit; NaN inputs give
    NaN in both. A mistake in the tie rule, the carry into the exponent or
    the sign fails here."""
    import chain_check as cc
    rng = np.random.default_rng(0xBF16)
    u = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    finite = u[(u & 0x7F800000) != 0x7F800000]
    hi = rng.integers(0, 1 << 16, 4096, dtype=np.uint64).astype(np.uint32) << 16
    hi = hi[(hi & 0x7F800000) != 0x7F800000]
    ties = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001])            # tie, just below, just above
    sub = np.concatenate([np.arange(1, 1 << 12, dtype=np.uint32), np.uint32(0x007FFFFF) - np.arange(4096, dtype=np.uint32),
                          np.uint32(0x00008000) + np.arange(-3, 4, dtype=np.int64).astype(np.uint32)])
    edge = np.array([0x00000000, 0x80000000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x7F800000, 0xFF800000,
                     0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000, 0x00008000, 0x00018000], dtype=np.uint32)
    vals = np.concatenate([finite, ties, sub, sub | 0x80000000, edge]).view(np.float32)
    got = cc.bf16_bits(vals)
    want = _torch_bf16_bits(vals)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(int(vals.view(np.uint32)[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
    # ties go to the even neighbour: 1 + 2^-8 (kept bit even) stays 1, 1 + 3 * 2^-8 (odd) rounds up
    assert cc.bf16_bits(np.float32([1 + 2 ** -8, 1 + 3 * 2 ** -8])).tolist() == [0x3F80, 0x3F82]
    # the largest finite f32 rounds up to infinity, as torch's does
    assert int(cc.bf16_bits(np.float32([3.4028235e38]))[0]) == 0x7F80
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FFFFFFF, 0xFF800001], dtype=np.uint32).view(np.float32)
    nb = cc.bf16_bits(nans)
    assert np.all((nb & 0x7F80) == 0x7F80) and np.all((nb & 0x7F) != 0), [hex(int(v)) for v in nb]
    assert int(nb[0]) == 0x7FC0
    tn = _torch_bf16_bits(nans)   # torch's NaN bits differ by path (0x7FC0 or 0xFFFF): NaN either way
    assert np.all((tn & 0x7F80) == 0x7F80) and np.all((tn & 0x7F) != 0)
