"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, and its host-side code (container validation, synthetic packing)
agrees with the oracle. No GPU call is made here."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

from conftest import GOLDEN, ROOT

HEADER = os.path.join(ROOT, "include", "sparkmv.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b((?:vqg|sparkmv)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_reference_abi():
    names = declared_functions()
    for ref_name in ["vqg_decode_error", "vqg_device_name", "vqg_driver_version", "vqg_gemv_ready", "vqg_gemv_t",
                     "vqg_gemv", "vqg_gemv_launch_t", "vqg_gemv_launch", "vqg_dequant", "vqg_row_dequant",
                     "vqg_prefill_ready", "vqg_prefill_cfg_count", "vqg_prefill_cfg", "vqg_prefill_cfg_ready",
                     "vqg_prefill", "vqg_prefill_tile", "vqg_prefill_launch", "vqg_prefill_launch_tile",
                     "vqg_gemv_f32"]:
        assert ref_name in names


def test_library_exports_every_declared_symbol(sm):
    L = ctypes.CDLL(sm.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol(sm):
    assert set(declared_functions()) <= set(sm.SIGNATURES)


def test_readiness_rules(sm):
    """vqg_gemv_ready is the reference's truth table (decode-gpu.cu:788-797):
    3 when the DQV3 block kernel's preconditions hold (v3, a 12-bit main
    stream, whole 32-index groups, 4-byte aligned streams; :62-64), 2 for
    dim 4, 1 always, 0 when the codebook fits the shared-codebook kernel
    (160 KB of LDS here). Geometries every launch refuses (a DQV3 codebook
    past 13 bits, cols not a multiple of dim) are ready for no variant."""
    L = sm.lib()
    table = [   # (dim, nc, rows, cols, v3) -> ready for variants 0, 1, 2, 3
        ((4, 4096, 10240, 2560, 1), (1, 1, 1, 1)),
        ((4, 8192, 16, 2560, 1), (1, 1, 1, 1)),      # 13-bit: 12-bit stream + plane
        ((4, 1024, 64, 2560, 1), (1, 1, 1, 0)),      # 10-bit stream
        ((8, 4096, 64, 2560, 1), (1, 1, 0, 1)),      # dim 8: block path yes, dim-4 path no
        ((4, 4096, 64, 2560, 0), (1, 1, 1, 0)),      # DQVQ
        ((4, 4096, 64, 2500, 1), (1, 1, 1, 0)),      # 625 indices per row: not whole 32-index groups
        ((4, 4096, 37, 12, 1), (1, 1, 1, 0)),
        ((2, 65536, 8, 256, 0), (0, 1, 0, 0)),       # 256 KB codebook: not the shared-codebook kernel
        ((4, 16384, 64, 2560, 0), (1, 1, 1, 0)),     # DQVQ has no 13-bit limit; 128 KB codebook fits
        ((4, 16384, 64, 2560, 1), (0, 0, 0, 0)),     # DQV3 is at most 13 bits
        ((4, 4096, 1, 10, 1), (0, 0, 0, 0)),         # cols not a multiple of dim
    ]
    for geom, want in table:
        got = tuple(L.vqg_gemv_ready(*geom, v) for v in range(4))
        assert got == want, (geom, got, want)
    assert L.vqg_gemv_ready(4, 4096, 64, 2560, 1, 4) == 0


def test_prefill_readiness_rules(sm):
    """The reference's prefill rules (decode-gpu.cu:527-558, :995-1025): its
    tuner's three tiles, tiled variants 1 and 2 for DQV3 dim 4/8 streams of
    at least 12 bits whose columns split into 64-column rounds, the legacy
    variant 3 and the picker 0 for anything."""
    L = sm.lib()
    assert L.vqg_prefill_cfg_count() == 3
    tiles = []
    for i in range(3):
        bn, bk = ctypes.c_int(), ctypes.c_int()
        assert L.vqg_prefill_cfg(i, ctypes.byref(bn), ctypes.byref(bk)) == 0
        tiles.append((bn.value, bk.value))
    assert tiles == [(64, 64), (128, 64), (256, 64)]
    assert L.vqg_prefill_cfg(3, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int())) == -1
    for v in (0, 1, 2, 3):
        assert L.vqg_prefill_ready(4, 4096, 10240, 2560, 1, v) == 1
        assert L.vqg_prefill_ready(4, 8192, 2560, 10240, 1, v) == 1
    for v in (1, 2):
        assert L.vqg_prefill_ready(4, 4096, 64, 2560, 0, v) == 0    # DQVQ: legacy only
        assert L.vqg_prefill_ready(4, 1024, 64, 2560, 1, v) == 0    # 10-bit stream
        assert L.vqg_prefill_ready(4, 4096, 64, 2592, 1, v) == 0    # 2592 columns: not whole 64-column rounds
        assert L.vqg_prefill_ready(8, 4096, 64, 2560, 1, v) == 1    # dim 8 runs (one thread per output here)
        assert L.vqg_prefill_cfg_ready(4, 4096, 64, 2560, 1, 128, 64, v) == 1
        assert L.vqg_prefill_cfg_ready(4, 4096, 64, 2560, 1, 128, 48, v) == 0   # 2560 % 48 != 0
    assert L.vqg_prefill_ready(4, 4096, 64, 2560, 0, 3) == 1
    assert L.vqg_prefill_cfg_ready(4, 4096, 64, 2560, 0, 1, 1, 3) == 1
    assert L.vqg_prefill_ready(4, 4096, 64, 2560, 1, 4) == 0
    assert L.vqg_prefill_cfg_ready(4, 4096, 64, 2560, 1, 128, 64, 0) == 0


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_container_open_agrees_with_oracle(sm, ref, path):
    with np.load(path, allow_pickle=False) as z:
        data = z["container"]
        seed, rows, cols, dim, nc, ns, v3 = [int(v) for v in z["geometry"]]
    c = sm.Container(data)
    assert (c.rows, c.cols, c.dim, c.nc, c.nstages, c.v3) == (rows, cols, dim, nc, ns, v3)
    ok, msg, info = ref.container_check(data)
    assert ok and info["stride"] == c.stage_bytes
    variants = [data[:-1], np.concatenate([data, np.zeros(1, np.uint8)])]
    e = data.copy(); e[24] ^= 1; variants.append(e)
    f = data.copy(); f[36:38] = np.frombuffer(np.uint16(2 * dim).tobytes(), np.uint8); variants.append(f)
    g = data.copy(); g[0] = 0; variants.append(g)
    h = data.copy(); h[4:6] = 0; variants.append(h)
    i = data.copy(); i[6:8] = np.frombuffer(np.uint16(16384).tobytes(), np.uint8)
    i[38:40] = np.frombuffer(np.uint16(16384).tobytes(), np.uint8); variants.append(i)
    for v in variants:
        ok, msg, _ = ref.container_check(v)
        with pytest.raises(sm.SparkmvError) as exc:
            sm.Container(v)
        if not ok:
            assert msg in str(exc.value)
        else:  # pragma: no cover - every variant above is refused
            pytest.fail("oracle accepted a damaged container")


@pytest.mark.parametrize("rows,cols,dim,nc,ns,v3", [(7, 64, 4, 4096, 2, 1), (3, 40, 4, 8192, 1, 1),
                                                    (5, 36, 4, 1024, 1, 1), (4, 48, 8, 300, 2, 1),
                                                    (6, 20, 4, 256, 1, 0), (3, 24, 4, 600, 2, 0),
                                                    (2, 4, 4, 4096, 1, 1)])
def test_synth_packing_matches_reference_writer(sm, ref, rows, cols, dim, nc, ns, v3):
    """The product's seeded writer lays indices out exactly as the reference's
    writers (build-vq-gpu.c:71-111 / vq_qc.h:241-264, restated in the oracle)."""
    data = sm.synth_container(1234 + rows, rows, cols, dim, nc, ns, v3)
    ok, msg, info = ref.container_check(data)
    assert ok, msg
    stride = info["stride"]
    for s in range(ns):
        payload = data[32 + s * stride:32 + (s + 1) * stride]
        idx = ref.stage_indices(payload)
        assert idx.max() < nc
        hdr = 24 if v3 else 16
        cb = payload[hdr:hdr + nc * dim * 2].view(np.uint16)
        gains = payload[hdr + nc * dim * 2:hdr + nc * dim * 2 + rows * 2].view(np.uint16)
        again = ref.pack(v3, cb, idx.ravel(), gains, rows, cols, dim, nc)
        assert np.array_equal(again, payload)


def test_synth_distributions(sm):
    data = sm.synth_container(7, 512, 256, 4, 4096, 1, 1)
    cb = data[32 + 24:32 + 24 + 4096 * 8].view(np.float16).astype(np.float64)
    assert abs(cb.std() - 0.02) < 0.001 and abs(cb.mean()) < 0.001
    g = data[32 + 24 + 4096 * 8:32 + 24 + 4096 * 8 + 1024].view(np.float16).astype(np.float64)
    assert g.min() >= 0.5 and g.max() <= 1.5 and abs(g.mean() - 1.0) < 0.05
    x = sm.bf16_to_f32(sm.synth_bf16(3, 100000))
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1.0) < 0.02
    q8 = sm.synth_q8_0(5, 64, 256)
    d = np.concatenate([q8[i * 34:i * 34 + 2] for i in range(64 * 8)]).view(np.float16).astype(np.float64)
    assert d.min() >= 1e-4 and d.max() <= 1e-3
    q6 = sm.synth_q6k(5, 16, 512)
    sc = np.concatenate([q6[i * 210 + 192:i * 210 + 208] for i in range(32)]).view(np.int8)
    assert sc.min() >= -32 and sc.max() <= 31


def test_synth_is_deterministic(sm):
    a = sm.synth_container(42, 33, 128, 4, 4096, 2, 1)
    b = sm.synth_container(42, 33, 128, 4, 4096, 2, 1)
    c = sm.synth_container(43, 33, 128, 4, 4096, 2, 1)
    assert np.array_equal(a, b) and not np.array_equal(a, c)


def test_stage_bytes_agree(sm, ref):
    for args in [(1, 10240, 2560, 4, 4096), (1, 16, 2560, 4, 8192), (0, 3, 16, 4, 512), (1, 5, 12, 4, 1024)]:
        assert sm.lib().sparkmv_stage_bytes(*args) == ref.stage_bytes(*args)


def test_model_config_refusals(sm):
    """sparkmv_model_create refuses a configuration before touching the
    device: each bad field with its own message."""
    import ctypes
    good = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=320, eps=1e-6,
                sliding_window=3, rope_full_theta=5e6, rope_full_partial=0.25, rope_slide_theta=1e4,
                rope_slide_partial=1.0, max_ctx=16, x_dtype=sm.X_F32, dim=4, nc=4096, nstages=2, v3=1)
    for bad, msg in ((dict(heads=3), "multiple of kv_heads"), (dict(head_dim=96), "not 64, 128 or 256"),
                     (dict(heads=16, kv_heads=2), "more than 4 query heads"), (dict(max_ctx=10 ** 6), "is above"),
                     (dict(x_dtype=7), "unknown x dtype"), (dict(nstages=5), "outside 1..4"),
                     (dict(eps=0.0), "eps must be positive"), (dict(vocab=0), "non-positive"),
                     (dict(rope_full_partial=0.05), "not a multiple")):
        cfg = sm.ModelCfg(**dict(good, **bad))
        if bad == dict(rope_full_partial=0.05):
            cfg = sm.ModelCfg(**dict(good, head_dim=256, rope_full_partial=0.05))   # 12 rotated: half 6, lanes hold 4
        assert not sm.lib().sparkmv_model_create(ctypes.byref(cfg)), bad
        assert msg in sm.last_error(), (bad, sm.last_error())


def test_chain_refusals(sm):
    """sparkmv_chain_add_vq refuses what the chain kernel cannot run, before
    any device call: indices other than 12-bit, columns that are not a
    multiple of 128, unaligned stages, a pair of unequal row counts, a
    matrix without an output, and tuning outside the built kernels."""
    import ctypes
    h = sm.lib().sparkmv_chain_create()
    try:
        def mats(n, rows=(64, 64), align=0, out=True):
            arr = (sm.ChainMatrix * n)()
            for i in range(n):
                arr[i].stages[0] = 0x10000 + align
                arr[i].stages[1] = 0x20000
                arr[i].y = 0x30000 if out else None
                arr[i].rows = rows[i]
            return arr
        x = ctypes.c_void_p(0x40000)

        def add(arr, n, nc=4096, cols=256, act=None, xx=x):
            return sm.lib().sparkmv_chain_add_vq(h, arr, n, 2, 4, nc, cols, 1, xx, 0, None, 1e-6, None, act, 1)

        for args, msg in (((mats(1), 1, 1024), "12-bit indices"), ((mats(1), 1, 4095), "12-bit indices"),
                          ((mats(1), 1, 4096, 200), "multiple of 128"), ((mats(1, align=2), 1), "not 4-byte aligned"),
                          ((mats(1, out=False), 1), "has no output"),
                          ((mats(2, rows=(64, 32)), 2, 4096, 256, ctypes.c_void_p(0x50000)), "equal row counts"),
                          ((mats(1), 1, 4096, 256, ctypes.c_void_p(0x50000)), "two matrices"),
                          ((mats(1), 1, 4096, 256, None, ctypes.c_void_p(0x40002)), "4-byte aligned")):
            assert add(*args) == -1, msg
            assert msg in sm.last_error(), (msg, sm.last_error())
        assert add(mats(1), 1) == 0 and sm.lib().sparkmv_chain_size(h) == 1
        assert sm.lib().sparkmv_chain_tune(h, 10, 2, 16) == -1 and "8, 12 or 16" in sm.last_error()
        assert sm.lib().sparkmv_chain_tune(h, 16, 3, 16) == -1 and "2, 4 or 8" in sm.last_error()
        assert sm.lib().sparkmv_chain_tune(h, 16, 8, 16) == -1 and "8 waves" in sm.last_error()
        assert sm.lib().sparkmv_chain_tune(h, 12, 4, -1) == -1 and "0..1024" in sm.last_error()
        assert sm.lib().sparkmv_chain_tune(h, 12, 4, 24) == 0
        assert sm.lib().sparkmv_chain_tune(h, 8, 8, 0) == 0
    finally:
        sm.lib().sparkmv_chain_destroy(h)


def test_probe_refusals(sm):
    """The measurement entries refuse what they cannot time before any device
    call: too many or too few sizes, sizes outside their range, repetitions
    outside 3..64, word counts outside 256..5120, and a missing output."""
    import ctypes
    L = sm.lib()
    out = (ctypes.c_double * 64)()

    def sizes(*v):
        return (ctypes.c_size_t * len(v))(*v)

    def words(*v):
        return (ctypes.c_int * len(v))(*v)

    for call, msg in ((lambda: L.sparkmv_probe_startup(sizes(1 << 20), 1, 2, out), "3..64 repetitions"),
                      (lambda: L.sparkmv_probe_startup(sizes(1000), 1, 5, out), "from 64 KB to 1 GB"),
                      (lambda: L.sparkmv_probe_startup(sizes(1 << 20), 1, 5, None), "output array"),
                      (lambda: L.sparkmv_probe_read_chain(sizes(1 << 20), 0, 5, out), "1..1024 sizes"),
                      (lambda: L.sparkmv_probe_read_chain(sizes(100), 1, 5, out), "from 4 KB to 1 GB"),
                      (lambda: L.sparkmv_probe_read_chain(sizes(1 << 20), 1, 99, out), "3..64 repetitions"),
                      (lambda: L.sparkmv_probe_read_chain(sizes(1 << 30, 1 << 30, 1 << 30), 3, 5, None), "output array"),
                      (lambda: L.sparkmv_probe_handoff(words(2560), 0, out), "1..8 word counts"),
                      (lambda: L.sparkmv_probe_handoff(words(100), 1, out), "256")):
        assert call() == -1, msg
        assert msg in sm.last_error(), (msg, sm.last_error())


def test_handles_are_released_at_interpreter_exit(sm):
    """Objects still alive when the interpreter exits are destroyed without
    an error: their destructors use only the library they captured, not
    module globals that teardown may already have cleared."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); import sparkmv as sm\n"
            "keep = [sm.Plan(), sm.Chain(), sm.Plan()]\n" % os.path.dirname(sm.__file__))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "Exception ignored" not in r.stderr and "Error" not in r.stderr, r.stderr
