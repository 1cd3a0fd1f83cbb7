"""Weight-artifact readers on the host: GGUF files (ggml's layout, as
tools/dspark/src/gguf.rs:95-190 reads it, plus the Q6_K tensors that reader
refuses) and the VQ manifest directory (tools/vq-runtime/src/vq_source.rs:
30-104, RawF32::open at tools/vq-format/src/lib.rs:325-350).

The GGUF files are written here by a small writer that follows ggml's
published format (magic "GGUF", version, tensor count, key/value count, typed
values, the tensor table, data at align_up(end of table, general.alignment)).
What a read must return is what the writer put there, byte for byte, and every
refusal the reference makes (bad magic, unsupported version, truncation,
manifest disagreements) is checked. No real artifact is available offline.
"""
import os
import struct

import numpy as np
import pytest

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _gstr(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gval(ty, v):
    if ty == STRING:
        return _gstr(v)
    if ty == ARRAY:
        elem, items = v
        return struct.pack("<IQ", elem, len(items)) + b"".join(_gval(elem, x) for x in items)
    return struct.pack(_FMT[ty], v)


def write_gguf(path, kv, tensors, version=3, alignment=None):
    """kv: [(key, type, value)]; tensors: [(name, dims fastest first, ggml
    type, bytes)]. Tensor data is placed at aligned offsets from the data
    section's start. Returns the data section's start in the file."""
    al = alignment or 32
    if alignment is not None:
        kv = list(kv) + [("general.alignment", U32, alignment)]
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv))
    head += b"".join(_gstr(k) + struct.pack("<I", t) + _gval(t, v) for k, t, v in kv)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + len(data) + al - 1) // al * al
    for (name, dims, ty, _), o in zip(tensors, offsets):
        head += _gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    start = (len(head) + al - 1) // al * al
    body = bytearray(off)
    for (_, _, _, data), o in zip(tensors, offsets):
        body[o:o + len(data)] = data
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)) + bytes(body))
    return start


def _model_file(sm, path, alignment=64):
    q8 = sm.synth_q8_0(7, 5, 64)
    q6 = sm.synth_q6k(8, 3, 512)
    f = np.arange(12, dtype=np.float32) * 0.5
    q4k = bytes(range(256)) * 1   # type 12 (Q4_K): listed, not handed out
    kv = [("general.architecture", STRING, "spark"), ("spark.block_count", U32, 36),
          ("spark.rope.freq_base", F32, 1.0e6), ("spark.context_length", U64, 1 << 20),
          ("spark.shift", I32, -3), ("tokenizer.scores", ARRAY, (F32, [0.5, -1.0, 2.0])),
          ("tokenizer.tokens", ARRAY, (STRING, ["a", "bc", ""])), ("spark.tied", BOOL, 1)]
    tensors = [("token_embd.weight", [64, 5], 8, q8.tobytes()), ("blk.0.ffn_down.weight", [512, 3], 14, q6.tobytes()),
               ("output_norm.weight", [4, 3], 0, f.tobytes()), ("blk.0.attn_q.weight", [256, 1], 12, q4k)]
    start = write_gguf(path, kv, tensors, alignment=alignment)
    return q8, q6, f, start


def test_gguf_tensors_and_metadata(sm, tmp_path):
    path = tmp_path / "m.gguf"
    q8, q6, f, start = _model_file(sm, path)
    with sm.Gguf(path) as g:
        assert g.version == 3
        ts = g.tensors()
        assert [t["name"] for t in ts] == ["token_embd.weight", "blk.0.ffn_down.weight", "output_norm.weight",
                                           "blk.0.attn_q.weight"]
        assert ts[0]["dims"] == [64, 5] and ts[0]["dtype"] == 8 and ts[0]["nbytes"] == 5 * 2 * 34
        assert ts[1]["dims"] == [512, 3] and ts[1]["dtype"] == 14 and ts[1]["nbytes"] == 3 * 2 * 210
        assert ts[2]["nbytes"] == 48 and ts[3]["nbytes"] == 0
        assert all(t["offset"] % 64 == 0 for t in ts)
        assert np.array_equal(g.tensor_bytes("token_embd.weight"), q8)
        assert np.array_equal(g.tensor_bytes("blk.0.ffn_down.weight"), q6)
        assert np.array_equal(g.tensor_bytes("output_norm.weight").view(np.float32), f)
        kind, rows, cols, blocks = g.kquant("blk.0.ffn_down.weight")
        assert (kind, rows, cols) == (6, 3, 512) and np.array_equal(blocks, q6)
        kind, rows, cols, blocks = g.kquant("token_embd.weight")
        assert (kind, rows, cols) == (8, 5, 64)
        with pytest.raises(sm.SparkmvError, match="ggml type 12 is not supported"):
            g.tensor_bytes("blk.0.attn_q.weight")
        with pytest.raises(sm.SparkmvError, match="not a 2-D Q8_0 or Q6_K"):
            g.kquant("output_norm.weight")
        with pytest.raises(sm.SparkmvError, match="no tensor"):
            g.tensor_bytes("missing")
        # metadata
        assert g.get_str("general.architecture") == "spark"
        assert g.get_u64("spark.block_count") == 36
        assert g.get_u64("spark.context_length") == 1 << 20
        assert g.get_f64("spark.rope.freq_base") == 1.0e6
        assert g.get_f64("spark.shift") == -3.0
        assert g.get_u64("spark.tied") == 1
        assert g.get_u64("general.alignment") == 64
        assert g.get_arr_len("tokenizer.scores") == (3, F32)
        assert g.get_arr_len("tokenizer.tokens") == (3, STRING)
        with pytest.raises(sm.SparkmvError):
            g.get_u64("spark.shift")   # negative: not a non-negative integer
        with pytest.raises(sm.SparkmvError):
            g.get_str("spark.block_count")
        assert ("spark.tied", BOOL) in g.keys()


def test_gguf_default_alignment_and_version_2(sm, tmp_path):
    path = tmp_path / "v2.gguf"
    f = np.linspace(-1, 1, 33, dtype=np.float32)
    start = write_gguf(path, [("a", U8, 1)], [("w", [33], 0, f.tobytes())], version=2)
    assert start % 32 == 0
    with sm.Gguf(path) as g:
        assert g.version == 2
        assert np.array_equal(g.tensor_bytes("w").view(np.float32), f)


def test_gguf_refusals(sm, tmp_path):
    path = tmp_path / "m.gguf"
    _model_file(sm, path)
    raw = path.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    with pytest.raises(sm.SparkmvError, match="not a GGUF file"):
        sm.Gguf(bad)
    bad.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    with pytest.raises(sm.SparkmvError, match="version 1 is not supported"):
        sm.Gguf(bad)
    bad.write_bytes(raw[:40])
    with pytest.raises(sm.SparkmvError, match="count does not fit the file"):
        sm.Gguf(bad)
    bad.write_bytes(raw[:200])
    with pytest.raises(sm.SparkmvError, match="unexpected end of file"):
        sm.Gguf(bad)
    # truncated inside the tensor data: the table reads, the last tensors do not
    bad.write_bytes(raw[:len(raw) - 300])
    with sm.Gguf(bad) as g:
        assert len(g.tensors()) == 4
        g.tensor_bytes("token_embd.weight")
        with pytest.raises(sm.SparkmvError, match="needs bytes"):
            g.tensor_bytes("output_norm.weight")
    with pytest.raises(sm.SparkmvError):
        sm.Gguf(tmp_path / "absent.gguf")
    # an array whose count cannot fit the file
    write_gguf(bad, [("x", ARRAY, (U32, []))], [])
    b = bytearray(bad.read_bytes())
    at = b.index(struct.pack("<IQ", U32, 0))
    b[at + 4:at + 12] = struct.pack("<Q", 1 << 40)
    bad.write_bytes(bytes(b))
    with pytest.raises(sm.SparkmvError, match="does not fit the file"):
        sm.Gguf(bad)


def _write_dir(sm, d, extra=""):
    cont = sm.synth_container(3, 48, 256)
    norm = (np.arange(2560, dtype=np.float32) - 7.0) / 3.0
    (d / "blk.0.mlp.up_proj.weight.bin").write_bytes(cont.tobytes())
    (d / "blk.0.norm.weight.bin").write_bytes(b"RQVF" + struct.pack("<II", 1, 2560) + norm.tobytes())
    (d / "manifest.txt").write_text(
        "# name rows cols stages file_bytes relL2\n\n"
        f"blk.0.mlp.up_proj.weight 48 256 2 {cont.nbytes} 3.2789\n"
        f"  blk.0.norm.weight\t1 2560 0 {12 + norm.nbytes} 0\n" + extra)
    return cont, norm


def test_manifest_directory(sm, tmp_path):
    cont, norm = _write_dir(sm, tmp_path)
    d = sm.VqDir(tmp_path)
    assert d.entries() == [("blk.0.mlp.up_proj.weight", 48, 256, 2), ("blk.0.norm.weight", 1, 2560, 0)]
    got = d.read("blk.0.mlp.up_proj.weight")
    assert np.array_equal(got, cont)
    c = sm.Container(got)
    assert (c.rows, c.cols, c.nstages) == (48, 256, 2)
    assert np.array_equal(d.read("blk.0.norm.weight"), norm.reshape(1, 2560))
    with pytest.raises(sm.SparkmvError, match="is not in the manifest"):
        d.read("blk.1.mlp.up_proj.weight")


def test_manifest_refusals(sm, tmp_path):
    cont, norm = _write_dir(sm, tmp_path, "blk.9.gone 4 256 2 100 1.0\n")
    d = sm.VqDir(tmp_path)
    with pytest.raises(sm.SparkmvError, match="gone.bin"):
        d.read("blk.9.gone")
    # the manifest disagrees with the container's header
    (tmp_path / "manifest.txt").write_text(f"blk.0.mlp.up_proj.weight 47 256 2 {cont.nbytes} 1\n")
    with pytest.raises(sm.SparkmvError, match="container is 48x256 with 2 stages, manifest says 47x256 with 2"):
        sm.VqDir(tmp_path).read("blk.0.mlp.up_proj.weight")
    (tmp_path / "manifest.txt").write_text("blk.0.norm.weight 2 1280 0 0 0\n")
    with pytest.raises(sm.SparkmvError, match="sidecar is 1x2560, manifest says 2x1280"):
        sm.VqDir(tmp_path).read("blk.0.norm.weight")
    # a sidecar whose length disagrees with its own header
    (tmp_path / "blk.0.norm.weight.bin").write_bytes(b"RQVF" + struct.pack("<II", 1, 2560) + norm.tobytes()[:-4])
    (tmp_path / "manifest.txt").write_text("blk.0.norm.weight 1 2560 0 0 0\n")
    with pytest.raises(sm.SparkmvError, match="RQVF file is"):
        sm.VqDir(tmp_path).read("blk.0.norm.weight")
    (tmp_path / "blk.0.norm.weight.bin").write_bytes(b"RQVF" + struct.pack("<II", 0, 2560))
    with pytest.raises(sm.SparkmvError, match="RQVF header is inconsistent"):
        sm.VqDir(tmp_path).read("blk.0.norm.weight")
    # malformed manifest lines
    (tmp_path / "manifest.txt").write_text("blk.0.norm.weight 1 2560 0\n")
    with pytest.raises(sm.SparkmvError, match="short manifest line"):
        sm.VqDir(tmp_path)
    (tmp_path / "manifest.txt").write_text("blk.0.norm.weight 1x 2560 0 0 0\n")
    with pytest.raises(sm.SparkmvError, match="bad rows in"):
        sm.VqDir(tmp_path)
    os.remove(tmp_path / "manifest.txt")
    with pytest.raises(sm.SparkmvError, match="manifest.txt"):
        sm.VqDir(tmp_path)
