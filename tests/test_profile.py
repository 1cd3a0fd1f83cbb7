"""The tuning profile (VQPROF 1, tools/vq/gpu/vq-profile.h:10-30): the
artifact fingerprint against the published FNV-1a 64 test vectors and an
independent restatement of the hashed sequence, the reader on files in the
reference's format, the writer's round trip and the trust gate."""
import os
import struct

import pytest

FNV_PRIME = 0x100000001B3
STD_BASIS = 14695981039346656037        # FNV-1a 64's published offset basis
# The reference's tuner and reader both start from 1469598103934665603
# (tools/vq-tune/src/artifact.rs:14, tools/vq/gpu/vq-profile.h:67), one digit
# short of the published basis; a profile must hash what its tuner hashed.
REF_BASIS = 1469598103934665603


def fnv1a(h, data):
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & 0xFFFFFFFFFFFFFFFF
    return h


def test_fnv1a_restatement_meets_the_published_vectors():
    assert fnv1a(STD_BASIS, b"") == 0xCBF29CE484222325
    assert fnv1a(STD_BASIS, b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a(STD_BASIS, b"foobar") == 0x85944171F73967E8


def test_fingerprint_of_a_bare_manifest(sm, tmp_path):
    for text in (b"a", b"foobar", b"# only a comment\n"):
        (tmp_path / "manifest.txt").write_bytes(text)
        assert sm.profile_fingerprint(tmp_path) == fnv1a(REF_BASIS, text)


def test_fingerprint_hashes_manifest_then_containers(sm, tmp_path):
    small = os.urandom(1000)
    large = os.urandom(10000)
    man = ("# comment line\n"
           "model.embed 320 256 2 %d 1.0\n"
           "model.norm 1 256 0 1036 0.0\n"
           "model.up 512 256 2 %d 2.5\n" % (len(small), len(large))).encode()
    (tmp_path / "manifest.txt").write_bytes(man)
    (tmp_path / "model.embed.bin").write_bytes(small)
    (tmp_path / "model.up.bin").write_bytes(large)
    h = fnv1a(REF_BASIS, man)
    for name, data in (("model.embed", small), ("model.up", large)):   # stages > 0 only, file order
        h = fnv1a(h, name.encode())
        h = fnv1a(h, struct.pack("<Q", len(data)))
        h = fnv1a(h, data[:4096])
        h = fnv1a(h, data[-4096:] if len(data) > 4096 else data[:4096])
    assert sm.profile_fingerprint(tmp_path) == h
    (tmp_path / "model.up.bin").unlink()
    with pytest.raises(sm.SparkmvError):
        sm.profile_fingerprint(tmp_path)
    assert "cannot be opened" in sm.last_error()


def test_reader_on_the_reference_format_and_trust_gate(sm, tmp_path):
    p = tmp_path / "vq-tune.profile"
    p.write_text("VQPROF 1\nartifact 00000000deadbeef\ngpu AMD Instinct MI355X\ndriver 70200\n"
                 "gemv 4 4096 10240 2560 1 3 256 2750.12\n"
                 "a line the reader skips\n"
                 "prefill 4 4096 10240 2560 1 2 128 64 30000.5\n")
    pf = sm.Profile(p)
    es = pf.entries()
    assert [(e.kind, e.rows, e.cols, e.variant) for e in es] == [(0, 10240, 2560, 3), (1, 10240, 2560, 2)]
    assert es[0].threads == 256 and abs(es[0].rate - 2750.12) < 1e-9
    assert (es[1].bn, es[1].bk) == (128, 64)
    e = pf.find(1, 4, 4096, 10240, 2560, 1)
    assert e is not None and e.variant == 2
    assert pf.find(0, 4, 4096, 2560, 10240, 1) is None
    assert pf.trusted(0xDEADBEEF, "AMD Instinct MI355X")
    assert not pf.trusted(0xDEADBEEE, "AMD Instinct MI355X")
    assert "does not match" in sm.last_error()
    assert not pf.trusted(0xDEADBEEF, "another GPU")
    assert "was measured on" in sm.last_error()


def test_writer_round_trip_and_version_refusal(sm, tmp_path):
    es = [sm.ProfileEntry(kind=0, dim=4, nc=4096, rows=2560, cols=10240, v3=1, variant=3, threads=0, rate=1999.5),
          sm.ProfileEntry(kind=1, dim=4, nc=8192, rows=512, cols=4096, v3=1, variant=1, bn=64, bk=64, rate=12.25)]
    p = tmp_path / "out.profile"
    sm.profile_write(p, 0x0123456789ABCDEF, "gfx950 test device", "7.2", es)
    text = p.read_text().splitlines()
    assert text[:4] == ["VQPROF 1", "artifact 0123456789abcdef", "gpu gfx950 test device", "driver 7.2"]
    pf = sm.Profile(p)
    got = [(e.kind, e.dim, e.nc, e.rows, e.cols, e.v3, e.variant, e.threads, e.bn, e.bk) for e in pf.entries()]
    assert got == [(0, 4, 4096, 2560, 10240, 1, 3, 0, 0, 0), (1, 4, 8192, 512, 4096, 1, 1, 0, 64, 64)]
    assert pf.trusted(0x0123456789ABCDEF, "gfx950 test device")
    p.write_text("VQPROF 2\nartifact 0\n")
    with pytest.raises(sm.SparkmvError):
        sm.Profile(p)
    assert "version 2" in sm.last_error()
