"""Write the golden fixtures under tests/golden/ (run in the build container).

Each fixture is a small RQVQ container plus the matrix that the reference's
own C decoder (tools/vq/decode.c, compiled from its source into
oracle/_ref/decode by oracle/Makefile) dumps for it, and the refusals that
decoder makes on damaged containers. The containers come from libsparkmv's
seeded generator; the decoded matrices and refusals are the reference's.

    python tests/golden/make_golden.py

Fixtures are data (inputs and expected outputs); no reference source is kept.
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "spark-x2.6-4b-q6k_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import sparkmv  # noqa: E402
import sparkref  # noqa: E402

# name: (seed, rows, cols, dim, nc, stages, v3)
CASES = {
    "v3_nc4096_s2": (11, 37, 256, 4, 4096, 2, 1),
    "v3_nc8192_s1": (12, 20, 128, 4, 8192, 1, 1),
    "v3_nc1024_s2": (13, 33, 96, 4, 1024, 2, 1),
    "v3_nc4096_dim8": (14, 16, 128, 8, 4096, 1, 1),
    "v3_nc3000_s1": (15, 18, 64, 4, 3000, 1, 1),
    "v3_nc4096_odd": (16, 5, 12, 4, 4096, 2, 1),
    "vq_nc256_s2": (17, 24, 64, 4, 256, 2, 0),
    "vq_nc512_s1": (18, 19, 60, 4, 512, 1, 0),
}


def ref_dump(decode, data):
    with tempfile.TemporaryDirectory() as d:
        src, out = os.path.join(d, "c.bin"), os.path.join(d, "w.f32")
        data.tofile(src)
        r = subprocess.run([decode, "dump", src, out], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
        if r.returncode != 0:
            return None, r.stderr.strip()
        return np.fromfile(out, dtype=np.float32), ""


def damaged(data, dim):
    """Damaged variants of one container: (name, bytes)."""
    d = data.copy()
    yield "truncated", d[:-1]
    e = data.copy()
    e[24] ^= 0x01                       # payload byte count off by one
    yield "payload_count", e
    f = data.copy()
    f[36:38] = np.frombuffer(np.uint16(2 * dim).tobytes(), np.uint8)   # stage dim disagrees with header
    yield "stage_dim", f
    g = data.copy()
    g[0] = ord("X")                     # not an RQVQ container
    yield "magic", g
    h = data.copy()                      # DQV3 with nc 16384 (14-bit) in both headers
    h[6:8] = np.frombuffer(np.uint16(16384).tobytes(), np.uint8)
    h[38:40] = np.frombuffer(np.uint16(16384).tobytes(), np.uint8)
    yield "nc16384", h


def main():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    decode = sparkref.REF_DECODE
    if not os.path.exists(decode):
        sys.exit("oracle/_ref/decode is missing: the reference tree is needed to write fixtures")
    for name, (seed, rows, cols, dim, nc, ns, v3) in CASES.items():
        data = sparkmv.synth_container(seed, rows, cols, dim, nc, ns, v3)
        w, err = ref_dump(decode, data)
        if w is None:
            sys.exit(f"{name}: reference decoder refused a valid container: {err}")
        refused = []
        for dname, dd in damaged(data, dim):
            if dname == "nc16384" and not v3:
                continue
            wd, _ = ref_dump(decode, dd)
            refused.append((dname, wd is None))
        np.savez_compressed(os.path.join(HERE, name + ".npz"), container=data, decoded=w.reshape(rows, cols),
                            geometry=np.array([seed, rows, cols, dim, nc, ns, v3], dtype=np.int64),
                            damaged_names=np.array([r[0] for r in refused]),
                            damaged_refused=np.array([r[1] for r in refused]))
        print(f"{name}: {rows}x{cols} dim {dim} nc {nc} stages {ns} v3 {v3}; refusals {refused}")


if __name__ == "__main__":
    main()
