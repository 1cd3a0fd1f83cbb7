"""Build libsparkmv.so (gfx950) in-tree with hipcc.

    python build.py            # compile every source, link lib/libsparkmv.so

HIP sources are compiled for gfx950 only, with packed FP32 instructions
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops); hipcc's host pass
warns that it does not know that feature, which is harmless. Host C++ sources
are compiled by hipcc as plain C++.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib", "libsparkmv.so")

HIP_SOURCES = ["vq_kernels.hip", "kq_kernels.hip", "prefill.hip", "forward.hip", "chain.hip", "probe.hip"]
CXX_SOURCES = ["abi.cpp", "plan.cpp", "host/vq_format.cpp", "host/synth.cpp", "host/artifacts.cpp", "host/profile.cpp",
               "host/model_load.cpp"]

ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _obj(src):
    return os.path.join(BUILD, src.replace("/", "_").rsplit(".", 1)[0] + ".o")


def _compile(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    return r.returncode, " ".join(cmd), out


def build(verbose=False):
    """Compile and link; returns the library path. Raises on any failure."""
    cc = hipcc()
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    jobs = []
    for s in HIP_SOURCES:
        jobs.append([cc, *COMMON, *HIP_FLAGS, "-c", os.path.join(CSRC, s), "-o", _obj(s)])
    for s in CXX_SOURCES:
        rocm = os.path.dirname(os.path.dirname(os.path.realpath(cc)))
        jobs.append([cc, *COMMON, "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(rocm, "include"),
                     "-c", os.path.join(CSRC, s), "-o", _obj(s)])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        results = list(ex.map(_compile, jobs))
    failed = False
    for rc, cmd, out in results:
        if verbose or rc:
            print(cmd)
        if out.strip() and (verbose or rc):
            print(out)
        failed |= rc != 0
    if failed:
        raise RuntimeError("libsparkmv compilation failed")
    tmp = LIB + ".tmp"
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
            *[_obj(s) for s in HIP_SOURCES + CXX_SOURCES]]
    rc, cmd, out = _compile(link)
    if rc:
        print(cmd)
        print(out)
        raise RuntimeError("libsparkmv link failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
