"""ctypes binding of the oracle (oracle/_build/libsparkref.so).

Test infrastructure only: tests/, the smoke check and bench.py's CPU-baseline
leg load it, to compare against. The product library never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libsparkref.so")
REF_DECODE = os.path.join(HERE, "_ref", "decode")

_lib = None
_P, _S, _I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int


class Stage(ctypes.Structure):
    _fields_ = [("dim", _I), ("nc", _I), ("rows", _I), ("cols", _I), ("nbit", _I), ("v3", _I),
                ("mrow", _S), ("prow", _S), ("bytes", _S), ("gains", _P), ("stream", _P), ("stream_len", _S),
                ("cb32", _P)]


def build():
    subprocess.run(["make", "-s", "-C", HERE, "_build/libsparkref.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "sr_f16": (ctypes.c_float, [ctypes.c_uint16]),
            "sr_bf16": (ctypes.c_float, [ctypes.c_uint16]),
            "sr_stage_open": (_I, [_P, _S, ctypes.POINTER(Stage), ctypes.c_char_p, _S]),
            "sr_stage_close": (None, [ctypes.POINTER(Stage)]),
            "sr_stage_index": (ctypes.c_uint32, [ctypes.POINTER(Stage), _S, _S]),
            "sr_stage_gain": (ctypes.c_float, [ctypes.POINTER(Stage), _S]),
            "sr_stage_add_into": (None, [ctypes.POINTER(Stage), _P]),
            "sr_stage_dot_row": (None, [ctypes.POINTER(Stage), _S, _P, _P]),
            "sr_container_check": (_I, [_P, _S, ctypes.POINTER(_I), ctypes.POINTER(_S), ctypes.POINTER(_I),
                                        ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
                                        ctypes.POINTER(_I), ctypes.c_char_p, _S]),
            "sr_container_decode": (_I, [_P, _S, _P, ctypes.c_char_p, _S]),
            "sr_container_gemv_fused": (_I, [_P, _S, _P, _P, _I, ctypes.c_char_p, _S]),
            "sr_dot": (ctypes.c_float, [_P, _P, _S]),
            "sr_matvec": (None, [_P, _S, _S, _P, _P, _I]),
            "sr_matvec_f64": (None, [_P, _S, _S, _P, _P, _I]),
            "sr_stage_bytes": (_S, [_I, _I, _I, _I, _I]),
            "sr_v3_pack": (_S, [_P, _P, _P, _I, _I, _I, _I, _P]),
            "sr_vq_pack": (_S, [_P, _P, _P, _I, _I, _I, _I, _P]),
            "sr_q6k_dequant": (None, [_P, _S, _P]),
            "sr_q8_0_dequant": (None, [_P, _S, _P]),
            "sr_q6k_matvec": (None, [_P, _S, _S, _P, _P, _I]),
            "sr_q8_0_matvec": (None, [_P, _S, _S, _P, _P, _I]),
            "sr_hardware_threads": (_I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def threads():
    return lib().sr_hardware_threads()


def _buf(a):
    return np.ascontiguousarray(a)


def container_check(data):
    """(ok, message, dict) as Container::open (lib.rs:240-306) decides."""
    d = _buf(np.asarray(data, dtype=np.uint8))
    err = ctypes.create_string_buffer(256)
    ns, rows, cols, dim, nc, v3 = (_I() for _ in range(6))
    per = _S()
    rc = lib().sr_container_check(d.ctypes.data, d.nbytes, ctypes.byref(ns), ctypes.byref(per), ctypes.byref(rows),
                                  ctypes.byref(cols), ctypes.byref(dim), ctypes.byref(nc), ctypes.byref(v3), err, 256)
    info = dict(nstages=ns.value, stride=per.value, rows=rows.value, cols=cols.value, dim=dim.value, nc=nc.value,
                v3=v3.value)
    return rc == 0, err.value.decode(), info


def decode(data):
    """Container::decode: the f32 matrix (rows x cols)."""
    d = _buf(np.asarray(data, dtype=np.uint8))
    ok, msg, info = container_check(d)
    if not ok:
        raise ValueError(msg)
    out = np.zeros((info["rows"], info["cols"]), dtype=np.float32)
    err = ctypes.create_string_buffer(256)
    if lib().sr_container_decode(d.ctypes.data, d.nbytes, out.ctypes.data, err, 256):
        raise ValueError(err.value.decode())
    return out


def gemv_fused(data, x, nthreads=0):
    """The fused stage-by-stage dot_row path (dqvq gemv --fused)."""
    d = _buf(np.asarray(data, dtype=np.uint8))
    ok, msg, info = container_check(d)
    if not ok:
        raise ValueError(msg)
    x = _buf(np.asarray(x, dtype=np.float32))
    y = np.zeros(info["rows"], dtype=np.float32)
    err = ctypes.create_string_buffer(256)
    if lib().sr_container_gemv_fused(d.ctypes.data, d.nbytes, x.ctypes.data, y.ctypes.data,
                                     nthreads or threads(), err, 256):
        raise ValueError(err.value.decode())
    return y


def matvec(W, x, nthreads=0):
    """model.rs matvec: 8-lane f32 dot per row."""
    W = _buf(np.asarray(W, dtype=np.float32))
    x = _buf(np.asarray(x, dtype=np.float32))
    y = np.zeros(W.shape[0], dtype=np.float32)
    lib().sr_matvec(W.ctypes.data, W.shape[0], W.shape[1], x.ctypes.data, y.ctypes.data, nthreads or threads())
    return y


def matvec_f64(W, x, nthreads=0):
    W = _buf(np.asarray(W, dtype=np.float32))
    x = _buf(np.asarray(x, dtype=np.float32))
    y = np.zeros(W.shape[0], dtype=np.float64)
    lib().sr_matvec_f64(W.ctypes.data, W.shape[0], W.shape[1], x.ctypes.data, y.ctypes.data, nthreads or threads())
    return y


def dot(a, b):
    a = _buf(np.asarray(a, dtype=np.float32))
    b = _buf(np.asarray(b, dtype=np.float32))
    return float(lib().sr_dot(a.ctypes.data, b.ctypes.data, a.size))


def f16(h):
    return lib().sr_f16(int(h))


def stage_bytes(v3, rows, cols, dim, nc):
    return lib().sr_stage_bytes(v3, rows, cols, dim, nc)


def pack(v3, cb_f16, idx, gains_f16, rows, cols, dim, nc):
    """sr_v3_pack / sr_vq_pack: one stage payload from fp16 bits and indices."""
    cb = _buf(np.asarray(cb_f16, dtype=np.uint16))
    ix = _buf(np.asarray(idx, dtype=np.uint32))
    g = _buf(np.asarray(gains_f16, dtype=np.uint16))
    out = np.zeros(stage_bytes(v3, rows, cols, dim, nc) + 8, dtype=np.uint8)
    fn = lib().sr_v3_pack if v3 else lib().sr_vq_pack
    n = fn(cb.ctypes.data, ix.ctypes.data, g.ctypes.data, rows, cols, dim, nc, out.ctypes.data)
    return out[:n]


def stage_indices(payload):
    """All indices of one stage payload, [rows][cols/dim], via Stage::index."""
    p = _buf(np.asarray(payload, dtype=np.uint8))
    st = Stage()
    err = ctypes.create_string_buffer(256)
    if lib().sr_stage_open(p.ctypes.data, p.nbytes, ctypes.byref(st), err, 256):
        raise ValueError(err.value.decode())
    try:
        n = st.cols // st.dim
        out = np.zeros((st.rows, n), dtype=np.uint32)
        for r in range(st.rows):
            for i in range(n):
                out[r, i] = lib().sr_stage_index(ctypes.byref(st), r, i)
        return out
    finally:
        lib().sr_stage_close(ctypes.byref(st))


def q6k_dequant(blocks, rows, cols):
    b = _buf(np.asarray(blocks, dtype=np.uint8))
    out = np.zeros((rows, cols), dtype=np.float32)
    lib().sr_q6k_dequant(b.ctypes.data, rows * cols // 256, out.ctypes.data)
    return out


def q8_0_dequant(blocks, rows, cols):
    b = _buf(np.asarray(blocks, dtype=np.uint8))
    out = np.zeros((rows, cols), dtype=np.float32)
    lib().sr_q8_0_dequant(b.ctypes.data, rows * cols // 32, out.ctypes.data)
    return out


def q6k_matvec(blocks, rows, cols, x, nthreads=0):
    b = _buf(np.asarray(blocks, dtype=np.uint8))
    x = _buf(np.asarray(x, dtype=np.float32))
    y = np.zeros(rows, dtype=np.float32)
    lib().sr_q6k_matvec(b.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, nthreads or threads())
    return y


def q8_0_matvec(blocks, rows, cols, x, nthreads=0):
    b = _buf(np.asarray(blocks, dtype=np.uint8))
    x = _buf(np.asarray(x, dtype=np.float32))
    y = np.zeros(rows, dtype=np.float32)
    lib().sr_q8_0_matvec(b.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, nthreads or threads())
    return y


def ref_decode_available():
    return os.path.exists(REF_DECODE)
