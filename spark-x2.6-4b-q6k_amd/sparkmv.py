"""Python binding of libsparkmv (ctypes over the C-ABI in include/sparkmv.h).

The library is the product: every function here forwards to an exported C
symbol. PyTorch is used only to own device memory and streams. There is no
CPU fallback: if the library is missing, ``lib()`` raises.

Interface mirror (the reference's Rust surface this stands beside):
  Container.open           tools/vq-format/src/lib.rs:240-306 (Container::open)
  DeviceContainer.gemv     tools/vq-runtime/src/model.rs:228-234 (matvec), fused
                           over stages as tools/vq/gpu/vq-model-gpu.cu:651-660 does
  DeviceContainer.dequant  lib.rs:309-315 (Container::decode) on the device
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libsparkmv.so")

X_BF16 = 0
X_F32 = 1

_lib = None


class SparkmvError(RuntimeError):
    pass


class ContainerInfo(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int), ("nc", ctypes.c_int), ("nstages", ctypes.c_int), ("rows", ctypes.c_int),
        ("cols", ctypes.c_int), ("v3", ctypes.c_int), ("nbit", ctypes.c_int),
        ("payload_bytes", ctypes.c_uint64), ("stage_offset", ctypes.c_uint64 * 4), ("stage_bytes", ctypes.c_uint64),
    ]


class VqMatrix(ctypes.Structure):
    _fields_ = [("stages", ctypes.c_void_p * 4), ("y", ctypes.c_void_p), ("rows", ctypes.c_int)]


_I, _P, _D, _S, _U64 = ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_double), ctypes.c_size_t, ctypes.c_uint64
_PP = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "vqg_decode_error": (ctypes.c_char_p, []),
    "vqg_device_name": (_I, [ctypes.c_char_p, _I]),
    "vqg_driver_version": (_I, []),
    "vqg_gemv_ready": (_I, [_I] * 6),
    "vqg_gemv_t": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _I, _I, _I, _D]),
    "vqg_gemv": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _I, _I, _D]),
    "vqg_gemv_launch_t": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _I, _I]),
    "vqg_gemv_launch": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _I]),
    "vqg_dequant": (_I, [_P, _I, _I, _I, _I, _I, _P, _I, _D]),
    "vqg_row_dequant": (_I, [_P, _I, _I, _I, _I, _I, _I, _P]),
    "vqg_prefill_ready": (_I, [_I] * 6),
    "vqg_prefill_cfg_count": (_I, []),
    "vqg_prefill_cfg": (_I, [_I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "vqg_prefill_cfg_ready": (_I, [_I] * 8),
    "vqg_prefill": (_I, [_P, _I, _I, _I, _I, _I, _P, _I, _P, _I, _D, _I]),
    "vqg_prefill_tile": (_I, [_P, _I, _I, _I, _I, _I, _P, _I, _P, _I, _D, _I, _I, _I]),
    "vqg_prefill_launch": (_I, [_P, _I, _I, _I, _I, _I, _P, _I, _P, _I]),
    "vqg_prefill_launch_tile": (_I, [_P, _I, _I, _I, _I, _I, _P, _I, _P, _I, _I, _I]),
    "vqg_gemv_f32": (_I, [_P, _P, _P, _I, _I, _I, _D]),
    "sparkmv_container_open": (_I, [_P, _S, ctypes.POINTER(ContainerInfo)]),
    "sparkmv_stage_bytes": (_S, [_I] * 5),
    "sparkmv_vq_gemv": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _I, _P]),
    "sparkmv_vq_gemv_multi": (_I, [ctypes.POINTER(VqMatrix), _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _I, _P]),
    "sparkmv_vq_dequant": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _P]),
    "sparkmv_q6k_gemv": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_q8_0_gemv": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_q6k_dequant": (_I, [_P, _I, _I, _P, _P]),
    "sparkmv_q8_0_dequant": (_I, [_P, _I, _I, _P, _P]),
    "sparkmv_vq_prefill": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_plan_create": (_P, []),
    "sparkmv_plan_destroy": (None, [_P]),
    "sparkmv_plan_size": (_I, [_P]),
    "sparkmv_plan_add_vq": (_I, [_P, ctypes.POINTER(VqMatrix), _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _I]),
    "sparkmv_plan_add_kquant": (_I, [_P, _I, _P, _I, _I, _P, _I, _I, _I, _P, _I, _I]),
    "sparkmv_plan_run": (_I, [_P, _P]),
    "sparkmv_plan_capture": (_I, [_P, _P]),
    "sparkmv_plan_launch": (_I, [_P, _P]),
    "sparkmv_plan_time_ops": (_I, [_P, _P, _I, _D]),
    "sparkmv_synth_container_bytes": (_S, [_I] * 6),
    "sparkmv_synth_vq_container": (_I, [_U64, _I, _I, _I, _I, _I, _I, _P, _S]),
    "sparkmv_synth_q6k": (_I, [_U64, _I, _I, _P]),
    "sparkmv_synth_q8_0": (_I, [_U64, _I, _I, _P]),
    "sparkmv_synth_bf16_normal": (_I, [_U64, _S, _P]),
}


def lib():
    """The loaded library; raises if it has not been built.

    torch is imported first: it loads its own HIP runtime (libamdhip64,
    soname libamdhip64.so.7), and libsparkmv's dependency on that soname then
    binds to the same runtime. Loading libsparkmv first would bring a second
    HIP runtime into the process, and the two do not share the device."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SparkmvError(f"{LIB_PATH} is missing: build it with spark-x2.6-4b-q6k_amd/build.py")
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().vqg_decode_error().decode(errors="replace")


def check(rc, what="sparkmv"):
    if rc != 0:
        raise SparkmvError(f"{what}: {last_error()}")
    return rc


# ----------------------------------------------------------------- host side


class Container:
    """A validated RQVQ container in host memory (lib.rs:240-306)."""

    def __init__(self, data):
        self.data = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        info = ContainerInfo()
        check(lib().sparkmv_container_open(self.data.ctypes.data, self.data.nbytes, ctypes.byref(info)),
              "container open")
        self.info = info
        self.dim, self.nc, self.rows, self.cols = info.dim, info.nc, info.rows, info.cols
        self.nstages, self.v3, self.nbit = info.nstages, info.v3, info.nbit
        self.stage_offsets = [int(info.stage_offset[s]) for s in range(info.nstages)]
        self.stage_bytes = int(info.stage_bytes)

    @classmethod
    def open(cls, data):
        return cls(data)


def synth_container(seed, rows, cols, dim=4, nc=4096, nstages=2, v3=1):
    n = lib().sparkmv_synth_container_bytes(rows, cols, dim, nc, nstages, v3)
    if n == 0:
        raise SparkmvError("invalid synthetic container geometry")
    buf = np.zeros(n, dtype=np.uint8)
    check(lib().sparkmv_synth_vq_container(seed, rows, cols, dim, nc, nstages, v3, buf.ctypes.data, n), "synth")
    return buf


def synth_q6k(seed, rows, cols):
    buf = np.zeros(rows * (cols // 256) * 210, dtype=np.uint8)
    check(lib().sparkmv_synth_q6k(seed, rows, cols, buf.ctypes.data), "synth q6k")
    return buf


def synth_q8_0(seed, rows, cols):
    buf = np.zeros(rows * (cols // 32) * 34, dtype=np.uint8)
    check(lib().sparkmv_synth_q8_0(seed, rows, cols, buf.ctypes.data), "synth q8_0")
    return buf


def synth_bf16(seed, n):
    out = np.zeros(n, dtype=np.uint16)
    check(lib().sparkmv_synth_bf16_normal(seed, n, out.ctypes.data), "synth bf16")
    return out


def bf16_to_f32(u16):
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------- device side


def _torch():
    import torch
    return torch


def _stream_ptr(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class DeviceContainer:
    """An RQVQ container resident in device memory (one buffer, stages at
    their file offsets) with the fused GEMV and dequant of all its stages."""

    def __init__(self, host_bytes, device="cuda"):
        torch = _torch()
        self.host = Container(host_bytes)
        self.buf = torch.from_numpy(np.ascontiguousarray(self.host.data)).to(device)
        base = self.buf.data_ptr()
        self.stage_ptrs = [base + off for off in self.host.stage_offsets]
        self.rows, self.cols = self.host.rows, self.host.cols

    def _stages(self):
        arr = (ctypes.c_void_p * len(self.stage_ptrs))(*self.stage_ptrs)
        return ctypes.cast(arr, _PP), arr

    def gemv(self, x, y, ncols=1, accumulate=False, variant=0, stream=None):
        """y[n, r] (+)= sum_c W[r, c] x[n, c]; x bf16 (as int16/uint16 or
        torch.bfloat16) or f32, shape [ncols, cols]; y f32 [ncols, rows]."""
        torch = _torch()
        xd = X_F32 if x.dtype == torch.float32 else X_BF16
        pp, keep = self._stages()
        h = self.host
        check(lib().sparkmv_vq_gemv(pp, h.nstages, h.dim, h.nc, h.rows, h.cols, h.v3, x.data_ptr(), xd,
                                    x.stride(0) if x.dim() > 1 else h.cols, ncols, y.data_ptr(),
                                    y.stride(0) if y.dim() > 1 else h.rows, int(accumulate), variant,
                                    _stream_ptr(stream)), "vq gemv")

    def dequant(self, out, accumulate=False, stream=None):
        pp, keep = self._stages()
        h = self.host
        check(lib().sparkmv_vq_dequant(pp, h.nstages, h.dim, h.nc, h.rows, h.cols, h.v3, out.data_ptr(),
                                       int(accumulate), _stream_ptr(stream)), "vq dequant")

    def prefill(self, x, y, accumulate=False, stream=None):
        """x [ntok, cols] token-major (bf16 or f32), y [ntok, rows] f32."""
        torch = _torch()
        xd = X_F32 if x.dtype == torch.float32 else X_BF16
        pp, keep = self._stages()
        h = self.host
        check(lib().sparkmv_vq_prefill(pp, h.nstages, h.dim, h.nc, h.rows, h.cols, h.v3, x.data_ptr(), xd,
                                       x.stride(0), x.shape[0], y.data_ptr(), y.stride(0), int(accumulate),
                                       _stream_ptr(stream)), "vq prefill")


def gemv_multi(mats, x, ys, ncols=1, accumulate=False, variant=0, stream=None):
    """One launch over several DeviceContainers that share x (same cols,
    stages, nc, dim, format); ys[i] is matrix i's output [ncols, rows_i]."""
    torch = _torch()
    arr = (VqMatrix * len(mats))()
    for i, (m, y) in enumerate(zip(mats, ys)):
        for s, p in enumerate(m.stage_ptrs):
            arr[i].stages[s] = p
        arr[i].y = y.data_ptr()
        arr[i].rows = m.rows
    h = mats[0].host
    ldy = ys[0].stride(0) if ys[0].dim() > 1 else h.rows
    xd = X_F32 if x.dtype == torch.float32 else X_BF16
    check(lib().sparkmv_vq_gemv_multi(arr, len(mats), h.nstages, h.dim, h.nc, h.cols, h.v3, x.data_ptr(), xd,
                                      x.stride(0) if x.dim() > 1 else h.cols, ncols, ldy, int(accumulate), variant,
                                      _stream_ptr(stream)), "vq gemv multi")


def kquant_gemv(kind, blocks, rows, cols, x, y, ncols=1, accumulate=False, stream=None):
    """kind 'q6_k' or 'q8_0'; blocks a device uint8 tensor of ggml blocks."""
    torch = _torch()
    xd = X_F32 if x.dtype == torch.float32 else X_BF16
    fn = lib().sparkmv_q6k_gemv if kind == "q6_k" else lib().sparkmv_q8_0_gemv
    check(fn(blocks.data_ptr(), rows, cols, x.data_ptr(), xd, x.stride(0) if x.dim() > 1 else cols, ncols,
             y.data_ptr(), y.stride(0) if y.dim() > 1 else rows, int(accumulate), _stream_ptr(stream)), kind + " gemv")


def kquant_dequant(kind, blocks, rows, cols, out, stream=None):
    fn = lib().sparkmv_q6k_dequant if kind == "q6_k" else lib().sparkmv_q8_0_dequant
    check(fn(blocks.data_ptr(), rows, cols, out.data_ptr(), _stream_ptr(stream)), kind + " dequant")


class Plan:
    """A recorded chain of matvec launches (sparkmv_plan_*): run eagerly or
    replayed as one HIP graph. Holds references to every tensor it uses."""

    def __init__(self):
        self.h = lib().sparkmv_plan_create()
        self.keep = []
        self.labels = []

    def __del__(self):
        if getattr(self, "h", None):
            lib().sparkmv_plan_destroy(self.h)
            self.h = None

    def __len__(self):
        return lib().sparkmv_plan_size(self.h)

    def add_vq(self, mats, x, ys, ncols=1, accumulate=False, variant=0, label="vq"):
        torch = _torch()
        arr = (VqMatrix * len(mats))()
        for i, (m, y) in enumerate(zip(mats, ys)):
            for s, p in enumerate(m.stage_ptrs):
                arr[i].stages[s] = p
            arr[i].y = y.data_ptr()
            arr[i].rows = m.rows
        h = mats[0].host
        ldy = ys[0].stride(0) if ys[0].dim() > 1 else h.rows
        xd = X_F32 if x.dtype == torch.float32 else X_BF16
        check(lib().sparkmv_plan_add_vq(self.h, arr, len(mats), h.nstages, h.dim, h.nc, h.cols, h.v3, x.data_ptr(),
                                        xd, x.stride(0) if x.dim() > 1 else h.cols, ncols, ldy, int(accumulate),
                                        variant), "plan add vq")
        self.keep.append((mats, x, ys))
        self.labels.append(label)

    def add_kquant(self, kind, blocks, rows, cols, x, y, ncols=1, accumulate=False, label=None):
        torch = _torch()
        xd = X_F32 if x.dtype == torch.float32 else X_BF16
        check(lib().sparkmv_plan_add_kquant(self.h, 6 if kind == "q6_k" else 8, blocks.data_ptr(), rows, cols,
                                            x.data_ptr(), xd, x.stride(0) if x.dim() > 1 else cols, ncols,
                                            y.data_ptr(), y.stride(0) if y.dim() > 1 else rows, int(accumulate)),
              "plan add kquant")
        self.keep.append((blocks, x, y))
        self.labels.append(label or kind)

    def run(self, stream=None):
        check(lib().sparkmv_plan_run(self.h, _stream_ptr(stream)), "plan run")

    def capture(self, stream):
        check(lib().sparkmv_plan_capture(self.h, _stream_ptr(stream)), "plan capture")

    def launch(self, stream=None):
        check(lib().sparkmv_plan_launch(self.h, _stream_ptr(stream)), "plan launch")

    def time_ops(self, stream=None, iters=5):
        n = len(self)
        out = (ctypes.c_double * n)()
        check(lib().sparkmv_plan_time_ops(self.h, _stream_ptr(stream), iters, out), "plan time")
        return np.array(out[:], dtype=np.float64)
