"""Python binding of libsparkmv (ctypes over the C-ABI in include/sparkmv.h).

The library is the product: every function here forwards to an exported C
symbol. PyTorch is used only to own device memory and streams. There is no
CPU fallback: if the library is missing, ``lib()`` raises.

Interface mirror (the reference's Rust surface this stands beside):
  Container.open           tools/vq-format/src/lib.rs:240-306 (Container::open)
  DeviceContainer.gemv     tools/vq-runtime/src/model.rs:228-234 (matvec), fused
                           over stages as tools/vq/gpu/vq-model-gpu.cu:651-660 does
  DeviceContainer.dequant  lib.rs:309-315 (Container::decode) on the device
  VqDir                    tools/vq-runtime/src/vq_source.rs:30-104 (VqDir: manifest
                           directory of RQVQ containers and RQVF sidecars)
  Gguf                     tools/dspark/src/gguf.rs:95-190 (Gguf::open,
                           tensor_bytes, get_*), with Q6_K tensors handed out
  Profile / tune_gemv      tools/vq/gpu/vq-profile.h (VQPROF 1 reader, trust gate),
                           tools/vq-tune/src/artifact.rs:148-171 (writer, sweep)
  Model.forward            tools/vq-runtime/src/model.rs:441-591 (Model::forward),
                           as the GPU runtime runs it, tools/vq/gpu/vq-model-gpu.cu:776-835
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


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("ndims", ctypes.c_int), ("dims", ctypes.c_uint64 * 4),
                ("dtype", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class ModelCfg(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("layers", ctypes.c_int), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("vocab", ctypes.c_int), ("eps", ctypes.c_float), ("sliding_window", ctypes.c_int),
                ("rope_full_theta", ctypes.c_double), ("rope_full_partial", ctypes.c_double),
                ("rope_slide_theta", ctypes.c_double), ("rope_slide_partial", ctypes.c_double),
                ("max_ctx", ctypes.c_int), ("x_dtype", ctypes.c_int), ("dim", ctypes.c_int), ("nc", ctypes.c_int),
                ("nstages", ctypes.c_int), ("v3", ctypes.c_int)]


class ModelLayer(ctypes.Structure):
    _fields_ = [("in_norm", ctypes.c_void_p), ("post_norm", ctypes.c_void_p), ("qkv", ctypes.c_void_p * 4),
                ("attn_gate", ctypes.c_void_p * 4), ("out", ctypes.c_void_p * 4), ("gate", ctypes.c_void_p * 4),
                ("up", ctypes.c_void_p * 4), ("down", ctypes.c_void_p * 4), ("full", ctypes.c_int)]


class ProfileEntry(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("dim", ctypes.c_int), ("nc", ctypes.c_int), ("rows", ctypes.c_int),
                ("cols", ctypes.c_int), ("v3", ctypes.c_int), ("variant", ctypes.c_int), ("threads", ctypes.c_int),
                ("bn", ctypes.c_int), ("bk", ctypes.c_int), ("rate", ctypes.c_double)]


class ChainMatrix(ctypes.Structure):
    _fields_ = [("stages", ctypes.c_void_p * 4), ("y", ctypes.c_void_p), ("y_bf16", ctypes.c_void_p),
                ("y_add", ctypes.c_void_p), ("rows", ctypes.c_int)]


# chain op input transforms (sparkmv_chain_add_vq x_mode)
X_MODE_BF16, X_MODE_F32, X_MODE_NORM = 0, 1, 2


# ggml tensor types the GGUF reader hands out
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q6_K, GGML_BF16 = 0, 1, 8, 14, 30


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
    "sparkmv_vq_gemv_ready": (_I, [_I] * 6),
    "sparkmv_vq_gemv": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _I, _P]),
    "sparkmv_vq_gemv_multi": (_I, [ctypes.POINTER(VqMatrix), _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _I, _P]),
    "sparkmv_vq_gemv_norm": (_I, [ctypes.POINTER(VqMatrix), _I, _I, _I, _I, _I, _I, _P, _P, ctypes.c_float, _P, _I,
                                  _P]),
    "sparkmv_vq_dequant": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _P]),
    "sparkmv_q6k_gemv": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_q8_0_gemv": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_q6k_dequant": (_I, [_P, _I, _I, _P, _P]),
    "sparkmv_q8_0_dequant": (_I, [_P, _I, _I, _P, _P]),
    "sparkmv_vq_prefill": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_vq_prefill_noalloc": (_I, [_PP, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P]),
    "sparkmv_prefill_fold": (_I, [_I]),
    "sparkmv_plan_create": (_P, []),
    "sparkmv_plan_destroy": (None, [_P]),
    "sparkmv_plan_size": (_I, [_P]),
    "sparkmv_plan_add_vq": (_I, [_P, ctypes.POINTER(VqMatrix), _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _I]),
    "sparkmv_plan_add_kquant": (_I, [_P, _I, _P, _I, _I, _P, _I, _I, _I, _P, _I, _I]),
    "sparkmv_plan_run": (_I, [_P, _P]),
    "sparkmv_plan_capture": (_I, [_P, _P]),
    "sparkmv_plan_launch": (_I, [_P, _P]),
    "sparkmv_plan_time_ops": (_I, [_P, _P, _I, _D]),
    "sparkmv_plan_apply_profile": (_I, [_P, _P, _U64, ctypes.c_char_p]),
    "sparkmv_plan_op_kernel": (_I, [_P, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "sparkmv_chain_create": (_P, []),
    "sparkmv_chain_destroy": (None, [_P]),
    "sparkmv_chain_size": (_I, [_P]),
    "sparkmv_chain_tune": (_I, [_P, _I, _I, _I]),
    "sparkmv_chain_add_vq": (_I, [_P, ctypes.POINTER(ChainMatrix), _I, _I, _I, _I, _I, _I, _P, _I, _P,
                                  ctypes.c_float, _P, _P, _I]),
    "sparkmv_chain_add_norm": (_I, [_P, _P, _I, _P, ctypes.c_float, _P, _I]),
    "sparkmv_chain_launch": (_I, [_P, _P]),
    "sparkmv_chain_status": (_I, [_P]),
    "sparkmv_chain_op_shape": (_I, [_P, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "sparkmv_chain_trace": (_I, [_P, _P, ctypes.c_long]),
    "sparkmv_probe_startup": (_I, [ctypes.POINTER(_S), _I, _I, _D]),
    "sparkmv_probe_handoff": (_I, [ctypes.POINTER(_I), _I, _D]),
    "sparkmv_probe_read_chain": (_I, [ctypes.POINTER(_S), _I, _I, _D]),
    "sparkmv_gguf_open": (_P, [ctypes.c_char_p]),
    "sparkmv_gguf_close": (None, [_P]),
    "sparkmv_gguf_version": (_I, [_P]),
    "sparkmv_gguf_tensor_count": (ctypes.c_int64, [_P]),
    "sparkmv_gguf_find": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "sparkmv_gguf_tensor_info": (_I, [_P, ctypes.c_int64, ctypes.POINTER(GgufTensor)]),
    "sparkmv_gguf_tensor_data": (_P, [_P, ctypes.c_int64, ctypes.POINTER(_U64)]),
    "sparkmv_gguf_kv_count": (ctypes.c_int64, [_P]),
    "sparkmv_gguf_kv_key": (_I, [_P, ctypes.c_int64, ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_uint32)]),
    "sparkmv_gguf_get_u64": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "sparkmv_gguf_get_f64": (_I, [_P, ctypes.c_char_p, _D]),
    "sparkmv_gguf_get_str": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p, _I]),
    "sparkmv_gguf_get_arr_len": (ctypes.c_int64, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]),
    "sparkmv_manifest_open": (_P, [ctypes.c_char_p]),
    "sparkmv_manifest_close": (None, [_P]),
    "sparkmv_manifest_count": (_I, [_P]),
    "sparkmv_manifest_entry": (_I, [_P, _I, ctypes.c_char_p, _I, ctypes.POINTER(_I), ctypes.POINTER(_I),
                                    ctypes.POINTER(_I)]),
    "sparkmv_manifest_read": (_I, [_P, ctypes.c_char_p, _PP, ctypes.POINTER(_S), ctypes.POINTER(_I)]),
    "sparkmv_model_create": (_P, [ctypes.POINTER(ModelCfg)]),
    "sparkmv_model_destroy": (None, [_P]),
    "sparkmv_model_set_layer": (_I, [_P, _I, ctypes.POINTER(ModelLayer)]),
    "sparkmv_model_set_head": (_I, [_P, _I, _PP, _P, _P]),
    "sparkmv_model_forward": (_I, [_P, ctypes.c_uint32, _I, _P, _P]),
    "sparkmv_model_capture": (_I, [_P, _P, _P]),
    "sparkmv_model_replay": (_I, [_P, ctypes.c_uint32, _I, _P]),
    "sparkmv_model_verify": (_I, [_P, ctypes.POINTER(ctypes.c_uint32), _I, _I, _P, _P]),
    "sparkmv_model_forward_batch": (_I, [_P, ctypes.POINTER(ctypes.c_uint32), _I, _I, _P, _P]),
    "sparkmv_model_reserve": (_I, [_P, _I]),
    "sparkmv_model_rollback": (_I, [_P, _I]),
    "sparkmv_model_len": (_I, [_P]),
    "sparkmv_model_kv": (_I, [_P, _I, _PP, _PP]),
    "sparkmv_model_enable_capture": (_I, [_P, ctypes.POINTER(_I), _I]),
    "sparkmv_model_captured": (_I, [_P, _I, _PP]),
    "sparkmv_model_embed_row": (_I, [_P, ctypes.c_uint32, _P, _P]),
    "sparkmv_argmax": (_I, [_P, _I, _P, _P]),
    "sparkmv_config_load": (_I, [ctypes.c_char_p, ctypes.POINTER(ModelCfg), ctypes.POINTER(_I), _I]),
    "sparkmv_model_load": (_P, [ctypes.c_char_p, ctypes.c_char_p, _I, _I, _I]),
    "sparkmv_model_apply_profile": (_I, [_P, _P, _U64, ctypes.c_char_p]),
    "sparkmv_model_matvec_kernel": (_I, [_P, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "sparkmv_profile_fingerprint": (_I, [ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "sparkmv_profile_load": (_P, [ctypes.c_char_p]),
    "sparkmv_profile_close": (None, [_P]),
    "sparkmv_profile_trusted": (_I, [_P, _U64, ctypes.c_char_p]),
    "sparkmv_profile_count": (_I, [_P]),
    "sparkmv_profile_entry_at": (_I, [_P, _I, ctypes.POINTER(ProfileEntry)]),
    "sparkmv_profile_find": (_I, [_P, _I, _I, _I, _I, _I, _I, ctypes.POINTER(ProfileEntry)]),
    "sparkmv_profile_write": (_I, [ctypes.c_char_p, _U64, ctypes.c_char_p, ctypes.c_char_p,
                                   ctypes.POINTER(ProfileEntry), _I]),
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


def _copy_out(ptr, n):
    """n bytes at a library-owned address, as a writable numpy array of our own"""
    out = np.empty(n, dtype=np.uint8)
    if n:
        ctypes.memmove(out.ctypes.data, ptr, n)
    return out


class Gguf:
    """A GGUF v2/v3 file, memory-mapped by the library (the layout
    tools/dspark/src/gguf.rs:95-190 reads; that reader refuses Q6_K). Tensor
    bytes come back as copies, so they outlive the handle."""

    def __init__(self, path):
        self._L = lib()   # kept for __del__, which must not use module globals at interpreter exit
        self.h = self._L.sparkmv_gguf_open(os.fsencode(path))
        if not self.h:
            raise SparkmvError(f"gguf open: {last_error()}")
        self.version = lib().sparkmv_gguf_version(self.h)

    def close(self):
        if self.h:
            lib().sparkmv_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_gguf_close(self.h)
            except Exception:
                pass
            self.h = None

    def tensors(self):
        """[{name, dims (fastest first), dtype, offset, nbytes}] in file order;
        nbytes is 0 for a type the reader does not hand out."""
        out = []
        for i in range(lib().sparkmv_gguf_tensor_count(self.h)):
            t = GgufTensor()
            check(lib().sparkmv_gguf_tensor_info(self.h, i, ctypes.byref(t)), "gguf tensor info")
            out.append({"name": t.name.decode(), "dims": [int(t.dims[d]) for d in range(t.ndims)],
                        "dtype": int(t.dtype), "offset": int(t.offset), "nbytes": int(t.nbytes)})
        return out

    def _index(self, name):
        i = lib().sparkmv_gguf_find(self.h, name.encode())
        if i < 0:
            raise SparkmvError(f"gguf: no tensor {name}")
        return i

    def tensor_bytes(self, name):
        n = _U64(0)
        p = lib().sparkmv_gguf_tensor_data(self.h, self._index(name), ctypes.byref(n))
        if not p:
            raise SparkmvError(f"gguf tensor {name}: {last_error()}")
        return _copy_out(p, n.value)

    def kquant(self, name):
        """A 2-D Q8_0 or Q6_K weight as (kind 8 or 6, rows, cols, blocks): ggml
        dims are {cols, rows}, the blocks row-major, as the GEMVs take them."""
        t = self.tensors()[self._index(name)]
        kind = {GGML_Q8_0: 8, GGML_Q6_K: 6}.get(t["dtype"])
        if kind is None or len(t["dims"]) != 2:
            raise SparkmvError(f"gguf tensor {name}: type {t['dtype']} with {len(t['dims'])} dims is not a "
                               "2-D Q8_0 or Q6_K weight")
        cols, rows = t["dims"]
        return kind, rows, cols, self.tensor_bytes(name)

    def keys(self):
        out = []
        buf = ctypes.create_string_buffer(4096)
        ty = ctypes.c_uint32(0)
        for i in range(lib().sparkmv_gguf_kv_count(self.h)):
            check(lib().sparkmv_gguf_kv_key(self.h, i, buf, len(buf), ctypes.byref(ty)), "gguf key")
            out.append((buf.value.decode(), ty.value))
        return out

    def get_u64(self, key):
        v = _U64(0)
        check(lib().sparkmv_gguf_get_u64(self.h, key.encode(), ctypes.byref(v)), "gguf get")
        return v.value

    def get_f64(self, key):
        v = ctypes.c_double(0.0)
        check(lib().sparkmv_gguf_get_f64(self.h, key.encode(), ctypes.byref(v)), "gguf get")
        return v.value

    def get_str(self, key, cap=1 << 16):
        buf = ctypes.create_string_buffer(cap)
        check(lib().sparkmv_gguf_get_str(self.h, key.encode(), buf, cap), "gguf get")
        return buf.value.decode()

    def get_arr_len(self, key):
        elem = ctypes.c_uint32(0)
        n = lib().sparkmv_gguf_get_arr_len(self.h, key.encode(), ctypes.byref(elem))
        if n < 0:
            raise SparkmvError(f"gguf get: {last_error()}")
        return n, elem.value


class VqDir:
    """A VQ artifact directory: manifest.txt and one <name>.bin per tensor
    (tools/vq-runtime/src/vq_source.rs:30-104). read() validates the file
    against its manifest line and returns an RQVQ container's bytes, or a
    norm sidecar as an f32 array [rows, cols]."""

    def __init__(self, path):
        self._L = lib()
        self.h = self._L.sparkmv_manifest_open(os.fsencode(path))
        if not self.h:
            raise SparkmvError(f"manifest open: {last_error()}")

    def close(self):
        if self.h:
            lib().sparkmv_manifest_close(self.h)
            self.h = None

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_manifest_close(self.h)
            except Exception:
                pass
            self.h = None

    def entries(self):
        out = []
        buf = ctypes.create_string_buffer(4096)
        r, c, s = _I(0), _I(0), _I(0)
        for i in range(lib().sparkmv_manifest_count(self.h)):
            check(lib().sparkmv_manifest_entry(self.h, i, buf, len(buf), ctypes.byref(r), ctypes.byref(c),
                                               ctypes.byref(s)), "manifest entry")
            out.append((buf.value.decode(), r.value, c.value, s.value))
        return out

    def read(self, name):
        p, n, kind = ctypes.c_void_p(), _S(0), _I(0)
        check(lib().sparkmv_manifest_read(self.h, name.encode(), ctypes.byref(p), ctypes.byref(n),
                                          ctypes.byref(kind)), "manifest read")
        raw = _copy_out(p.value, n.value)
        if kind.value == 1:
            return raw
        e = [e for e in self.entries() if e[0] == name][0]
        return raw.view(np.float32).reshape(e[1], e[2])


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


def gemv_norm(mats, h, norm_w, ys, eps=1e-6, x_out=None, accumulate=False, stream=None):
    """One launch over up to 4 DeviceContainers of x = bf16(rms_norm(h) *
    norm_w), staged by the kernel from the f32 residual h (device f32
    [cols]); x_out (device int16 [cols]), when given, receives x."""
    arr = (VqMatrix * len(mats))()
    for i, (m, y) in enumerate(zip(mats, ys)):
        for s, p in enumerate(m.stage_ptrs):
            arr[i].stages[s] = p
        arr[i].y = y.data_ptr()
        arr[i].rows = m.rows
    h0 = mats[0].host
    check(lib().sparkmv_vq_gemv_norm(arr, len(mats), h0.nstages, h0.dim, h0.nc, h0.cols, h0.v3, h.data_ptr(),
                                     norm_w.data_ptr(), float(eps), x_out.data_ptr() if x_out is not None else None,
                                     int(accumulate), _stream_ptr(stream)), "vq gemv norm")


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


def prefill_fold(on=None):
    """The two-stage prefill's mode, process-wide: True (default) folds the
    stages into one f16 weight, False runs each stage's exact codewords
    apart. With no argument, returns the current setting; else sets it and
    returns the previous one."""
    prev = lib().sparkmv_prefill_fold(-1 if on is None else int(bool(on)))
    return bool(prev)


class prefill_mode:
    """Context manager: the two-stage prefill folded (True) or with its
    stages apart (False) inside the block, the previous mode after it."""

    def __init__(self, fold):
        self.fold = bool(fold)

    def __enter__(self):
        self.prev = prefill_fold(self.fold)
        return self

    def __exit__(self, *exc):
        prefill_fold(self.prev)
        return False


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


_CFG_FIELDS = ("hidden", "layers", "heads", "kv_heads", "head_dim", "intermediate", "vocab", "eps", "sliding_window",
               "rope_full_theta", "rope_full_partial", "rope_slide_theta", "rope_slide_partial")


def config_load(path, max_layers=4096):
    """config.json (tools/vq-runtime/src/config.rs:39-85): a dict of the
    model fields and the per-layer full-attention flags."""
    c = ModelCfg()
    full = (_I * max_layers)()
    check(lib().sparkmv_config_load(os.fsencode(str(path)), ctypes.byref(c), full, max_layers), "config load")
    cfg = {k: getattr(c, k) for k in _CFG_FIELDS}
    return cfg, [bool(full[i]) for i in range(min(c.layers, max_layers))]


class Model:
    """The decode forward on the GPU (sparkmv_model_*): one token through
    every layer, tools/vq-runtime/src/model.rs:441-591 (Model::forward).

    cfg: dict of the sparkmv_model_cfg fields. layers: per layer a dict with
    in_norm, post_norm (device f32 tensors), qkv, attn_gate, out, gate, up,
    down (DeviceContainers) and full (bool). head: a DeviceContainer (VQ) or
    a device uint8 tensor of Q8_0 blocks; final_norm a device f32 tensor.
    The model keeps references to everything it was given."""

    def __init__(self, cfg, layers, head, final_norm):
        c = ModelCfg(**cfg)
        self.cfg = dict(cfg)
        self._L = lib()
        self.h = self._L.sparkmv_model_create(ctypes.byref(c))
        if not self.h:
            raise SparkmvError("model create: " + last_error())
        self.keep = [layers, head, final_norm]
        for i, L in enumerate(layers):
            w = ModelLayer()
            w.in_norm = L["in_norm"].data_ptr()
            w.post_norm = L["post_norm"].data_ptr()
            for name in ("qkv", "attn_gate", "out", "gate", "up", "down"):
                arr = getattr(w, name)
                for s, p in enumerate(L[name].stage_ptrs):
                    arr[s] = p
            w.full = int(bool(L["full"]))
            check(lib().sparkmv_model_set_layer(self.h, i, ctypes.byref(w)), "model layer %d" % i)
        if isinstance(head, DeviceContainer):
            arr = (ctypes.c_void_p * 4)(*(head.stage_ptrs + [None] * (4 - len(head.stage_ptrs))))
            check(lib().sparkmv_model_set_head(self.h, 0, ctypes.cast(arr, _PP), None, final_norm.data_ptr()),
                  "model head")
        else:
            check(lib().sparkmv_model_set_head(self.h, 8, None, head.data_ptr(), final_norm.data_ptr()), "model head")

    @classmethod
    def load(cls, directory, config_path, max_ctx, x_dtype=X_BF16, apply_profile=True):
        """The whole model from a VQ artifact directory and config.json
        (sparkmv_model_load: model.rs:121-185 over VqDir); the model owns
        the weights it uploaded. profile_note says what became of
        DIR/vq-tune.profile (a bad or foreign profile keeps the heuristic)."""
        self = cls.__new__(cls)
        self._L = lib()
        self.h = self._L.sparkmv_model_load(os.fsencode(str(directory)), os.fsencode(str(config_path)), int(max_ctx),
                                          int(x_dtype), int(bool(apply_profile)))
        if not self.h:
            raise SparkmvError("model load: " + last_error())
        self.profile_note = last_error()
        cfg, _ = config_load(config_path)
        self.cfg = dict(cfg, max_ctx=int(max_ctx), x_dtype=int(x_dtype))
        self.keep = []
        return self

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_model_destroy(self.h)
            except Exception:
                pass
            self.h = None

    def forward(self, token, pos, logits, stream=None):
        """logits: device f32 [vocab]; asynchronous on stream."""
        check(lib().sparkmv_model_forward(self.h, int(token), int(pos), logits.data_ptr(), _stream_ptr(stream)),
              "model forward")

    def capture(self, logits, stream):
        """Record one token's launches as a HIP graph writing logits (run
        forward once first); stream must be a created torch stream."""
        check(lib().sparkmv_model_capture(self.h, logits.data_ptr(), _stream_ptr(stream)), "model capture")
        self.keep.append(logits)

    def replay(self, token, pos, stream):
        check(lib().sparkmv_model_replay(self.h, int(token), int(pos), _stream_ptr(stream)), "model replay")

    def verify(self, tokens, pos, logits, stream=None):
        """A block of up to 8 tokens at pos .. (vq-model-gpu.cu:955-969);
        logits: device f32 [len(tokens), vocab]."""
        arr = (ctypes.c_uint32 * len(tokens))(*[int(t) for t in tokens])
        check(lib().sparkmv_model_verify(self.h, arr, len(tokens), int(pos), logits.data_ptr(), _stream_ptr(stream)),
              "model verify")

    def forward_batch(self, tokens, pos, logits=None, stream=None):
        """A prompt chunk of up to 512 tokens at pos .. (vq-model-gpu.cu:858-953
        forward_batch + tail_logits): fills their cache rows; logits (device
        f32 [vocab]), when given, gets the last token's."""
        arr = (ctypes.c_uint32 * len(tokens))(*[int(t) for t in tokens])
        check(lib().sparkmv_model_forward_batch(self.h, arr, len(tokens), int(pos),
                                                logits.data_ptr() if logits is not None else None,
                                                _stream_ptr(stream)), "model forward batch")

    def reserve(self, ntok):
        """Allocate the block buffers for up to ntok tokens now."""
        check(lib().sparkmv_model_reserve(self.h, int(ntok)), "model reserve")

    def rollback(self, pos):
        """Keep the first pos cached positions (model.rs:361-381)."""
        check(lib().sparkmv_model_rollback(self.h, int(pos)), "model rollback")

    def __len__(self):
        return lib().sparkmv_model_len(self.h)

    def apply_profile(self, profile, artifact, gpu):
        n = lib().sparkmv_model_apply_profile(self.h, profile.h, artifact, gpu.encode())
        check(0 if n >= 0 else -1, "model apply profile")
        return n

    def matvec_kernel(self, rows, cols):
        v, t = ctypes.c_int(), ctypes.c_int()
        check(lib().sparkmv_model_matvec_kernel(self.h, rows, cols, ctypes.byref(v), ctypes.byref(t)), "model kernel")
        return v.value, t.value

    def kv(self, layer):
        """(k, v) device pointers of the layer's cache, [max_ctx][kv_dim] f32 each."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib().sparkmv_model_kv(self.h, layer, ctypes.byref(k), ctypes.byref(v)), "model kv")
        return k.value, v.value

    def reset(self):
        """Forget every cached position (model.rs:384-397)."""
        self.rollback(0)

    def enable_capture(self, layers):
        """Capture the residual entering each listed layer at every position
        from now on (model.rs:322-348); slot k is layers[k]."""
        arr = (_I * len(layers))(*[int(x) for x in layers])
        check(lib().sparkmv_model_enable_capture(self.h, arr, len(layers)), "model capture")
        self.capture_layers = [int(x) for x in layers]

    def captured(self, k):
        """Slot k's current rows as a new device f32 tensor [positions, hidden]
        (model.rs:346-348)."""
        torch = _torch()
        rows = ctypes.c_void_p()
        n = lib().sparkmv_model_captured(self.h, int(k), ctypes.byref(rows))
        check(0 if n >= 0 else -1, "model captured")
        hidden = self.cfg["hidden"]
        out = torch.empty((n, hidden), dtype=torch.float32, device="cuda")
        if n:
            _hip_copy(out.data_ptr(), rows.value, n * hidden * 4)
        return out

    def embed_row(self, token, out=None, stream=None):
        """The tied embedding row of token (model.rs:352-354), device f32 [hidden]."""
        torch = _torch()
        if out is None:
            out = torch.empty(self.cfg["hidden"], dtype=torch.float32, device="cuda")
        check(lib().sparkmv_model_embed_row(self.h, int(token), out.data_ptr(), _stream_ptr(stream)),
              "model embed row")
        return out


def argmax(logits, stream=None):
    """Model::argmax (model.rs:594-605) of a device f32 vector on the GPU:
    the first of equal maxima; returns a device int32 tensor of one element."""
    torch = _torch()
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    check(lib().sparkmv_argmax(logits.data_ptr(), logits.numel(), out.data_ptr(), _stream_ptr(stream)), "argmax")
    return out


def _hip_copy(dst, src, nbytes):
    """A device-to-device copy between raw pointers (the HIP runtime torch
    already loaded), synchronous."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemcpy.argtypes = [_P, _P, _S, _I]
    rc = hip.hipMemcpy(dst, src, nbytes, 3)
    if rc != 0:
        raise SparkmvError(f"device copy failed ({rc})")


def profile_fingerprint(dirpath):
    """The VQ artifact directory's FNV-1a fingerprint (tools/vq/gpu/vq-profile.h:118-146)."""
    h = ctypes.c_uint64()
    check(lib().sparkmv_profile_fingerprint(os.fsencode(dirpath), ctypes.byref(h)), "profile fingerprint")
    return h.value


class Profile:
    """A VQPROF 1 tuning profile (tools/vq/gpu/vq-profile.h): entries per
    geometry, trusted only for the artifact and device that measured it."""

    def __init__(self, path):
        self._L = lib()
        self.h = self._L.sparkmv_profile_load(os.fsencode(path))
        if not self.h:
            raise SparkmvError("profile load: " + last_error())

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_profile_close(self.h)
            except Exception:
                pass
            self.h = None

    def trusted(self, artifact, gpu):
        rc = lib().sparkmv_profile_trusted(self.h, artifact, gpu.encode())
        check(0 if rc >= 0 else -1, "profile trust")
        return rc == 1

    def entries(self):
        out = []
        for i in range(lib().sparkmv_profile_count(self.h)):
            e = ProfileEntry()
            check(lib().sparkmv_profile_entry_at(self.h, i, ctypes.byref(e)), "profile entry")
            out.append(e)
        return out

    def find(self, kind, dim, nc, rows, cols, v3):
        """The entry for a geometry, or None (kind 0 gemv, 1 prefill)."""
        e = ProfileEntry()
        if lib().sparkmv_profile_find(self.h, kind, dim, nc, rows, cols, v3, ctypes.byref(e)) != 0:
            return None
        return e


def profile_write(path, artifact, gpu, driver, entries):
    arr = (ProfileEntry * max(1, len(entries)))(*entries)
    check(lib().sparkmv_profile_write(os.fsencode(path), artifact, gpu.encode(), driver.encode(), arr, len(entries)),
          "profile write")


TUNE_GATE = 1e-4   # tools/vq-tune/src/main.rs:107-108 (GEMV_GATE, PREFILL_GATE)


def _tune_activations(n):
    """tools/vq-tune/src/main.rs:89-91: sin(0.001 i) in f64, rounded to f32."""
    return np.sin(np.arange(n, dtype=np.float64) * 0.001).astype(np.float32)


def _tune_rel_l2(a, b):
    """tools/vq-tune/src/kernels.rs:241-253: ||a - b|| / ||b||, 0/0 = 0."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d, n = float(np.sum((a - b) ** 2)), float(np.sum(b * b))
    if n == 0.0:
        return 0.0 if d == 0.0 else float("inf")
    return (d / n) ** 0.5


def tune(mats, iters=20, tokens=512, prefill=True):
    """tools/vq-tune's sweep (main.rs:110-225) on the current device, per
    distinct geometry of the DeviceContainers, every stage through the
    reference ABI with the tuner's activations:

      gemv: a reference output from variant 3, else 2, else 1, at 256 threads;
        then every ready variant (3, 2, 1, 0) at each width (0 at 256, the
        others at 128, 256 and 512). A candidate whose output differs from
        the reference's by more than 1e-4 relative L2 is rejected; the fastest
        survivor (GB/s of container) is the entry.
      prefill (`tokens` tokens, xT [cols][tokens] f32): the reference is tile
        128 x 64 of variant 1 when ready, else the legacy variant 3; the
        candidates are every ready tile of variants 1 and 2 (only 3 when no
        tile is ready), gated the same way; the fastest (tokens/s) wins.

    Returns (entries, rejected): ProfileEntry records (kind 0 gemv, 1 prefill)
    and (kind, geometry, candidate, relL2) for every gated-out candidate."""
    torch = _torch()
    L = lib()
    entries, rejected, seen = [], [], set()
    for m in mats:
        h = m.host
        g = (h.dim, h.nc, h.rows, h.cols, h.v3)
        if g in seen:
            continue
        seen.add(g)
        nbytes = float(h.data.nbytes) if hasattr(h, "data") else float(h.stage_bytes * h.nstages)
        x = torch.from_numpy(_tune_activations(h.cols)).to("cuda")
        y = torch.zeros(h.rows, device="cuda")

        def gemv(variant, threads, n):
            y.zero_()
            total = 0.0
            for p in m.stage_ptrs:
                ms = ctypes.c_double()
                check(L.vqg_gemv_t(p, *g, x.data_ptr(), y.data_ptr(), variant, threads, n, ctypes.byref(ms)),
                      "vqg_gemv_t")
                total += ms.value
            return total, (y.cpu().numpy().copy() if n == 1 else None)

        ready = lambda v: L.vqg_gemv_ready(*g, v) != 0  # noqa: E731
        ref_v = 3 if ready(3) else (2 if ready(2) else 1)
        _, ref_out = gemv(ref_v, 256, 1)
        best = None
        for variant in (3, 2, 1, 0):
            if not ready(variant):
                continue
            for th in ((256,) if variant == 0 else (128, 256, 512)):
                _, out = gemv(variant, th, 1)
                rel = _tune_rel_l2(out, ref_out)
                if rel > TUNE_GATE:
                    rejected.append((0, g, (variant, th), rel))
                    continue
                ms, _ = gemv(variant, th, iters)
                gbs = nbytes / (ms * 1e-3) / 1e9
                if best is None or gbs > best[2]:
                    best = (variant, th, gbs)
        if best is None:
            raise SparkmvError(f"no runnable gemv variant for {g}")
        entries.append(ProfileEntry(kind=0, dim=h.dim, nc=h.nc, rows=h.rows, cols=h.cols, v3=h.v3,
                                    variant=best[0], threads=best[1], rate=best[2]))
        if not prefill:
            continue
        xt = torch.from_numpy(_tune_activations(h.cols * tokens).reshape(h.cols, tokens)).to("cuda")
        yb = torch.zeros(tokens, h.rows, device="cuda")

        def pre(variant, bn, bk, n):
            yb.zero_()
            total = 0.0
            for p in m.stage_ptrs:
                ms = ctypes.c_double()
                check(L.vqg_prefill_tile(p, *g, xt.data_ptr(), tokens, yb.data_ptr(), n, ctypes.byref(ms), bn, bk,
                                         variant), "vqg_prefill_tile")
                total += ms.value
            return total, (yb.cpu().numpy().copy() if n == 1 else None)

        tile_ready = lambda bn, bk, v: L.vqg_prefill_cfg_ready(*g, bn, bk, v) != 0  # noqa: E731
        ref_t = (1, 128, 64) if tile_ready(128, 64, 1) else (3, 0, 0)
        _, ref_out = pre(*ref_t, 1)
        cands = []
        if ref_t[0] == 3:
            cands.append((3, 0, 0))
        else:
            for i in range(L.vqg_prefill_cfg_count()):
                bn, bk = ctypes.c_int(), ctypes.c_int()
                check(L.vqg_prefill_cfg(i, ctypes.byref(bn), ctypes.byref(bk)), "vqg_prefill_cfg")
                for variant in (1, 2):
                    if tile_ready(bn.value, bk.value, variant):
                        cands.append((variant, bn.value, bk.value))
        best = None
        for cand in cands:
            _, out = pre(*cand, 1)
            rel = _tune_rel_l2(out, ref_out)
            if rel > TUNE_GATE:
                rejected.append((1, g, cand, rel))
                continue
            ms, _ = pre(*cand, iters)
            tps = tokens / (ms * 1e-3)
            if best is None or tps > best[3]:
                best = (*cand, tps)
        if best is None:
            raise SparkmvError(f"no runnable prefill path for {g}")
        entries.append(ProfileEntry(kind=1, dim=h.dim, nc=h.nc, rows=h.rows, cols=h.cols, v3=h.v3,
                                    variant=best[0], bn=best[1], bk=best[2], rate=best[3]))
    return entries, rejected


def device_name():
    """vqg_device_name: the name a profile's trust check compares."""
    buf = ctypes.create_string_buffer(256)
    check(lib().vqg_device_name(buf, 256), "device name")
    return buf.value.decode()


class Plan:
    """A recorded chain of matvec launches (sparkmv_plan_*): run eagerly or
    replayed as one HIP graph. Holds references to every tensor it uses."""

    def __init__(self):
        self._L = lib()
        self.h = self._L.sparkmv_plan_create()
        self.keep = []
        self.labels = []

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_plan_destroy(self.h)
            except Exception:
                pass
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

    def apply_profile(self, profile, artifact, gpu):
        """Apply a trusted Profile (sparkmv_plan_apply_profile): returns the
        number of ops changed; last_error() then counts refused entries."""
        n = lib().sparkmv_plan_apply_profile(self.h, profile.h, artifact, gpu.encode())
        check(0 if n >= 0 else -1, "plan apply profile")
        return n

    def op_kernel(self, i):
        v, t = ctypes.c_int(), ctypes.c_int()
        check(lib().sparkmv_plan_op_kernel(self.h, i, ctypes.byref(v), ctypes.byref(t)), "plan op kernel")
        return v.value, t.value

    def time_ops(self, stream=None, iters=5):
        n = len(self)
        out = (ctypes.c_double * n)()
        check(lib().sparkmv_plan_time_ops(self.h, _stream_ptr(stream), iters, out), "plan time")
        return np.array(out[:], dtype=np.float64)


def _ptr(t):
    return None if t is None else t.data_ptr()


class Chain:
    """A chain of VQ matvecs run as one persistent launch (sparkmv_chain_*).
    Each op waits (wait=True) until every workgroup has published the ops
    before it; holds references to every tensor it uses."""

    def __init__(self):
        self._L = lib()
        self.h = self._L.sparkmv_chain_create()
        self.keep = []
        self.labels = []

    def __del__(self):
        # only attributes of self: at interpreter exit the module's globals may be gone
        L = getattr(self, "_L", None)
        if getattr(self, "h", None) and L is not None:
            try:
                L.sparkmv_chain_destroy(self.h)
            except Exception:
                pass
            self.h = None

    def __len__(self):
        return lib().sparkmv_chain_size(self.h)

    def tune(self, waves=12, look=2, min_units=0):
        check(lib().sparkmv_chain_tune(self.h, waves, look, min_units), "chain tune")

    def add_vq(self, mats, x, x_mode, ys=None, ys_bf16=None, y_add=None, norm_w=None, eps=1e-6, x_out=None,
               act=None, wait=True, label="vq"):
        """mats: DeviceContainers sharing x (two stages, dim 4, DQV3). x: the
        input (bf16 as int16/uint16 for X_MODE_BF16, f32 otherwise). ys,
        ys_bf16, y_add: per matrix tensors or None. act: bf16 output of a
        gate/up pair (mats = [gate, up])."""
        n = len(mats)
        ys = ys or [None] * n
        ys_bf16 = ys_bf16 or [None] * n
        y_add = y_add or [None] * n
        arr = (ChainMatrix * n)()
        for i, m in enumerate(mats):
            for s_, p in enumerate(m.stage_ptrs):
                arr[i].stages[s_] = p
            arr[i].y = _ptr(ys[i])
            arr[i].y_bf16 = _ptr(ys_bf16[i])
            arr[i].y_add = _ptr(y_add[i])
            arr[i].rows = m.rows
        h = mats[0].host
        check(lib().sparkmv_chain_add_vq(self.h, arr, n, h.nstages, h.dim, h.nc, h.cols, h.v3, x.data_ptr(), x_mode,
                                         _ptr(norm_w), eps, _ptr(x_out), _ptr(act), int(wait)), "chain add vq")
        self.keep.append((mats, x, ys, ys_bf16, y_add, norm_w, x_out, act))
        self.labels.append(label)

    def add_norm(self, x, out, norm_w=None, eps=1e-6, wait=True, label="norm"):
        check(lib().sparkmv_chain_add_norm(self.h, x.data_ptr(), x.numel(), _ptr(norm_w), eps, out.data_ptr(),
                                           int(wait)), "chain add norm")
        self.keep.append((x, out, norm_w))
        self.labels.append(label)

    def launch(self, stream=None):
        check(lib().sparkmv_chain_launch(self.h, _stream_ptr(stream)), "chain launch")

    def status(self):
        check(lib().sparkmv_chain_status(self.h), "chain")

    def trace(self, on=True, device="cuda"):
        """Record a phase trace in every later launch (on=False stops it).
        Returns the int32 device tensor [workgroups, ops, 10] that each launch
        overwrites: the 100 MHz clock (low 32 bits) at each op's start, x
        arrived, x staged, step loop entered, wave 0's steps done, every unit
        done, epilogue issued and x requested, then the shader clock at the
        op's start and end."""
        torch = _torch()
        if not on:
            if lib().sparkmv_chain_trace(self.h, None, 0) < 0:
                check(-1, "chain trace")
            self.trace_buf = None
            return None
        need = lib().sparkmv_chain_trace(self.h, None, 0)
        if need < 0:
            check(need, "chain trace")
        n = len(self)
        buf = torch.zeros(need // (10 * n), n, 10, dtype=torch.int32, device=device)
        if lib().sparkmv_chain_trace(self.h, ctypes.c_void_p(buf.data_ptr()), need) < 0:
            check(-1, "chain trace")
        self.trace_buf = buf
        return buf

    def op_shape(self, i):
        S, C, msc = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().sparkmv_chain_op_shape(self.h, i, ctypes.byref(S), ctypes.byref(C), ctypes.byref(msc)),
              "chain shape")
        return S.value, C.value, msc.value


def probe_startup(sizes=(8 << 20, 20 << 20, 40 << 20), reps=20):
    """Launch start-up split (sparkmv_probe_startup), kernel-exact medians
    in µs: {"empty", "empty_1wave", "empty_1wg", "empty_stream",
    "empty_graph", "stage_64k", sizes[i]: {"cold", "page_warm",
    "line_warm"}}."""
    n = len(sizes)
    sz = (_S * n)(*sizes)
    out = (ctypes.c_double * (6 + 3 * n))()
    check(lib().sparkmv_probe_startup(sz, n, int(reps), out), "probe startup")
    res = {"empty": out[0], "empty_1wave": out[1], "stage_64k": out[2], "empty_1wg": out[3 + 3 * n],
           "empty_stream": out[4 + 3 * n], "empty_graph": out[5 + 3 * n]}
    for i, b in enumerate(sizes):
        res[int(b)] = {"cold": out[3 + 3 * i], "page_warm": out[4 + 3 * i], "line_warm": out[5 + 3 * i]}
    return res


def probe_handoff(nwords=(1280, 2560, 5120)):
    """µs per dependent op over every workgroup (sparkmv_probe_handoff):
    {"epoch_words" | "sentinel" | "fence_counter": {n: us}}."""
    n = len(nwords)
    arr = (_I * n)(*nwords)
    out = (ctypes.c_double * (3 * n))()
    check(lib().sparkmv_probe_handoff(arr, n, out), "probe handoff")
    return {name: {int(w): out[m * n + i] for i, w in enumerate(nwords)}
            for m, name in enumerate(("epoch_words", "sentinel", "fence_counter"))}


def probe_read_chain(sizes, reps=10):
    """The floor of one launch per matvec with no compute
    (sparkmv_probe_read_chain): plain reads of the given byte counts back to
    back, {"graph_us": per replay, "stream_us": per eager pass}."""
    n = len(sizes)
    arr = (ctypes.c_size_t * n)(*sizes)
    out = (ctypes.c_double * 2)()
    check(lib().sparkmv_probe_read_chain(arr, n, reps, out), "probe read chain")
    return {"graph_us": out[0], "stream_us": out[1]}


# The decode token's matvecs in the order the forward issues them
# (tools/vq-runtime/src/model.rs:481-590; tools/vq/gpu/vq-model-gpu.cu:776-835).
DECODE_MATS = ("q", "k", "v", "g", "o", "gate", "up", "down")


class DecodeChain:
    """The per-token matvec chain of the decode forward, without attention,
    as one chain launch plus the tied Q8_0 head:

        per layer l (h[l] the f32 residual):
          q, k, v, g = W_qkvg  bf16(rms_norm(h[l]))         one op, four matrices
          hm[l]      = h[l]  + W_o    bf16(q)                 attention left out: o reads q
          gate, up   = W_gu   bf16(rms_norm(hm[l]))           a pair: act = bf16(gelu(gate) * up)
          h[l + 1]   = hm[l] + W_down act
        hn = bf16(rms_norm(h[L])); logits = Q8_0 head . hn    (a second launch)

    Every op waits for the one before it, as in the forward. Every
    intermediate is kept in its own buffer, so each op can be checked from
    what the GPU actually read. layers: per layer a dict of DeviceContainers
    keyed by DECODE_MATS; head: device Q8_0 blocks (head_rows x hidden)."""

    def __init__(self, layers, head, head_rows, h0, eps=1e-6, device="cuda", record_inputs=False):
        """record_inputs: every op also writes its staged bf16 input to
        self.xouts[op] (4 ops per layer), for checks."""
        torch = _torch()
        self.L = len(layers)
        self.layers = layers
        self.eps = eps
        hid = layers[0]["q"].cols
        self.hidden = hid
        qd, kvd, gd = layers[0]["q"].rows, layers[0]["k"].rows, layers[0]["g"].rows
        ffn = layers[0]["gate"].rows
        L = self.L
        z = lambda *shape: torch.zeros(*shape, device=device)  # noqa: E731
        zi = lambda *shape: torch.zeros(*shape, dtype=torch.int16, device=device)  # noqa: E731
        self.h = z(L + 1, hid)
        self.h[0].copy_(h0)
        self.hm = z(L, hid)
        self.q, self.k, self.v, self.g = z(L, qd), z(L, kvd), z(L, kvd), z(L, gd)
        self.q16 = zi(L, qd)
        self.gate, self.up = z(L, ffn), z(L, ffn)
        self.act = zi(L, ffn)
        self.hn = zi(hid)
        self.head, self.head_rows = head, head_rows
        self.logits = z(head_rows)
        self.xouts = None
        if record_inputs:
            self.xouts = [zi(n) for _ in range(L) for n in (hid, qd, hid, ffn)]
        xo = (lambda i: self.xouts[i]) if record_inputs else (lambda i: None)  # noqa: E731
        c = Chain()
        for l, m in enumerate(layers):
            c.add_vq([m["q"], m["k"], m["v"], m["g"]], self.h[l], X_MODE_NORM,
                     ys=[self.q[l], self.k[l], self.v[l], self.g[l]], ys_bf16=[self.q16[l], None, None, None],
                     eps=eps, x_out=xo(4 * l), wait=l > 0, label=f"L{l}:q+k+v+g")
            c.add_vq([m["o"]], self.q16[l], X_MODE_BF16, ys=[self.hm[l]], y_add=[self.h[l]], x_out=xo(4 * l + 1),
                     label=f"L{l}:o")
            c.add_vq([m["gate"], m["up"]], self.hm[l], X_MODE_NORM, ys=[self.gate[l], self.up[l]], eps=eps,
                     act=self.act[l], x_out=xo(4 * l + 2), label=f"L{l}:gate+up")
            c.add_vq([m["down"]], self.act[l], X_MODE_BF16, ys=[self.h[l + 1]], y_add=[self.hm[l]],
                     x_out=xo(4 * l + 3), label=f"L{l}:down")
        c.add_norm(self.h[L], self.hn, eps=eps, label="final norm")
        self.chain = c

    def launch(self, stream=None):
        self.chain.launch(stream)
        kquant_gemv("q8_0", self.head, self.head_rows, self.hidden, self.hn.view(1, -1), self.logits.view(1, -1),
                    stream=stream)
