"""ctypes binding of the GGUF reader and the Qwen3 host forward in
libfence_ops.so (include/fence/gguf.h, include/fence/model.h).

GGUF mirrors the reference's GGUFFile (src/gguf/gguf_parser.h:130-217):
find_tensor returns None when absent, the get_* methods raise KeyError for a
missing key and TypeError for a value of another type (the reference throws
std::runtime_error for both).  Model mirrors Qwen3Model
(src/model/qwen3.h:115-155).  Failures raise fence_ops.FenceError with the
library's status.
"""
from __future__ import annotations

import ctypes

import fence_ops
from fence_ops import FenceError

NOT_FOUND = 2
OUT_OF_MEMORY = 12
BAD_FILE = 74
TYPE_MISMATCH = 75
UNSUPPORTED = 95
SEQUENCE_FUSED = 0
SEQUENCE_REFERENCE = 1

# GGUF value and tensor type numbers (the file format's)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
F32, F16, Q8_0, Q6_K = 0, 1, 8, 14


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p),
                ("data_size_bytes", ctypes.c_uint64)]


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "embed_dim", "ff_dim", "n_heads", "n_kv_heads",
                                             "head_dim", "vocab_size", "max_ctx")] + \
               [("rope_freq_base", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("has_qk_norm", ctypes.c_int), ("has_qkv_bias", ctypes.c_int)]


_P = ctypes.c_void_p
_S = ctypes.c_char_p
_I = ctypes.c_int
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (argument types, result type), in the order of the headers
SIGNATURES = {
    "fence_gguf_open": ((_S, _PP, ctypes.c_char_p, _SZ), _I),
    "fence_gguf_close": ((_P,), None),
    "fence_gguf_version": ((_P,), _U32),
    "fence_gguf_tensor_count": ((_P,), _U64),
    "fence_gguf_metadata_count": ((_P,), _U64),
    "fence_gguf_file_size": ((_P,), _U64),
    "fence_gguf_data_offset": ((_P,), _U64),
    "fence_gguf_alignment": ((_P,), _U32),
    "fence_gguf_find_tensor": ((_P, _S, ctypes.POINTER(TensorInfo)), _I),
    "fence_gguf_tensor_at": ((_P, _U64, ctypes.POINTER(TensorInfo)), _I),
    "fence_gguf_metadata_type": ((_P, _S, ctypes.POINTER(_U32)), _I),
    "fence_gguf_get_u32": ((_P, _S, ctypes.POINTER(_U32)), _I),
    "fence_gguf_get_i32": ((_P, _S, ctypes.POINTER(ctypes.c_int32)), _I),
    "fence_gguf_get_u64": ((_P, _S, ctypes.POINTER(_U64)), _I),
    "fence_gguf_get_f32": ((_P, _S, ctypes.POINTER(ctypes.c_float)), _I),
    "fence_gguf_get_bool": ((_P, _S, ctypes.POINTER(_I)), _I),
    "fence_gguf_get_string": ((_P, _S, ctypes.POINTER(ctypes.c_char_p)), _I),
    "fence_model_load": ((_S, _I, _P, _PP, ctypes.c_char_p, _SZ), _I),
    "fence_model_free": ((_P,), None),
    "fence_model_get_config": ((_P, ctypes.POINTER(ModelConfig)), _I),
    "fence_model_set_sequence": ((_P, _I), _I),
    "fence_model_forward": ((_P, _I, _I, _PP), _I),
    "fence_model_sample_greedy": ((_P, _P, ctypes.POINTER(_I)), _I),
    "fence_model_read_tensor": ((_P, _S, _P, _U64, ctypes.POINTER(_U64)), _I),
    "fence_model_kv_cache": ((_P, _I, _PP, _PP), _I),
    "fence_model_stream": ((_P,), _P),
}

_bound = None


def lib() -> ctypes.CDLL:
    global _bound
    if _bound is None:
        handle = fence_ops.lib()
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = list(argtypes)
            fn.restype = restype
        _bound = handle
    return _bound


def _check(name, st):
    if st != 0:
        raise FenceError(name, st)


class GGUF:
    """A memory-mapped GGUF file (GGUFFile::open ... close)."""

    def __init__(self, path: str):
        self._h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        st = lib().fence_gguf_open(str(path).encode(), ctypes.byref(self._h), err, len(err))
        self.error = err.value.decode(errors="replace")
        if st != 0:
            e = FenceError("fence_gguf_open", st)
            e.reason = self.error
            raise e

    def close(self):
        if self._h:
            lib().fence_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    version = property(lambda s: lib().fence_gguf_version(s._h))
    tensor_count = property(lambda s: lib().fence_gguf_tensor_count(s._h))
    metadata_count = property(lambda s: lib().fence_gguf_metadata_count(s._h))
    file_size = property(lambda s: lib().fence_gguf_file_size(s._h))
    data_offset = property(lambda s: lib().fence_gguf_data_offset(s._h))
    alignment = property(lambda s: lib().fence_gguf_alignment(s._h))

    @staticmethod
    def _info(ti: TensorInfo) -> dict:
        return {"name": ti.name.decode(), "n_dims": ti.n_dims, "dims": tuple(ti.dims), "type": ti.type,
                "offset": ti.offset, "data": ti.data, "data_size_bytes": ti.data_size_bytes}

    def find_tensor(self, name: str):
        ti = TensorInfo()
        st = lib().fence_gguf_find_tensor(self._h, name.encode(), ctypes.byref(ti))
        if st == NOT_FOUND:
            return None
        _check("fence_gguf_find_tensor", st)
        return self._info(ti)

    def tensor_at(self, i: int) -> dict:
        ti = TensorInfo()
        _check("fence_gguf_tensor_at", lib().fence_gguf_tensor_at(self._h, i, ctypes.byref(ti)))
        return self._info(ti)

    def tensor_bytes(self, name: str) -> bytes:
        t = self.find_tensor(name)
        if t is None:
            raise KeyError(name)
        return ctypes.string_at(t["data"], t["data_size_bytes"])

    def metadata_type(self, key: str):
        t = _U32()
        st = lib().fence_gguf_metadata_type(self._h, key.encode(), ctypes.byref(t))
        return None if st == NOT_FOUND else t.value

    def _get(self, fn, ctype, key):
        v = ctype()
        st = getattr(lib(), fn)(self._h, key.encode(), ctypes.byref(v))
        if st == NOT_FOUND:
            raise KeyError(key)
        if st == TYPE_MISMATCH:
            raise TypeError(f"{key} has another type")
        _check(fn, st)
        return v.value

    def get_u32(self, key):
        return self._get("fence_gguf_get_u32", _U32, key)

    def get_i32(self, key):
        return self._get("fence_gguf_get_i32", ctypes.c_int32, key)

    def get_u64(self, key):
        return self._get("fence_gguf_get_u64", _U64, key)

    def get_f32(self, key):
        return self._get("fence_gguf_get_f32", ctypes.c_float, key)

    def get_bool(self, key):
        return bool(self._get("fence_gguf_get_bool", _I, key))

    def get_string(self, key):
        return self._get("fence_gguf_get_string", ctypes.c_char_p, key).decode()


_hip = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime libfence_ops.so is linked against (already loaded)."""
    global _hip
    if _hip is None:
        lib()
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    return _hip


def device_to_host(ptr: int, nbytes: int, stream=None) -> bytes:
    """Copies nbytes of device memory at ptr once `stream` has finished."""
    hip = _hip_runtime()
    if stream:
        st = hip.hipStreamSynchronize(stream)
        if st != 0:
            raise FenceError("hipStreamSynchronize", fence_ops.HIP_BASE + st)
    buf = ctypes.create_string_buffer(max(nbytes, 1))
    st = hip.hipMemcpy(buf, ptr, nbytes, 2)  # hipMemcpyDeviceToHost
    if st != 0:
        raise FenceError("hipMemcpy", fence_ops.HIP_BASE + st)
    return buf.raw[:nbytes]


class Model:
    """Qwen3Model::load ... unload on the current device."""

    def __init__(self, path: str, max_ctx: int = 4096, stream=None):
        self._h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(1024)
        st = lib().fence_model_load(str(path).encode(), max_ctx, stream, ctypes.byref(self._h), err, len(err))
        self.error = err.value.decode(errors="replace")
        if st != 0:
            e = FenceError("fence_model_load", st)
            e.reason = self.error
            raise e
        c = ModelConfig()
        _check("fence_model_get_config", lib().fence_model_get_config(self._h, ctypes.byref(c)))
        self.config = {name: getattr(c, name) for name, _ in ModelConfig._fields_}

    def close(self):
        if self._h:
            lib().fence_model_free(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return lib().fence_model_stream(self._h) or 0

    def set_sequence(self, seq: int):
        _check("fence_model_set_sequence", lib().fence_model_set_sequence(self._h, seq))

    def forward(self, token_id: int, pos: int) -> int:
        """Device address of the logits [vocab]."""
        out = ctypes.c_void_p()
        _check("fence_model_forward", lib().fence_model_forward(self._h, token_id, pos, ctypes.byref(out)))
        return out.value

    def sample_greedy(self, logits: int) -> int:
        t = _I()
        _check("fence_model_sample_greedy", lib().fence_model_sample_greedy(self._h, logits, ctypes.byref(t)))
        return t.value

    def logits(self, ptr: int):
        """The vocab fp32 logits at device address ptr, as numpy."""
        import numpy as np
        n = self.config["vocab_size"]
        return np.frombuffer(device_to_host(ptr, 4 * n, self.stream), np.float32).copy()

    def read_tensor(self, name: str) -> bytes:
        n = _U64()
        _check("fence_model_read_tensor", lib().fence_model_read_tensor(self._h, name.encode(), None, 0,
                                                                        ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _check("fence_model_read_tensor", lib().fence_model_read_tensor(self._h, name.encode(), buf, n.value,
                                                                        ctypes.byref(n)))
        return buf.raw[:n.value]

    def kv_cache(self, layer: int):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        _check("fence_model_kv_cache", lib().fence_model_kv_cache(self._h, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value
