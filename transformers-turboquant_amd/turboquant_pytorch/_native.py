"""ctypes binding of libtq_amd.so, the gfx950 C-ABI library (include/tq_api.h).

Torch supplies device memory and the current HIP stream; every call passes raw
data pointers plus shapes and strides.  The library is mandatory for tensors on
a GPU: if it is missing or fails to load, :func:`lib` raises instead of letting
callers drop to another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = "libtq_amd.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

TQ_F32, TQ_F16, TQ_BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: TQ_F32, torch.float16: TQ_F16, torch.bfloat16: TQ_BF16}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> argument types (return type is int status unless listed in _RESTYPE)
_SIGNATURES = {
    "tq_version": [],
    "tq_last_error": [],
    "tq_out_cols": [_i64, _i32],
    "tq_pack_bits": [_p, _i64, _i32, _i64, _i32, _p, _i64, _p],
    "tq_unpack_bits": [_p, _i64, _i32, _i64, _i32, _p, _i64, _p],
    "tq_quantize_pack": [_p, _i64, _i32, _i64, _p, _i32, _p, _i64, _p],
    "tq_dequantize": [_p, _i64, _i32, _i64, _p, _i32, _p, _i64, _p],
    "tq_compress_keys": [_p, _i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64,
                         _p, _p, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p],
    "tq_compress_values": [_p, _i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64,
                           _p, _p, _i32, _p, _p, _p, _p],
    "tq_decompress_values": [_p, _p, _i64, _i32, _p, _p, _i32, _p, _i32, _i64, _p],
    "tq_query_prep": [_p, _i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _p, _p, _p],
    "tq_cache_append": [_p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64,
                        _p, _p, _p, _p, _i32, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _i64, _i64,
                        _p, _i32, _i64, _i64, _i64, _p, _p, _p, _p],
    "tq_attention_scores": [_p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                            _i32, _f32, _p, _p],
    "tq_attention_fwd": [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i32, _p,
                         _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _i32,
                         _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64, _p],
    "tq_attention_scores_kv": [_p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i32,
                               _i32, _f32, _p, _p],
    "tq_attention_fwd_kv": [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i32, _p,
                            _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _f32, _i32,
                            _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64, _p],
    "tq_attention_workspace_size": [_i32, _i32, _i32, _i32, _i32, _i32, _i32],
    "tq_attention_fwd_kv_noalloc": [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i32, _p,
                                    _i32, _i32, _i32, _i32, _i32, _i64, _i32, _f32, _f32, _i32,
                                    _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p],
    "tq_noalloc_scratch_bytes": [],
}
_RESTYPE = {"tq_last_error": ctypes.c_char_p, "tq_out_cols": _i64, "tq_attention_workspace_size": _i64,
            "tq_noalloc_scratch_bytes": _i64}

EXPORTED = tuple(_SIGNATURES)


def library_path() -> str:
    return _LIB_PATH


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the shared library and declare every entry point's signature."""
    cdll = ctypes.CDLL(path or _LIB_PATH, mode=ctypes.RTLD_LOCAL)
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return cdll


def lib() -> ctypes.CDLL:
    """The process-wide library handle; raises RuntimeError if it cannot load."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(_LIB_PATH):
                    raise RuntimeError(
                        f"TurboQuant HIP library not built: {_LIB_PATH} is missing. "
                        "Run `python -c 'import __graft_entry__ as g; g.build()'` "
                        "or `make -C transformers-turboquant_amd/csrc`."
                    )
                _lib = load()
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().tq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported activation dtype {dt}; expected float32, float16 or bfloat16")


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what}: expected a GPU tensor, got device {t.device}")
