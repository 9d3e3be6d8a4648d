"""ctypes binding of libesda.so (the C ABI declared in include/esda.h).

The library is loaded from the package directory only (built in-tree by
``apertura_amd/build.py``); a missing library raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(HERE, "libesda.so")
_lib: ctypes.CDLL | None = None

ESDA_OK = 0
ERROR_NAMES = {1: "invalid argument", 2: "runtime error", 3: "HIP error", 4: "workspace",
               5: "device"}

# Every symbol include/esda.h declares (checked by tests/test_abi.py).
EXPORTS = (
    "esda_decode_workspace_size", "esda_decode", "esda_decode_stages", "esda_decode_status",
    "esda_kv_append",
    "esda_last_error", "esda_version",
)


class EsdaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"esda error {code} ({ERROR_NAMES.get(code, '?')}): {msg}")
        self.code = code


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("cap", ctypes.c_int32), ("window", ctypes.c_int32), ("ring", ctypes.c_int32),
        ("kv_shared", ctypes.c_int32), ("seq_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64), ("max_visible", ctypes.c_int32),
        ("split_rows", ctypes.c_int32), ("scale", ctypes.c_float),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("pos", ctypes.c_void_p),
        ("row_base", ctypes.c_void_p), ("out", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libesda.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise ImportError(f"{_LIB_PATH} is missing: build it with `python apertura_amd/build.py` "
                              "(no CPU fallback exists)")
        L = ctypes.CDLL(_LIB_PATH)
        P, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
        L.esda_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.POINTER(sz)]
        L.esda_decode.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.POINTER(DecodeArgs), P]
        L.esda_decode_stages.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.POINTER(DecodeArgs),
                                         ctypes.c_int, P]
        L.esda_decode_status.argtypes = [ctypes.POINTER(DecodeDesc), P, ctypes.POINTER(i32), P]
        L.esda_kv_append.argtypes = [P, i64, i64, i32, i32, i32, i32, P, i32, P, P]
        L.esda_last_error.restype = ctypes.c_char_p
        L.esda_last_error.argtypes = []
        L.esda_version.argtypes = []
        for name in EXPORTS:
            if name not in ("esda_last_error", "esda_version"):
                getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != ESDA_OK:
        raise EsdaError(rc, lib().esda_last_error().decode())
