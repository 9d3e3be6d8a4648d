"""ctypes binding of libesda.so (the C ABI declared in include/esda.h,
include/esda_cache.h and include/esda_prefill.h).

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

# Every function include/*.h declares (checked by tests/test_abi.py).
EXPORTS = (
    # include/esda.h
    "esda_decode_workspace_size", "esda_decode", "esda_decode_stages", "esda_decode_status",
    "esda_decode_noalloc",
    "esda_kv_append", "esda_decode_raw_workspace_size", "esda_decode_raw",
    "esda_decode_raw_stages", "esda_decode_raw_q8", "esda_decode_raw_q8_stages", "esda_quantize_raw_rows", "esda_rope_table",
    "esda_fill_i32", "esda_stream_read", "esda_last_error", "esda_version",
    # include/esda_cache.h
    "esda_cache_create", "esda_cache_destroy", "esda_cache_update", "esda_cache_update_raw",
    "esda_cache_current", "esda_cache_current_raw",
    "esda_cache_begin_step", "esda_cache_end_step", "esda_cache_set_slot", "esda_cache_slot_kv", "esda_cache_take_slot", "esda_cache_decode", "esda_cache_decode_raw", "esda_cache_slot",
    "esda_cache_seq_len", "esda_cache_mark_step", "esda_cache_reset", "esda_cache_save_snapshot",
    "esda_cache_restore_snapshot", "esda_cache_restore_snapshot_ex", "esda_cache_mark_prefix",
    "esda_cache_mark_rewind_point", "esda_cache_rewind_to_mark", "esda_cache_clear_rewind_mark",
    "esda_decode_attn_global", "esda_cache_update_raw_q8", "esda_cache_current_raw_q8",
    "esda_cache_decode_raw_q8", "esda_decode_attn_global_q8",
    # include/esda_prefill.h
    "esda_prefill_workspace_size", "esda_prefill", "esda_prefill_stages", "esda_raw_prefill_kv",
    "esda_raw_q8_prefill_kv", "esda_cache_prefill", "esda_cache_prefill_raw", "esda_lds_read",
)
_VOID = ("esda_cache_destroy", "esda_cache_mark_step", "esda_cache_reset", "esda_cache_clear_rewind_mark")

# const char *(*)(int32_t pos, void *user): the caller's prefix fingerprint at a marker
# (declared returning void *: the callback hands back the address of a buffer it keeps alive)
PREFIX_FP_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p)


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


class RawDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("cap", ctypes.c_int32), ("seq_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64), ("max_visible", ctypes.c_int32),
        ("split_rows", ctypes.c_int32), ("scale", ctypes.c_float), ("eps", ctypes.c_float),
    ]


class RawArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_new", ctypes.c_void_p), ("raw_cache", ctypes.c_void_p),
        ("pos", ctypes.c_void_p), ("kw", ctypes.c_void_p), ("inv_freq", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("rope_table", ctypes.c_void_p), ("rope_table_rows", ctypes.c_int32),
    ]


class RawQ8Args(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_new", ctypes.c_void_p), ("q8_cache", ctypes.c_void_p),
        ("scale", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("sb_seq_stride", ctypes.c_int64), ("sb_head_stride", ctypes.c_int64),
        ("pos", ctypes.c_void_p), ("kw", ctypes.c_void_p), ("inv_freq", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("rope_table", ctypes.c_void_p), ("rope_table_rows", ctypes.c_int32),
    ]


class View(ctypes.Structure):
    """esda_view: element (h, r, d) at data[h*head_stride + r*head_dim + d]."""
    _fields_ = [
        ("data", ctypes.c_void_p), ("kv_heads", ctypes.c_int32), ("rows", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("head_stride", ctypes.c_int64),
    ]


class PrefillDesc(ctypes.Structure):
    _fields_ = [
        ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("seq_q", ctypes.c_int32), ("seq_k", ctypes.c_int32), ("q_pos0", ctypes.c_int32),
        ("k_pos0", ctypes.c_int32), ("window", ctypes.c_int32),
        ("q_head_stride", ctypes.c_int64), ("q_row_stride", ctypes.c_int64),
        ("kv_head_stride", ctypes.c_int64), ("out_row_stride", ctypes.c_int64),
        ("out_head_stride", ctypes.c_int64), ("split_keys", ctypes.c_int32), ("scale", ctypes.c_float),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class Q8View(ctypes.Structure):
    """esda_q8_view: u8 rows q [kv_heads, pitch, 512], f32 scale / bias [kv_heads, pitch]."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("kv_heads", ctypes.c_int32), ("len", ctypes.c_int32), ("pitch", ctypes.c_int32),
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
        L.esda_decode_noalloc.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.POINTER(DecodeArgs), P]
        L.esda_kv_append.argtypes = [P, i64, i64, i32, i32, i32, i32, P, i32, P, P]
        L.esda_decode_raw_workspace_size.argtypes = [ctypes.POINTER(RawDesc), ctypes.POINTER(sz)]
        L.esda_decode_raw.argtypes = [ctypes.POINTER(RawDesc), ctypes.POINTER(RawArgs), P]
        L.esda_decode_raw_stages.argtypes = [ctypes.POINTER(RawDesc), ctypes.POINTER(RawArgs),
                                             ctypes.c_int, P]
        L.esda_decode_raw_q8.argtypes = [ctypes.POINTER(RawDesc), ctypes.POINTER(RawQ8Args), P]
        L.esda_decode_raw_q8_stages.argtypes = [ctypes.POINTER(RawDesc), ctypes.POINTER(RawQ8Args),
                                                ctypes.c_int, P]
        L.esda_quantize_raw_rows.argtypes = [P, i32, i32, P, i64, P, P, i64, i32, P]
        L.esda_rope_table.argtypes = [P, i32, P, P]
        L.esda_fill_i32.argtypes = [P, i32, i32, P]
        L.esda_stream_read.argtypes = [P, sz, i32, P, P]
        L.esda_lds_read.argtypes = [i32, i32, i32, i32, P, P]
        L.esda_last_error.restype = ctypes.c_char_p
        L.esda_last_error.argtypes = []
        L.esda_version.argtypes = []
        f32, VP = ctypes.c_float, ctypes.POINTER(View)
        pi32 = ctypes.POINTER(i32)
        L.esda_cache_create.argtypes = [i32, ctypes.POINTER(P)]
        L.esda_cache_destroy.argtypes = [P]
        L.esda_cache_update.argtypes = [P, i32, P, P, i32, i32, i32, i32, i32, P, VP, VP]
        L.esda_cache_update_raw.argtypes = [P, i32, P, i32, i32, i32, i32, P, VP, pi32, pi32]
        L.esda_cache_current.argtypes = [P, i32, i32, VP, VP]
        L.esda_cache_begin_step.argtypes = [P, P, P]
        L.esda_cache_end_step.argtypes = [P]
        L.esda_cache_set_slot.argtypes = [P, i32, P, P, i32, i32, i32]
        L.esda_cache_slot_kv.argtypes = [P, i32, VP, VP]
        L.esda_cache_take_slot.argtypes = [P, i32, VP, VP]
        L.esda_cache_current_raw.argtypes = [P, i32, VP, pi32, pi32]
        L.esda_cache_decode.argtypes = [P, i32, P, i32, P, P, i32, i32, i32, i32, f32, P, P]
        L.esda_cache_decode_raw.argtypes = [P, i32, P, i32, P, i32, P, f32, P, i32, P, P]
        L.esda_cache_slot.argtypes = [P, i32, pi32, pi32, pi32, pi32]
        L.esda_cache_seq_len.argtypes = [P]
        L.esda_cache_mark_step.argtypes = [P, i32]
        L.esda_cache_reset.argtypes = [P]
        L.esda_cache_save_snapshot.argtypes = [P, ctypes.c_char_p, ctypes.c_char_p, i32]
        L.esda_cache_restore_snapshot.argtypes = [P, ctypes.c_char_p, ctypes.c_char_p]
        L.esda_cache_restore_snapshot_ex.argtypes = [P, ctypes.c_char_p, ctypes.c_char_p, i32, PREFIX_FP_FN, P]
        L.esda_cache_mark_prefix.argtypes = [P, i32, ctypes.c_char_p]
        L.esda_cache_clear_rewind_mark.argtypes = [P]
        L.esda_cache_mark_rewind_point.argtypes = [P, i32]
        L.esda_cache_rewind_to_mark.argtypes = [P]
        L.esda_decode_attn_global.argtypes = [P, i32, P, i32, i32, i32, P, f32, P, i32, P, P]
        QVP = ctypes.POINTER(Q8View)
        L.esda_cache_update_raw_q8.argtypes = [P, i32, P, i32, i32, P, QVP]
        L.esda_cache_current_raw_q8.argtypes = [P, i32, QVP]
        L.esda_cache_decode_raw_q8.argtypes = [P, i32, P, i32, P, i32, P, f32, P, i32, P, P]
        L.esda_decode_attn_global_q8.argtypes = [P, i32, P, P, P, i32, i32, i32, P, f32, P, i32, P, P]
        PD = ctypes.POINTER(PrefillDesc)
        L.esda_prefill_workspace_size.argtypes = [PD, ctypes.POINTER(sz)]
        L.esda_prefill.argtypes = [PD, ctypes.POINTER(PrefillArgs), P]
        L.esda_prefill_stages.argtypes = [PD, ctypes.POINTER(PrefillArgs), ctypes.c_int, P]
        L.esda_cache_prefill.argtypes = [P, i32, P, i32, i32, P, P, i32, i32, i32, i32, f32, i32, i32, P, P]
        L.esda_cache_prefill_raw.argtypes = [P, i32, P, i32, i32, P, i32, P, f32, P, i32, i32, f32, i32, P, P]
        L.esda_raw_prefill_kv.argtypes = [P, i64, i32, i32, i32, P, f32, P, i32, P, P, i64, P]
        L.esda_raw_q8_prefill_kv.argtypes = [P, i64, P, P, i64, i32, i32, P, f32, P, i32, P, P, i64, P]
        for name in EXPORTS:
            if name in _VOID:
                getattr(L, name).restype = None
            elif name not in ("esda_last_error", "esda_version"):
                getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != ESDA_OK:
        raise EsdaError(rc, lib().esda_last_error().decode())
