"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Loaded by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` as the checker / CPU baseline; the product
package ``apertura_amd`` never imports it.

Every array argument is a numpy array; bf16 tensors travel as ``np.uint16`` bit
patterns.  See ``oracle.h`` for which reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so from oracle.c (gcc, no GPU)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class Desc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("D", ctypes.c_int32), ("cap", ctypes.c_int32), ("window", ctypes.c_int32),
        ("ring", ctypes.c_int32), ("seq_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64), ("scale", ctypes.c_float),
    ]


_P = ctypes.c_void_p


def _declare(L: ctypes.CDLL) -> None:
    i32 = ctypes.c_int32
    L.orc_f32_to_bf16_n.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_bf16_to_f32_n.argtypes = [_P, _P, ctypes.c_size_t]
    L.orc_visible.argtypes = [ctypes.POINTER(Desc), i32, i32, _P]
    L.orc_visible.restype = i32
    L.orc_append.argtypes = [ctypes.POINTER(Desc), _P, _P, _P, _P, _P, _P]
    L.orc_append.restype = i32
    for name in ("orc_decode_f64", "orc_decode_refround"):
        f = getattr(L, name)
        f.argtypes = [ctypes.POINTER(Desc), _P, _P, _P, _P, _P, _P, i32]
        f.restype = i32
    L.orc_decode_splitk.argtypes = [ctypes.POINTER(Desc), _P, _P, _P, _P, _P, i32, _P, i32]
    L.orc_decode_splitk.restype = i32
    L.orc_decode_refround_grouped.argtypes = [ctypes.POINTER(Desc), _P, _P, _P, _P, _P, i32, _P, i32]
    L.orc_decode_refround_grouped.restype = i32
    L.orc_rope_inv_freq.argtypes = [i32, ctypes.c_float, ctypes.c_float, _P]
    L.orc_rms_norm_rows.argtypes = [_P, _P, ctypes.c_int64, i32, ctypes.c_float, _P]
    L.orc_decode_raw_f64.argtypes = [_P, _P, i32, i32, i32, _P, ctypes.c_float, _P,
                                     ctypes.c_float, _P, i32]
    L.orc_decode_raw_f64.restype = i32
    L.orc_decode_raw_q8_f64.argtypes = [_P, _P, _P, _P, i32, i32, i32, _P, ctypes.c_float, _P,
                                        ctypes.c_float, _P, i32]
    L.orc_decode_raw_q8_f64.restype = i32
    L.orc_quantize_rows.argtypes = [_P, ctypes.c_int64, i32, _P, _P, _P]
    i64 = ctypes.c_int64
    L.orc_prefill_f64.argtypes = [_P, i64, i64, _P, _P, i64, i32, i32, i32, i32, i32, i32, i32, i32,
                                  ctypes.c_float, _P, i32]
    L.orc_prefill_f64.restype = i32
    L.orc_raw_prefill_kv.argtypes = [_P, i32, i32, i32, _P, ctypes.c_float, _P, i32, _P, _P]
    L.orc_raw_prefill_kv.restype = None
    L.orc_set_fault.argtypes = [i32]
    L.orc_set_rinv_ulps.argtypes = [i32]


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _threads(n: int | None) -> int:
    return int(n) if n else min(os.cpu_count() or 1, 16)


# ----------------------------------------------------------------- bf16 helpers

def to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def from_bf16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


# ---------------------------------------------------------------- descriptions

@dataclass
class Step:
    """One decode step's shapes and cache mode (mirrors orc_desc)."""

    B: int
    Hq: int
    Hkv: int
    D: int
    cap: int
    window: int = 0
    ring: bool = False
    scale: float = 1.0
    seq_stride: int | None = None
    head_stride: int | None = None

    def desc(self) -> Desc:
        hs = self.head_stride if self.head_stride is not None else self.cap * self.D
        ss = self.seq_stride if self.seq_stride is not None else self.Hkv * hs
        return Desc(self.B, self.Hq, self.Hkv, self.D, self.cap, self.window,
                    1 if self.ring else 0, ss, hs, self.scale)

    def cache_elems(self) -> int:
        d = self.desc()
        return int(d.seq_stride) * self.B


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def visible(step: Step, pos: int, row_base: int = 0) -> np.ndarray:
    rows = np.empty(step.cap + 1, dtype=np.int32)
    d = step.desc()
    n = lib().orc_visible(ctypes.byref(d), int(pos), int(row_base), _ptr(rows))
    if n < 0:
        raise ValueError("invalid step description")
    return rows[:n].copy()


def append(step: Step, k_cache: np.ndarray, v_cache: np.ndarray | None, k_new: np.ndarray,
           v_new: np.ndarray | None, pos, row_base=None) -> None:
    """In-place append of the new rows (v_cache None or identical = shared buffer)."""
    d = step.desc()
    vc = k_cache if v_cache is None else v_cache
    pos_a = _i32(pos)  # keep the converted arrays alive across the C call
    rb_a = None if row_base is None else _i32(row_base)
    rc = lib().orc_append(ctypes.byref(d), _ptr(k_cache), _ptr(vc), _ptr(k_new),
                          _ptr(v_new), _ptr(pos_a), _ptr(rb_a))
    if rc != 0:
        raise ValueError("orc_append rejected the description")


def _decode(fn: str, step: Step, q, k_cache, v_cache, pos, row_base, out, threads, *extra):
    d = step.desc()
    vc = k_cache if v_cache is None else v_cache
    pos_a = _i32(pos)
    rb_a = None if row_base is None else _i32(row_base)
    args = [ctypes.byref(d), _ptr(q), _ptr(k_cache), _ptr(vc), _ptr(pos_a), _ptr(rb_a)]
    if fn in ("orc_decode_splitk", "orc_decode_refround_grouped"):
        args.append(ctypes.c_int32(extra[0]))
    args += [_ptr(out), _threads(threads)]
    rc = getattr(lib(), fn)(*args)
    if rc != 0:
        raise ValueError(f"{fn} rejected the description")
    return out


def decode_f64(step: Step, q, k_cache, v_cache, pos, row_base=None, threads=None) -> np.ndarray:
    out = np.empty((step.B, step.Hq, step.D), dtype=np.float64)
    return _decode("orc_decode_f64", step, q, k_cache, v_cache, pos, row_base, out, threads)


def decode_refround(step: Step, q, k_cache, v_cache, pos, row_base=None, threads=None) -> np.ndarray:
    out = np.empty((step.B, step.Hq, step.D), dtype=np.uint16)
    return _decode("orc_decode_refround", step, q, k_cache, v_cache, pos, row_base, out, threads)


def decode_refround_grouped(step: Step, q, k_cache, v_cache, pos, row_base=None, threads=None,
                            nsplit: int = 0) -> np.ndarray:
    """decode_refround with each K / V row read once per kv head and the rows split over
    threads (the CPU baseline); equal to decode_refround bit for bit when nsplit == 1."""
    out = np.empty((step.B, step.Hq, step.D), dtype=np.uint16)
    return _decode("orc_decode_refround_grouped", step, q, k_cache, v_cache, pos, row_base, out,
                   threads, nsplit)


def decode_splitk(step: Step, q, k_cache, v_cache, pos, nsplit: int, row_base=None,
                  threads=None) -> np.ndarray:
    out = np.empty((step.B, step.Hq, step.D), dtype=np.float32)
    return _decode("orc_decode_splitk", step, q, k_cache, v_cache, pos, row_base, out,
                   threads, nsplit)


def rope_inv_freq(head_dim: int, theta: float, partial: float) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().orc_rope_inv_freq(head_dim, ctypes.c_float(theta), ctypes.c_float(partial), _ptr(out))
    return out


def rms_norm_rows(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm_rows(_ptr(x), _ptr(w), x.size // n, n, ctypes.c_float(eps), _ptr(y))
    return y


def _other_groups(q, Hkv, call):
    """GQA groups other than the reference kernel's 8 query heads per kv head: each query
    head's output depends only on its own q row and its kv head's rows, so the group is run
    in calls of 8 heads on that kv head alone (q padded with zero heads, their outputs
    dropped).  call(kvh, q8) returns the [8, 512] outputs of q8 against kv head kvh."""
    G = q.shape[0] // Hkv
    out = np.empty((Hkv * G, 512), dtype=np.float64)
    for kvh in range(Hkv):
        for g0 in range(0, G, 8):
            n = min(8, G - g0)
            q8 = np.zeros((8, 512), dtype=np.uint16)
            q8[:n] = q[kvh * G + g0:kvh * G + g0 + n]
            out[kvh * G + g0:kvh * G + g0 + n] = call(kvh, q8)[:n]
    return out


def decode_raw_f64(q, raw, len_: int, kw, eps: float, inv_freq, scale: float = 1.0,
                   threads=None) -> np.ndarray:
    Hkv, pitch, D = raw.shape
    assert D == 512 and q.shape[1] == 512 and q.shape[0] % Hkv == 0
    if q.shape[0] != Hkv * 8:
        return _other_groups(q, Hkv, lambda kvh, q8: decode_raw_f64(
            q8, raw[kvh:kvh + 1], len_, kw, eps, inv_freq, scale, threads))
    out = np.empty((Hkv * 8, 512), dtype=np.float64)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    rc = lib().orc_decode_raw_f64(_ptr(q), _ptr(raw), Hkv, int(len_), pitch, _ptr(kw),
                                  ctypes.c_float(eps), _ptr(inv), ctypes.c_float(scale),
                                  _ptr(out), _threads(threads))
    if rc != 0:
        raise ValueError("orc_decode_raw_f64 rejected the shapes")
    return out


def decode_raw_q8_f64(q, qraw, sc, bs, len_: int, kw, eps: float, inv_freq, scale: float = 1.0,
                      threads=None) -> np.ndarray:
    """q8 raw stream: qraw [Hkv, pitch, 512] u8, sc / bs [Hkv, pitch] (or [Hkv, pitch, 1]) f32."""
    Hkv, pitch, D = qraw.shape
    assert D == 512 and q.shape[1] == 512 and q.shape[0] % Hkv == 0
    qraw = np.ascontiguousarray(qraw, dtype=np.uint8)
    sc = np.ascontiguousarray(sc, dtype=np.float32).reshape(Hkv, pitch)
    bs = np.ascontiguousarray(bs, dtype=np.float32).reshape(Hkv, pitch)
    if q.shape[0] != Hkv * 8:
        return _other_groups(q, Hkv, lambda kvh, q8: decode_raw_q8_f64(
            q8, qraw[kvh:kvh + 1], sc[kvh:kvh + 1], bs[kvh:kvh + 1], len_, kw, eps, inv_freq, scale, threads))
    out = np.empty((Hkv * 8, 512), dtype=np.float64)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    rc = lib().orc_decode_raw_q8_f64(_ptr(q), _ptr(qraw), _ptr(sc), _ptr(bs), Hkv, int(len_), pitch,
                                     _ptr(kw), ctypes.c_float(eps), _ptr(inv), ctypes.c_float(scale),
                                     _ptr(out), _threads(threads))
    if rc != 0:
        raise ValueError("orc_decode_raw_q8_f64 rejected the shapes")
    return out


def quantize_rows(x: np.ndarray):
    """Per-row affine u8 of bf16 rows x [..., n] -> (q u8 [..., n], scale f32 [...], bias f32 [...])."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    n = x.shape[-1]
    rows = x.size // n
    q = np.empty(x.shape, dtype=np.uint8)
    sc = np.empty(x.shape[:-1], dtype=np.float32)
    bs = np.empty(x.shape[:-1], dtype=np.float32)
    lib().orc_quantize_rows(_ptr(x), rows, n, _ptr(q), _ptr(sc), _ptr(bs))
    return q, sc, bs


def prefill_f64(q, k, v, q_pos0: int, k_pos0: int, window: int, scale: float, threads=None) -> np.ndarray:
    """Prefill attention: q [Hq, Sq, D], k / v [Hkv, Sk, D] bf16 bits; query i at absolute
    position q_pos0 + i, key j at k_pos0 + j; returns out [Sq, Hq, D] fp64."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    Hq, Sq, D = q.shape
    Hkv, Sk, _ = k.shape
    assert v.shape == k.shape and k.shape[2] == D
    out = np.empty((Sq, Hq, D), dtype=np.float64)
    rc = lib().orc_prefill_f64(_ptr(q), Sq * D, D, _ptr(k), _ptr(v), Sk * D, Hq, Hkv, D, Sq, Sk,
                               int(q_pos0), int(k_pos0), int(window), ctypes.c_float(scale), _ptr(out),
                               _threads(threads))
    if rc != 0:
        raise ValueError("orc_prefill_f64: a query sees no key, or the shapes are invalid")
    return out


def raw_prefill_kv(raw, kw, eps: float, inv_freq, pos0: int = 0):
    """Raw-K prefill reconstruction: raw [Hkv, Sk, D] bf16 bits -> (K, V) bf16 bits."""
    raw = np.ascontiguousarray(raw, dtype=np.uint16)
    Hkv, Sk, D = raw.shape
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    assert inv.shape == (D // 2,)
    k = np.empty_like(raw)
    v = np.empty_like(raw)
    lib().orc_raw_prefill_kv(_ptr(raw), Hkv, Sk, D, _ptr(np.ascontiguousarray(kw, dtype=np.uint16)),
                             ctypes.c_float(eps), _ptr(inv), int(pos0), _ptr(k), _ptr(v))
    return k, v


class rinv_nudge:
    """Context manager: the raw-K oracles move every row's rinv by `ulps` fp32 ulps (a
    conditioning probe for tests, not a mistake)."""

    def __init__(self, ulps: int):
        self.ulps = ulps

    def __enter__(self):
        lib().orc_set_rinv_ulps(self.ulps)
        return self

    def __exit__(self, *exc):
        lib().orc_set_rinv_ulps(0)
        return False


class planted_fault:
    """Context manager that plants a mistake in the oracle (CPU self-tests only)."""

    def __init__(self, code: int):
        self.code = code

    def __enter__(self):
        lib().orc_set_fault(self.code)
        return self

    def __exit__(self, *exc):
        lib().orc_set_fault(0)
        return False
