"""Python front end of the ES* C++ layer (include/esda_cache.h): ``ESKVCache`` and
``es_decode_attn_global`` with the reference's method names and argument meaning
(Apertura ESKVCache.h:44-224, ESDecodeAttn.h:22-28).

Row tensors are torch bf16 GPU tensors [kvHeads, n, headDim] with contiguous rows.
Views returned by update / current are ``CacheView`` records (non-owning device
pointers into the cache's buffers, valid until the slot next grows or is reset);
``CacheView.torch()`` copies one out as a torch tensor.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import Q8View, View, check, lib
from .decode import _dev_ptr, _stream_ptr


@dataclass
class CacheView:
    data: int
    kv_heads: int
    rows: int
    head_dim: int
    head_stride: int  # elements

    @classmethod
    def of(cls, v: View) -> "CacheView":
        return cls(int(v.data or 0), v.kv_heads, v.rows, v.head_dim, int(v.head_stride))

    def torch(self, device="cuda") -> torch.Tensor:
        """Copy of the viewed rows, [kv_heads, rows, head_dim] bf16 on `device`."""
        out = torch.empty((self.kv_heads, self.rows, self.head_dim), dtype=torch.bfloat16, device=device)
        _hip_copy_2d(out.data_ptr(), self.rows * self.head_dim * 2, self.data, self.head_stride * 2,
                     self.rows * self.head_dim * 2, self.kv_heads)
        return out


_hip = None


def _hip_copy_2d(dst: int, dpitch: int, src: int, spitch: int, width: int, height: int) -> None:
    """Synchronous device-to-device 2-D copy through the HIP runtime torch already uses."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy2D.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                     ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy2D.restype = ctypes.c_int
    torch.cuda.synchronize()
    rc = _hip.hipMemcpy2D(dst, dpitch, src, spitch, width, height, 3)  # hipMemcpyDeviceToDevice
    if rc != 0:
        raise RuntimeError(f"hipMemcpy2D failed ({rc})")


@dataclass
class RawQ8View:
    """A q8 raw slot (ESKVCache::RawQ8): u8 rows [kv_heads, pitch, 512] and f32 scale /
    bias [kv_heads, pitch] at device addresses q / scale / bias; rows 0 .. len-1 live."""
    q: int
    scale: int
    bias: int
    kv_heads: int
    len: int
    pitch: int

    @classmethod
    def of(cls, v: Q8View) -> "RawQ8View":
        return cls(int(v.q or 0), int(v.scale or 0), int(v.bias or 0), v.kv_heads, v.len, v.pitch)

    def torch(self, device="cuda") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Copies of the live rows: (q u8 [kv_heads, len, 512], scale, bias f32 [kv_heads, len])."""
        h, n, p = self.kv_heads, self.len, self.pitch
        q = torch.empty((h, n, 512), dtype=torch.uint8, device=device)
        sc = torch.empty((h, n), dtype=torch.float32, device=device)
        bs = torch.empty((h, n), dtype=torch.float32, device=device)
        if n:
            _hip_copy_2d(q.data_ptr(), n * 512, self.q, p * 512, n * 512, h)
            _hip_copy_2d(sc.data_ptr(), n * 4, self.scale, p * 4, n * 4, h)
            _hip_copy_2d(bs.data_ptr(), n * 4, self.bias, p * 4, n * 4, h)
        return q, sc, bs


def _rows(t: torch.Tensor, what: str):
    if t.dim() != 3 or t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous bf16 [kvHeads, n, headDim] tensor")
    return t.shape


class ESKVCache:
    """Per-layer KV storage on the GPU (the reference's ESKVCache)."""

    kGrowChunk = 256

    def __init__(self, num_layers: int):
        h = ctypes.c_void_p()
        check(lib().esda_cache_create(num_layers, ctypes.byref(h)))
        self._h = h
        self._num_layers = num_layers

    def close(self) -> None:
        if self._h:
            lib().esda_cache_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def update(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, max_keep: int = 0,
               prealloc: bool = False, stream=None) -> tuple[CacheView, CacheView]:
        kvh, n, hd = _rows(k_new, "k_new")
        _rows(v_new, "v_new")
        kv, vv = View(), View()
        check(lib().esda_cache_update(self._h, layer, _dev_ptr(k_new), _dev_ptr(v_new), kvh, n, hd, max_keep,
                                      1 if prealloc else 0, _stream_ptr(stream), ctypes.byref(kv),
                                      ctypes.byref(vv)))
        return CacheView.of(kv), CacheView.of(vv)

    def update_raw(self, layer: int, k_new: torch.Tensor, prealloc: bool, stream=None):
        """Returns (view, len, pitch) (ESKVCache::Raw without the buffer handle)."""
        kvh, n, hd = _rows(k_new, "k_new")
        v, ln, pitch = View(), ctypes.c_int32(), ctypes.c_int32()
        check(lib().esda_cache_update_raw(self._h, layer, _dev_ptr(k_new), kvh, n, hd, 1 if prealloc else 0,
                                          _stream_ptr(stream), ctypes.byref(v), ctypes.byref(ln),
                                          ctypes.byref(pitch)))
        return CacheView.of(v), int(ln.value), int(pitch.value)

    def current(self, layer: int, prealloc: bool) -> tuple[CacheView, CacheView]:
        kv, vv = View(), View()
        check(lib().esda_cache_current(self._h, layer, 1 if prealloc else 0, ctypes.byref(kv), ctypes.byref(vv)))
        return CacheView.of(kv), CacheView.of(vv)

    # -------------------------------------------- compiled-step mode (ESKVCache.h:93-112)

    def begin_step(self, global_idx: torch.Tensor, sliding_idx: torch.Tensor) -> None:
        """Until end_step, update() writes its one row at the cache row held in the int32
        device word global_idx (max_keep == 0) or sliding_idx (max_keep > 0)."""
        for t in (global_idx, sliding_idx):
            if t.dtype != torch.int32 or t.numel() < 1 or not t.is_cuda:
                raise ValueError("step indices must be int32 device tensors")
        self._step_idx = (global_idx, sliding_idx)  # kept alive while the step runs
        check(lib().esda_cache_begin_step(self._h, _dev_ptr(global_idx), _dev_ptr(sliding_idx)))

    def end_step(self) -> None:
        check(lib().esda_cache_end_step(self._h))
        self._step_idx = None

    def set_slot(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Install [kv_heads, cap, head_dim] bf16 buffers (v may be k: shared K=V); the
        caller keeps them alive while the cache refers to them."""
        kvh, cap, hd = _rows(k, "k")
        if v.shape != k.shape:
            raise ValueError("set_slot: k and v differ in shape")
        _rows(v, "v")
        check(lib().esda_cache_set_slot(self._h, layer, _dev_ptr(k), _dev_ptr(v), kvh, cap, hd))

    def slot_kv(self, layer: int) -> tuple[CacheView, CacheView]:
        kv, vv = View(), View()
        check(lib().esda_cache_slot_kv(self._h, layer, ctypes.byref(kv), ctypes.byref(vv)))
        return CacheView.of(kv), CacheView.of(vv)

    def take_slot(self, layer: int) -> tuple[CacheView, CacheView]:
        kv, vv = View(), View()
        check(lib().esda_cache_take_slot(self._h, layer, ctypes.byref(kv), ctypes.byref(vv)))
        return CacheView.of(kv), CacheView.of(vv)

    def current_raw(self, layer: int):
        """(view, len, pitch) of a prealloc raw-K slot without appending."""
        v, ln, pitch = View(), ctypes.c_int32(), ctypes.c_int32()
        check(lib().esda_cache_current_raw(self._h, layer, ctypes.byref(v), ctypes.byref(ln), ctypes.byref(pitch)))
        return CacheView.of(v), int(ln.value), int(pitch.value)

    def decode(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, max_keep: int,
               window: int, scale: float, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """Fused append + attention of one decode step; v_new may be k_new itself
        (attention_k_eq_v: one shared K=V buffer).  window > 0: the sliding mask (last
        `window` positions), whatever max_keep evicts.  Returns [numQHeads, headDim] bf16."""
        kvh, n, hd = _rows(k_new, "k_new")
        _rows(v_new, "v_new")
        if n != 1:
            raise ValueError("decode appends exactly one row")
        hq = q.numel() // hd
        if out is None:
            out = torch.empty((hq, hd), dtype=torch.bfloat16, device=q.device)
        check(lib().esda_cache_decode(self._h, layer, _dev_ptr(q, torch.bfloat16), hq, _dev_ptr(k_new),
                                      _dev_ptr(v_new), kvh, hd, max_keep, window, scale,
                                      _dev_ptr(out, torch.bfloat16),
                                      _stream_ptr(stream)))
        return out

    def decode_raw(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, kw: torch.Tensor, eps: float,
                   inv_freq, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """Fused updateRaw + esDecodeAttnGlobal of one decode step (head dim 512)."""
        kvh, n, hd = _rows(k_new, "k_new")
        if n != 1 or hd != 512:
            raise ValueError("decode_raw appends one 512-dim row per kv head")
        hq = q.numel() // 512
        if out is None:
            out = torch.empty((hq, 512), dtype=torch.bfloat16, device=q.device)
        f = (ctypes.c_float * len(inv_freq))(*[float(x) for x in inv_freq])
        check(lib().esda_cache_decode_raw(self._h, layer, _dev_ptr(q, torch.bfloat16), hq, _dev_ptr(k_new), kvh,
                                          _dev_ptr(kw, torch.bfloat16), eps, f, len(inv_freq),
                                          _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
        return out

    def update_raw_q8(self, layer: int, k_new: torch.Tensor, stream=None) -> RawQ8View:
        """ESKVCache::updateRawQ8: quantize k_new [kvHeads, n, 512] bf16 raw rows into the
        layer's q8 slot (a bf16 raw slot migrates first)."""
        kvh, n, hd = _rows(k_new, "k_new")
        if hd != 512:
            raise ValueError("q8 raw rows are 512 wide")
        v = Q8View()
        check(lib().esda_cache_update_raw_q8(self._h, layer, _dev_ptr(k_new), kvh, n, _stream_ptr(stream),
                                             ctypes.byref(v)))
        return RawQ8View.of(v)

    def current_raw_q8(self, layer: int) -> RawQ8View:
        v = Q8View()
        check(lib().esda_cache_current_raw_q8(self._h, layer, ctypes.byref(v)))
        return RawQ8View.of(v)

    def decode_raw_q8(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, kw: torch.Tensor, eps: float,
                      inv_freq, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """Fused updateRawQ8 + esDecodeAttnGlobalQ8 of one decode step (the new row is
        quantized inside the kernel)."""
        kvh, n, hd = _rows(k_new, "k_new")
        if n != 1 or hd != 512:
            raise ValueError("decode_raw_q8 appends one 512-dim row per kv head")
        hq = q.numel() // 512
        if out is None:
            out = torch.empty((hq, 512), dtype=torch.bfloat16, device=q.device)
        f = (ctypes.c_float * len(inv_freq))(*[float(x) for x in inv_freq])
        check(lib().esda_cache_decode_raw_q8(self._h, layer, _dev_ptr(q, torch.bfloat16), hq, _dev_ptr(k_new),
                                             kvh, _dev_ptr(kw, torch.bfloat16), eps, f, len(inv_freq),
                                             _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
        return out

    def prefill(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, max_keep: int,
                window: int, scale: float, past_len: int, prealloc: bool = True, out: torch.Tensor | None = None,
                stream=None) -> torch.Tensor:
        """ESKVCache::prefill: append a chunk (k_new / v_new [kvHeads, seq, headDim]; v_new may
        be k_new itself) and attend q [numQHeads, seq, headDim] over the live rows with the
        reference's mask.  Returns [seq, numQHeads * headDim] bf16."""
        kvh, n, hd = _rows(k_new, "k_new")
        _rows(v_new, "v_new")
        if q.dim() != 3 or q.shape[1] != n or q.shape[2] != hd or not q.is_contiguous():
            raise ValueError("q must be contiguous [numQHeads, seq, headDim] with seq = k_new rows")
        hq = q.shape[0]
        if out is None:
            out = torch.empty((n, hq * hd), dtype=torch.bfloat16, device=q.device)
        check(lib().esda_cache_prefill(self._h, layer, _dev_ptr(q, torch.bfloat16), hq, n, _dev_ptr(k_new),
                                       _dev_ptr(v_new), kvh, hd, max_keep, window, scale, past_len,
                                       1 if prealloc else 0, _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
        return out

    def prefill_raw(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, kw: torch.Tensor, eps: float, inv_freq,
                    past_len: int, scale: float, q8: bool = False, out: torch.Tensor | None = None,
                    stream=None) -> torch.Tensor:
        """ESKVCache::prefillRaw: append the chunk's raw rows (into the q8 stream when q8)
        and attend over the whole raw stream (head dim 512)."""
        kvh, n, hd = _rows(k_new, "k_new")
        if hd != 512 or q.dim() != 3 or q.shape[1:] != (n, 512) or not q.is_contiguous():
            raise ValueError("raw prefill: q [numQHeads, seq, 512] contiguous, k_new [kvHeads, seq, 512]")
        hq = q.shape[0]
        if out is None:
            out = torch.empty((n, hq * 512), dtype=torch.bfloat16, device=q.device)
        f = (ctypes.c_float * len(inv_freq))(*[float(x) for x in inv_freq])
        check(lib().esda_cache_prefill_raw(self._h, layer, _dev_ptr(q, torch.bfloat16), hq, n, _dev_ptr(k_new), kvh,
                                           _dev_ptr(kw, torch.bfloat16), eps, f, len(inv_freq), past_len, scale,
                                           1 if q8 else 0, _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
        return out

    def slot(self, layer: int) -> dict:
        ln, st, cap, fl = (ctypes.c_int32() for _ in range(4))
        check(lib().esda_cache_slot(self._h, layer, ctypes.byref(ln), ctypes.byref(st), ctypes.byref(cap),
                                    ctypes.byref(fl)))
        f = int(fl.value)
        return {"len": int(ln.value), "start": int(st.value), "capacity": int(cap.value),
                "lost": bool(f & 1), "shared": bool(f & 2), "raw": bool(f & 4), "q8": bool(f & 8)}

    def seq_len(self) -> int:
        return lib().esda_cache_seq_len(self._h)

    def mark_step(self, n_new: int) -> None:
        lib().esda_cache_mark_step(self._h, n_new)

    def reset(self) -> None:
        lib().esda_cache_reset(self._h)

    # Persistence and rewind (ESKVCache.h:102-174).
    RAW_MODES = {"composite": 0, "raw": 1, "rawQ8": 2, "asStored": 3}

    def save_snapshot(self, path: str, fingerprint: str, pos: int) -> bool:
        return bool(lib().esda_cache_save_snapshot(self._h, path.encode(), fingerprint.encode(), pos))

    def restore_snapshot(self, path: str, fingerprint: str, mode: str = "asStored", prefix_fp=None) -> int:
        """Restored position or -1.  prefix_fp(pos) -> the caller's prefix fingerprint at a
        marker position ("" = none)."""
        from ._lib import PREFIX_FP_FN
        keep = []

        def cb(pos, _user):
            buf = ctypes.create_string_buffer((prefix_fp(int(pos)) or "").encode())
            keep.append(buf)  # alive until the restore returns
            return ctypes.addressof(buf)

        fn = PREFIX_FP_FN(cb) if prefix_fp is not None else PREFIX_FP_FN()
        return lib().esda_cache_restore_snapshot_ex(self._h, path.encode(), fingerprint.encode(),
                                                    self.RAW_MODES[mode], fn, None)

    def mark_prefix(self, pos: int, fingerprint: str) -> None:
        check(lib().esda_cache_mark_prefix(self._h, pos, fingerprint.encode()))

    def mark_rewind_point(self, pos: int) -> bool:
        return bool(lib().esda_cache_mark_rewind_point(self._h, pos))

    def rewind_to_mark(self) -> int:
        return lib().esda_cache_rewind_to_mark(self._h)

    def clear_rewind_mark(self) -> None:
        lib().esda_cache_clear_rewind_mark(self._h)


def es_decode_attn_global(q: torch.Tensor, raw_buf: torch.Tensor, length: int, pitch: int, kw: torch.Tensor,
                          eps: float, inv_freq, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """esDecodeAttnGlobal: q [numQ, 512], raw_buf the unsliced [numKV, pitch, 512] buffer
    whose rows 0 .. length-1 are attended; returns [numQ, 512] bf16."""
    if raw_buf.dim() != 3 or not raw_buf.is_contiguous():
        raise ValueError("raw_buf must be a contiguous [numKV, pitch, 512] tensor")
    hq = q.numel() // 512
    if out is None:
        out = torch.empty((hq, 512), dtype=torch.bfloat16, device=q.device)
    f = (ctypes.c_float * len(inv_freq))(*[float(x) for x in inv_freq])
    check(lib().esda_decode_attn_global(_dev_ptr(q, torch.bfloat16), hq, _dev_ptr(raw_buf, torch.bfloat16),
                                        raw_buf.shape[0], length, pitch, _dev_ptr(kw, torch.bfloat16), eps, f,
                                        len(inv_freq), _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
    return out


def es_decode_attn_global_q8(q: torch.Tensor, q8_buf: torch.Tensor, scale_buf: torch.Tensor,
                             bias_buf: torch.Tensor, length: int, pitch: int, kw: torch.Tensor, eps: float,
                             inv_freq, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """esDecodeAttnGlobalQ8: q [numQ, 512]; q8_buf the unsliced u8 [numKV, pitch, 512]
    buffer, scale_buf / bias_buf f32 [numKV, pitch(, 1)]; rows 0 .. length-1 attended."""
    if q8_buf.dim() != 3 or q8_buf.dtype != torch.uint8 or not q8_buf.is_contiguous():
        raise ValueError("q8_buf must be a contiguous uint8 [numKV, pitch, 512] tensor")
    for t in (scale_buf, bias_buf):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != q8_buf.shape[0] * q8_buf.shape[1]:
            raise ValueError("scale_buf / bias_buf must be contiguous float32 [numKV, pitch]")
    hq = q.numel() // 512
    if out is None:
        out = torch.empty((hq, 512), dtype=torch.bfloat16, device=q.device)
    f = (ctypes.c_float * len(inv_freq))(*[float(x) for x in inv_freq])
    check(lib().esda_decode_attn_global_q8(_dev_ptr(q, torch.bfloat16), hq, _dev_ptr(q8_buf),
                                           _dev_ptr(scale_buf), _dev_ptr(bias_buf), q8_buf.shape[0], length,
                                           pitch, _dev_ptr(kw, torch.bfloat16), eps, f, len(inv_freq),
                                           _dev_ptr(out, torch.bfloat16), _stream_ptr(stream)))
    return out
