"""Torch-tensor front end of esda_decode (one decode step: append + attend + merge).

Mirrors the reference's decode call pair -- ESKVCache::update (ESKVCache.mm:64-109)
followed by the SDPA call of ESAttention.mm:188 -- as one call.  Tensors are torch
CUDA (HIP) tensors; torch is only the allocator and stream provider here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import DecodeArgs, DecodeDesc, RawArgs, RawDesc, RawQ8Args, check, lib

STAGE_ATTEND = 1
STAGE_MERGE = 2


@dataclass
class DecodeStep:
    """Shapes and cache mode of a decode step (esda_decode_desc).

    Caches are [B, Hkv, cap, D] bf16 views (any sequence / head strides, rows dense).
    ``ring`` selects slot = pos mod cap with a sliding ``window``; otherwise row =
    pos - row_base.  ``kv_shared`` means V aliases K (attention_k_eq_v)."""

    batch: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    cap: int
    window: int = 0
    ring: bool = False
    kv_shared: bool = False
    scale: float = 1.0
    max_visible: int = 0
    split_rows: int = 0
    seq_stride: int | None = None
    head_stride: int | None = None

    def desc(self) -> DecodeDesc:
        hs = self.head_stride if self.head_stride is not None else self.cap * self.head_dim
        ss = self.seq_stride if self.seq_stride is not None else self.num_kv_heads * hs
        return DecodeDesc(self.batch, self.num_q_heads, self.num_kv_heads, self.head_dim,
                          self.cap, self.window, 1 if self.ring else 0, 1 if self.kv_shared else 0,
                          ss, hs, self.max_visible, self.split_rows, self.scale)

    @classmethod
    def for_cache(cls, cache: torch.Tensor, num_q_heads: int, **kw) -> "DecodeStep":
        B, Hkv, cap, D = cache.shape
        if cache.stride(3) != 1 or cache.stride(2) != D:
            raise ValueError("cache rows must be dense ([B, Hkv, cap, D] with unit inner strides)")
        return cls(batch=B, num_q_heads=num_q_heads, num_kv_heads=Hkv, head_dim=D, cap=cap,
                   seq_stride=cache.stride(0), head_stride=cache.stride(1), **kw)


def workspace_bytes(step: DecodeStep) -> int:
    n = ctypes.c_size_t(0)
    d = step.desc()
    check(lib().esda_decode_workspace_size(ctypes.byref(d), ctypes.byref(n)))
    return int(n.value)


def new_workspace(step: DecodeStep, device) -> torch.Tensor:
    """Workspace for ``step`` with its status word zeroed (the only part that needs
    initialising; the kernels keep it at zero unless a sequence is out of range)."""
    return torch.zeros(workspace_bytes(step), dtype=torch.uint8, device=device)


def _dev_ptr(t: torch.Tensor | None, dtype=None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("esda tensors must live in GPU memory")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    return t.data_ptr()


def _check_cache(step, t: torch.Tensor | None, what: str, elem_bytes: int = 2) -> None:
    """The cache tensor must hold every element the step addresses: (b, kvh, row, d) at
    b*seq_stride + kvh*head_stride + row*head_dim + d for rows < cap; a 4-D view must be
    [B, Hkv, cap, D] with exactly the step's strides."""
    if t is None:
        return
    if not t.is_cuda:
        raise ValueError(f"{what} must live in GPU memory")
    d = step.desc()
    B, Hkv, cap, D = step.batch, step.num_kv_heads, step.cap, step.head_dim
    need = (B - 1) * d.seq_stride + (Hkv - 1) * d.head_stride + cap * D
    avail = t.untyped_storage().nbytes() // elem_bytes - t.storage_offset()
    if avail < need:
        raise ValueError(f"{what} holds {avail} elements from its start; the step addresses {need}")
    if t.dim() == 4 and (tuple(t.shape) != (B, Hkv, cap, D) or t.stride() != (d.seq_stride, d.head_stride, D, 1)):
        raise ValueError(f"{what} is {tuple(t.shape)} with strides {t.stride()}; the step describes "
                         f"({B}, {Hkv}, {cap}, {D}) with strides ({d.seq_stride}, {d.head_stride}, {D}, 1)")
    if t.dim() != 4 and not t.is_contiguous():
        raise ValueError(f"{what}: pass a contiguous buffer or a [B, Hkv, cap, D] view")


def _check_row_base(step, row_base: torch.Tensor | None) -> None:
    if row_base is not None and (row_base.dtype != torch.int32 or row_base.shape != (step.batch,)
                                 or not row_base.is_contiguous()):
        raise ValueError("row_base must be contiguous int32 [B]")


def _stream_ptr(stream) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def decode_step(step: DecodeStep, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor | None,
                k_cache: torch.Tensor, v_cache: torch.Tensor | None, pos: torch.Tensor,
                row_base: torch.Tensor | None = None, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, stream=None,
                stages: int = STAGE_ATTEND | STAGE_MERGE) -> torch.Tensor:
    """Append the new rows and attend; returns out [B, Hq, D] bf16."""
    bf = torch.bfloat16
    if q.shape != (step.batch, step.num_q_heads, step.head_dim) or not q.is_contiguous():
        raise ValueError(f"q must be contiguous [B, Hq, D], got {tuple(q.shape)}")
    if k_new.shape != (step.batch, step.num_kv_heads, step.head_dim) or not k_new.is_contiguous():
        raise ValueError("k_new must be contiguous [B, Hkv, D]")
    if v_new is not None and (v_new.shape != k_new.shape or not v_new.is_contiguous()):
        raise ValueError("v_new must be contiguous [B, Hkv, D]")
    if pos.dtype != torch.int32 or pos.shape != (step.batch,):
        raise ValueError("pos must be int32 [B]")
    vc = k_cache if (v_cache is None or step.kv_shared) else v_cache
    _check_cache(step, k_cache, "k_cache")
    _check_cache(step, vc, "v_cache")
    _check_row_base(step, row_base)
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = new_workspace(step, q.device)
    args = DecodeArgs(_dev_ptr(q, bf), _dev_ptr(k_new, bf),
                      _dev_ptr(v_new, bf) if (v_new is not None and not step.kv_shared) else None,
                      _dev_ptr(k_cache, bf), _dev_ptr(vc, bf), _dev_ptr(pos),
                      _dev_ptr(row_base), _dev_ptr(out, bf), _dev_ptr(workspace),
                      workspace.numel() * workspace.element_size())
    d = step.desc()
    check(lib().esda_decode_stages(ctypes.byref(d), ctypes.byref(args), stages, _stream_ptr(stream)))
    return out


def decode_step_noalloc(step: DecodeStep, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor | None,
                        k_cache: torch.Tensor, v_cache: torch.Tensor | None, pos: torch.Tensor,
                        out: torch.Tensor, row_base: torch.Tensor | None = None,
                        status: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """esda_decode_noalloc: decode_step with the library's static scratch instead of a
    workspace; nothing is allocated (``out`` is required).  ``status``: an optional int32
    device word counting skipped sequences (read with decode_status)."""
    bf = torch.bfloat16
    if q.shape != (step.batch, step.num_q_heads, step.head_dim) or not q.is_contiguous():
        raise ValueError(f"q must be contiguous [B, Hq, D], got {tuple(q.shape)}")
    if k_new.shape != (step.batch, step.num_kv_heads, step.head_dim) or not k_new.is_contiguous():
        raise ValueError("k_new must be contiguous [B, Hkv, D]")
    if v_new is not None and (v_new.shape != k_new.shape or not v_new.is_contiguous()):
        raise ValueError("v_new must be contiguous [B, Hkv, D]")
    if pos.dtype != torch.int32 or pos.shape != (step.batch,):
        raise ValueError("pos must be int32 [B]")
    if out.shape != q.shape or not out.is_contiguous():
        raise ValueError("out must be contiguous [B, Hq, D]")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1):
        raise ValueError("status must be an int32 device tensor")
    vc = k_cache if (v_cache is None or step.kv_shared) else v_cache
    _check_cache(step, k_cache, "k_cache")
    _check_cache(step, vc, "v_cache")
    _check_row_base(step, row_base)
    args = DecodeArgs(_dev_ptr(q, bf), _dev_ptr(k_new, bf),
                      _dev_ptr(v_new, bf) if (v_new is not None and not step.kv_shared) else None,
                      _dev_ptr(k_cache, bf), _dev_ptr(vc, bf), _dev_ptr(pos),
                      _dev_ptr(row_base), _dev_ptr(out, bf), _dev_ptr(status),
                      0 if status is None else status.numel() * 4)
    d = step.desc()
    check(lib().esda_decode_noalloc(ctypes.byref(d), ctypes.byref(args), _stream_ptr(stream)))
    return out


def decode_status(step: DecodeStep, workspace: torch.Tensor, stream=None) -> int:
    """Number of sequences the kernels skipped (position outside the cache) since the
    last call; clears the counter."""
    n = ctypes.c_int32(0)
    d = step.desc()
    check(lib().esda_decode_status(ctypes.byref(d), _dev_ptr(workspace), ctypes.byref(n),
                                   _stream_ptr(stream)))
    return int(n.value)


def kv_append(cache: torch.Tensor, src: torch.Tensor, row0: torch.Tensor, stream=None) -> None:
    """Copy src [B, Hkv, n, D] into cache rows row0[b] .. row0[b]+n-1 (slice_update)."""
    B, Hkv, cap, D = cache.shape
    if src.shape[:2] != (B, Hkv) or src.shape[3] != D or not src.is_contiguous():
        raise ValueError("src must be contiguous [B, Hkv, n, D]")
    check(lib().esda_kv_append(_dev_ptr(cache, torch.bfloat16), cache.stride(0), cache.stride(1),
                               B, Hkv, D, cap, _dev_ptr(src, torch.bfloat16), src.shape[2],
                               _dev_ptr(row0), _stream_ptr(stream)))


class DecodeCall:
    """A decode step with its C-ABI arguments marshalled once (the host-side cost of a
    launch is then one ctypes call).  Tensors are referenced, not copied: refill q,
    k_new, v_new and pos in place between calls.  Also usable under HIP graph capture
    (the library issues only kernel launches on the given stream)."""

    def __init__(self, step: DecodeStep, q, k_new, v_new, k_cache, v_cache, pos, row_base=None,
                 out=None, workspace=None, stages: int = STAGE_ATTEND | STAGE_MERGE):
        if out is None:
            out = torch.empty_like(q)
        if workspace is None:
            workspace = new_workspace(step, q.device)
        _check_cache(step, k_cache, "k_cache")
        _check_cache(step, k_cache if (v_cache is None or step.kv_shared) else v_cache, "v_cache")
        _check_row_base(step, row_base)
        self._keep = (q, k_new, v_new, k_cache, v_cache, pos, row_base, out, workspace)
        self.step, self.out, self.workspace, self.stages = step, out, workspace, stages
        bf = torch.bfloat16
        vc = k_cache if (v_cache is None or step.kv_shared) else v_cache
        self._desc = step.desc()
        self._args = DecodeArgs(_dev_ptr(q, bf), _dev_ptr(k_new, bf),
                                _dev_ptr(v_new, bf) if (v_new is not None and not step.kv_shared) else None,
                                _dev_ptr(k_cache, bf), _dev_ptr(vc, bf), _dev_ptr(pos),
                                _dev_ptr(row_base), _dev_ptr(out, bf), _dev_ptr(workspace),
                                workspace.numel() * workspace.element_size())
        self._fn = lib().esda_decode_stages
        self._pd, self._pa = ctypes.byref(self._desc), ctypes.byref(self._args)

    def __call__(self, stream=None, stages: int | None = None) -> torch.Tensor:
        rc = self._fn(self._pd, self._pa, self.stages if stages is None else stages,
                      _stream_ptr(stream))
        if rc:
            check(rc)
        return self.out


# ----------------------------------------------------------------------- raw-K mode

@dataclass
class RawStep:
    """Shapes of a raw-K decode step (esda_raw_desc): the cache holds pre-norm k_proj rows
    [B, Hkv, cap, 512]; sequence b attends rows 0 .. pos[b] with K and V rebuilt from them
    (ESDecodeAttn.mm:17-117)."""

    batch: int
    num_q_heads: int
    num_kv_heads: int
    cap: int
    eps: float = 1e-6
    scale: float = 1.0
    max_visible: int = 0
    split_rows: int = 0
    seq_stride: int | None = None
    head_stride: int | None = None
    head_dim: int = 512

    def desc(self) -> RawDesc:
        hs = self.head_stride if self.head_stride is not None else self.cap * self.head_dim
        ss = self.seq_stride if self.seq_stride is not None else self.num_kv_heads * hs
        return RawDesc(self.batch, self.num_q_heads, self.num_kv_heads, self.head_dim, self.cap,
                       ss, hs, self.max_visible, self.split_rows, self.scale, self.eps)

    @classmethod
    def for_cache(cls, cache: torch.Tensor, num_q_heads: int, **kw) -> "RawStep":
        B, Hkv, cap, D = cache.shape
        if D != 512 or cache.stride(3) != 1 or cache.stride(2) != D:
            raise ValueError("raw cache rows must be dense [B, Hkv, cap, 512]")
        return cls(batch=B, num_q_heads=num_q_heads, num_kv_heads=Hkv, cap=cap,
                   seq_stride=cache.stride(0), head_stride=cache.stride(1), **kw)


def raw_workspace_bytes(step: RawStep) -> int:
    n = ctypes.c_size_t(0)
    d = step.desc()
    check(lib().esda_decode_raw_workspace_size(ctypes.byref(d), ctypes.byref(n)))
    return int(n.value)


def new_raw_workspace(step: RawStep, device) -> torch.Tensor:
    return torch.zeros(raw_workspace_bytes(step), dtype=torch.uint8, device=device)


def rope_table(inv_freq: torch.Tensor, rows: int, stream=None) -> torch.Tensor:
    """The raw-K rotary table (esda_rope_table): int32 [rows, 64], entry (t, d) = bf16
    cos | bf16 sin << 16 of float(t) * inv_freq[d] -- what the raw-K kernels otherwise
    compute per step."""
    if inv_freq.dtype != torch.float32 or inv_freq.numel() < 64 or not inv_freq.is_contiguous():
        raise ValueError("inv_freq must be contiguous f32 [>= 64]")
    tab = torch.empty((rows, 64), dtype=torch.int32, device=inv_freq.device)
    check(lib().esda_rope_table(_dev_ptr(inv_freq), rows, _dev_ptr(tab), _stream_ptr(stream)))
    return tab


def _table(tab: torch.Tensor | None):
    """(pointer, rows) of an optional rope_table."""
    if tab is None:
        return None, 0
    if tab.dtype != torch.int32 or tab.dim() != 2 or tab.shape[1] != 64 or not tab.is_contiguous():
        raise ValueError("rope_table must be contiguous int32 [rows, 64] (rope_table())")
    return _dev_ptr(tab), tab.shape[0]


def decode_raw(step: RawStep, q: torch.Tensor, k_new: torch.Tensor | None, raw_cache: torch.Tensor,
               pos: torch.Tensor, kw: torch.Tensor, inv_freq: torch.Tensor,
               out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, stream=None,
               stages: int = STAGE_ATTEND | STAGE_MERGE, rope_table: torch.Tensor | None = None) -> torch.Tensor:
    """Raw-K decode step: write k_new (raw rows, or None) at row pos[b], then attend rows
    0 .. pos[b]; returns out [B, Hq, 512] bf16.  rope_table: an optional precomputed
    rotary table (rope_table(), >= cap rows), bit-identical to the kernel's own."""
    bf = torch.bfloat16
    if q.shape != (step.batch, step.num_q_heads, 512) or not q.is_contiguous():
        raise ValueError("q must be contiguous [B, Hq, 512]")
    if k_new is not None and (k_new.shape != (step.batch, step.num_kv_heads, 512) or not k_new.is_contiguous()):
        raise ValueError("k_new must be contiguous [B, Hkv, 512]")
    if pos.dtype != torch.int32 or pos.shape != (step.batch,):
        raise ValueError("pos must be int32 [B]")
    if kw.dtype != bf or kw.numel() != 512 or inv_freq.dtype != torch.float32 or inv_freq.numel() < 64:
        raise ValueError("kw must be bf16 [512] and inv_freq f32 [>= 64]")
    _check_cache(step, raw_cache, "raw_cache")
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = new_raw_workspace(step, q.device)
    args = RawArgs(_dev_ptr(q, bf), _dev_ptr(k_new, bf), _dev_ptr(raw_cache, bf), _dev_ptr(pos),
                   _dev_ptr(kw, bf), _dev_ptr(inv_freq), _dev_ptr(out, bf), _dev_ptr(workspace),
                   workspace.numel() * workspace.element_size(), *_table(rope_table))
    d = step.desc()
    check(lib().esda_decode_raw_stages(ctypes.byref(d), ctypes.byref(args), stages, _stream_ptr(stream)))
    return out


class RawCall:
    """decode_raw with its arguments marshalled once (see DecodeCall)."""

    def __init__(self, step: RawStep, q, k_new, raw_cache, pos, kw, inv_freq, out=None, workspace=None,
                 stages: int = STAGE_ATTEND | STAGE_MERGE, rope_table=None):
        if out is None:
            out = torch.empty_like(q)
        if workspace is None:
            workspace = new_raw_workspace(step, q.device)
        _check_cache(step, raw_cache, "raw_cache")
        self._keep = (q, k_new, raw_cache, pos, kw, inv_freq, out, workspace, rope_table)
        self.step, self.out, self.workspace, self.stages = step, out, workspace, stages
        bf = torch.bfloat16
        self._desc = step.desc()
        self._args = RawArgs(_dev_ptr(q, bf), _dev_ptr(k_new, bf), _dev_ptr(raw_cache, bf), _dev_ptr(pos),
                             _dev_ptr(kw, bf), _dev_ptr(inv_freq), _dev_ptr(out, bf), _dev_ptr(workspace),
                             workspace.numel() * workspace.element_size(), *_table(rope_table))
        self._fn = lib().esda_decode_raw_stages
        self._pd, self._pa = ctypes.byref(self._desc), ctypes.byref(self._args)

    def __call__(self, stream=None, stages: int | None = None) -> torch.Tensor:
        rc = self._fn(self._pd, self._pa, self.stages if stages is None else stages, _stream_ptr(stream))
        if rc:
            check(rc)
        return self.out


# ----------------------------------------------------------------- q8 raw-K mode

def quantize_raw_rows(src: torch.Tensor, q8: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor,
                      row0: int = 0, stream=None) -> None:
    """Quantize src [Hkv, n, 512] bf16 into rows row0 .. row0+n-1 of a q8 cache for one
    sequence: q8 [Hkv, cap, 512] u8, scale / bias [Hkv, cap] f32 (esQuantizeRawRows)."""
    Hkv, n, D = src.shape
    if D != 512 or not src.is_contiguous() or src.dtype != torch.bfloat16:
        raise ValueError("src must be contiguous bf16 [Hkv, n, 512]")
    if q8.dtype != torch.uint8 or q8.dim() != 3 or q8.shape[0] != Hkv or q8.stride(2) != 1 or q8.stride(1) != 512:
        raise ValueError("q8 must be u8 [Hkv, cap, 512] with dense rows")
    if scale.shape != q8.shape[:2] or bias.shape != q8.shape[:2] or scale.stride(1) != 1 or bias.stride() != scale.stride():
        raise ValueError("scale / bias must be f32 [Hkv, cap]")
    check(lib().esda_quantize_raw_rows(_dev_ptr(src, torch.bfloat16), Hkv, n, _dev_ptr(q8), q8.stride(0),
                                       _dev_ptr(scale), _dev_ptr(bias), scale.stride(0), row0,
                                       _stream_ptr(stream)))


def _q8_args(step: RawStep, q, k_new, q8, scale, bias, pos, kw, inv_freq, out, workspace,
             rope_table=None) -> RawQ8Args:
    bf = torch.bfloat16
    if q.shape != (step.batch, step.num_q_heads, 512) or not q.is_contiguous():
        raise ValueError("q must be contiguous [B, Hq, 512]")
    if k_new is not None and (k_new.shape != (step.batch, step.num_kv_heads, 512) or not k_new.is_contiguous()):
        raise ValueError("k_new must be contiguous [B, Hkv, 512]")
    if q8.dtype != torch.uint8 or q8.shape != (step.batch, step.num_kv_heads, step.cap, 512):
        raise ValueError("q8 cache must be u8 [B, Hkv, cap, 512]")
    _check_cache(step, q8, "q8 cache", elem_bytes=1)
    if scale.dtype != torch.float32 or scale.shape != (step.batch, step.num_kv_heads, step.cap) or \
            bias.shape != scale.shape or bias.stride() != scale.stride() or scale.stride(2) != 1:
        raise ValueError("scale / bias must be f32 [B, Hkv, cap] with the same strides")
    if pos.dtype != torch.int32 or pos.shape != (step.batch,):
        raise ValueError("pos must be int32 [B]")
    return RawQ8Args(_dev_ptr(q, bf), _dev_ptr(k_new, bf), _dev_ptr(q8), _dev_ptr(scale), _dev_ptr(bias),
                     scale.stride(0), scale.stride(1), _dev_ptr(pos), _dev_ptr(kw, bf), _dev_ptr(inv_freq),
                     _dev_ptr(out, bf), _dev_ptr(workspace), workspace.numel() * workspace.element_size(),
                     *_table(rope_table))


def q8_step_for(q8: torch.Tensor, num_q_heads: int, **kw) -> RawStep:
    """RawStep of a q8 cache [B, Hkv, cap, 512] u8 (strides in bytes)."""
    B, Hkv, cap, D = q8.shape
    if D != 512 or q8.stride(3) != 1 or q8.stride(2) != D:
        raise ValueError("q8 cache rows must be dense [B, Hkv, cap, 512]")
    return RawStep(batch=B, num_q_heads=num_q_heads, num_kv_heads=Hkv, cap=cap,
                   seq_stride=q8.stride(0), head_stride=q8.stride(1), **kw)


def decode_raw_q8(step: RawStep, q: torch.Tensor, k_new: torch.Tensor | None, q8: torch.Tensor,
                  scale: torch.Tensor, bias: torch.Tensor, pos: torch.Tensor, kw: torch.Tensor,
                  inv_freq: torch.Tensor, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None, stream=None,
                  stages: int = STAGE_ATTEND | STAGE_MERGE, rope_table: torch.Tensor | None = None) -> torch.Tensor:
    """q8 raw-K decode step: quantize k_new (or None) into row pos[b], then attend rows
    0 .. pos[b] of the q8 stream; returns out [B, Hq, 512] bf16."""
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = new_raw_workspace(step, q.device)
    args = _q8_args(step, q, k_new, q8, scale, bias, pos, kw, inv_freq, out, workspace, rope_table)
    d = step.desc()
    check(lib().esda_decode_raw_q8_stages(ctypes.byref(d), ctypes.byref(args), stages, _stream_ptr(stream)))
    return out


class RawQ8Call:
    """decode_raw_q8 with its arguments marshalled once (see DecodeCall)."""

    def __init__(self, step: RawStep, q, k_new, q8, scale, bias, pos, kw, inv_freq, out=None, workspace=None,
                 stages: int = STAGE_ATTEND | STAGE_MERGE, rope_table=None):
        if out is None:
            out = torch.empty_like(q)
        if workspace is None:
            workspace = new_raw_workspace(step, q.device)
        self._keep = (q, k_new, q8, scale, bias, pos, kw, inv_freq, out, workspace, rope_table)
        self.step, self.out, self.workspace, self.stages = step, out, workspace, stages
        self._desc = step.desc()
        self._args = _q8_args(step, q, k_new, q8, scale, bias, pos, kw, inv_freq, out, workspace, rope_table)
        self._fn = lib().esda_decode_raw_q8_stages
        self._pd, self._pa = ctypes.byref(self._desc), ctypes.byref(self._args)

    def __call__(self, stream=None, stages: int | None = None) -> torch.Tensor:
        rc = self._fn(self._pd, self._pa, self.stages if stages is None else stages, _stream_ptr(stream))
        if rc:
            check(rc)
        return self.out
