"""Torch-tensor front end of esda_prefill (include/esda_prefill.h): attention of a chunk
of new tokens over the cache, and the raw-K stream's K / V reconstruction.

Mirrors mx::fast::scaled_dot_product_attention at ESAttention.mm:188 (seq > 1) with the
additive mask of ESGemma4TextModel.mm:68-83 aligned by ESAttention.mm:17-22, and the
raw-K prefill of ESAttention.mm:306-332.  Tensors are torch CUDA (HIP) tensors; torch is
only the allocator and stream provider here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import PrefillArgs, PrefillDesc, check, lib
from .decode import _dev_ptr, _stream_ptr


@dataclass
class PrefillStep:
    """One prefill attention call (esda_prefill_desc).

    Query i sits at absolute position q_pos0 + i, key j at k_pos0 + j; key j is visible
    to query i iff kAbs <= qAbs and (window == 0 or kAbs > qAbs - window)."""

    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    seq_q: int
    seq_k: int
    q_pos0: int = 0
    k_pos0: int = 0
    window: int = 0
    scale: float = 1.0
    split_keys: int = 0
    q_head_stride: int | None = None
    q_row_stride: int | None = None
    kv_head_stride: int | None = None
    out_row_stride: int | None = None
    out_head_stride: int | None = None

    def desc(self) -> PrefillDesc:
        D = self.head_dim
        qhs = self.q_head_stride if self.q_head_stride is not None else self.seq_q * D
        qrs = self.q_row_stride if self.q_row_stride is not None else D
        kvhs = self.kv_head_stride if self.kv_head_stride is not None else self.seq_k * D
        ors = self.out_row_stride if self.out_row_stride is not None else self.num_q_heads * D
        ohs = self.out_head_stride if self.out_head_stride is not None else D
        return PrefillDesc(self.num_q_heads, self.num_kv_heads, D, self.seq_q, self.seq_k, self.q_pos0,
                           self.k_pos0, self.window, qhs, qrs, kvhs, ors, ohs, self.split_keys, self.scale)

    @classmethod
    def for_tensors(cls, q: torch.Tensor, k: torch.Tensor, out: torch.Tensor | None = None, **kw) -> "PrefillStep":
        """q: an [Hq, Sq, D] view, k: an [Hkv, Sk, D] view with dense rows, out: an
        [Sq, Hq, D] view (unit inner strides); strides are taken from the tensors."""
        Hq, Sq, D = q.shape
        Hkv, Sk, Dk = k.shape
        if Dk != D or q.stride(2) != 1 or k.stride(2) != 1 or k.stride(1) != D:
            raise ValueError("q must be an [Hq, Sq, D] view and k an [Hkv, Sk, D] view with dense rows")
        st = dict(q_head_stride=q.stride(0), q_row_stride=q.stride(1), kv_head_stride=k.stride(0))
        if out is not None:
            if out.shape != (Sq, Hq, D) or out.stride(2) != 1:
                raise ValueError("out must be an [Sq, Hq, D] view with unit inner stride")
            st.update(out_row_stride=out.stride(0), out_head_stride=out.stride(1))
        st.update(kw)
        return cls(num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, seq_q=Sq, seq_k=Sk, **st)


def prefill_workspace_bytes(step: PrefillStep) -> int:
    n = ctypes.c_size_t(0)
    d = step.desc()
    check(lib().esda_prefill_workspace_size(ctypes.byref(d), ctypes.byref(n)))
    return int(n.value)


STAGE_ATTEND = 1
STAGE_MERGE = 2


def prefill(step: PrefillStep, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None,
            workspace: torch.Tensor | None = None, stream=None, stages: int = STAGE_ATTEND | STAGE_MERGE) -> torch.Tensor:
    """O [Sq, Hq, D] bf16 of ``step`` (strides as in ``step``; defaults: q [Hq, Sq, D],
    k / v [Hkv, Sk, D], out [Sq, Hq, D], all dense).  ``stages`` selects the launches
    (timing only: the output is complete only with both)."""
    bf = torch.bfloat16
    D = step.head_dim
    if out is None:
        out = torch.empty((step.seq_q, step.num_q_heads, D), dtype=bf, device=q.device)
    d = step.desc()
    # the extent each tensor must cover (elements), checked before the pointers go down
    need = {
        "q": (step.num_q_heads - 1) * d.q_head_stride + (step.seq_q - 1) * d.q_row_stride + D,
        "k": (step.num_kv_heads - 1) * d.kv_head_stride + step.seq_k * D,
        "out": (step.seq_q - 1) * d.out_row_stride + (step.num_q_heads - 1) * d.out_head_stride + D,
    }
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.dtype != bf or not t.is_cuda:
            raise ValueError(f"{name} must be a bf16 GPU tensor")
        avail = t.untyped_storage().nbytes() // 2 - t.storage_offset()
        if avail < need["k" if name == "v" else name]:
            raise ValueError(f"{name} is smaller than the description's extent")
    nbytes = prefill_workspace_bytes(step)
    if nbytes and (workspace is None or workspace.numel() * workspace.element_size() < nbytes):
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    a = PrefillArgs(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(out),
                    _dev_ptr(workspace) if nbytes else None, nbytes)
    check(lib().esda_prefill_stages(ctypes.byref(d), ctypes.byref(a), int(stages), _stream_ptr(stream)))
    return out


def raw_prefill_kv(raw: torch.Tensor, kw: torch.Tensor, eps: float, inv_freq: torch.Tensor, pos0: int = 0,
                   k_out: torch.Tensor | None = None, v_out: torch.Tensor | None = None, stream=None):
    """K, V [Hkv, Sk, D] bf16 of a raw-K view raw [Hkv, Sk, D] (dense rows) by the
    reference's prefill ops (ESAttention.mm:306-326); key t at position pos0 + t."""
    Hkv, Sk, D = raw.shape
    if raw.dtype != torch.bfloat16 or raw.stride(2) != 1 or raw.stride(1) != D:
        raise ValueError("raw must be a bf16 [Hkv, Sk, D] view with dense rows")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != D // 2 or not inv_freq.is_contiguous():
        raise ValueError("inv_freq must be contiguous float32 [D/2]")
    if kw.dtype != torch.bfloat16 or kw.numel() != D or not kw.is_contiguous():
        raise ValueError("kw must be contiguous bf16 [D]")
    k_out = torch.empty((Hkv, Sk, D), dtype=torch.bfloat16, device=raw.device) if k_out is None else k_out
    v_out = torch.empty((Hkv, Sk, D), dtype=torch.bfloat16, device=raw.device) if v_out is None else v_out
    for t in (k_out, v_out):
        if t.shape != (Hkv, Sk, D) or not t.is_contiguous():
            raise ValueError("k_out / v_out must be contiguous [Hkv, Sk, D]")
    check(lib().esda_raw_prefill_kv(_dev_ptr(raw), raw.stride(0), Hkv, Sk, D, _dev_ptr(kw), eps, _dev_ptr(inv_freq),
                                    pos0, _dev_ptr(k_out), _dev_ptr(v_out), Sk * D, _stream_ptr(stream)))
    return k_out, v_out


def raw_q8_prefill_kv(q8: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, kw: torch.Tensor, eps: float,
                      inv_freq: torch.Tensor, pos0: int = 0, k_out: torch.Tensor | None = None,
                      v_out: torch.Tensor | None = None, stream=None):
    """As raw_prefill_kv over a q8 raw view: q8 [Hkv, Sk, 512] u8 (dense rows), scale /
    bias [Hkv, Sk] f32 views (unit row stride); rows dequantised to bf16(q*scale + bias)."""
    Hkv, Sk, D = q8.shape
    if D != 512 or q8.dtype != torch.uint8 or q8.stride(2) != 1 or q8.stride(1) != 512:
        raise ValueError("q8 must be a u8 [Hkv, Sk, 512] view with dense rows")
    for t in (scale, bias):
        if t.dtype != torch.float32 or t.shape[:2] != (Hkv, Sk) or t.stride(1) != 1 or t.stride(0) != scale.stride(0):
            raise ValueError("scale / bias must be float32 [Hkv, Sk] views with unit row stride")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != 256 or not inv_freq.is_contiguous():
        raise ValueError("inv_freq must be contiguous float32 [256]")
    if kw.dtype != torch.bfloat16 or kw.numel() != D or not kw.is_contiguous():
        raise ValueError("kw must be contiguous bf16 [512]")
    k_out = torch.empty((Hkv, Sk, D), dtype=torch.bfloat16, device=q8.device) if k_out is None else k_out
    v_out = torch.empty((Hkv, Sk, D), dtype=torch.bfloat16, device=q8.device) if v_out is None else v_out
    for t in (k_out, v_out):
        if t.shape != (Hkv, Sk, D) or not t.is_contiguous():
            raise ValueError("k_out / v_out must be contiguous [Hkv, Sk, 512]")
    check(lib().esda_raw_q8_prefill_kv(_dev_ptr(q8), q8.stride(0), _dev_ptr(scale), _dev_ptr(bias), scale.stride(0),
                                       Hkv, Sk, _dev_ptr(kw), eps, _dev_ptr(inv_freq), pos0, _dev_ptr(k_out),
                                       _dev_ptr(v_out), Sk * D, _stream_ptr(stream)))
    return k_out, v_out
