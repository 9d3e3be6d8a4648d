"""GPU checks of the ES* layer's prefill branch (ESKVCache::prefill / prefillRaw through
include/esda_cache.h): chunked prefill as the reference's ESAttention runs it at seq > 1
(ESAttention.mm:77-108 append, :168-193 SDPA with buildMask / alignMask; raw-K and q8
raw-K :253-332), each chunk compared with the fp64 prefill oracle over a host model of
the cache's live rows (sliding layers keep window + chunk keys), then decode steps on
the same cache continue from it.  Tolerance max-abs <= 2e-2, mean-abs <= 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from _synth import rms_rows

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3
EPS = 1e-6


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _check(out, ref, what):
    o = orc.from_bf16(_host(out)).astype(np.float64).reshape(ref.shape)
    err = np.abs(o - ref)
    print(f"[es-prefill] {what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, what


def _close_bf16(ours, ref, what):
    """The reconstruction kernel against the oracle's: equal but for rare bf16
    rounding-boundary cases (two bf16 steps of the value, or one step of the row's
    largest element where the rotated products nearly cancel)."""
    a, b = orc.from_bf16(ours), orc.from_bf16(ref)
    floor = np.abs(b).max(axis=-1, keepdims=True) * 2.0 ** -8
    assert not (np.abs(a - b) > np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -6 + floor).any(), what
    assert np.mean(ours != ref) < 1e-2, what


@pytest.mark.parametrize("shared,D,Hq,Hkv,window,chunks", [
    (False, 256, 8, 4, 64, [100, 37, 80]),     # local: sliding window, chunked eviction
    (True, 512, 16, 2, 0, [300, 200, 40]),     # global k_eq_v: one shared buffer, growth
])
def test_chunked_prefill_then_decode(shared, D, Hq, Hkv, window, chunks):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(D + len(chunks))
    scale = D ** -0.5
    cache = ESKVCache(1)
    mk = np.zeros((Hkv, 0, D), np.uint16)
    mv = mk.copy()
    past = 0
    for ci, n in enumerate(chunks):
        q = rms_rows(rng, (Hq, n, D))
        kn = rms_rows(rng, (Hkv, n, D))
        vn = kn if shared else rms_rows(rng, (Hkv, n, D))
        max_keep = window + n if window else 0
        kd = _dev(kn)
        out = cache.prefill(0, _dev(q), kd, kd if shared else _dev(vn), max_keep, window, scale, past)
        torch.cuda.synchronize()
        mk = np.concatenate([mk, kn], axis=1)
        mv = mk if shared else np.concatenate([mv, vn], axis=1)
        if max_keep and mk.shape[1] > max_keep:
            mk = mk[:, -max_keep:]
            mv = mk if shared else mv[:, -max_keep:]
        live = mk.shape[1]
        ref = orc.prefill_f64(q, mk, mv, past, past + n - live, window, scale)  # [n, Hq, D]
        _check(out, ref, f"chunk {ci} (rows {n}, live {live})")
        past += n
    # decode continues on the prefilled cache (maxKeep = window on a sliding layer)
    for i in range(3):
        q = rms_rows(rng, (Hq, D))
        kn = rms_rows(rng, (Hkv, 1, D))
        vn = kn if shared else rms_rows(rng, (Hkv, 1, D))
        kd = _dev(kn)
        out = cache.decode(0, _dev(q), kd, kd if shared else _dev(vn), window, window, scale)
        torch.cuda.synchronize()
        mk = np.concatenate([mk, kn], axis=1)
        mv = mk if shared else np.concatenate([mv, vn], axis=1)
        if window and mk.shape[1] > window:
            mk = mk[:, -window:]
            mv = mk if shared else mv[:, -window:]
        ref = orc.prefill_f64(q[:, None], mk, mv, past, past + 1 - mk.shape[1], window, scale)
        _check(out, ref, f"decode {i}")
        past += 1


@pytest.mark.parametrize("q8", [False, True])
def test_raw_prefill_chunks_then_decode(q8):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(50 + q8)
    Hq, Hkv = 16, 2
    kw = orc.to_bf16((1.0 + 0.2 * rng.standard_normal(512)).astype(np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)   # 256 entries, 64 nonzero
    kw_d = _dev(kw)
    cache = ESKVCache(1)
    model = np.zeros((Hkv, 0, 512), np.uint16)
    past = 0

    def view_of(m):
        if not q8:
            return m
        qc, sc, bs = orc.quantize_rows(m)
        return orc.to_bf16((qc.astype(np.float32) * sc[..., None]).astype(np.float32) + bs[..., None])

    from apertura_amd.prefill import raw_prefill_kv, raw_q8_prefill_kv
    inv_d = torch.from_numpy(inv).cuda()
    for ci, n in enumerate([150, 90]):
        q = rms_rows(rng, (Hq, n, 512))
        kn = orc.to_bf16((rng.standard_normal((Hkv, n, 512), dtype=np.float32) * 2.0).astype(np.float32))
        out = cache.prefill_raw(0, _dev(q), _dev(kn), kw_d, EPS, list(inv), past, 1.0, q8=q8)
        torch.cuda.synchronize()
        model = np.concatenate([model, kn], axis=1)
        # The K / V the call rebuilt: the same kernel over the slot's stored rows (bitwise
        # the same input), checked against the oracle's reconstruction; the attention is
        # then checked over exactly those K / V.  (At in-model scale 1.0 logits spread by
        # tens, and a near tie turns one bf16 step of a K element into ~1e-2 of output.)
        if q8:
            gq, gsc, gbs = cache.current_raw_q8(0).torch()
            gk, gv = raw_q8_prefill_kv(gq, gsc, gbs, kw_d, EPS, inv_d)
        else:
            view, ln, _ = cache.current_raw(0)
            gk, gv = raw_prefill_kv(view.torch(), kw_d, EPS, inv_d)
        torch.cuda.synchronize()
        gk, gv = _host(gk), _host(gv)
        ek, ev = orc.raw_prefill_kv(view_of(model), kw, EPS, inv, 0)
        _close_bf16(gk, ek, f"chunk {ci} K")
        _close_bf16(gv, ev, f"chunk {ci} V")
        _check(out, orc.prefill_f64(q, gk, gv, past, 0, 0, 1.0), f"raw chunk {ci} q8={q8}")
        past += n
    assert cache.slot(0)["q8" if q8 else "raw"] and cache.slot(0)["len"] == past
    # one decode step continues on the same stream (the fused raw / q8 decode kernels)
    q = rms_rows(rng, (Hq, 512))
    one = orc.to_bf16((rng.standard_normal((Hkv, 1, 512), dtype=np.float32) * 2.0).astype(np.float32))
    out = (cache.decode_raw_q8 if q8 else cache.decode_raw)(0, _dev(q), _dev(one), kw_d, EPS, list(inv))
    torch.cuda.synchronize()
    model = np.concatenate([model, one], axis=1)
    if q8:
        qc, sc, bs = orc.quantize_rows(model)
        ref = orc.decode_raw_q8_f64(q, qc, sc, bs, model.shape[1], kw, EPS, inv, 1.0)
    else:
        ref = orc.decode_raw_f64(q, model, model.shape[1], kw, EPS, inv, 1.0)
    _check(out, ref, f"raw decode after prefill q8={q8}")
