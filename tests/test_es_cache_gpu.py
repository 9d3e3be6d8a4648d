"""GPU checks of the ES* C++ layer (ESKVCache through include/esda_cache.h).

update() in both storage modes is compared byte for byte with a host model of the
reference's semantics (concatenate along the sequence axis, keep the last maxKeep rows:
ESKVCache.mm:35-55 and 64-109); decode() is compared with the CPU oracle on the rows
that model says are live, across buffer growth and compaction; the mode-mismatch
guards raise the reference's error class.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from _synth import rms_rows

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _view(v) -> np.ndarray:
    return _host(v.torch())


@pytest.mark.parametrize("max_keep", [0, 48])
def test_update_modes_match_the_concat_model(max_keep):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(max_keep + 1)
    kvh, hd = 2, 128
    cache = ESKVCache(2)
    model_k = np.zeros((kvh, 0, hd), np.uint16)
    model_v = np.zeros((kvh, 0, hd), np.uint16)
    # a prefill of 70 rows, then single-row appends across two capacity growths
    sizes = [70] + [1] * 500
    for i, n in enumerate(sizes):
        kn, vn = rms_rows(rng, (kvh, n, hd)), rms_rows(rng, (kvh, n, hd))
        model_k = np.concatenate([model_k, kn], axis=1)
        model_v = np.concatenate([model_v, vn], axis=1)
        if max_keep and model_k.shape[1] > max_keep and n == 1:
            model_k, model_v = model_k[:, -max_keep:], model_v[:, -max_keep:]
        lk, lv = cache.update(0, _dev(kn), _dev(vn), max_keep if n == 1 else 0, prealloc=False)
        pk, pv = cache.update(1, _dev(kn), _dev(vn), max_keep if n == 1 else 0, prealloc=True)
        if i % 61 == 0 or i == len(sizes) - 1:
            for v, m in ((lk, model_k), (lv, model_v), (pk, model_k), (pv, model_v)):
                assert v.rows == m.shape[1]
                assert np.array_equal(_view(v), m), f"step {i}: view differs from the model"
    s = cache.slot(1)
    assert s["len"] - s["start"] == model_k.shape[1]
    assert s["capacity"] % 256 == 0 and s["capacity"] >= s["len"]
    assert s["lost"] == bool(max_keep)  # a compaction dropped evicted rows only when sliding
    ck, cv = cache.current(1, True)
    assert np.array_equal(_view(ck), model_k) and np.array_equal(_view(cv), model_v)


def test_first_prealloc_store_has_capacity_equal_to_content_then_grows_by_chunks():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(3)
    cache = ESKVCache(1)
    kn = rms_rows(rng, (4, 100, 64))
    cache.update(0, _dev(kn), _dev(kn), 0, prealloc=True)
    assert cache.slot(0)["capacity"] == 100
    one = rms_rows(rng, (4, 1, 64))
    cache.update(0, _dev(one), _dev(one), 0, prealloc=True)
    assert cache.slot(0)["capacity"] == 512  # roundUp(100 + 1 + 256, 256)


def _decode_run(cache, layer, rng, *, kvh, hq, hd, shared, max_keep, steps, prefill, scale, window=None):
    """Prefill with update(prealloc), then decode() steps, each checked against the oracle
    on the live rows of the host model under the sliding mask of `window` (default: a
    sliding layer's window = max_keep; 0 = full causal)."""
    window = max_keep if window is None else window
    model_k = rms_rows(rng, (kvh, prefill, hd)) if prefill else np.zeros((kvh, 0, hd), np.uint16)
    model_v = model_k if shared else (rms_rows(rng, (kvh, prefill, hd)) if prefill else model_k.copy())
    if prefill:
        k_d = _dev(model_k)
        cache.update(layer, k_d, k_d if shared else _dev(model_v), 0, prealloc=True)
    worst = 0.0
    for i in range(steps):
        q = rms_rows(rng, (hq, hd))
        kn = rms_rows(rng, (kvh, 1, hd))
        vn = kn if shared else rms_rows(rng, (kvh, 1, hd))
        kn_d = _dev(kn)
        out = cache.decode(layer, _dev(q), kn_d, kn_d if shared else _dev(vn), max_keep, window, scale)
        model_k = np.concatenate([model_k, kn], axis=1)
        model_v = model_k if shared else np.concatenate([model_v, vn], axis=1)
        if max_keep and model_k.shape[1] > max_keep:
            model_k = model_k[:, -max_keep:]
            model_v = model_k if shared else model_v[:, -max_keep:]
        live = model_k.shape[1]
        if i % 7 == 0 or i == steps - 1:
            step = orc.Step(B=1, Hq=hq, Hkv=kvh, D=hd, cap=live, window=min(window, live), scale=scale)
            ref = orc.decode_f64(step, q.reshape(1, hq, hd), np.ascontiguousarray(model_k).reshape(-1),
                                 np.ascontiguousarray(model_v).reshape(-1), [live - 1])
            o = orc.from_bf16(_host(out)).reshape(1, hq, hd).astype(np.float64)
            err = np.abs(o - ref)
            worst = max(worst, err.max())
            assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, f"step {i}"
    ck, cv = cache.current(layer, True)
    assert np.array_equal(_view(ck), model_k) and np.array_equal(_view(cv), model_v)
    return worst


def test_decode_sliding_layer_across_compaction():
    from apertura_amd.cache import ESKVCache
    cache = ESKVCache(1)
    w = _decode_run(cache, 0, np.random.default_rng(5), kvh=4, hq=8, hd=256, shared=False, max_keep=96,
                    steps=480, prefill=40, scale=1 / 16)
    s = cache.slot(0)
    assert s["len"] - s["start"] == 96 and s["lost"] and not s["shared"]
    print(f"sliding worst max_abs {w:.3e}")


def test_decode_sliding_mask_without_eviction():
    """A sliding layer whose cache keeps every row (maxKeep = 0: the reference's
    --no-swa-cache, or a layer storing its full K/V, ESAttention.mm:99-103) still masks
    all but the last `window` positions (ESGemma4TextModel.mm:68-83)."""
    from apertura_amd.cache import ESKVCache
    cache = ESKVCache(1)
    w = _decode_run(cache, 0, np.random.default_rng(15), kvh=4, hq=8, hd=256, shared=False, max_keep=0,
                    window=64, steps=300, prefill=40, scale=1 / 16)
    s = cache.slot(0)
    assert s["len"] == 340 and s["start"] == 0 and not s["lost"]
    print(f"unevicted sliding worst max_abs {w:.3e}")


def test_decode_global_k_eq_v_across_growth():
    from apertura_amd.cache import ESKVCache
    cache = ESKVCache(2)
    w = _decode_run(cache, 1, np.random.default_rng(7), kvh=2, hq=16, hd=512, shared=True, max_keep=0,
                    steps=300, prefill=230, scale=512 ** -0.5)
    s = cache.slot(1)
    assert s["len"] == 530 and s["start"] == 0 and s["shared"] and s["capacity"] >= 530
    print(f"global worst max_abs {w:.3e}")


def test_decode_on_an_empty_slot_starts_the_cache():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(9)
    cache = ESKVCache(1)
    w = _decode_run(cache, 0, rng, kvh=1, hq=4, hd=128, shared=True, max_keep=0, steps=20, prefill=0,
                    scale=1.0)
    assert w <= TOL_MAX
    s = cache.slot(0)
    assert s["len"] == 20 and s["shared"]


def test_mode_mismatch_guards_raise_runtime_error():
    from apertura_amd import EsdaError
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(11)
    cache = ESKVCache(2)
    kv = _dev(rms_rows(rng, (2, 3, 512)))
    cache.update(0, kv, kv, 0, prealloc=True)
    with pytest.raises(EsdaError) as ei:
        cache.update_raw(0, kv, True)
    assert ei.value.code == 2 and "composite" in str(ei.value)
    cache.update_raw(1, kv, True)
    with pytest.raises(EsdaError) as ei:
        cache.update(1, kv, kv, 0, prealloc=True)
    assert ei.value.code == 2 and "raw-K" in str(ei.value)
    with pytest.raises(EsdaError) as ei:
        cache.decode(1, _dev(rms_rows(rng, (16, 512))), kv[:, :1].contiguous(), kv[:, :1].contiguous(), 0, 0, 1.0)
    assert ei.value.code == 2
    assert cache.slot(1)["raw"] and not cache.slot(0)["raw"]
    # a shared K=V slot refuses a distinct V row
    c2 = ESKVCache(1)
    one = _dev(rms_rows(rng, (2, 1, 128)))
    c2.decode(0, _dev(rms_rows(rng, (4, 128))), one, one, 0, 0, 1.0)
    other = _dev(rms_rows(rng, (2, 1, 128)))
    with pytest.raises(EsdaError) as ei:
        c2.decode(0, _dev(rms_rows(rng, (4, 128))), one, other, 0, 0, 1.0)
    assert ei.value.code == 2


def test_update_raw_layout_and_growth():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(13)
    cache = ESKVCache(1)
    model = rms_rows(rng, (4, 300, 512))
    view, ln, pitch = cache.update_raw(0, _dev(model), True)
    assert (ln, pitch) == (300, 300)
    for _ in range(3):
        one = rms_rows(rng, (4, 1, 512))
        view, ln, pitch = cache.update_raw(0, _dev(one), True)
        model = np.concatenate([model, one], axis=1)
    assert (ln, pitch) == (303, 768)  # roundUp(300 + 1 + 256, 256)
    assert np.array_equal(_view(view), model)


def test_decode_raw_through_the_cache_matches_oracle():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(15)
    kvh, hq, eps = 2, 16, 1e-6
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    kw = orc.to_bf16((1.0 + 0.2 * rng.standard_normal(512)).astype(np.float32))
    kw_d = _dev(kw)
    cache = ESKVCache(1)
    model = orc.to_bf16(rng.standard_normal((kvh, 200, 512), dtype=np.float32) * 2.0)
    cache.update_raw(0, _dev(model), True)
    for i in range(70):
        q = rms_rows(rng, (hq, 512))
        one = orc.to_bf16(rng.standard_normal((kvh, 1, 512), dtype=np.float32) * 2.0)
        out = cache.decode_raw(0, _dev(q), _dev(one), kw_d, eps, list(inv))
        model = np.concatenate([model, one], axis=1)
        if i % 10 == 0 or i == 69:
            ref = orc.decode_raw_f64(q, np.ascontiguousarray(model), model.shape[1], kw, eps, inv, 1.0)
            o = orc.from_bf16(_host(out)).reshape(hq, 512).astype(np.float64)
            err = np.abs(o - ref)
            assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, f"step {i}"
    view, ln, pitch = cache.update_raw(0, _dev(np.zeros((kvh, 1, 512), np.uint16)), True)
    assert ln == 271 and np.array_equal(_view(view)[:, :270], model)


def test_unprimed_cache_failure_values_and_step_counter(tmp_path):
    """An unprimed cache: nothing to snapshot or rewind (the reference's false / -1);
    seqLen counts markStep calls until reset."""
    from apertura_amd.cache import ESKVCache
    cache = ESKVCache(3)
    assert cache.save_snapshot(str(tmp_path / "kv.safetensors"), "fp", 10) is False
    assert cache.restore_snapshot(str(tmp_path / "kv.safetensors"), "fp") == -1
    assert cache.mark_rewind_point(5) is False
    assert cache.rewind_to_mark() == -1
    cache.mark_step(5)
    cache.mark_step(2)
    assert cache.seq_len() == 7
    cache.reset()
    assert cache.seq_len() == 0


def test_compiled_step_mode_scatters_at_device_positions():
    """Compiled-step mode (ESKVCache.h:93-112, driven as ESGenerationLoop.mm:104-238 does):
    slots adopted with setSlot, then update() inside beginStep .. endStep writes the one
    new row at the row the device index words hold -- the sliding index for maxKeep > 0,
    the global index otherwise -- and returns the full-capacity buffers.  The appends are
    captured once in a HIP graph and replayed for several positions set on the device
    between replays; every byte of both slots matches a host model after each replay.
    takeSlot empties a slot; the fused calls refuse to run inside a step."""
    from apertura_amd._lib import EsdaError
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(71)
    W, capS, capG = 16, 32, 96
    cache = ESKVCache(2)
    # layer 0: sliding, separate K / V (hd 256); layer 1: global, one shared K=V buffer (hd 512)
    sk = torch.zeros((2, capS, 256), dtype=torch.bfloat16, device="cuda")
    sv = torch.zeros_like(sk)
    g = torch.zeros((2, capG, 512), dtype=torch.bfloat16, device="cuda")
    cache.set_slot(0, sk, sv)
    cache.set_slot(1, g, g)
    model = {"sk": np.zeros((2, capS, 256), np.uint16), "sv": np.zeros((2, capS, 256), np.uint16),
             "g": np.zeros((2, capG, 512), np.uint16)}
    gidx = torch.zeros(1, dtype=torch.int32, device="cuda")
    sidx = torch.zeros(1, dtype=torch.int32, device="cuda")
    kn_s, vn_s = torch.empty((2, 1, 256), dtype=torch.bfloat16, device="cuda"), torch.empty(
        (2, 1, 256), dtype=torch.bfloat16, device="cuda")
    kn_g = torch.empty((2, 1, 512), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()

    def appends():
        ks, vs = cache.update(0, kn_s, vn_s, W, True, stream)
        kg, vg = cache.update(1, kn_g, kn_g, 0, True, stream)
        return ks, vs, kg, vg

    print("\n[case] compiled-step mode: eager step, then a captured graph", flush=True)
    cache.begin_step(gidx, sidx)
    with pytest.raises(EsdaError) as ei:
        cache.decode(1, torch.zeros((16, 512), dtype=torch.bfloat16, device="cuda"), kn_g, kn_g, 0, 0, 1.0)
    assert ei.value.code == 2
    graph = None
    base = 40 - W  # sliding slot 0 holds this position (the adopted window ends at 39)
    for step, pos in enumerate(range(40, 52)):
        srow = pos - base
        rows = {k: rms_rows(rng, (2, 1, d)) for k, d in (("ks", 256), ("vs", 256), ("kg", 512))}
        kn_s.copy_(_dev(rows["ks"]))
        vn_s.copy_(_dev(rows["vs"]))
        kn_g.copy_(_dev(rows["kg"]))
        gidx.fill_(pos)
        sidx.fill_(srow)
        torch.cuda.synchronize()
        if step == 0:
            ks, vs, kg, vg = appends()  # eager
            assert ks.rows == capS and kg.rows == capG and kg.data == vg.data
            with torch.cuda.stream(stream):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    appends()
        else:
            with torch.cuda.stream(stream):
                graph.replay()
        torch.cuda.synchronize()
        model["sk"][:, srow] = rows["ks"][:, 0]
        model["sv"][:, srow] = rows["vs"][:, 0]
        model["g"][:, pos] = rows["kg"][:, 0]
        assert np.array_equal(_host(sk), model["sk"]) and np.array_equal(_host(sv), model["sv"]), f"pos {pos}"
        assert np.array_equal(_host(g), model["g"]), f"pos {pos}"
    cache.end_step()
    k0, v0 = cache.slot_kv(0)
    assert k0.data == sk.data_ptr() and v0.data == sv.data_ptr() and k0.rows == capS
    tk, tv = cache.take_slot(1)
    assert tk.data == g.data_ptr() and tv.data == g.data_ptr()
    with pytest.raises(EsdaError) as ei:
        cache.slot_kv(1)
    assert ei.value.code == 2


def test_compiled_step_shared_slot_refuses_a_distinct_v():
    """A compiled-step slot adopted with one shared K=V buffer (setSlot(k, k)) takes one row per
    update: a vNew that does not alias kNew would be scattered over the K row just written, so
    update() refuses it with invalid_argument before any launch, and the buffer is unchanged.
    The aliased update of the same step then writes its row."""
    from apertura_amd._lib import EsdaError
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(72)
    cap = 64
    cache = ESKVCache(1)
    g = _dev(rms_rows(rng, (2, cap, 512)))
    before = _host(g)
    cache.set_slot(0, g, g)
    gidx = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    sidx = torch.zeros(1, dtype=torch.int32, device="cuda")
    kn = _dev(rms_rows(rng, (2, 1, 512)))
    vn = _dev(rms_rows(rng, (2, 1, 512)))
    print("\n[case] compiled step, shared slot, distinct vNew", flush=True)
    cache.begin_step(gidx, sidx)
    with pytest.raises(EsdaError) as ei:
        cache.update(0, kn, vn, 0, True)
    assert ei.value.code == 1 and "alias" in str(ei.value)
    torch.cuda.synchronize()
    assert np.array_equal(_host(g), before), "a refused step wrote the slot"
    cache.update(0, kn, kn, 0, True)
    torch.cuda.synchronize()
    cache.end_step()
    want = before.copy()
    want[:, 7] = _host(kn)[:, 0]
    assert np.array_equal(_host(g), want)
