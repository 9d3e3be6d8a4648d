"""GPU checks of KV snapshots, prefix markers and turn rewind (es::ESKVCache through
include/esda_cache.h), after ESKVCache.mm:121-456.

The file format is checked from the other side with the `safetensors` package: files the
library writes are read back with it (names, dtypes, shapes, bytes, metadata), and files
written with it in the reference's layout (k_<i>/v_<i>, raw k_<i>, q8 rq_/rs_/rb_) are
restored by the library.  Restores are compared byte for byte with the saved live rows,
and a decode step after a restore or a rewind must give the same bits as the same step
on a cache that never went through it.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from _synth import rms_rows

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _view(v) -> np.ndarray:
    return _host(v.torch())


# Layer kinds of the test cache: a sliding layer (separate K/V, window 64), a global
# k_eq_v layer (one shared buffer), a raw-K layer, a global layer with separate K/V.
SLIDE, SHARED, RAW, GLOBAL = 0, 1, 2, 3
WINDOW = 64


def _prime(cache, rng, prefill, steps, hd=128, raw_hd=512):
    """Prefill `prefill` rows into every layer, then `steps` single-row appends (decode
    for the composite layers, updateRaw for the raw one).  Returns the host model of
    each layer's live rows."""
    model = {}
    k = rms_rows(rng, (2, prefill, hd))
    v = rms_rows(rng, (2, prefill, hd))
    cache.update(SLIDE, _dev(k), _dev(v), WINDOW, prealloc=True)
    model[SLIDE] = [k[:, -WINDOW:], v[:, -WINDOW:]]
    s = rms_rows(rng, (1, prefill, hd))
    sd = _dev(s)
    cache.update(SHARED, sd, sd, 0, prealloc=True)
    model[SHARED] = [s, s]
    r = (rms_rows(rng, (1, prefill, raw_hd)).view(np.uint16))
    cache.update_raw(RAW, _dev(r), True)
    model[RAW] = [r]
    gk, gv = rms_rows(rng, (1, prefill, hd)), rms_rows(rng, (1, prefill, hd))
    cache.update(GLOBAL, _dev(gk), _dev(gv), 0, prealloc=True)
    model[GLOBAL] = [gk, gv]
    for _ in range(steps):
        _step(cache, rng, model, hd, raw_hd)
    return model


def _step(cache, rng, model, hd=128, raw_hd=512, q_seed=None):
    """One decode step on every layer; returns the outputs (bf16 host arrays)."""
    outs = []
    k, v = rms_rows(rng, (2, 1, hd)), rms_rows(rng, (2, 1, hd))
    q = rms_rows(rng, (4, hd))
    outs.append(_host(cache.decode(SLIDE, _dev(q), _dev(k), _dev(v), WINDOW, WINDOW, 1.0)))
    model[SLIDE] = [np.concatenate([m, x], axis=1)[:, -WINDOW:] for m, x in zip(model[SLIDE], (k, v))]
    s = rms_rows(rng, (1, 1, hd))
    sd = _dev(s)
    q = rms_rows(rng, (8, hd))
    outs.append(_host(cache.decode(SHARED, _dev(q), sd, sd, 0, 0, 1.0)))
    model[SHARED] = [np.concatenate([model[SHARED][0], s], axis=1)] * 2
    r = rms_rows(rng, (1, 1, raw_hd))
    cache.update_raw(RAW, _dev(r), True)
    model[RAW] = [np.concatenate([model[RAW][0], r], axis=1)]
    gk, gv = rms_rows(rng, (1, 1, hd)), rms_rows(rng, (1, 1, hd))
    q = rms_rows(rng, (8, hd))
    outs.append(_host(cache.decode(GLOBAL, _dev(q), _dev(gk), _dev(gv), 0, 0, 1.0)))
    model[GLOBAL] = [np.concatenate([m, x], axis=1) for m, x in zip(model[GLOBAL], (gk, gv))]
    return outs


def _live(cache, layer):
    if cache.slot(layer)["raw"]:
        return [_view(cache.current_raw(layer)[0])]
    kv, vv = cache.current(layer, True)
    return [_view(kv), _view(vv)]


def _snapshot_state(cache, n):
    return [(cache.slot(i), [a.copy() for a in _live(cache, i)]) for i in range(n)]


def test_snapshot_round_trip_is_bit_exact(tmp_path):
    from apertura_amd.cache import ESKVCache
    from safetensors import safe_open
    rng = np.random.default_rng(1)
    a = ESKVCache(4)
    model = _prime(a, rng, prefill=300, steps=20)
    path = str(tmp_path / "snap.safetensors")
    assert a.save_snapshot(path, "fp-A", 320)
    # the file, read by the safetensors package: the reference's names and layout
    with safe_open(path, framework="pt") as f:
        meta = f.metadata()
        names = set(f.keys())
        assert meta["fingerprint"] == "fp-A" and meta["pos"] == "320" and meta["layers"] == "4"
        assert meta["marker_count"] == "0" and meta.get("shared_1") == "1"
        assert names == {"k_0", "v_0", "k_1", "v_1", "k_2", "k_3", "v_3"}
        for name, arr in (("k_0", model[SLIDE][0]), ("v_0", model[SLIDE][1]), ("k_1", model[SHARED][0]),
                          ("v_1", model[SHARED][1]), ("k_2", model[RAW][0]), ("k_3", model[GLOBAL][0]),
                          ("v_3", model[GLOBAL][1])):
            t = f.get_tensor(name)
            assert t.dtype == torch.bfloat16 and tuple(t.shape) == arr.shape, name
            assert np.array_equal(_host(t), arr), name
    b = ESKVCache(4)
    assert b.restore_snapshot(path, "fp-A") == 320
    for i in range(4):
        sa, sb = a.slot(i), b.slot(i)
        live = sa["len"] - sa["start"]
        assert sb["start"] == 0 and sb["len"] == live
        assert sb["capacity"] == (live + 256 + 255) // 256 * 256  # roundUp(content + kGrowChunk)
        assert (sb["shared"], sb["raw"]) == (sa["shared"], sa["raw"])
        assert sb["lost"] == (live < 320)  # a window is not a full prefix
        for x, y in zip(_live(a, i), _live(b, i)):
            assert np.array_equal(x, y), f"layer {i} differs after restore"
    # continuing from the restored cache gives the same bits as continuing the original
    oa = _step(a, np.random.default_rng(99), model)
    ob = _step(b, np.random.default_rng(99), {k: [x.copy() for x in v] for k, v in model.items()})
    for x, y in zip(oa, ob):
        assert np.array_equal(x, y)


def test_refused_restores_leave_the_cache_untouched(tmp_path):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(2)
    a = ESKVCache(4)
    _prime(a, rng, prefill=100, steps=3)
    good = str(tmp_path / "good.safetensors")
    assert a.save_snapshot(good, "fp", 103)
    target = ESKVCache(4)
    _prime(target, np.random.default_rng(3), prefill=50, steps=2)
    before = _snapshot_state(target, 4)
    raw_bytes = open(good, "rb").read()
    bad = {}
    bad["truncated"] = raw_bytes[: len(raw_bytes) - 100]
    bad["header_garbage"] = raw_bytes[:8] + b"{" + b"x" * 40 + raw_bytes[49:]
    bad["huge_header_len"] = (1 << 40).to_bytes(8, "little") + raw_bytes[8:]
    bad["empty"] = b""
    for name, blob in bad.items():
        p = str(tmp_path / f"{name}.safetensors")
        open(p, "wb").write(blob)
        assert target.restore_snapshot(p, "fp") == -1, name
    assert target.restore_snapshot(str(tmp_path / "missing.safetensors"), "fp") == -1
    assert target.restore_snapshot(good, "other-fp") == -1                 # fingerprint miss, no markers
    assert target.restore_snapshot(good, "fp", mode="composite") == -1    # the file holds a raw layer
    comp_only = str(tmp_path / "composite.safetensors")
    _save_composite_only(comp_only, 4)
    assert target.restore_snapshot(comp_only, "fp", mode="rawQ8") == -1   # composite -> raw q8
    assert target.restore_snapshot(comp_only, "fp", mode="raw") == -1     # composite -> raw
    assert ESKVCache(3).restore_snapshot(good, "fp") == -1                 # layer count
    after = _snapshot_state(target, 4)
    for (s0, l0), (s1, l1) in zip(before, after):
        assert s0 == s1
        for x, y in zip(l0, l1):
            assert np.array_equal(x, y)
    # an unprimed layer: nothing to save
    assert not ESKVCache(2).save_snapshot(str(tmp_path / "x.safetensors"), "fp", 0)


def _save_composite_only(path, layers):
    from safetensors.torch import save_file
    rng = np.random.default_rng(40)
    t = {}
    for i in range(layers):
        for n in ("k_", "v_"):
            t[n + str(i)] = torch.from_numpy(rms_rows(rng, (1, 20, 128)).view(np.int16)).view(torch.bfloat16)
    save_file(t, path, metadata={"fingerprint": "fp", "pos": "20", "layers": str(layers)})


def test_reference_layout_files_restore(tmp_path):
    """Files written by the safetensors package in the reference's layout: a composite
    layer (k_0/v_0), a raw-K layer (k_1), and a q8 raw layer (rq_2/rs_2/rb_2).  As stored
    the q8 layer keeps its bytes; mode raw rehydrates it to bf16(float(q) * scale + bias)
    (ESKVCache.mm:366-383); mode rawQ8 quantizes the bf16 raw layer (ESKVCache.mm:394-408)."""
    from apertura_amd.cache import ESKVCache
    from safetensors.torch import save_file
    rng = np.random.default_rng(4)
    k0, v0 = rms_rows(rng, (2, 77, 256)), rms_rows(rng, (2, 77, 256))
    k1 = rms_rows(rng, (1, 90, 512))
    q2 = rng.integers(0, 256, size=(1, 90, 512), dtype=np.uint8)
    sc2 = (rng.random((1, 90, 1)) * 0.05 + 1e-3).astype(np.float32)
    bs2 = (-rng.random((1, 90, 1)) * 3).astype(np.float32)
    tensors = {"k_0": torch.from_numpy(k0.view(np.int16)).view(torch.bfloat16),
               "v_0": torch.from_numpy(v0.view(np.int16)).view(torch.bfloat16),
               "k_1": torch.from_numpy(k1.view(np.int16)).view(torch.bfloat16),
               "rq_2": torch.from_numpy(q2), "rs_2": torch.from_numpy(sc2), "rb_2": torch.from_numpy(bs2)}
    path = str(tmp_path / "ref.safetensors")
    save_file(tensors, path, metadata={"fingerprint": "ref", "pos": "90", "layers": "3"})
    c = ESKVCache(3)
    assert c.restore_snapshot(path, "ref", mode="composite") == -1
    assert c.restore_snapshot(path, "ref") == 90                  # as stored
    assert c.slot(1)["raw"] and not c.slot(1)["q8"] and np.array_equal(_live(c, 1)[0], k1)
    s2 = c.slot(2)
    assert s2["q8"] and not s2["raw"] and s2["len"] == 90 and s2["capacity"] == 512  # roundUp(90 + 256)
    gq, gsc, gbs = (t.cpu().numpy() for t in c.current_raw_q8(2).torch())
    assert np.array_equal(gq, q2) and np.array_equal(gsc, sc2[..., 0]) and np.array_equal(gbs, bs2[..., 0])
    assert c.restore_snapshot(path, "ref", mode="rawQ8") == 90    # bf16 raw layer quantized
    eq, esc, ebs = orc.quantize_rows(k1)
    gq, gsc, gbs = (t.cpu().numpy() for t in c.current_raw_q8(1).torch())
    assert c.slot(1)["q8"] and np.array_equal(gq, eq)
    assert np.array_equal(gsc.view(np.uint32), esc.view(np.uint32)) and np.array_equal(gbs.view(np.uint32), ebs.view(np.uint32))
    assert c.restore_snapshot(path, "ref", mode="raw") == 90
    assert np.array_equal(_live(c, 0)[0], k0) and np.array_equal(_live(c, 0)[1], v0)
    assert c.slot(0)["lost"] and c.slot(0)["len"] == 77           # 77 rows of a 90-position prefix
    assert c.slot(1)["raw"] and np.array_equal(_live(c, 1)[0], k1)
    expect = orc.to_bf16((q2.astype(np.float32) * sc2) + bs2)
    assert c.slot(2)["raw"] and not c.slot(2)["q8"] and np.array_equal(_live(c, 2)[0], expect)
    assert not c.slot(1)["q8"] and np.array_equal(_live(c, 1)[0], k1)


def test_prefix_marker_restores_the_longest_reproducible_prefix(tmp_path):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(5)
    hd = 128
    a = ESKVCache(2)  # 0: sliding (window 64), 1: global
    k, v = rms_rows(rng, (1, 4096, hd)), rms_rows(rng, (1, 4096, hd))
    gk, gv = rms_rows(rng, (1, 4096, hd)), rms_rows(rng, (1, 4096, hd))
    a.update(0, _dev(k), _dev(v), WINDOW, prealloc=True)
    a.update(1, _dev(gk), _dev(gv), 0, prealloc=True)
    with pytest.raises(Exception):
        a.mark_prefix(4095, "too-early")
    a.mark_prefix(4096, "prefix-4096")
    win_k, win_v = _live(a, 0)
    for _ in range(40):  # the turn goes on past the marker
        kn, vn = rms_rows(rng, (1, 1, hd)), rms_rows(rng, (1, 1, hd))
        a.decode(0, _dev(rms_rows(rng, (2, hd))), _dev(kn), _dev(vn), WINDOW, WINDOW, 1.0)
        a.decode(1, _dev(rms_rows(rng, (2, hd))), _dev(kn), _dev(vn), 0, 0, 1.0)
    path = str(tmp_path / "marked.safetensors")
    assert a.save_snapshot(path, "full-4136", 4136)
    b = ESKVCache(2)
    asked = []

    def prefix_fp(pos):
        asked.append(pos)
        return "prefix-4096" if pos == 4096 else ""

    assert b.restore_snapshot(path, "different-turn", prefix_fp=prefix_fp) == 4096
    assert asked == [4096]
    # global layer truncated to the marker; sliding layer = the marker's window
    assert b.slot(1)["len"] == 4096 and not b.slot(1)["lost"]
    assert np.array_equal(_live(b, 1)[0], gk) and np.array_equal(_live(b, 1)[1], gv)
    assert b.slot(0)["len"] == WINDOW and b.slot(0)["lost"]
    assert np.array_equal(_live(b, 0)[0], win_k) and np.array_equal(_live(b, 0)[1], win_v)
    # no reproducible marker: refused
    assert ESKVCache(2).restore_snapshot(path, "different-turn", prefix_fp=lambda p: "nope") == -1
    # reset drops the markers: the next snapshot carries none
    a.reset()


def test_rewind_to_mark_matches_a_cache_that_never_decoded_the_turn():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(6)
    a, ref = ESKVCache(4), ESKVCache(4)
    _prime(a, np.random.default_rng(7), prefill=200, steps=0)
    model = _prime(ref, np.random.default_rng(7), prefill=200, steps=0)
    assert a.rewind_to_mark() == -1                    # no mark yet
    assert not a.mark_rewind_point(0)
    assert a.mark_rewind_point(200)
    for _ in range(30):                                 # the excised turn
        _step(a, rng, {k: [x.copy() for x in v] for k, v in model.items()})
    assert a.rewind_to_mark() == 200
    assert a.rewind_to_mark() == -1                    # the mark is consumed
    assert a.slot(GLOBAL)["len"] == 200 and a.slot(RAW)["len"] == 200 and a.slot(SHARED)["len"] == 200
    for i in (SHARED, RAW, GLOBAL):
        for x, y in zip(_live(a, i), _live(ref, i)):
            assert np.array_equal(x, y), f"layer {i}"
    for x, y in zip(_live(a, SLIDE), _live(ref, SLIDE)):  # the window copied at the mark
        assert np.array_equal(x, y)
    oa = _step(a, np.random.default_rng(8), {k: [x.copy() for x in v] for k, v in model.items()})
    ob = _step(ref, np.random.default_rng(8), model)
    for x, y in zip(oa, ob):
        assert np.array_equal(x, y)
    # legacy storage has no rewind
    legacy = ESKVCache(1)
    kk = rms_rows(rng, (1, 10, 128))
    legacy.update(0, _dev(kk), _dev(kk), 0, prealloc=False)
    assert not legacy.mark_rewind_point(5)
