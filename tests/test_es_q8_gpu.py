"""GPU checks of the q8 raw-K storage of the ES* C++ layer (ESKVCache::updateRawQ8,
the fused decodeRawQ8 and esDecodeAttnGlobalQ8, through include/esda_cache.h), after
ESKVCache.mm:513-556, ESAttention.mm:270-277 and ESDecodeAttn.mm:440-492.

Stored rows, scales and biases are compared bit for bit with the oracle's quantizer
applied to a host model of the raw stream (IEEE fp32 arithmetic, round half away from
zero); decode outputs are held to max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp64
q8 oracle over the model's quantized rows.  Slot growth follows the reference: the first
store has capacity == content, growth goes to roundUp(len + n + 256, 256), and a bf16 raw
slot migrates to q8 with capacity roundUp(len + 256, 256).
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


def _raw(rng, shape):
    return orc.to_bf16((rng.standard_normal(shape, dtype=np.float32) * 2.0).astype(np.float32))


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _assert_slot_matches(cache, layer, model):
    """The layer's q8 rows, scales and biases equal the oracle's quantization of model."""
    eq, esc, ebs = orc.quantize_rows(model)
    gq, gsc, gbs = (t.cpu().numpy() for t in cache.current_raw_q8(layer).torch())
    assert gq.shape == eq.shape, (gq.shape, eq.shape)
    assert np.array_equal(gq, eq), "q8 rows differ"
    assert np.array_equal(_bits(gsc), _bits(esc)), "scales differ"
    assert np.array_equal(_bits(gbs), _bits(ebs)), "biases differ"


def _check_decode(out, q, model, kw, inv, what):
    qc, sc, bs = orc.quantize_rows(model)
    ref = orc.decode_raw_q8_f64(q, qc, sc, bs, model.shape[1], kw, EPS, inv, 1.0)
    o = orc.from_bf16(_host(out)).reshape(q.shape).astype(np.float64)
    err = np.abs(o - ref)
    assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, f"{what}: {err.max():.3e} {err.mean():.3e}"
    return err.max()


def _decode_inputs(rng):
    kw = orc.to_bf16((1.0 + 0.2 * rng.standard_normal(512)).astype(np.float32))
    return kw, _dev(kw), orc.rope_inv_freq(512, 1.0e6, 0.25)


def test_update_raw_q8_layout_growth_and_bytes():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(1)
    cache = ESKVCache(2)
    model = _raw(rng, (4, 300, 512))
    v = cache.update_raw_q8(1, _dev(model))
    assert (v.kv_heads, v.len, v.pitch) == (4, 300, 300)  # first store: capacity == content
    for _ in range(3):
        one = _raw(rng, (4, 1, 512))
        v = cache.update_raw_q8(1, _dev(one))
        model = np.concatenate([model, one], axis=1)
    assert (v.len, v.pitch) == (303, 768)  # roundUp(300 + 1 + 256, 256)
    big = _raw(rng, (4, 500, 512))
    v = cache.update_raw_q8(1, _dev(big))
    model = np.concatenate([model, big], axis=1)
    assert (v.len, v.pitch) == (803, 1280)  # roundUp(303 + 500 + 256, 256)
    _assert_slot_matches(cache, 1, model)
    s = cache.slot(1)
    assert s["q8"] and not s["raw"] and s["len"] == 803 and s["capacity"] == 1280
    assert not cache.slot(0)["q8"]
    cache.reset()
    assert not cache.slot(1)["q8"] and cache.slot(1)["len"] == 0


def test_decode_raw_q8_through_the_cache_matches_oracle():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(2)
    kvh, hq = 2, 16
    kw, kw_d, inv = _decode_inputs(rng)
    cache = ESKVCache(1)
    model = _raw(rng, (kvh, 200, 512))
    cache.update_raw_q8(0, _dev(model))
    worst = 0.0
    for i in range(70):
        q = rms_rows(rng, (hq, 512))
        one = _raw(rng, (kvh, 1, 512))
        out = cache.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv))
        model = np.concatenate([model, one], axis=1)
        if i % 10 == 0 or i == 69:
            torch.cuda.synchronize()
            worst = max(worst, _check_decode(out, q, model, kw, inv, f"step {i}"))
    s = cache.slot(0)
    assert s["q8"] and s["len"] == 270 and s["capacity"] == 512  # grown once: roundUp(200 + 1 + 256)
    _assert_slot_matches(cache, 0, model)  # the kernel's in-place quantization of each new row
    print(f"q8 cache decode worst max_abs {worst:.3e}")


def test_decode_raw_q8_on_an_empty_slot_starts_the_stream():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(3)
    kw, kw_d, inv = _decode_inputs(rng)
    cache = ESKVCache(1)
    model = np.zeros((1, 0, 512), np.uint16)
    for i in range(20):
        q = rms_rows(rng, (8, 512))
        one = _raw(rng, (1, 1, 512))
        out = cache.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv))
        model = np.concatenate([model, one], axis=1)
        torch.cuda.synchronize()
        _check_decode(out, q, model, kw, inv, f"step {i}")
    assert cache.slot(0)["len"] == 20
    _assert_slot_matches(cache, 0, model)


@pytest.mark.parametrize("via_decode", [False, True])
def test_bf16_raw_slot_migrates_to_q8(via_decode):
    """A bf16 raw slot (e.g. restored from a raw snapshot) is quantized once on the first
    q8 append and retired (ESKVCache.mm:518-536)."""
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(4 + via_decode)
    kw, kw_d, inv = _decode_inputs(rng)
    cache = ESKVCache(1)
    model = _raw(rng, (2, 300, 512))
    cache.update_raw(0, _dev(model), True)
    assert cache.slot(0)["raw"]
    one = _raw(rng, (2, 1, 512))
    if via_decode:
        q = rms_rows(rng, (16, 512))
        out = cache.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv))
    else:
        cache.update_raw_q8(0, _dev(one))
    model = np.concatenate([model, one], axis=1)
    torch.cuda.synchronize()
    s = cache.slot(0)
    assert s["q8"] and not s["raw"] and s["len"] == 301 and s["capacity"] == 768  # roundUp(300 + 256)
    _assert_slot_matches(cache, 0, model)
    if via_decode:
        _check_decode(out, q, model, kw, inv, "migrating decode")


def test_q8_mode_guards():
    from apertura_amd import EsdaError
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(6)
    kw, kw_d, inv = _decode_inputs(rng)
    cache = ESKVCache(2)
    kv = _dev(rms_rows(rng, (2, 3, 512)))
    one = kv[:, :1].contiguous()
    q = _dev(rms_rows(rng, (16, 512)))
    cache.update(0, kv, kv, 0, prealloc=True)  # composite
    for call in (lambda: cache.update_raw_q8(0, kv), lambda: cache.decode_raw_q8(0, q, one, kw_d, EPS, list(inv))):
        with pytest.raises(EsdaError) as ei:
            call()
        assert ei.value.code == 2 and "composite" in str(ei.value)
    cache.update_raw_q8(1, kv)  # q8
    for call in (lambda: cache.update(1, kv, kv, 0, prealloc=True),
                 lambda: cache.decode(1, q, one, one, 0, 0, 1.0),
                 lambda: cache.update_raw(1, kv, True),
                 lambda: cache.decode_raw(1, q, one, kw_d, EPS, list(inv))):
        with pytest.raises(EsdaError) as ei:
            call()
        assert ei.value.code == 2
    with pytest.raises(EsdaError) as ei:
        cache.current_raw_q8(0)
    assert ei.value.code == 2
    with pytest.raises(EsdaError) as ei:
        cache.update_raw_q8(1, _dev(rms_rows(rng, (3, 1, 512))))  # kv heads differ
    assert ei.value.code == 1
    with pytest.raises(ValueError):
        cache.update_raw_q8(1, _dev(rms_rows(rng, (2, 1, 256))))  # q8 rows are 512 wide
    assert cache.slot(1)["len"] == 3 and cache.slot(1)["q8"]


def test_es_decode_attn_global_q8_over_unsliced_buffers():
    """esDecodeAttnGlobalQ8 on the unsliced buffers of a q8 slot, rows 0 .. len-1 already
    appended (the reference's updateRawQ8 + esDecodeAttnGlobalQ8 pair)."""
    from apertura_amd.cache import es_decode_attn_global_q8
    from apertura_amd.decode import quantize_raw_rows
    rng = np.random.default_rng(7)
    kw, kw_d, inv = _decode_inputs(rng)
    kvh, n, pitch = 3, 1500, 2048
    model = _raw(rng, (kvh, n, 512))
    qb = torch.zeros((kvh, pitch, 512), dtype=torch.uint8, device="cuda")
    sb = torch.zeros((kvh, pitch, 1), dtype=torch.float32, device="cuda")
    bb = torch.zeros((kvh, pitch, 1), dtype=torch.float32, device="cuda")
    quantize_raw_rows(_dev(model), qb, sb.view(kvh, pitch), bb.view(kvh, pitch), row0=0)
    for length in (n, 1, 777):
        q = rms_rows(rng, (kvh * 8, 512))
        out = es_decode_attn_global_q8(_dev(q), qb, sb, bb, length, pitch, kw_d, EPS, list(inv))
        torch.cuda.synchronize()
        _check_decode(out, q, model[:, :length], kw, inv, f"len {length}")


def test_q8_snapshot_round_trip_and_conversions(tmp_path):
    """q8 layers save as rq_/rs_/rb_ (u8, f32 [kvHeads, rows, 1]); as stored they restore
    byte for byte, mode raw rehydrates them to bf16(float(q) * scale + bias), and a bf16 raw
    snapshot restored as rawQ8 quantizes its rows."""
    from apertura_amd.cache import ESKVCache
    from safetensors.torch import load_file
    rng = np.random.default_rng(8)
    kw, kw_d, inv = _decode_inputs(rng)
    a = ESKVCache(2)
    m0 = _raw(rng, (2, 130, 512))
    a.update_raw_q8(0, _dev(m0))
    kc = rms_rows(rng, (2, 40, 128))
    a.update(1, _dev(kc), _dev(kc), 0, prealloc=True)
    for _ in range(5):
        one = _raw(rng, (2, 1, 512))
        a.decode_raw_q8(0, _dev(rms_rows(rng, (16, 512))), _dev(one), kw_d, EPS, list(inv))
        m0 = np.concatenate([m0, one], axis=1)
    path = str(tmp_path / "q8.safetensors")
    assert a.save_snapshot(path, "fp", 135)
    t = {k: (v.numpy() if v.dtype != torch.bfloat16 else v) for k, v in load_file(path).items()}
    eq, esc, ebs = orc.quantize_rows(m0)
    assert t["rq_0"].dtype == np.uint8 and t["rq_0"].shape == (2, 135, 512) and np.array_equal(t["rq_0"], eq)
    assert t["rs_0"].shape == (2, 135, 1) and np.array_equal(_bits(t["rs_0"][..., 0]), _bits(esc))
    assert t["rb_0"].shape == (2, 135, 1) and np.array_equal(_bits(t["rb_0"][..., 0]), _bits(ebs))
    assert "k_0" not in t and "k_1" in t and "v_1" in t

    b = ESKVCache(2)
    assert b.restore_snapshot(path, "fp") == 135  # as stored
    assert b.slot(0)["q8"] and b.slot(0)["capacity"] == 512  # roundUp(135 + 256)
    _assert_slot_matches(b, 0, m0)
    # continuing on the restored cache and on the original gives the same bits
    q, one = rms_rows(rng, (16, 512)), _raw(rng, (2, 1, 512))
    oa = _host(a.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv)))
    ob = _host(b.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv)))
    assert np.array_equal(oa, ob)

    c = ESKVCache(2)
    assert c.restore_snapshot(path, "fp", mode="raw") == 135  # rehydration
    assert c.slot(0)["raw"] and not c.slot(0)["q8"]
    view, ln, _ = c.current_raw(0)
    expect = orc.to_bf16(eq.astype(np.float32) * esc[..., None] + ebs[..., None])
    assert ln == 135 and np.array_equal(_host(view.torch()), expect)

    # bf16 raw snapshot -> rawQ8
    path2 = str(tmp_path / "raw.safetensors")
    assert c.save_snapshot(path2, "fp2", 135)
    d = ESKVCache(2)
    assert d.restore_snapshot(path2, "fp2", mode="rawQ8") == 135
    assert d.slot(0)["q8"]
    _assert_slot_matches(d, 0, expect)
    assert d.restore_snapshot(path, "fp", mode="composite") == -1
    assert d.slot(0)["q8"] and d.slot(0)["len"] == 135  # refused restore left the cache as it was


def test_q8_prefix_marker_truncates_the_q8_stream(tmp_path):
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(9)
    cache = ESKVCache(1)
    model = _raw(rng, (1, 5000, 512))
    cache.update_raw_q8(0, _dev(model))
    cache.mark_prefix(4200, "persona")
    path = str(tmp_path / "m.safetensors")
    assert cache.save_snapshot(path, "full", 5000)
    r = ESKVCache(1)
    assert r.restore_snapshot(path, "other", prefix_fp=lambda pos: "persona" if pos == 4200 else "") == 4200
    assert r.slot(0)["q8"] and r.slot(0)["len"] == 4200 and r.slot(0)["capacity"] == 4608
    _assert_slot_matches(r, 0, model[:, :4200])


def test_q8_rewind_truncates_and_refuses_a_short_slot():
    from apertura_amd.cache import ESKVCache
    rng = np.random.default_rng(10)
    kw, kw_d, inv = _decode_inputs(rng)
    cache = ESKVCache(1)
    model = _raw(rng, (2, 300, 512))
    cache.update_raw_q8(0, _dev(model))
    assert cache.mark_rewind_point(300)
    for _ in range(6):
        cache.decode_raw_q8(0, _dev(rms_rows(rng, (16, 512))), _dev(_raw(rng, (2, 1, 512))), kw_d, EPS, list(inv))
    assert cache.rewind_to_mark() == 300
    assert cache.slot(0)["len"] == 300
    q, one = rms_rows(rng, (16, 512)), _raw(rng, (2, 1, 512))
    out = cache.decode_raw_q8(0, _dev(q), _dev(one), kw_d, EPS, list(inv))
    model = np.concatenate([model, one], axis=1)
    torch.cuda.synchronize()
    _check_decode(out, q, model, kw, inv, "after rewind")
    _assert_slot_matches(cache, 0, model)
    # a mark beyond the slot's rows cannot be rebuilt: -1, the cache unchanged
    assert cache.mark_rewind_point(400)
    assert cache.rewind_to_mark() == -1
    assert cache.slot(0)["len"] == 301
