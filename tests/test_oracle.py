"""Pins of the CPU oracle (oracle/liboracle.so) -- CPU only.

The reference holds no attention goldens (its fixtures are gitignored and need the
31B weights), so each oracle function is pinned by something other than itself:

  bf16 rounding      torch's RNE bf16 conversion + hand-computed tie cases
  visibility rule    HF transformers masking_utils (causal / sliding-window mask
                     functions, the rule ESGemma4TextModel.mm:68-83 restates)
  append             numpy row assignment; every other byte unchanged
  decode_f64         HF transformers gemma4 eager_attention_forward in fp64 (library),
                     closed forms (single key, q = 0, identical keys, dominant key),
                     invariants (permutation / ring-vs-linear, masked rows inert,
                     score shift)
  GQA order          ESPrimitivesTests.mm:118-128 (repeatKV is kv-major: [h0,h0,h1,h1])
  decode_refround    within the north-star tolerance of fp64; bit-level spot checks
                     of its rounding points on a hand-computed case
  refround_grouped   decode_refround bit for bit with one split; within one bf16 ulp
                     with several
  decode_splitk      S = 1 vs many splits vs fp64 (split invariance)
  rope inv_freq      ESPrimitivesTests.mm:130-139, 191-210 (zero tail, full rotation)
  rms norm           ESPrimitivesTests.mm:93-116 (unit weight, weightless [2,2,2,2])
  raw-K decode       HF apply_rotary_pos_emb + rms norm composition feeding decode_f64
  quantize_rows      quantisation bounds, ties away from zero, constant rows, endpoints
  raw q8 decode      equals the raw-K decode on rows q8 represents exactly
  prefill_f64        HF eager_attention_forward with HF masks over a query chunk; every
                     row equals decode_f64 at its position; closed forms
  raw_prefill_kv     torch bf16 ops with HF rotate_half (two bf16 steps at most)
  ES primitives      the reference's own ESPrimitivesTests.mm assertions, transcribed into
                     tests/golden/es_primitives.json

Planted-mistake tests (orc_set_fault) show that a plausible bug in the oracle is
caught by at least one pin.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from _synth import make_step_inputs, rms_rows

TOL_MAX, TOL_MEAN = 2e-2, 2e-3


# --------------------------------------------------------------------- bf16

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100_000),
        np.array([0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    ours = orc.to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_bf16_ties_to_even():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 spacing at 1.0
    vals = np.array([one + ulp / 2, one + 3 * ulp / 2, one + ulp / 2 + np.float32(2 ** -20)],
                    np.float32)
    got = orc.to_bf16(vals)
    assert list(got) == [0x3F80, 0x3F82, 0x3F81]
    assert np.isnan(orc.from_bf16(orc.to_bf16(np.array([np.nan], np.float32))))[0]


# -------------------------------------------------------------- visibility

def _hf_mask_fn(window: int):
    from transformers import masking_utils as mu
    return mu.sliding_window_causal_mask_function(window) if window else mu.causal_mask_function


def _hf_allowed(window: int, pos: int, kv_positions) -> list:
    fn = _hf_mask_fn(window)
    z = torch.tensor(0)
    ok = fn(z, z, torch.tensor(pos), torch.as_tensor(list(kv_positions), dtype=torch.long))
    return ok.tolist()


def _hf_visible(pos: int, window: int, n_pos: int):
    ok = _hf_allowed(window, pos, range(n_pos))
    return [kv for kv in range(n_pos) if ok[kv]]


@pytest.mark.parametrize("pos,window", [(0, 0), (5, 0), (1023, 1024), (1024, 1024),
                                        (3000, 1024), (7, 3), (2, 3), (4095, 512)])
def test_visible_linear_matches_hf_mask(pos, window):
    step = orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=pos + 1, window=window)
    rows = orc.visible(step, pos)
    assert list(rows) == _hf_visible(pos, window, pos + 1)


@pytest.mark.parametrize("pos,window,cap", [(0, 4, 4), (3, 4, 4), (10, 4, 4), (10, 3, 8),
                                            (2048, 1024, 1024), (32767, 1024, 1024)])
def test_visible_ring_matches_hf_mask(pos, window, cap):
    step = orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=cap, window=window, ring=True)
    rows = orc.visible(step, pos)
    want = [p % cap for p in _hf_visible(pos, window, pos + 1)]
    assert list(rows) == want
    assert len(set(rows)) == len(rows)  # no slot twice


def test_visible_linear_row_base():
    # After a compaction the buffer's row 0 holds absolute position row_base
    # (ESKVCache.mm:76-94); rows below the window are gone, rows in it are re-based.
    step = orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=1536, window=1024)
    rows = orc.visible(step, 5000, row_base=5000 - 1100)
    assert rows[0] == 5000 - 1023 - (5000 - 1100) and rows[-1] == 1100 and len(rows) == 1024


def test_visible_rejects_bad_descriptions():
    with pytest.raises(ValueError):
        orc.visible(orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=4, window=0, ring=True), 3)
    with pytest.raises(ValueError):
        orc.visible(orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=4, window=8, ring=True), 3)
    with pytest.raises(ValueError):
        orc.visible(orc.Step(B=1, Hq=3, Hkv=2, D=8, cap=4), 3)
    with pytest.raises(ValueError):
        orc.visible(orc.Step(B=1, Hq=2, Hkv=1, D=8, cap=4), 4)  # linear overflow


# ------------------------------------------------------------------- append

@pytest.mark.parametrize("ring,shared", [(False, False), (True, False), (False, True)])
def test_append_writes_exactly_one_row(ring, shared):
    step = orc.Step(B=3, Hq=4, Hkv=2, D=16, cap=8, window=8 if ring else 0, ring=ring,
                    head_stride=8 * 16 + 16, seq_stride=2 * (8 * 16 + 16) + 32)
    pos = [3, 7, 13] if ring else [0, 4, 7]
    q, kc, vc, kn, vn = make_step_inputs(step, 11, pos, shared_kv=shared)
    k0, v0 = kc.copy(), vc.copy()
    orc.append(step, kc, None if shared else vc, kn, None if shared else vn, pos)
    k_exp = k0.copy()
    v_exp = v0.copy()
    d = step.desc()
    for b in range(step.B):
        r = pos[b] % step.cap if ring else pos[b]
        for h in range(step.Hkv):
            off = b * d.seq_stride + h * d.head_stride + r * step.D
            k_exp[off:off + step.D] = kn[b, h]
            v_exp[off:off + step.D] = (kn if shared else vn)[b, h]
    np.testing.assert_array_equal(kc, k_exp)
    if not shared:
        np.testing.assert_array_equal(vc, v_exp)


# ---------------------------------------------------------------- fp64 mode

def _hf_attention_f64(step, q, kc, vc, pos):
    """transformers' gemma4 eager_attention_forward in fp64 over the full cache rows
    with an HF-rule additive mask on absolute positions."""
    from transformers.models.gemma4.modeling_gemma4 import eager_attention_forward
    d = step.desc()
    G = step.Hq // step.Hkv

    class M(torch.nn.Module):
        num_key_value_groups = G
        head_dim = step.D
        training = False

    outs = []
    for b in range(step.B):
        # positions held by the cache, derived without the oracle: linear rows hold
        # p = row; ring slot j holds the newest p <= pos with p = j (mod cap)
        if step.ring:
            held = [(pos[b] - ((pos[b] - j) % step.cap), j) for j in range(step.cap)]
            held = sorted((p, j) for p, j in held if p >= 0)
        else:
            held = [(p, p) for p in range(pos[b] + 1)]
        K = np.empty((step.Hkv, len(held), step.D), np.float64)
        V = np.empty_like(K)
        for h in range(step.Hkv):
            base = b * d.seq_stride + h * d.head_stride
            for t, (_, r) in enumerate(held):
                K[h, t] = orc.from_bf16(kc[base + r * step.D: base + (r + 1) * step.D])
                V[h, t] = orc.from_bf16(vc[base + r * step.D: base + (r + 1) * step.D])
        ok = _hf_allowed(step.window, pos[b], [p for p, _ in held])
        mask = torch.tensor([[0.0 if a else -1e30 for a in ok]], dtype=torch.float64)
        Q = torch.from_numpy(orc.from_bf16(q[b]).astype(np.float64))[None, :, None, :]
        o, _ = eager_attention_forward(M(), Q, torch.from_numpy(K)[None], torch.from_numpy(V)[None],
                                       mask[None, None], scaling=step.scale)
        outs.append(o[0, 0].numpy())
    return np.stack(outs)


@pytest.mark.parametrize("cfg", [
    dict(B=1, Hq=16, Hkv=8, D=64, cap=40, window=0, ring=False, pos=[39], shared=False),
    dict(B=2, Hq=8, Hkv=1, D=64, cap=64, window=0, ring=False, pos=[10, 63], shared=True),
    dict(B=2, Hq=4, Hkv=2, D=32, cap=16, window=16, ring=True, pos=[40, 9], shared=False),
    dict(B=1, Hq=4, Hkv=2, D=32, cap=64, window=10, ring=False, pos=[50], shared=False),
])
def test_f64_matches_hf_eager_attention(cfg):
    step = orc.Step(B=cfg["B"], Hq=cfg["Hq"], Hkv=cfg["Hkv"], D=cfg["D"], cap=cfg["cap"],
                    window=cfg["window"], ring=cfg["ring"], scale=cfg["D"] ** -0.5)
    q, kc, vc, kn, vn = make_step_inputs(step, 3, cfg["pos"], shared_kv=cfg["shared"])
    orc.append(step, kc, None if cfg["shared"] else vc, kn, None if cfg["shared"] else vn,
               cfg["pos"])
    ours = orc.decode_f64(step, q, kc, vc, cfg["pos"])
    ref = _hf_attention_f64(step, q, kc, vc, cfg["pos"])
    # HF's eager softmax runs in fp32 (dtype=torch.float32) even for fp64 inputs.
    np.testing.assert_allclose(ours, ref, rtol=0, atol=2e-6)


def _one_step(D=32, Hq=4, Hkv=2, cap=12, pos=None, scale=None, ring=False, window=0, seed=5):
    step = orc.Step(B=1, Hq=Hq, Hkv=Hkv, D=D, cap=cap, ring=ring, window=window,
                    scale=scale if scale is not None else D ** -0.5)
    pos = [cap - 1] if pos is None else pos
    return step, make_step_inputs(step, seed, pos), pos


def test_closed_form_single_key_returns_v_row():
    step, (q, kc, vc, kn, vn), _ = _one_step(cap=4, pos=[0])
    orc.append(step, kc, vc, kn, vn, [0])
    out = orc.decode_f64(step, q, kc, vc, [0])
    for h in range(step.Hq):
        np.testing.assert_array_equal(out[0, h], orc.from_bf16(vn[0, h // 2]).astype(np.float64))


def test_closed_form_zero_query_is_mean_of_visible_v():
    step, (q, kc, vc, kn, vn), pos = _one_step(cap=64, pos=[40], window=17)
    q[:] = 0
    orc.append(step, kc, vc, kn, vn, pos)
    out = orc.decode_f64(step, q, kc, vc, pos)
    d = step.desc()
    for h in range(step.Hq):
        base = (h // 2) * d.head_stride
        rows = range(40 - 16, 41)
        mean = np.mean([orc.from_bf16(vc[base + r * 32: base + r * 32 + 32]) for r in rows], axis=0)
        np.testing.assert_allclose(out[0, h], mean, atol=1e-12)


def test_closed_form_identical_keys_uniform_weights():
    step, (q, kc, vc, kn, vn), pos = _one_step(cap=20, pos=[19])
    d = step.desc()
    for h in range(step.Hkv):
        base = h * d.head_stride
        for r in range(20):
            kc[base + r * 32: base + r * 32 + 32] = kn[0, h]
    orc.append(step, kc, vc, kn, vn, pos)
    out = orc.decode_f64(step, q, kc, vc, pos)
    for h in range(step.Hq):
        base = (h // 2) * d.head_stride
        mean = np.mean([orc.from_bf16(vc[base + r * 32: base + r * 32 + 32]) for r in range(20)], 0)
        np.testing.assert_allclose(out[0, h], mean, atol=1e-12)


def test_closed_form_dominant_key_wins():
    step, (q, kc, vc, kn, vn), pos = _one_step(D=32, Hq=2, Hkv=1, cap=30, pos=[29], scale=1.0)
    d = step.desc()
    r = 7
    kc[r * 32:(r + 1) * 32] = orc.to_bf16(orc.from_bf16(q[0, 0]) * 50.0)
    orc.append(step, kc, vc, kn, vn, pos)
    out = orc.decode_f64(step, q, kc, vc, pos)
    np.testing.assert_allclose(out[0, 0], orc.from_bf16(vc[r * 32:(r + 1) * 32]), atol=1e-9)


def test_invariant_non_visible_rows_are_inert():
    step, (q, kc, vc, kn, vn), pos = _one_step(cap=64, pos=[50], window=8)
    orc.append(step, kc, vc, kn, vn, pos)
    a = orc.decode_f64(step, q, kc, vc, pos)
    d = step.desc()
    vis = set(orc.visible(step, 50))
    rng = np.random.default_rng(9)
    for h in range(step.Hkv):
        for r in range(64):
            if r not in vis:
                o = h * d.head_stride + r * 32
                kc[o:o + 32] = orc.to_bf16(rng.standard_normal(32).astype(np.float32) * 100)
                vc[o:o + 32] = orc.to_bf16(rng.standard_normal(32).astype(np.float32) * 100)
    b = orc.decode_f64(step, q, kc, vc, pos)
    np.testing.assert_array_equal(a, b)


def test_invariant_ring_equals_linear_layout():
    D, W, pos = 32, 16, 45
    lin = orc.Step(B=1, Hq=4, Hkv=2, D=D, cap=pos + 1, window=W, scale=0.3)
    ring = orc.Step(B=1, Hq=4, Hkv=2, D=D, cap=W, window=W, ring=True, scale=0.3)
    q, kc, vc, kn, vn = make_step_inputs(lin, 21, [pos])
    orc.append(lin, kc, vc, kn, vn, [pos])
    kr = np.zeros(ring.cache_elems(), np.uint16)
    vr = np.zeros_like(kr)
    for h in range(2):
        for p in range(pos - W + 1, pos + 1):
            src = h * lin.desc().head_stride + p * D
            dst = h * ring.desc().head_stride + (p % W) * D
            kr[dst:dst + D] = kc[src:src + D]
            vr[dst:dst + D] = vc[src:src + D]
    a = orc.decode_f64(lin, q, kc, vc, [pos])
    b = orc.decode_f64(ring, q, kr, vr, [pos])
    np.testing.assert_allclose(a, b, atol=1e-13)


def test_gqa_order_is_kv_major():
    # ESPrimitivesTests.mm:118-128: repeatKV([h0, h1], 2) == [h0, h0, h1, h1].
    step = orc.Step(B=1, Hq=4, Hkv=2, D=8, cap=3, scale=1.0)
    q = orc.to_bf16(np.zeros((1, 4, 8), np.float32))
    kc = orc.to_bf16(np.zeros(step.cache_elems(), np.float32))
    vc = kc.copy()
    d = step.desc()
    for h in range(2):
        vc[h * d.head_stride: h * d.head_stride + 3 * 8] = orc.to_bf16(np.full(24, float(h), np.float32))
    out = orc.decode_f64(step, q, kc, vc, [2])
    np.testing.assert_array_equal(out[0, :, 0], [0.0, 0.0, 1.0, 1.0])


# ------------------------------------------------- refround and split-K modes

@pytest.mark.parametrize("shared", [False, True])
def test_refround_within_tolerance_of_f64(shared):
    step = orc.Step(B=2, Hq=8, Hkv=2, D=128, cap=300, scale=128 ** -0.5)
    pos = [299, 120]
    q, kc, vc, kn, vn = make_step_inputs(step, 13, pos, shared_kv=shared)
    orc.append(step, kc, None if shared else vc, kn, None if shared else vn, pos)
    ref = orc.decode_f64(step, q, kc, vc, pos)
    rr = orc.from_bf16(orc.decode_refround(step, q, kc, vc, pos)).astype(np.float64)
    err = np.abs(rr - ref)
    assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN
    assert err.max() > 0  # it really rounds


def test_refround_rounding_points_hand_case():
    # Two keys, D=2: q=(1,0), k0=(1,0), k1=(0,0), v0=(1,0), v1=(0,1), scale 1.
    # scores bf16(1), bf16(0); softmax = (e/(e+1), 1/(e+1)) -> bf16 each;
    # out = bf16(w0*v0 + w1*v1).
    step = orc.Step(B=1, Hq=1, Hkv=1, D=2, cap=2, scale=1.0)
    q = orc.to_bf16(np.array([[[1.0, 0.0]]], np.float32))
    kc = orc.to_bf16(np.array([1.0, 0.0, 0.0, 0.0], np.float32))
    vc = orc.to_bf16(np.array([1.0, 0.0, 0.0, 1.0], np.float32))
    out = orc.from_bf16(orc.decode_refround(step, q, kc, vc, [1]))[0, 0]
    e = np.float32(np.e)
    w0 = orc.from_bf16(orc.to_bf16(np.array([np.float32(1) / (np.float32(1) + np.exp(np.float32(-1)))], np.float32)))[0]
    w1 = orc.from_bf16(orc.to_bf16(np.array([np.exp(np.float32(-1)) / (np.float32(1) + np.exp(np.float32(-1)))], np.float32)))[0]
    assert out[0] == orc.from_bf16(orc.to_bf16(np.array([w0], np.float32)))[0]
    assert out[1] == orc.from_bf16(orc.to_bf16(np.array([w1], np.float32)))[0]
    assert abs(out[0] - e / (e + 1)) < 4e-3


@pytest.mark.parametrize("cfg", [
    dict(B=2, Hq=8, Hkv=2, D=128, cap=300, window=0, ring=False, shared=False, pos=[299, 120]),
    dict(B=1, Hq=32, Hkv=4, D=512, cap=700, window=0, ring=False, shared=True, pos=[650]),
    dict(B=3, Hq=16, Hkv=8, D=256, cap=256, window=256, ring=True, shared=False, pos=[900, 300, 255]),
    dict(B=2, Hq=24, Hkv=1, D=128, cap=400, window=100, ring=False, shared=False, pos=[399, 50]),
])
def test_refround_grouped_equals_refround(cfg):
    """The CPU baseline's grouped restatement: one split per (sequence, kv head) gives
    orc_decode_refround bit for bit (G = 24 covers a partial block of 8 heads); many splits
    differ only where the order of the split sums moves a bf16 rounding (one ulp)."""
    step = orc.Step(B=cfg["B"], Hq=cfg["Hq"], Hkv=cfg["Hkv"], D=cfg["D"], cap=cfg["cap"],
                    window=cfg["window"], ring=cfg["ring"], scale=cfg["D"] ** -0.5)
    pos, shared = cfg["pos"], cfg["shared"]
    q, kc, vc, kn, vn = make_step_inputs(step, 29, pos, shared_kv=shared)
    orc.append(step, kc, None if shared else vc, kn, None if shared else vn, pos)
    ref = orc.decode_refround(step, q, kc, vc, pos)
    np.testing.assert_array_equal(orc.decode_refround_grouped(step, q, kc, vc, pos, nsplit=1), ref)
    many = orc.decode_refround_grouped(step, q, kc, vc, pos, nsplit=5, threads=4)
    a, b = orc.from_bf16(ref).astype(np.float64), orc.from_bf16(many).astype(np.float64)
    assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.maximum(np.abs(a), 2.0 ** -8))
    assert (ref != many).mean() < 0.02


def test_refround_grouped_planted_gqa_fault_is_refused():
    step = orc.Step(B=1, Hq=8, Hkv=2, D=64, cap=64, scale=0.125)
    q, kc, vc, _, _ = make_step_inputs(step, 3, [63])
    with orc.planted_fault(1):
        with pytest.raises(ValueError):
            orc.decode_refround_grouped(step, q, kc, vc, [63])


@pytest.mark.parametrize("nsplit", [1, 2, 7, 64])
def test_splitk_is_split_invariant(nsplit):
    step = orc.Step(B=1, Hq=8, Hkv=1, D=64, cap=500, scale=0.125)
    pos = [499]
    q, kc, vc, kn, vn = make_step_inputs(step, 17, pos, shared_kv=True)
    orc.append(step, kc, None, kn, None, pos)
    ref = orc.decode_f64(step, q, kc, kc, pos)
    sk = orc.decode_splitk(step, q, kc, kc, pos, nsplit).astype(np.float64)
    assert np.abs(sk - ref).max() < 1e-5


def test_splitk_peaked_keys_merge():
    # A few keys with +8 logits concentrated in one split: the merge must weight
    # that split by exp(m_s - mMax) (empty/low splits vanish) -- ESDecodeAttn.mm:253-273.
    step = orc.Step(B=1, Hq=2, Hkv=1, D=64, cap=1000, scale=1.0 / 8)
    pos = [999]
    q, kc, vc, kn, vn = make_step_inputs(step, 19, pos, shared_kv=True)
    qd = orc.from_bf16(q[0, 0]).astype(np.float64)
    alpha = 8.0 / (step.scale * np.linalg.norm(qd))  # raises head 0's logit by +8
    for r in (3, 5, 8):
        k = orc.from_bf16(kc[r * 64:(r + 1) * 64]) + alpha * qd / np.linalg.norm(qd)
        kc[r * 64:(r + 1) * 64] = orc.to_bf16(k.astype(np.float32))
    orc.append(step, kc, None, kn, None, pos)
    ref = orc.decode_f64(step, q, kc, kc, pos)
    sk = orc.decode_splitk(step, q, kc, kc, pos, 100).astype(np.float64)
    assert np.abs(sk - ref).max() < 1e-5


# ----------------------------------------------------------- rope and norms

def test_rope_proportional_zero_tail():
    # ESPrimitivesTests.mm:191-210: head_dim 512, partial 0.25 -> 64 real freqs, 192 zeros.
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    assert inv.shape == (256,)
    assert np.all(inv[64:] == 0) and np.all(inv[:64] > 0)
    assert inv[0] == 1.0 and abs(np.sin(1.0 * inv[0])) > 1e-3
    # HF default rope: inv_freq = 1 / base ** (arange(0, dim, 2) / dim) over the rotated dims
    ref = 1.0 / (1.0e6 ** (np.arange(0, 128, 2, dtype=np.float64) / 512))
    np.testing.assert_allclose(inv[:64], ref.astype(np.float32), rtol=1e-6)


def test_rope_local_full_rotation():
    # ESPrimitivesTests.mm:130-139: full rotation, position 0 -> cos 1, sin 0.
    inv = orc.rope_inv_freq(8, 1.0e4, 1.0)
    assert np.all(inv > 0) and inv.shape == (4,)
    assert np.all(np.cos(0.0 * inv) == 1.0) and np.all(np.sin(0.0 * inv) == 0.0)


def test_rms_norm_weightless_and_unit_weight():
    # ESPrimitivesTests.mm:107-116 and :93-105.
    y = orc.from_bf16(orc.rms_norm_rows(orc.to_bf16(np.full((1, 4), 2.0, np.float32)), None, 1e-6))
    assert np.all(np.abs(y - 1.0) <= 1e-3)
    x = orc.to_bf16((np.arange(8, dtype=np.float32) - 3.0)[None])
    y = orc.from_bf16(orc.rms_norm_rows(x, orc.to_bf16(np.ones(8, np.float32)), 1e-6))
    assert abs(float(np.mean(y.astype(np.float64) ** 2)) - 1.0) <= 1e-2


# --------------------------------------------------------------- raw-K mode

def _hf_raw_reference(q, raw, len_, kw, eps, inv, scale):
    """K = bf16(rope(rmsnorm_w(kraw))) with HF's apply_rotary_pos_emb / rotate_half on
    bf16-rounded cos/sin; V = rmsnorm(kraw) without weight; fp64 attention."""
    from transformers.models.gemma4.modeling_gemma4 import rotate_half
    Hkv, pitch, D = raw.shape
    x = torch.from_numpy(orc.from_bf16(raw[:, :len_]))
    ss = (x.double() ** 2).sum(-1, keepdim=True)
    rinv = 1.0 / torch.sqrt((ss / 512.0).float() + eps)
    kn = x * rinv * torch.from_numpy(orc.from_bf16(kw))
    pos_ = torch.arange(len_, dtype=torch.float32)[:, None]
    freqs = pos_ * torch.from_numpy(inv)[None, :256]
    emb = torch.cat([freqs, freqs], -1)
    c = torch.cos(emb).to(torch.bfloat16).float()
    s = torch.sin(emb).to(torch.bfloat16).float()
    k = (kn * c + rotate_half(kn) * s).to(torch.bfloat16).double()
    v = (x * rinv).double()
    G = q.shape[0] // Hkv
    qq = torch.from_numpy(orc.from_bf16(q)).double().view(Hkv, G, D)
    sc = torch.einsum("hgd,htd->hgt", qq, k) * scale
    w = torch.softmax(sc, -1)
    return torch.einsum("hgt,htd->hgd", w, v).reshape(Hkv * G, D).numpy()


def test_raw_decode_matches_hf_rope_composition():
    rng = np.random.default_rng(23)
    Hkv, pitch, L = 1, 80, 70
    raw = orc.to_bf16(rng.standard_normal((Hkv, pitch, 512)).astype(np.float32) * 3)
    q = rms_rows(rng, (8, 512))
    kw = orc.to_bf16((1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    ours = orc.decode_raw_f64(q, raw, L, kw, 1e-6, inv, scale=512 ** -0.5)
    ref = _hf_raw_reference(q, raw, L, kw, 1e-6, inv, 512 ** -0.5)
    assert np.abs(ours - ref).max() < 2e-3


@pytest.mark.parametrize("G", [1, 3, 16])
def test_raw_decode_other_gqa_groups(G):
    """Groups other than 8 query heads per kv head (run as calls of 8 heads on one kv head):
    every head against the HF composition, and each head's output the same as in a call that
    holds it among 8 heads of the group-8 form."""
    rng = np.random.default_rng(50 + G)
    Hkv, pitch, L = 2, 48, 41
    raw = orc.to_bf16(rng.standard_normal((Hkv, pitch, 512)).astype(np.float32) * 3)
    q = rms_rows(rng, (Hkv * G, 512))
    kw = orc.to_bf16((1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    ours = orc.decode_raw_f64(q, raw, L, kw, 1e-6, inv, scale=512 ** -0.5)
    assert ours.shape == (Hkv * G, 512)
    assert np.abs(ours - _hf_raw_reference(q, raw, L, kw, 1e-6, inv, 512 ** -0.5)).max() < 2e-3
    # head h of kv head 1 placed at slot 5 of a group-8 call on both kv heads
    h = Hkv * G - 1
    q8 = rms_rows(rng, (Hkv * 8, 512))
    q8[8 + 5] = q[h]
    assert np.array_equal(orc.decode_raw_f64(q8, raw, L, kw, 1e-6, inv, scale=512 ** -0.5)[8 + 5], ours[h])
    qraw, sc, bs = orc.quantize_rows(raw)
    a = orc.decode_raw_q8_f64(q, qraw, sc, bs, L, kw, 1e-6, inv, scale=512 ** -0.5)
    b = orc.decode_raw_q8_f64(q8, qraw, sc, bs, L, kw, 1e-6, inv, scale=512 ** -0.5)
    assert a.shape == (Hkv * G, 512) and np.array_equal(b[8 + 5], a[h])


def test_rinv_nudge_moves_the_row_norm_by_whole_ulps():
    """The conditioning probe: with one visible row the output is rinv * kraw exactly (the
    softmax weight is 1), so under a nudge of n ulps every element scales by rinv_n / rinv,
    where rinv_n is rinv stepped n times with nextafter; n = 0 is the plain oracle."""
    rng = np.random.default_rng(41)
    raw = orc.to_bf16(rng.standard_normal((1, 4, 512)).astype(np.float32) * 3)
    q = rms_rows(rng, (8, 512))
    kw = orc.to_bf16(np.ones(512, np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    x = orc.from_bf16(raw[0, 0]).astype(np.float64)
    ss = float((x * x).sum())
    rinv = np.float32(1.0) / np.sqrt(np.float32(ss / 512.0) + np.float32(1e-6))
    base = orc.decode_raw_f64(q, raw, 1, kw, 1e-6, inv, 1.0)
    assert np.array_equal(base, np.broadcast_to(float(rinv) * x, base.shape))
    for n in (1, -1, 3):
        want = rinv
        for _ in range(abs(n)):
            want = np.nextafter(want, np.float32(np.inf if n > 0 else -np.inf))
        with orc.rinv_nudge(n):
            got = orc.decode_raw_f64(q, raw, 1, kw, 1e-6, inv, 1.0)
        assert np.array_equal(got, np.broadcast_to(float(want) * x, got.shape)), n
    assert np.array_equal(orc.decode_raw_f64(q, raw, 1, kw, 1e-6, inv, 1.0), base)  # the probe is off again


# ------------------------------------------------------------ q8 raw stream

def test_quantize_rows_properties():
    """Per-row affine u8 (ESDecodeAttn.mm:491-509): the row's min maps to 0 and its max
    to 255, every value dequantises to within half a step, scale = (max - min) / 255 in
    fp32 and bias = min."""
    rng = np.random.default_rng(31)
    x = orc.to_bf16((rng.standard_normal((40, 512)) * rng.uniform(0.01, 5, (40, 1))).astype(np.float32))
    q, sc, bs = orc.quantize_rows(x)
    xf = orc.from_bf16(x).astype(np.float32)
    mn, mx = xf.min(axis=1), xf.max(axis=1)
    assert np.array_equal(bs, mn)
    assert np.array_equal(sc, np.maximum((mx - mn) / np.float32(255), np.float32(1e-8)))
    assert (q[np.arange(40), xf.argmin(axis=1)] == 0).all() and (q[np.arange(40), xf.argmax(axis=1)] == 255).all()
    deq = q.astype(np.float64) * sc[:, None] + bs[:, None]
    assert (np.abs(deq - xf) <= sc[:, None] * 0.5 * (1 + 1e-5) + np.abs(xf) * 1e-6).all()


def test_quantize_rows_rounds_ties_away_from_zero():
    # range 255/16 gives scale 1/16 exactly; 2.5/16 sits on a tie (round-half-even would give 2)
    row = np.zeros(512, np.float32)
    row[1], row[2], row[3] = 255 / 16, 2.5 / 16, 7.5 / 16
    q, sc, bs = orc.quantize_rows(orc.to_bf16(row)[None])
    assert sc[0] == np.float32(1 / 16) and bs[0] == 0
    assert q[0, 1] == 255 and q[0, 2] == 3 and q[0, 3] == 8 and q[0, 0] == 0


def test_quantize_rows_constant_row_keeps_a_finite_scale():
    x = orc.to_bf16(np.full((2, 512), [[0.75], [-3.0]], np.float32))
    q, sc, bs = orc.quantize_rows(x)
    assert (q == 0).all() and (sc == np.float32(1e-8)).all() and list(bs) == [0.75, -3.0]


def test_q8_decode_equals_raw_decode_on_exactly_representable_rows():
    """With power-of-two scales and integer biases every dequantised value q * scale + bias
    is exact in fp32 and in bf16, so the q8 decode must reproduce the (pinned) raw-K decode
    of those bf16 rows bit for bit."""
    rng = np.random.default_rng(37)
    Hkv, pitch, L = 2, 60, 53
    qraw = rng.integers(0, 256, size=(Hkv, pitch, 512), dtype=np.uint8)
    sc = (2.0 ** -rng.integers(4, 7, size=(Hkv, pitch))).astype(np.float32)
    bs = -rng.integers(1, 5, size=(Hkv, pitch)).astype(np.float32)
    deq = qraw.astype(np.float32) * sc[..., None] + bs[..., None]
    raw = orc.to_bf16(deq)
    assert np.array_equal(orc.from_bf16(raw), deq)
    q = rms_rows(rng, (Hkv * 8, 512))
    kw = orc.to_bf16((1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    a = orc.decode_raw_q8_f64(q, qraw, sc, bs, L, kw, 1e-6, inv, scale=512 ** -0.5)
    b = orc.decode_raw_f64(q, raw, L, kw, 1e-6, inv, scale=512 ** -0.5)
    assert np.array_equal(a, b)


# ------------------------------------------------------------ planted faults

def _pins_fail(fn) -> bool:
    try:
        fn()
    except AssertionError:
        return True
    return False


@pytest.mark.parametrize("fault,pin", [
    (1, lambda: test_gqa_order_is_kv_major()),
    (1, lambda: test_f64_matches_hf_eager_attention(dict(B=1, Hq=16, Hkv=8, D=64, cap=40,
                                                         window=0, ring=False, pos=[39],
                                                         shared=False))),
    (2, lambda: test_visible_linear_matches_hf_mask(3000, 1024)),
    (3, lambda: test_f64_matches_hf_eager_attention(dict(B=1, Hq=4, Hkv=2, D=32, cap=64,
                                                         window=10, ring=False, pos=[50],
                                                         shared=False))),
    (4, lambda: test_append_writes_exactly_one_row(False, False)),
    (5, lambda: test_raw_decode_matches_hf_rope_composition()),
    (6, lambda: test_quantize_rows_properties()),
    (7, lambda: test_prefill_matches_hf_eager_attention(dict(Hq=8, Hkv=1, D=64, Sq=12, Sk=40, q_pos0=28,
                                                             k_pos0=0, window=0))),
    (8, lambda: test_raw_prefill_kv_matches_torch_bf16_ops(512, 0.25)),
])
def test_planted_fault_is_caught(fault, pin):
    with orc.planted_fault(fault):
        assert _pins_fail(pin), f"planted fault {fault} went unnoticed"
    pin()  # and the clean oracle passes again


def test_append_with_row_base_writes_the_rebased_row():
    # Regression: the row_base / pos arrays must stay alive across the C call.
    step = orc.Step(B=2, Hq=4, Hkv=2, D=16, cap=64, window=32)
    pos, rb = [100, 70], [60, 40]
    q, kc, vc, kn, vn = make_step_inputs(step, 4, pos)
    k0 = kc.copy()
    orc.append(step, kc, vc, kn, vn, pos, rb)
    d = step.desc()
    changed = np.nonzero(kc != k0)[0]
    rows = {(int(i // d.seq_stride), int((i % d.head_stride) // 16)) for i in changed}
    assert rows <= {(0, 40), (1, 30)} and len(rows) == 2


def test_refround_coarse_at_in_model_scale():
    # Scale 1.0 (in-model, ESAttention.mm:56) on unit-RMS q/k at D=512: logits ~ 512, where
    # one bf16 ulp of a score (ESAttention.mm:153) is 2..4 -- the reference composite's own
    # rounding exceeds the 2e-2 bar, so GPU parity at this scale is gated on fp64 only.
    step = orc.Step(B=1, Hq=8, Hkv=1, D=512, cap=512, scale=1.0)
    q, kc, vc, kn, vn = make_step_inputs(step, 6, [511], shared_kv=True)
    orc.append(step, kc, None, kn, None, [511])
    ref = orc.decode_f64(step, q, kc, kc, [511])
    rr = orc.from_bf16(orc.decode_refround(step, q, kc, kc, [511])).astype(np.float64)
    assert np.abs(rr - ref).max() > TOL_MAX


# ---------------------------------------------------------------- prefill

def _prefill_inputs(rng, Hq, Hkv, D, Sq, Sk):
    q = rms_rows(rng, (Hq, Sq, D))
    k = rms_rows(rng, (Hkv, Sk, D))
    v = rms_rows(rng, (Hkv, Sk, D))
    return q, k, v


def _hf_prefill_f64(q, k, v, q_pos0, k_pos0, window, scale):
    """transformers' gemma4 eager_attention_forward in fp64 over a query chunk, with the
    HF-rule additive mask on absolute positions (query i at q_pos0 + i, key j at k_pos0 + j)."""
    from transformers.models.gemma4.modeling_gemma4 import eager_attention_forward
    Hq, Sq, D = q.shape
    Hkv, Sk, _ = k.shape

    class M(torch.nn.Module):
        num_key_value_groups = Hq // Hkv
        head_dim = D
        training = False

    rows = [_hf_allowed(window, q_pos0 + i, range(k_pos0, k_pos0 + Sk)) for i in range(Sq)]
    mask = torch.tensor([[0.0 if a else -1e30 for a in r] for r in rows], dtype=torch.float64)
    f = lambda a: torch.from_numpy(orc.from_bf16(a).astype(np.float64))[None]
    o, _ = eager_attention_forward(M(), f(q), f(k), f(v), mask[None, None], scaling=scale)
    return o[0].numpy()  # [Sq, Hq, D]


@pytest.mark.parametrize("cfg", [
    dict(Hq=4, Hkv=2, D=32, Sq=24, Sk=24, q_pos0=0, k_pos0=0, window=0),     # fresh causal prefill
    dict(Hq=8, Hkv=1, D=64, Sq=12, Sk=40, q_pos0=28, k_pos0=0, window=0),    # a chunk after 28 cached
    dict(Hq=4, Hkv=2, D=32, Sq=12, Sk=27, q_pos0=20, k_pos0=5, window=8),    # sliding, evicted keys
    dict(Hq=6, Hkv=3, D=16, Sq=30, Sk=30, q_pos0=0, k_pos0=0, window=4),     # sliding inside the chunk
])
def test_prefill_matches_hf_eager_attention(cfg):
    rng = np.random.default_rng(31)
    q, k, v = _prefill_inputs(rng, cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["Sq"], cfg["Sk"])
    scale = cfg["D"] ** -0.5
    ours = orc.prefill_f64(q, k, v, cfg["q_pos0"], cfg["k_pos0"], cfg["window"], scale)
    ref = _hf_prefill_f64(q, k, v, cfg["q_pos0"], cfg["k_pos0"], cfg["window"], scale)
    # HF's eager softmax runs in fp32 (dtype=torch.float32) even for fp64 inputs.
    np.testing.assert_allclose(ours, ref, rtol=0, atol=2e-6)


def test_prefill_rows_equal_decode_steps():
    """Query row i of a prefill is the decode step at position q_pos0 + i over the same
    cache rows (row_base = k_pos0), for causal and sliding layers."""
    rng = np.random.default_rng(32)
    Hq, Hkv, D, Sq, Sk, q_pos0, k_pos0 = 8, 2, 32, 10, 50, 45, 5
    q, k, v = _prefill_inputs(rng, Hq, Hkv, D, Sq, Sk)
    for window in (0, 7):
        out = orc.prefill_f64(q, k, v, q_pos0, k_pos0, window, 0.3)
        step = orc.Step(B=1, Hq=Hq, Hkv=Hkv, D=D, cap=Sk, window=window, scale=0.3)
        for i in range(Sq):
            dec = orc.decode_f64(step, np.ascontiguousarray(q[:, i])[None], k.reshape(-1), v.reshape(-1),
                                 [q_pos0 + i], row_base=[k_pos0])
            np.testing.assert_allclose(out[i], dec[0], rtol=0, atol=1e-12)


def test_prefill_closed_forms():
    rng = np.random.default_rng(33)
    q, k, v = _prefill_inputs(rng, 4, 2, 16, 6, 1)
    out = orc.prefill_f64(q, k, v, 0, 0, 0, 1.0)  # query 0 at position 0 sees only key 0
    np.testing.assert_allclose(out[0], np.repeat(orc.from_bf16(v[:, 0]), 2, axis=0), rtol=0, atol=1e-12)
    q, k, v = _prefill_inputs(rng, 4, 2, 16, 6, 9)
    out = orc.prefill_f64(q, k, v, 3, 0, 1, 1.0)  # window 1: each query sees its own key only
    for i in range(6):
        np.testing.assert_allclose(out[i], np.repeat(orc.from_bf16(v[:, 3 + i]), 2, axis=0), rtol=0, atol=1e-12)
    with pytest.raises(ValueError):  # keys all after the first query: nothing visible
        orc.prefill_f64(q, k, v, 0, 2, 0, 1.0)


def _torch_raw_prefill_kv(raw, kw, eps, inv):
    """ESAttention.mm:306-326 in torch bf16 ops: kNorm / vNorm in fp32 then cast; cos / sin
    of fp32 angles cast to bf16; K*c + rotate_half(K)*s with every product and the sum in
    bf16 (HF's rotate_half)."""
    from transformers.models.gemma4.modeling_gemma4 import rotate_half
    Hkv, Sk, D = raw.shape
    x = torch.from_numpy(orc.from_bf16(raw))
    rinv = 1.0 / torch.sqrt((x * x).sum(-1, keepdim=True) / D + eps)
    K = (x * rinv * torch.from_numpy(orc.from_bf16(kw))).to(torch.bfloat16)
    V = (x * rinv).to(torch.bfloat16)
    freqs = torch.arange(Sk, dtype=torch.float32)[:, None] * torch.from_numpy(inv)[None, :]
    emb = torch.cat([freqs, freqs], -1)
    c, s = torch.cos(emb).to(torch.bfloat16), torch.sin(emb).to(torch.bfloat16)
    K = K * c + rotate_half(K) * s
    f = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return f(K), f(V)


@pytest.mark.parametrize("D,partial", [(512, 0.25), (256, 1.0)])
def test_raw_prefill_kv_matches_torch_bf16_ops(D, partial):
    rng = np.random.default_rng(34)
    raw = orc.to_bf16(rng.standard_normal((2, 300, D)).astype(np.float32) * 2)
    kw = orc.to_bf16((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    inv = orc.rope_inv_freq(D, 1.0e6 if D == 512 else 1.0e4, partial)
    k, v = orc.raw_prefill_kv(raw, kw, 1e-6, inv)
    tk, tv = _torch_raw_prefill_kv(raw, kw, 1e-6, inv)
    # fp32 summation order (rinv) and cos / sin last-ulp differences move a value across a
    # bf16 rounding boundary only rarely: a rotated element sums two bf16 products, so it
    # can move by two bf16 steps, on a tiny fraction of elements.
    for ours, ref in ((k, tk), (v, tv)):
        a, b = orc.from_bf16(ours), orc.from_bf16(ref)
        assert (np.abs(a - b) <= np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -6).all()
        assert np.mean(ours != ref) < 2e-3
    # the rotated pairs really rotate: position 0 leaves K = kNorm(x); later positions do not
    k0 = orc.to_bf16(orc.from_bf16(raw[:, 0]) / np.sqrt((orc.from_bf16(raw[:, 0]) ** 2).mean(-1, keepdims=True) + 1e-6)
                     * orc.from_bf16(kw))
    assert np.mean(k[:, 0] == k0) > 0.99 and np.mean(k[:, 100, :64] != k0[:, :64]) > 0.5


# ------------------------------------------- the reference's own primitive test cases

def _golden():
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "es_primitives.json")) as f:
        return json.load(f)["cases"]


def test_golden_es_primitives():
    """The assertions of the reference's ESPrimitivesTests.mm for the primitives on this path
    (tests/golden/es_primitives.json), evaluated on the oracle."""
    g = _golden()
    c = g["rms_norm_weightless"]
    y = orc.from_bf16(orc.rms_norm_rows(orc.to_bf16(np.array([c["x"]], np.float32)), None, c["eps"]))
    assert np.abs(y[0] - np.array(c["expect"])).max() <= c["atol"]
    c = g["rms_norm_unit_weight_mean_square"]
    y = orc.from_bf16(orc.rms_norm_rows(orc.to_bf16(np.array([c["x"]], np.float32)),
                                        orc.to_bf16(np.array(c["weight"], np.float32)), c["eps"]))
    assert abs(float(np.mean(y.astype(np.float64) ** 2)) - c["expect_mean_square"]) <= c["atol"]
    c = g["repeat_kv_order"]
    # GQA kv-major: query head h reads kv head h // n_rep (the oracle's mapping, seen through
    # decode_f64 with one visible row per kv head whose V row is the head's value)
    n_rep, kv = c["n_rep"], c["kv_heads"]
    step = orc.Step(B=1, Hq=len(kv) * n_rep, Hkv=len(kv), D=8, cap=1, scale=1.0)
    v = orc.to_bf16(np.repeat(np.array(kv, np.float32)[:, None, None], 8, axis=2))
    q = orc.to_bf16(np.zeros((1, step.Hq, 8), np.float32))
    out = orc.decode_f64(step, q, v.reshape(-1), v.reshape(-1), [0])
    assert list(out[0, :, 0]) == c["expect"]
    for name in ("local_rope_full_rotation_position_0", "global_prope_zero_tail_position_1"):
        c = g[name]
        inv = orc.rope_inv_freq(c["head_dim"], c["theta"], c["partial"])
        ang = np.concatenate([inv, inv]).astype(np.float64) * c["position"]
        cos, sin = np.cos(ang), np.sin(ang)
        lo, hi = c.get("tail_dims", [0, c["head_dim"] // 2])
        for base in (0, c["head_dim"] // 2):
            assert np.abs(cos[base + lo:base + hi] - c.get("expect_tail_cos", c.get("expect_cos"))).max() <= c["atol"]
            assert np.abs(sin[base + lo:base + hi] - c.get("expect_tail_sin", c.get("expect_sin"))).max() <= c["atol"]
        if "first_dim_min_abs_sin" in c:
            assert abs(sin[0]) > c["first_dim_min_abs_sin"]
