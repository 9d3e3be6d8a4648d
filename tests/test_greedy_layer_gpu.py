"""Greedy-argmax agreement with the decode attention slotted into a random-init model.

A two-layer Gemma-4-shaped toy (one sliding layer: D=256, window 64, separate K/V; one
global layer: D=512, attention_k_eq_v with a shared buffer; q/k/v RMS-normed per head,
scale 1.0 as in the model) runs greedy decode steps twice: once with attention from the
GPU path (es::ESKVCache::decode through the C ABI, fused append included) and once with
the CPU oracle in reference-rounding mode (the composite of ESAttention.mm:136-165).
Projections, residuals, the final norm and the tied head are the same fp32 host code for
both.  Tokens are teacher-forced from the oracle run so both see the same inputs; the
greedy argmax of every step is compared (the decoder-layer shape of
ESDecoderLayer.mm:47-89 and the argmax of ESSampler.mm:6-10, with random weights).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HIDDEN, VOCAB, HQ = 512, 1024, 8
LAYERS = [
    dict(D=256, hkv=2, window=64, shared=False),   # sliding
    dict(D=512, hkv=1, window=0, shared=True),     # global, k_eq_v
]


def _bf(x):
    return orc.to_bf16(np.ascontiguousarray(x, dtype=np.float32))


def _f(h):
    return orc.from_bf16(h).astype(np.float32)


def _rms(x, eps=1e-6):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


class Toy:
    def __init__(self, seed):
        rng = np.random.default_rng(seed)
        self.emb = rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32)
        self.w = []
        for L in LAYERS:
            D, hkv = L["D"], L["hkv"]
            s = 1.0 / np.sqrt(HIDDEN)
            self.w.append(dict(
                q=rng.standard_normal((HIDDEN, HQ * D)).astype(np.float32) * s,
                k=rng.standard_normal((HIDDEN, hkv * D)).astype(np.float32) * s,
                v=rng.standard_normal((HIDDEN, hkv * D)).astype(np.float32) * s,
                o=rng.standard_normal((HQ * D, HIDDEN)).astype(np.float32) / np.sqrt(HQ * D),
            ))

    def qkv(self, li, x):
        L, W = LAYERS[li], self.w[li]
        D, hkv = L["D"], L["hkv"]
        h = _rms(x)
        q = _bf(_rms((h @ W["q"]).reshape(HQ, D)))
        k = _bf(_rms((h @ W["k"]).reshape(hkv, D)))
        v = k if L["shared"] else _bf(_rms((h @ W["v"]).reshape(hkv, D)))
        return q, k, v

    def out(self, li, x, o_bf16):
        return x + _f(o_bf16).reshape(-1) @ self.w[li]["o"]

    def logits(self, x, token):
        # The head reads what the two attention layers added to the residual stream (the
        # input embedding subtracted): with it left in, the input token's own logit wins
        # every step by ~20 and the argmax would not depend on attention at all.  These
        # logits are O(1) with a median top-2 margin of ~0.3, and the greedy tokens vary.
        return _rms(x - self.emb[token]) @ self.emb.T / np.sqrt(HIDDEN)


def _oracle_attend(L, q, kc, vc):
    D, hkv = L["D"], L["hkv"]
    n = kc.shape[1]
    step = orc.Step(B=1, Hq=HQ, Hkv=hkv, D=D, cap=n, scale=1.0)
    return orc.decode_refround(step, q.reshape(1, HQ, D), np.ascontiguousarray(kc).reshape(-1),
                               np.ascontiguousarray(vc).reshape(-1), [n - 1]).reshape(HQ, D)


def test_greedy_argmax_agreement_in_a_random_init_model():
    from apertura_amd.cache import ESKVCache
    toy = Toy(2024)
    rng = np.random.default_rng(7)
    prefill, steps = 150, 64
    cache = ESKVCache(len(LAYERS))
    host_k, host_v = [], []
    # prefill rows: random unit-RMS K/V rows (the same for both paths)
    for li, L in enumerate(LAYERS):
        k = _bf(_rms(rng.standard_normal((L["hkv"], prefill, L["D"])).astype(np.float32)))
        v = k if L["shared"] else _bf(_rms(rng.standard_normal((L["hkv"], prefill, L["D"])).astype(np.float32)))
        kd = _dev(k)
        cache.update(li, kd, kd if L["shared"] else _dev(v), 0, prealloc=True)
        host_k.append(k)
        host_v.append(v)
    token = int(rng.integers(VOCAB))
    agree, margins, dlogit, tokens = 0, [], [], set()
    for _ in range(steps):
        x_ref = toy.emb[token].copy()
        x_gpu = toy.emb[token].copy()
        for li, L in enumerate(LAYERS):
            # oracle path
            q, k, v = toy.qkv(li, x_ref)
            host_k[li] = np.concatenate([host_k[li], k[:, None]], axis=1)
            host_v[li] = host_k[li] if L["shared"] else np.concatenate([host_v[li], v[:, None]], axis=1)
            if L["window"] and host_k[li].shape[1] > L["window"]:
                host_k[li] = host_k[li][:, -L["window"]:]
                host_v[li] = host_k[li] if L["shared"] else host_v[li][:, -L["window"]:]
            x_ref = toy.out(li, x_ref, _oracle_attend(L, q, host_k[li], host_v[li]))
            # GPU path (its own residual stream)
            qg, kg, vg = toy.qkv(li, x_gpu)
            kd = _dev(kg[:, None])
            o = cache.decode(li, _dev(qg), kd, kd if L["shared"] else _dev(vg[:, None]), L["window"], L["window"],
                             1.0)
            x_gpu = toy.out(li, x_gpu, _host(o))
        lr, lg = toy.logits(x_ref, token), toy.logits(x_gpu, token)
        top = np.sort(lr)[-2:]
        margins.append(float(top[1] - top[0]))
        dlogit.append(float(np.abs(lr - lg).max()))
        agree += int(np.argmax(lr) == np.argmax(lg))
        token = int(np.argmax(lr))  # teacher forcing from the oracle path
        tokens.add(token)
    print(f"greedy agreement {agree}/{steps}; {len(tokens)} distinct tokens; smallest top-2 "
          f"margin {min(margins):.4f}; max |logit diff| {max(dlogit):.4f}")
    # the test is only meaningful if the argmax moves with the attention output
    assert len(tokens) >= steps // 2
    # The two residual streams (and so the appended K/V rows) drift apart by rounding over
    # the 64 steps: the fp64 oracle against the reference-rounding one drifts by up to 0.3
    # in a logit on this toy.  The fp64 oracle with a planted fault in place of the GPU
    # path (sliding window one row too long, kv heads swapped, the appended row not
    # attended) moves a logit by 1.6 to 5.9 here, so the drift bound is 1.0; a flip is
    # acceptable only where the oracle's own top-2 margin is below 0.1.
    assert max(dlogit) < 1.0
    assert agree >= steps - sum(m < 0.1 for m in margins)
    # the sliding layer kept exactly its window; the global layer every row
    assert cache.slot(0)["len"] - cache.slot(0)["start"] == LAYERS[0]["window"]
    assert cache.slot(1)["len"] == prefill + steps and cache.slot(1)["shared"]


# ------------------------------------------------------------------ raw-K global layer lockstep
#
# The reference's in-model global path: a rawKV layer keeps pre-norm k_proj rows and attends
# through esDecodeAttnGlobal (ESAttention.mm:253-302; q8: updateRawQ8 + esDecodeAttnGlobalQ8,
# ESAttention.mm:270-277), and its numerics are gated by rawLockstep (AperturaResearch/main.mm:
# 776-821): two arms decode one forced token stream in lockstep and report max / mean |dlogit|
# and argmax flips.  Here the arms are the GPU path (es::ESKVCache::decodeRaw / decodeRawQ8
# through the C ABI, fused append included) and the fp64 raw oracle (orc_decode_raw_f64 /
# orc_decode_raw_q8_f64 over the rows the oracle appends and quantizes itself).

RAW_HQ, RAW_HKV = 16, 2          # 8 query heads per kv head (ESDecodeAttn.mm:419-422); kv heads pair up
RAW_EPS = 1e-6
RAW_INV = orc.rope_inv_freq(512, 1.0e6, 0.25)  # Gemma-4 global rotary: theta 1e6, 64 of 256 pairs turn


def _rope_q(q, pos):
    """Rotary of the query heads at `pos` (pairs (d, d + 256), d < 64, fp32 angle pos * invFreq)."""
    out = q.copy()
    ang = np.float32(pos) * RAW_INV[:64]
    c, s = np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)
    x0, x1 = q[:, :64], q[:, 256:320]
    out[:, :64] = x0 * c - x1 * s
    out[:, 256:320] = x1 * c + x0 * s
    return out


class RawToy:
    """Layer 0: the sliding layer of Toy (D=256, window 64, separate K/V).  Layer 1: a global
    raw-K layer (D=512, 16 query heads over 2 kv heads): q = bf16(rope(rms(q_proj))) at the
    token's position, the cache keeps kRaw = bf16(k_proj) un-normalised (row RMS ~2), and the
    kernel rebuilds K = rope(rms(kRaw) * kw) and V = rms(kRaw) with a non-trivial k-norm
    weight kw; scale 1.0 (the model's)."""

    def __init__(self, seed):
        rng = np.random.default_rng(seed)
        self.emb = rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32)
        s = 1.0 / np.sqrt(HIDDEN)
        D0, h0 = LAYERS[0]["D"], LAYERS[0]["hkv"]
        self.w0 = dict(q=rng.standard_normal((HIDDEN, HQ * D0)).astype(np.float32) * s,
                       k=rng.standard_normal((HIDDEN, h0 * D0)).astype(np.float32) * s,
                       v=rng.standard_normal((HIDDEN, h0 * D0)).astype(np.float32) * s,
                       o=rng.standard_normal((HQ * D0, HIDDEN)).astype(np.float32) / np.sqrt(HQ * D0))
        self.wq = rng.standard_normal((HIDDEN, RAW_HQ * 512)).astype(np.float32) * s
        self.wk = rng.standard_normal((HIDDEN, RAW_HKV * 512)).astype(np.float32) * (2.0 * s)
        self.wo = rng.standard_normal((RAW_HQ * 512, HIDDEN)).astype(np.float32) / np.sqrt(RAW_HQ * 512)
        self.kw = _bf((1.0 + 0.25 * rng.standard_normal(512)).astype(np.float32))

    def sliding_qkv(self, x):
        D, hkv = LAYERS[0]["D"], LAYERS[0]["hkv"]
        h = _rms(x)
        return (_bf(_rms((h @ self.w0["q"]).reshape(HQ, D))), _bf(_rms((h @ self.w0["k"]).reshape(hkv, D))),
                _bf(_rms((h @ self.w0["v"]).reshape(hkv, D))))

    def global_q_kraw(self, x, pos):
        h = _rms(x)
        return _bf(_rope_q(_rms((h @ self.wq).reshape(RAW_HQ, 512)), pos)), _bf((h @ self.wk).reshape(RAW_HKV, 512))

    def logits(self, x, token):
        return _rms(x - self.emb[token]) @ self.emb.T / np.sqrt(HIDDEN)


def _oracle_attend_f64(L, q, kc, vc):
    """The sliding layer's attention by the fp64 oracle, rounded to bf16 as the GPU's output is
    (the reference-rounding oracle's bf16 scores would add a drift of their own at scale 1.0)."""
    D, hkv = L["D"], L["hkv"]
    n = kc.shape[1]
    step = orc.Step(B=1, Hq=HQ, Hkv=hkv, D=D, cap=n, scale=1.0)
    o = orc.decode_f64(step, q.reshape(1, HQ, D), np.ascontiguousarray(kc).reshape(-1),
                       np.ascontiguousarray(vc).reshape(-1), [n - 1])
    return _bf(o.reshape(HQ, D).astype(np.float32))


class _OracleArm:
    """One oracle arm's state: the sliding layer's live rows, the global layer's raw rows (q8:
    quantized by orc_quantize_rows as they arrive), and a planted oracle fault for the global
    layer's attention (0: none).  Both layers' attention is the fp64 oracle's."""

    def __init__(self, k0, v0, raw, q8, fault=0):
        self.k0, self.v0, self.q8, self.fault = k0.copy(), v0.copy(), q8, fault
        self.raw = raw.copy()
        if q8:
            self.qr, self.sc, self.bs = orc.quantize_rows(raw)

    def step(self, toy, token, pos):
        x = toy.emb[token].copy()
        q, k, v = toy.sliding_qkv(x)
        W = LAYERS[0]["window"]
        self.k0 = np.concatenate([self.k0, k[:, None]], axis=1)[:, -W:]
        self.v0 = np.concatenate([self.v0, v[:, None]], axis=1)[:, -W:]
        x = x + _f(_oracle_attend_f64(LAYERS[0], q, self.k0, self.v0)).reshape(-1) @ toy.w0["o"]
        qg, kr = toy.global_q_kraw(x, pos)
        self.raw = np.concatenate([self.raw, kr[:, None]], axis=1)
        n = self.raw.shape[1]
        with orc.planted_fault(self.fault):
            if self.q8:
                qn, sn, bn = orc.quantize_rows(kr[:, None])
                self.qr = np.concatenate([self.qr, qn], axis=1)
                self.sc = np.concatenate([self.sc, sn], axis=1)
                self.bs = np.concatenate([self.bs, bn], axis=1)
                o = orc.decode_raw_q8_f64(qg, self.qr, self.sc, self.bs, n, toy.kw, RAW_EPS, RAW_INV, 1.0)
            else:
                o = orc.decode_raw_f64(qg, np.ascontiguousarray(self.raw), n, toy.kw, RAW_EPS, RAW_INV, 1.0)
        x = x + _f(_bf(o.astype(np.float32))).reshape(-1) @ toy.wo
        return toy.logits(x, token)


@pytest.mark.parametrize("mode", ["raw", "q8"])
def test_raw_global_layer_lockstep(mode):
    """rawLockstep (AperturaResearch/main.mm:776-821) over the GPU raw-K (or q8 raw-K) global
    layer: 64 decode steps teacher-forced from the fp64 oracle arm, max / mean |dlogit| and
    argmax flips reported.  A third arm, the oracle with the RoPE sign of the K rebuild flipped
    (a planted mistake, on the CPU), calibrates the drift bound: it must move a logit by far
    more than the bound the GPU arm stays within."""
    from apertura_amd.cache import ESKVCache
    toy = RawToy(2025)
    rng = np.random.default_rng(11)
    # Bound: the GPU arm drifts by 0.05 (raw) and 0.07 (q8) in a logit over the 64 steps; the
    # oracle arm with the planted RoPE-sign fault moves one by ~4.  0.25 sits between them.
    prefill, steps, bound = 200, 64, 0.25
    q8 = mode == "q8"
    D0, h0 = LAYERS[0]["D"], LAYERS[0]["hkv"]
    k0 = _bf(_rms(rng.standard_normal((h0, prefill, D0)).astype(np.float32)))
    v0 = _bf(_rms(rng.standard_normal((h0, prefill, D0)).astype(np.float32)))
    scales = 2.0 * (0.5 + rng.random((RAW_HKV, prefill, 1))).astype(np.float32)
    raw = _bf(rng.standard_normal((RAW_HKV, prefill, 512)).astype(np.float32) * scales)
    cache = ESKVCache(2)
    cache.update(0, _dev(k0), _dev(v0), 0, prealloc=True)
    if q8:
        cache.update_raw_q8(1, _dev(raw))
    else:
        cache.update_raw(1, _dev(raw), True)
    kw_d = _dev(toy.kw)
    ref = _OracleArm(k0[:, -LAYERS[0]["window"]:], v0[:, -LAYERS[0]["window"]:], raw, q8)
    bad = _OracleArm(k0[:, -LAYERS[0]["window"]:], v0[:, -LAYERS[0]["window"]:], raw, q8, fault=5)
    print(f"\n[case] raw-K global layer lockstep, mode {mode}: prefill {prefill}, {steps} steps", flush=True)

    token = int(rng.integers(VOCAB))
    d_gpu, mean_gpu, d_bad, margins, flips, tokens = [], [], [], [], [], set()
    for i in range(steps):
        pos = prefill + i
        lr = ref.step(toy, token, pos)
        lb = bad.step(toy, token, pos)
        # GPU arm: its own residual stream and caches
        x = toy.emb[token].copy()
        q, k, v = toy.sliding_qkv(x)
        W = LAYERS[0]["window"]
        o = cache.decode(0, _dev(q), _dev(k[:, None]), _dev(v[:, None]), W, W, 1.0)
        x = x + _f(_host(o)).reshape(-1) @ toy.w0["o"]
        qg, kr = toy.global_q_kraw(x, pos)
        call = cache.decode_raw_q8 if q8 else cache.decode_raw
        og = call(1, _dev(qg), _dev(kr[:, None]), kw_d, RAW_EPS, list(RAW_INV))
        x = x + _f(_host(og)).reshape(-1) @ toy.wo
        lg = toy.logits(x, token)
        top = np.sort(lr)[-2:]
        margins.append(float(top[1] - top[0]))
        d_gpu.append(float(np.abs(lr - lg).max()))
        mean_gpu.append(float(np.abs(lr - lg).mean()))
        d_bad.append(float(np.abs(lr - lb).max()))
        if np.argmax(lr) != np.argmax(lg):
            flips.append(i)
        token = int(np.argmax(lr))  # teacher forcing from the oracle arm
        tokens.add(token)
    print(f"[{mode}] GPU vs oracle: max |dlogit| {max(d_gpu):.4f} mean {np.mean(mean_gpu):.5f} argmax flips "
          f"{len(flips)}/{steps} (oracle top-2 margins there: {[round(margins[i], 4) for i in flips]}); "
          f"planted RoPE-sign fault: max |dlogit| {max(d_bad):.4f}; "
          f"{len(tokens)} distinct tokens; smallest top-2 margin {min(margins):.4f}", flush=True)
    assert len(tokens) >= steps // 2  # the argmax moves with the attention output
    assert max(d_bad) > 8 * bound, "the planted fault does not clear the drift bound"
    assert max(d_gpu) < bound
    assert all(margins[i] < 0.1 for i in flips)
    s = cache.slot(1)
    assert s["len"] == prefill + steps and s["raw"] != q8 and s["q8"] == q8
