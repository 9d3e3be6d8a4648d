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
