// ESPrefillAttn.cpp -- the prefill branch of the ES* layer over esda_prefill and the raw-K
// reconstruction kernels: esPrefillAttention / esPrefillAttnRaw / esPrefillAttnRawQ8, and
// ESKVCache::prefill / prefillRaw (the chunk's append followed by its attention, as the
// reference's ESAttention does at seq > 1: ESAttention.mm:77-108 + :168-193, :253-332).
#include "es/ESPrefillAttn.h"

#include <algorithm>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>

#include "es/ESKVCache.h"
#include "es/stream_scratch.h"
#include "esda.h"
#include "esda_prefill.h"

namespace es {
namespace {

void hipCheck(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void esdaCheck(int rc) {
    if (rc == ESDA_OK) return;
    if (rc == ESDA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(esda_last_error());
    throw std::runtime_error(esda_last_error());
}

// Per-thread, per-device, per-stream scratch: the split workspace, the rebuilt K / V of a raw-K
// prefill and the last rotary table uploaded.  Growth waits for the stream so that no
// queued kernel still reads a buffer being released.
struct Scratch {
    std::optional<Tensor> workspace, k, v, invFreq;
    std::vector<float> invFreqHost;
};

// One scratch set per (device, stream) of the calling thread (at most kMaxStreamScratch of
// them; stream_scratch.h): calls on different streams never share a position word,
// workspace or rebuilt rows, so they may overlap.
Scratch &scratch(hipStream_t st) { return streamScratch<Scratch>(st); }

Tensor &grown(std::optional<Tensor> &slot, size_t elems, Dtype dt, hipStream_t st) {
    if (!slot || slot->numel() < (int64_t) elems) {
        if (slot) hipCheck(hipStreamSynchronize(st), "esPrefill scratch growth");
        slot = Tensor::empty({(int64_t) std::max<size_t>(elems, 16)}, dt);
    }
    return *slot;
}

// The rotary table on the device, hd/2 floats (zero-extended).
const float *deviceInvFreq(const std::vector<float> &invFreq, int hd, hipStream_t st) {
    Scratch &s = scratch(st);
    std::vector<float> want(hd / 2, 0.0f);
    std::copy_n(invFreq.begin(), std::min<size_t>(invFreq.size(), want.size()), want.begin());
    if (!s.invFreq || s.invFreqHost != want) {
        if (s.invFreq) hipCheck(hipStreamSynchronize(st), "esPrefill rotary table");
        s.invFreqHost = want;
        s.invFreq = Tensor::empty({(int64_t) want.size()}, Dtype::f32);
        hipCheck(hipMemcpyAsync(s.invFreq->data, want.data(), want.size() * sizeof(float), hipMemcpyHostToDevice, st),
                 "esPrefill rotary table upload");
        hipCheck(hipStreamSynchronize(st), "esPrefill rotary table upload");
    }
    return static_cast<const float *>(s.invFreq->data);
}

void checkQ(const Tensor &q, const char *what) {
    if (!q.defined() || q.dim() != 3 || q.dtype != Dtype::bf16 || q.strides[2] != 1)
        throw std::invalid_argument(std::string(what) + ": q must be a bf16 [numQ, seq, hd] view with dense head dims");
}

void checkKV(const Tensor &t, const char *what) {
    if (!t.defined() || t.dim() != 3 || t.dtype != Dtype::bf16 || t.strides[2] != 1 || t.strides[1] != t.shape[2])
        throw std::invalid_argument(std::string(what) + ": K / V must be bf16 [numKV, seqK, hd] views with dense rows");
}

// The attention itself: query i at q_pos0 + i, key j at k_pos0 + j.
Tensor attend(const Tensor &q, const Tensor &K, const Tensor &V, int qPos0, int kPos0, int window, float scale,
              hipStream_t st, Tensor *out, const char *what) {
    const int numQ = (int) q.shape[0], seq = (int) q.shape[1], hd = (int) q.shape[2];
    const int numKV = (int) K.shape[0], seqK = (int) K.shape[1];
    if (K.shape != V.shape || K.strides != V.strides || K.shape[2] != hd)
        throw std::invalid_argument(std::string(what) + ": K and V must be views of one shape and layout");
    esda_prefill_desc d{};
    d.num_q_heads = numQ;
    d.num_kv_heads = numKV;
    d.head_dim = hd;
    d.seq_q = seq;
    d.seq_k = seqK;
    d.q_pos0 = qPos0;
    d.k_pos0 = kPos0;
    d.window = window;
    d.q_head_stride = q.strides[0];
    d.q_row_stride = q.strides[1];
    d.kv_head_stride = K.strides[0];
    d.out_row_stride = (int64_t) numQ * hd;
    d.out_head_stride = hd;
    d.split_keys = 0;
    d.scale = scale;
    size_t wsBytes = 0;
    esdaCheck(esda_prefill_workspace_size(&d, &wsBytes));
    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) seq * numQ * hd)
            throw std::invalid_argument(std::string(what) + ": out must be contiguous bf16 [seq, numQ * hd]");
        o = *out;
    } else {
        o = Tensor::empty({seq, (int64_t) numQ * hd}, Dtype::bf16);
    }
    esda_prefill_args a{};
    a.q = q.data;
    a.k = K.data;
    a.v = V.data;
    a.out = o.data;
    if (wsBytes) {
        Tensor &ws = grown(scratch(st).workspace, wsBytes, Dtype::u8, st);
        a.workspace = ws.data;
        a.workspace_bytes = ws.nbytes();
    }
    esdaCheck(esda_prefill(&d, &a, st));
    return o;
}

}  // namespace

Tensor esPrefillAttention(const Tensor &q, const Tensor &K, const Tensor &V, int pastLen, int window, float scale,
                          hipStream_t st, Tensor *out) {
    checkQ(q, "esPrefillAttention");
    checkKV(K, "esPrefillAttention");
    checkKV(V, "esPrefillAttention");
    if (pastLen < 0 || window < 0) throw std::invalid_argument("esPrefillAttention: pastLen and window must be >= 0");
    const int seq = (int) q.shape[1], seqK = (int) K.shape[1];
    // alignMask keeps the last seqK of the pastLen + seq columns (ESAttention.mm:17-22)
    const int kPos0 = pastLen + seq - seqK;
    if (kPos0 < 0) throw std::invalid_argument("esPrefillAttention: more keys than pastLen + seq positions");
    return attend(q, K, V, pastLen, kPos0, window, scale, st, out, "esPrefillAttention");
}

Tensor esPrefillAttnRaw(const Tensor &q, const Tensor &rawView, const Tensor &kw, float eps,
                        const std::vector<float> &invFreq, int pastLen, float scale, hipStream_t st, Tensor *out) {
    checkQ(q, "esPrefillAttnRaw");
    checkKV(rawView, "esPrefillAttnRaw");
    const int numKV = (int) rawView.shape[0], seqK = (int) rawView.shape[1], hd = (int) rawView.shape[2];
    if (pastLen < 0 || pastLen + q.shape[1] != seqK)
        throw std::invalid_argument("esPrefillAttnRaw: the raw stream must hold pastLen + seq rows");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != hd || !kw.contiguous())
        throw std::invalid_argument("esPrefillAttnRaw: kw must be contiguous bf16 [hd]");
    Scratch &s = scratch(st);
    const size_t n = (size_t) numKV * seqK * hd;
    Tensor &kb = grown(s.k, n, Dtype::bf16, st);
    Tensor &vb = grown(s.v, n, Dtype::bf16, st);
    const float *inv = deviceInvFreq(invFreq, hd, st);
    esdaCheck(esda_raw_prefill_kv(rawView.data, rawView.strides[0], numKV, seqK, hd, kw.data, eps, inv, 0, kb.data,
                                  vb.data, (int64_t) seqK * hd, st));
    const Tensor K = Tensor::wrap(kb.data, {numKV, seqK, hd}, Dtype::bf16);
    const Tensor V = Tensor::wrap(vb.data, {numKV, seqK, hd}, Dtype::bf16);
    return attend(q, K, V, pastLen, 0, 0, scale, st, out, "esPrefillAttnRaw");
}

Tensor esPrefillAttnRawQ8(const Tensor &q, const Tensor &qView, const Tensor &scView, const Tensor &bsView,
                          const Tensor &kw, float eps, const std::vector<float> &invFreq, int pastLen, float scale,
                          hipStream_t st, Tensor *out) {
    checkQ(q, "esPrefillAttnRawQ8");
    if (!qView.defined() || qView.dim() != 3 || qView.dtype != Dtype::u8 || qView.shape[2] != 512 ||
        qView.strides[2] != 1 || qView.strides[1] != 512)
        throw std::invalid_argument("esPrefillAttnRawQ8: qView must be a u8 [numKV, seqK, 512] view with dense rows");
    const int numKV = (int) qView.shape[0], seqK = (int) qView.shape[1];
    for (const Tensor *t : {&scView, &bsView})
        if (!t->defined() || t->dtype != Dtype::f32 || t->dim() != 3 || t->shape[0] != numKV || t->shape[1] != seqK ||
            t->strides[1] != 1 || t->strides[0] != scView.strides[0])
            throw std::invalid_argument("esPrefillAttnRawQ8: scale / bias must be f32 [numKV, seqK, 1] views");
    if (pastLen < 0 || pastLen + q.shape[1] != seqK)
        throw std::invalid_argument("esPrefillAttnRawQ8: the raw stream must hold pastLen + seq rows");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != 512 || !kw.contiguous())
        throw std::invalid_argument("esPrefillAttnRawQ8: kw must be contiguous bf16 [512]");
    Scratch &s = scratch(st);
    const size_t n = (size_t) numKV * seqK * 512;
    Tensor &kb = grown(s.k, n, Dtype::bf16, st);
    Tensor &vb = grown(s.v, n, Dtype::bf16, st);
    const float *inv = deviceInvFreq(invFreq, 512, st);
    esdaCheck(esda_raw_q8_prefill_kv(qView.data, qView.strides[0], static_cast<const float *>(scView.data),
                                     static_cast<const float *>(bsView.data), scView.strides[0], numKV, seqK, kw.data,
                                     eps, inv, 0, kb.data, vb.data, (int64_t) seqK * 512, st));
    const Tensor K = Tensor::wrap(kb.data, {numKV, seqK, 512}, Dtype::bf16);
    const Tensor V = Tensor::wrap(vb.data, {numKV, seqK, 512}, Dtype::bf16);
    return attend(q, K, V, pastLen, 0, 0, scale, st, out, "esPrefillAttnRawQ8");
}

// ------------------------------------------------------------ ESKVCache prefill chunks

Tensor ESKVCache::prefill(int layer, const Tensor &q, const Tensor &kNew, const Tensor &vNew, int maxKeep, int window,
                          float scale, int pastLen, bool prealloc, hipStream_t st, Tensor *out) {
    lastStream_ = st;
    if (stepMode_) throw std::runtime_error("ESKVCache::prefill: not available in compiled-step mode (beginStep .. endStep)");
    checkQ(q, "ESKVCache::prefill");
    if (kNew.dim() != 3 || kNew.shape[1] != q.shape[1])
        throw std::invalid_argument("ESKVCache::prefill: kNew must hold one row per query");
    auto kv = update(layer, kNew, vNew, maxKeep, prealloc, st);
    return esPrefillAttention(q, kv.first, kv.second, pastLen, window, scale, st, out);
}

Tensor ESKVCache::prefillRaw(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                             const std::vector<float> &invFreq, int pastLen, float scale, bool q8, hipStream_t st,
                             Tensor *out) {
    lastStream_ = st;
    if (stepMode_) throw std::runtime_error("ESKVCache::prefillRaw: not available in compiled-step mode (beginStep .. endStep)");
    checkQ(q, "ESKVCache::prefillRaw");
    if (kNew.dim() != 3 || kNew.shape[1] != q.shape[1])
        throw std::invalid_argument("ESKVCache::prefillRaw: kNew must hold one row per query");
    if (q8) {
        const RawQ8 r = updateRawQ8(layer, kNew, st);
        return esPrefillAttnRawQ8(q, r.qview, r.sc, r.bs, kw, eps, invFreq, pastLen, scale, st, out);
    }
    const Raw r = updateRaw(layer, kNew, /*prealloc=*/true, st);
    return esPrefillAttnRaw(q, r.view, kw, eps, invFreq, pastLen, scale, st, out);
}

}  // namespace es
