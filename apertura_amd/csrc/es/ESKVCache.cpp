// ESKVCache.cpp -- GPU KV cache with the reference's update / updateRaw / current /
// reset behaviour (Apertura ESKVCache.mm:19-119, 458-504, 622-638).  Device work goes
// through the HIP runtime (buffer copies) and the esda C ABI (decode kernels).
#include "es/ESKVCache.h"

#include <algorithm>
#include <stdexcept>
#include <string>

#include "es/ESDecodeAttn.h"
#include "es/es_fill.h"
#include "esda.h"

namespace es {
namespace {

int roundUpChunk(int n) {
    return (n + ESKVCache::kGrowChunk - 1) / ESKVCache::kGrowChunk * ESKVCache::kGrowChunk;
}

void hipCheck(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// esda status -> the exception type the reference throws for the same condition.
void esdaCheck(int rc) {
    if (rc == ESDA_OK) return;
    if (rc == ESDA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(esda_last_error());
    throw std::runtime_error(esda_last_error());
}

// A [kvHeads, n, headDim] bf16 tensor whose rows are contiguous inside each head.
void checkRows(const Tensor &t, const char *what) {
    if (!t.defined() || t.dim() != 3 || t.dtype != Dtype::bf16)
        throw std::invalid_argument(std::string(what) + ": expected a [kvHeads, n, headDim] bf16 tensor");
    if (t.strides[2] != 1 || t.strides[1] != t.shape[2] || t.strides[0] < t.shape[1] * t.shape[2])
        throw std::invalid_argument(std::string(what) + ": rows must be contiguous within each head");
    if (t.shape[0] <= 0 || t.shape[1] <= 0 || t.shape[2] <= 0 || (t.shape[2] % 8))
        throw std::invalid_argument(std::string(what) + ": empty tensor or headDim not a multiple of 8");
}

// dst[h, dr0 + i, :] = src[h, sr0 + i, :] for i < n and every head h.
void copyRows(const Tensor &dst, int dr0, const Tensor &src, int sr0, int n, hipStream_t st) {
    if (n <= 0) return;
    const size_t rowBytes = (size_t) src.shape[2] * 2;
    auto *d = static_cast<char *>(dst.data) + (size_t) dr0 * dst.strides[1] * 2;
    auto *s = static_cast<const char *>(src.data) + (size_t) sr0 * src.strides[1] * 2;
    hipCheck(hipMemcpy2DAsync(d, (size_t) dst.strides[0] * 2, s, (size_t) src.strides[0] * 2,
                              (size_t) n * rowBytes, (size_t) src.shape[0], hipMemcpyDeviceToDevice, st),
             "ESKVCache row copy");
}

Tensor zeros(const std::vector<int64_t> &shape, hipStream_t st) {
    Tensor t = Tensor::empty(shape, Dtype::bf16);
    zeroFill(t.data, t.nbytes(), st);
    return t;
}

// An owned copy of `src` (the reference stores the caller's array itself; here the
// caller keeps ownership of its memory, so the value is copied).
Tensor clone(const Tensor &src, hipStream_t st) {
    Tensor t = Tensor::empty(src.shape, Dtype::bf16);
    copyRows(t, 0, src, 0, (int) src.shape[1], st);
    return t;
}

// Along the sequence axis: [a ; b] (a view-aware concatenate).
Tensor concatRows(const Tensor &a, const Tensor &b, hipStream_t st) {
    if (a.shape[0] != b.shape[0] || a.shape[2] != b.shape[2])
        throw std::invalid_argument("ESKVCache::update: kv heads / head dim differ from the cached rows");
    Tensor t = Tensor::empty({a.shape[0], a.shape[1] + b.shape[1], a.shape[2]}, Dtype::bf16);
    copyRows(t, 0, a, 0, (int) a.shape[1], st);
    copyRows(t, (int) a.shape[1], b, 0, (int) b.shape[1], st);
    return t;
}

Tensor liveView(const Tensor &buf, int start, int len) {
    if (start == 0 && len == buf.shape[1]) return buf;
    return buf.slice(1, start, len);
}

}  // namespace

ESKVCache::ESKVCache(int numLayers)
    : k_(numLayers), v_(numLayers), slots_(numLayers), rq8slots_(numLayers) {
    if (numLayers <= 0) throw std::invalid_argument("ESKVCache: numLayers must be positive");
}

void ESKVCache::checkLayer(int layer) const {
    if (layer < 0 || layer >= (int) slots_.size()) throw std::invalid_argument("ESKVCache: layer out of range");
}

const ESKVCache::Slot &ESKVCache::slotAt(int layer) const {
    checkLayer(layer);
    return slots_[layer];
}

int ESKVCache::slotCapacity(int layer) const {
    const Slot &s = slotAt(layer);
    if (rq8slots_[layer].q) return (int) rq8slots_[layer].q->shape[1];
    return s.k ? (int) s.k->shape[1] : 0;
}

// Make room for nNew rows at s.len (ESKVCache.mm:74-94): when they do not fit, the live
// range [start, len) moves to the front of a zeroed buffer of roundUpChunk(content +
// nNew + kGrowChunk) rows.  Raw slots (no v) keep rows from 0 (ESKVCache.mm:490-496).
void ESKVCache::growSlot(Slot &s, int nNew, hipStream_t st, bool compactStart) {
    const int cap = (int) s.k->shape[1];
    if (s.len + nNew <= cap) return;
    const int from = compactStart ? s.start : 0;
    const int content = s.len - from;
    const int newCap = roundUpChunk(content + nNew + kGrowChunk);
    const int64_t kvH = s.k->shape[0], hd = s.k->shape[2];
    Tensor nk = zeros({kvH, newCap, hd}, st);
    copyRows(nk, 0, *s.k, from, content, st);
    std::optional<Tensor> nv;
    if (s.v) {
        if (s.shared) {
            nv = nk;
        } else {
            nv = zeros({kvH, newCap, hd}, st);
            copyRows(*nv, 0, *s.v, from, content, st);
        }
    }
    // The old buffers may still be read by queued work: finish it before releasing them.
    hipCheck(hipStreamSynchronize(st), "ESKVCache compaction");
    s.k = nk;
    s.v = nv;
    if (compactStart) {
        if (s.start > 0) s.lost = true;
        s.len = content;
        s.start = 0;
    }
}

std::pair<Tensor, Tensor> ESKVCache::update(int layer, const Tensor &kNew, const Tensor &vNew, int maxKeep,
                                            bool prealloc, hipStream_t st) {
    lastStream_ = st;
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::update kNew");
    checkRows(vNew, "ESKVCache::update vNew");
    if (kNew.shape[1] != vNew.shape[1])
        throw std::invalid_argument("ESKVCache::update: kNew and vNew hold different row counts");
    if (stepMode_) {
        // Compiled-step append (ESKVCache.mm:21-33): the row comes from the step's index
        // tensor on the device, so the same launches serve every position; the whole
        // fixed-capacity buffers are returned (the step's mask hides unwritten rows).
        Slot &s = slots_[layer];
        if (!s.k || !s.v) throw std::runtime_error("ESKVCache::update: compiled-step slot not set (setSlot)");
        if (kNew.shape[1] != 1) throw std::invalid_argument("ESKVCache::update: a compiled step appends one row");
        const Tensor &idx = maxKeep > 0 ? *stepSlidingIdx_ : *stepGlobalIdx_;
        const bool slotShared = s.v->data == s.k->data;
        // One shared K=V buffer takes one row: a distinct vNew would overwrite the K row just
        // scattered (the reference's functional scatter keeps two arrays instead), so it is refused.
        if (slotShared && vNew.data != kNew.data)
            throw std::invalid_argument("ESKVCache::update: compiled-step slot holds one shared K=V buffer; "
                                        "vNew must alias kNew");
        // Every check runs before the first launch, so a refused step writes nothing.  The rows
        // must be packed [kvH, 1, hd] (what esda_kv_append reads): a strided row would need a
        // copy whose release waits on the stream, which a graph capture of the step forbids.
        auto check = [&](const Tensor &buf, const Tensor &row) {
            if (buf.dim() != 3 || buf.shape[0] != row.shape[0] || buf.shape[2] != row.shape[2] ||
                buf.strides[2] != 1 || buf.strides[1] != buf.shape[2])
                throw std::invalid_argument("ESKVCache::update: kNew / vNew do not match the compiled-step slot");
            if (row.strides[0] != row.shape[2])
                throw std::invalid_argument("ESKVCache::update: a compiled step needs packed [kvH, 1, hd] rows");
        };
        check(*s.k, kNew);
        check(*s.v, vNew);
        auto scatter = [&](const Tensor &buf, const Tensor &row) {
            const int cap = (int) buf.shape[1], hd = (int) buf.shape[2], kvH = (int) buf.shape[0];
            esdaCheck(esda_kv_append(buf.data, buf.strides[0] * kvH, buf.strides[0], 1, kvH, hd, cap, row.data, 1,
                                     static_cast<const int32_t *>(idx.data), st));
        };
        scatter(*s.k, kNew);
        if (!slotShared) scatter(*s.v, vNew);
        return {*s.k, *s.v};
    }
    if (!prealloc) {
        // Legacy mode (ESKVCache.mm:35-55): concat-grow, then keep the last maxKeep keys.
        auto &K = k_[layer];
        auto &V = v_[layer];
        if (!K) {
            K = clone(kNew, st);
            V = clone(vNew, st);
        } else {
            K = concatRows(*K, kNew, st);
            V = concatRows(*V, vNew, st);
        }
        if (maxKeep > 0 && K->shape[1] > maxKeep) {
            const int len = (int) K->shape[1], vlen = (int) V->shape[1];
            K = K->slice(1, len - maxKeep, len);
            V = V->slice(1, vlen - maxKeep, vlen);
        }
        return {*K, *V};
    }

    Slot &s = slots_[layer];
    // Mode-mismatch guard (ESKVCache.mm:59-62): raw rows (bf16 or q8) are pre-norm, not K/V.
    if ((s.k && !s.v) || rq8slots_[layer].q)
        throw std::runtime_error("ESKVCache::update: slot holds raw-K content — not usable "
                                 "by the composite path; re-prime the cache");
    const bool aliased = kNew.data == vNew.data;
    if (s.shared && !aliased)
        throw std::runtime_error("ESKVCache::update: slot holds one shared K=V buffer; vNew must alias kNew");
    const int nNew = (int) kNew.shape[1];
    if (!s.k) {
        // First append: capacity == content (ESKVCache.mm:69-73).  vNew aliasing kNew
        // (attention_k_eq_v) starts one shared K=V buffer.
        s.k = clone(kNew, st);
        s.shared = aliased;
        s.v = aliased ? *s.k : clone(vNew, st);
        s.len = nNew;
        s.start = 0;
    } else {
        if (kNew.shape[0] != s.k->shape[0] || kNew.shape[2] != s.k->shape[2])
            throw std::invalid_argument("ESKVCache::update: kv heads / head dim differ from the slot");
        growSlot(s, nNew, st, true);
        // In-place append at row len (ESKVCache.mm:95-99).
        copyRows(*s.k, s.len, kNew, 0, nNew, st);
        if (!s.shared) copyRows(*s.v, s.len, vNew, 0, nNew, st);
        s.len += nNew;
    }
    // Sliding-window eviction advances the logical start (ESKVCache.mm:102-104).
    if (maxKeep > 0 && s.len - s.start > maxKeep) s.start = s.len - maxKeep;
    return {liveView(*s.k, s.start, s.len), liveView(*s.v, s.start, s.len)};
}

ESKVCache::QKV ESKVCache::updateQuant(int layer, const Tensor &, const Tensor &, int, int, bool) {
    checkLayer(layer);
    throw std::runtime_error("ESKVCache::updateQuant: quantized-KV storage (quantized_matmul groups) is not "
                             "built by this library; use bf16, raw-K or q8 raw-K storage");
}

// ------------------------------------------------------------------ compiled-step mode

void ESKVCache::beginStep(const Tensor &globalIdx, const Tensor &slidingIdx) {
    for (const Tensor *t : {&globalIdx, &slidingIdx})
        if (!t->defined() || t->dtype != Dtype::i32 || t->numel() < 1)
            throw std::invalid_argument("ESKVCache::beginStep: indices must be device int32 [1] tensors");
    stepGlobalIdx_ = globalIdx;
    stepSlidingIdx_ = slidingIdx;
    stepMode_ = true;
}

void ESKVCache::endStep() {
    stepMode_ = false;
    stepGlobalIdx_.reset();
    stepSlidingIdx_.reset();
}

const Tensor &ESKVCache::slotK(int layer) const {
    const Slot &s = slotAt(layer);
    if (!s.k) throw std::runtime_error("ESKVCache::slotK: slot holds no buffer");
    return *s.k;
}

const Tensor &ESKVCache::slotV(int layer) const {
    const Slot &s = slotAt(layer);
    if (!s.v) throw std::runtime_error("ESKVCache::slotV: slot holds no buffer");
    return *s.v;
}

void ESKVCache::setSlot(int layer, Tensor k, Tensor v) {
    checkLayer(layer);
    checkRows(k, "ESKVCache::setSlot k");
    checkRows(v, "ESKVCache::setSlot v");
    Slot &s = slots_[layer];
    s.shared = k.data == v.data;
    s.k = std::move(k);
    s.v = std::move(v);
}

Tensor ESKVCache::takeSlotK(int layer) {
    checkLayer(layer);
    Slot &s = slots_[layer];
    if (!s.k) throw std::runtime_error("ESKVCache::takeSlotK: slot holds no buffer");
    Tensor t = std::move(*s.k);
    s.k.reset();
    return t;
}

Tensor ESKVCache::takeSlotV(int layer) {
    checkLayer(layer);
    Slot &s = slots_[layer];
    if (!s.v) throw std::runtime_error("ESKVCache::takeSlotV: slot holds no buffer");
    Tensor t = std::move(*s.v);
    s.v.reset();
    return t;
}

std::pair<Tensor, Tensor> ESKVCache::current(int layer, bool prealloc) const {
    checkLayer(layer);
    if (!prealloc) {
        if (!k_[layer]) throw std::runtime_error("ESKVCache::current: layer holds no rows");
        return {*k_[layer], *v_[layer]};
    }
    const Slot &s = slots_[layer];
    if (!s.k || !s.v) throw std::runtime_error("ESKVCache::current: layer holds no composite rows");
    return {liveView(*s.k, s.start, s.len), liveView(*s.v, s.start, s.len)};
}

ESKVCache::Raw ESKVCache::currentRaw(int layer) const {
    checkLayer(layer);
    const Slot &s = slots_[layer];
    if (!s.k || s.v) throw std::runtime_error("ESKVCache::currentRaw: layer holds no raw rows");
    return {liveView(*s.k, s.start, s.len), *s.k, s.len, (int) s.k->shape[1]};
}

ESKVCache::Raw ESKVCache::updateRaw(int layer, const Tensor &kNew, bool prealloc, hipStream_t st) {
    lastStream_ = st;
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::updateRaw kNew");
    const int nNew = (int) kNew.shape[1];
    if (!prealloc) {
        // Legacy concat-grow (ESKVCache.mm:460-466).
        auto &K = k_[layer];
        K = K ? concatRows(*K, kNew, st) : clone(kNew, st);
        const int len = (int) K->shape[1];
        return {*K, *K, len, len};
    }
    Slot &s = slots_[layer];
    if (s.k && s.v)
        throw std::runtime_error("ESKVCache::updateRaw: slot holds composite K/V content "
                                 "(post-norm) — not derivable as raw; re-prime the cache");
    // a bf16 slot beside the q8 rows would split the stream in two
    if (rq8slots_[layer].q)
        throw std::runtime_error("ESKVCache::updateRaw: slot holds q8 raw rows; use updateRawQ8");
    if (!s.k) {
        s.k = clone(kNew, st);
        s.len = nNew;
        s.start = 0;
    } else {
        if (kNew.shape[0] != s.k->shape[0] || kNew.shape[2] != s.k->shape[2])
            throw std::invalid_argument("ESKVCache::updateRaw: kv heads / head dim differ from the slot");
        growSlot(s, nNew, st, false);
        copyRows(*s.k, s.len, kNew, 0, nNew, st);
        s.len += nNew;
    }
    return {liveView(*s.k, 0, s.len), *s.k, s.len, (int) s.k->shape[1]};
}

void *ESKVCache::workspace(size_t bytes, hipStream_t st) {
    if (!workspace_ || workspace_->nbytes() < bytes) {
        if (workspace_) hipCheck(hipStreamSynchronize(st), "ESKVCache workspace growth");
        const size_t n = std::max<size_t>(bytes, 1 << 20);
        workspace_ = Tensor::empty({(int64_t) n}, Dtype::u8);
        // The status word at the front starts at zero (esda workspace contract).
        zeroFill(workspace_->data, 256, st);
    }
    return workspace_->data;
}

const void *ESKVCache::ropeTable(int rows, hipStream_t st) {
    if (!ropeTab_ || ropeRows_ < rows) {
        if (ropeTab_) hipCheck(hipStreamSynchronize(st), "ESKVCache rope table growth");
        const int n = (rows + 4095) / 4096 * 4096;
        ropeTab_ = Tensor::empty({(int64_t) n * 256}, Dtype::u8);
        esdaCheck(esda_rope_table(static_cast<const float *>(invFreqDev_->data), n, ropeTab_->data, st));
        ropeRows_ = n;
    }
    return ropeTab_->data;
}

int *ESKVCache::positionWord(int layer, int value, hipStream_t st) {
    if (!posDev_) posDev_ = Tensor::empty({(int64_t) slots_.size()}, Dtype::i32);
    int32_t *p = static_cast<int32_t *>(posDev_->data) + layer;
    esdaCheck(esda_fill_i32(p, value, 1, st));
    return p;
}

Tensor ESKVCache::decode(int layer, const Tensor &q, const Tensor &kNew, const Tensor &vNew, int maxKeep,
                         int window, float scale, hipStream_t st, Tensor *out) {
    lastStream_ = st;
    if (stepMode_) throw std::runtime_error("ESKVCache::decode: not available in compiled-step mode (beginStep .. endStep)");
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::decode kNew");
    checkRows(vNew, "ESKVCache::decode vNew");
    if (kNew.shape[1] != 1 || vNew.shape != kNew.shape)
        throw std::invalid_argument("ESKVCache::decode: kNew / vNew must be [kvHeads, 1, headDim]");
    if (window < 0) throw std::invalid_argument("ESKVCache::decode: window must be >= 0");
    const int kvH = (int) kNew.shape[0], hd = (int) kNew.shape[2];
    if (!q.defined() || q.dtype != Dtype::bf16 || !q.contiguous() || q.numel() % hd)
        throw std::invalid_argument("ESKVCache::decode: q must be contiguous bf16 [numQHeads, headDim]");
    const int Hq = (int) (q.numel() / hd);
    Slot &s = slots_[layer];
    if ((s.k && !s.v) || rq8slots_[layer].q)
        throw std::runtime_error("ESKVCache::decode: slot holds raw-K content — not usable "
                                 "by the composite path; re-prime the cache");
    const bool aliased = kNew.data == vNew.data;
    if (!s.k) {
        // First row: capacity == content, as for the reference's first store.
        s.k = Tensor::empty({kvH, 1, hd}, Dtype::bf16);
        s.shared = aliased;
        s.v = aliased ? *s.k : Tensor::empty({kvH, 1, hd}, Dtype::bf16);
        s.len = 0;
        s.start = 0;
    } else {
        if (kvH != s.k->shape[0] || hd != s.k->shape[2])
            throw std::invalid_argument("ESKVCache::decode: kv heads / head dim differ from the slot");
        if (s.shared && !aliased)
            throw std::runtime_error("ESKVCache::decode: slot holds one shared K=V buffer; vNew must alias kNew");
        growSlot(s, 1, st, true);
    }
    const int cap = (int) s.k->shape[1];
    // Rows attended after the append: the live range the reference's update() leaves,
    // then the sliding mask's last `window` positions of it.  Rows are positions here
    // (the slot's row 0 is position 0 until an eviction starts the window elsewhere),
    // so the window counts back from the new row.
    const int live = s.len + 1 - s.start;
    int w = maxKeep > 0 ? std::min(maxKeep, live) : live;
    if (window > 0) w = std::min(w, window);

    esda_decode_desc d{};
    d.batch = 1;
    d.num_q_heads = Hq;
    d.num_kv_heads = kvH;
    d.head_dim = hd;
    d.cap = cap;
    d.window = w;
    d.ring = 0;
    d.kv_shared = s.shared ? 1 : 0;
    d.head_stride = (int64_t) cap * hd;
    d.seq_stride = (int64_t) kvH * cap * hd;
    d.max_visible = w;
    d.split_rows = 0;
    d.scale = scale;
    size_t wsBytes = 0;
    esdaCheck(esda_decode_workspace_size(&d, &wsBytes));

    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) Hq * hd)
            throw std::invalid_argument("ESKVCache::decode: out must be contiguous bf16 [numQHeads, headDim]");
        o = *out;
    } else {
        o = Tensor::empty({Hq, hd}, Dtype::bf16);
    }
    esda_decode_args a{};
    a.q = q.data;
    a.k_new = kNew.data;
    a.v_new = s.shared ? nullptr : vNew.data;
    a.k_cache = s.k->data;
    a.v_cache = s.v->data;
    a.pos = positionWord(layer, s.len, st);
    a.row_base = nullptr;
    a.out = o.data;
    a.workspace = workspace(wsBytes, st);
    a.workspace_bytes = workspace_->nbytes();
    esdaCheck(esda_decode(&d, &a, st));
    s.len += 1;
    if (maxKeep > 0 && s.len - s.start > maxKeep) s.start = s.len - maxKeep;
    return o;
}

Tensor ESKVCache::decodeRaw(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                            const std::vector<float> &invFreq, hipStream_t st, Tensor *out) {
    lastStream_ = st;
    if (stepMode_) throw std::runtime_error("ESKVCache::decodeRaw: not available in compiled-step mode (beginStep .. endStep)");
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::decodeRaw kNew");
    if (kNew.shape[1] != 1 || kNew.shape[2] != 512)
        throw std::invalid_argument("ESKVCache::decodeRaw: kNew must be [kvHeads, 1, 512]");
    if (invFreq.size() < 64)
        throw std::invalid_argument("ESKVCache::decodeRaw: invFreq needs at least 64 entries");
    const int kvH = (int) kNew.shape[0];
    Slot &s = slots_[layer];
    if (s.k && s.v)
        throw std::runtime_error("ESKVCache::decodeRaw: slot holds composite K/V content "
                                 "(post-norm) — not derivable as raw; re-prime the cache");
    if (rq8slots_[layer].q)
        throw std::runtime_error("ESKVCache::decodeRaw: slot holds q8 raw rows; use decodeRawQ8");
    if (!s.k) {
        s.k = Tensor::empty({kvH, 1, 512}, Dtype::bf16);
        s.len = 0;
        s.start = 0;
    } else {
        if (kvH != s.k->shape[0] || s.k->shape[2] != 512)
            throw std::invalid_argument("ESKVCache::decodeRaw: kv heads / head dim differ from the slot");
        growSlot(s, 1, st, false);
    }
    if (!invFreqDev_ || !std::equal(invFreqHost_.begin(), invFreqHost_.end(), invFreq.begin()) ||
        invFreqHost_.size() != 64) {
        if (invFreqDev_) hipCheck(hipStreamSynchronize(st), "ESKVCache rotary table");
        invFreqHost_.assign(invFreq.begin(), invFreq.begin() + 64);
        invFreqDev_ = Tensor::empty({64}, Dtype::f32);
        ropeTab_.reset();
        ropeRows_ = 0;
        hipCheck(hipMemcpyAsync(invFreqDev_->data, invFreqHost_.data(), 64 * sizeof(float),
                                hipMemcpyHostToDevice, st),
                 "ESKVCache rotary table upload");
        hipCheck(hipStreamSynchronize(st), "ESKVCache rotary table upload");
    }
    if (!q.defined() || q.dtype != Dtype::bf16 || !q.contiguous() || q.numel() % 512)
        throw std::invalid_argument("ESKVCache::decodeRaw: q must be contiguous bf16 [numQHeads, 512]");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != 512 || !kw.contiguous())
        throw std::invalid_argument("ESKVCache::decodeRaw: kw must be contiguous bf16 [512]");
    const int Hq = (int) (q.numel() / 512);
    const int cap = (int) s.k->shape[1];

    esda_raw_desc d{};
    d.batch = 1;
    d.num_q_heads = Hq;
    d.num_kv_heads = kvH;
    d.head_dim = 512;
    d.cap = cap;
    d.head_stride = (int64_t) cap * 512;
    d.seq_stride = (int64_t) kvH * cap * 512;
    d.max_visible = s.len + 1;
    d.split_rows = 0;
    d.scale = 1.0f;
    d.eps = eps;
    size_t wsBytes = 0;
    esdaCheck(esda_decode_raw_workspace_size(&d, &wsBytes));
    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) Hq * 512)
            throw std::invalid_argument("ESKVCache::decodeRaw: out must be contiguous bf16 [numQHeads, 512]");
        o = *out;
    } else {
        o = Tensor::empty({Hq, 512}, Dtype::bf16);
    }
    esda_raw_args a{};
    a.q = q.data;
    a.k_new = kNew.data;
    a.raw_cache = s.k->data;
    a.pos = positionWord(layer, s.len, st);
    a.kw = kw.data;
    a.inv_freq = static_cast<const float *>(invFreqDev_->data);
    a.rope_table = ropeTable(d.cap, st);
    a.rope_table_rows = ropeRows_;
    a.out = o.data;
    a.workspace = workspace(wsBytes, st);
    a.workspace_bytes = workspace_->nbytes();
    esdaCheck(esda_decode_raw(&d, &a, st));
    s.len += 1;
    return o;
}

// ------------------------------------------------------------------ q8 raw-K storage

std::array<Tensor, 3> ESKVCache::quantizeRawRows(const Tensor &kNew, hipStream_t st) {
    checkRows(kNew, "ESKVCache::quantizeRawRows kNew");
    if (kNew.shape[2] != 512) throw std::invalid_argument("esQuantizeRawRows: expects headDim 512");
    const int64_t kvH = kNew.shape[0], n = kNew.shape[1];
    // packed rows (the reference copies a transposed view packed first, ESDecodeAttn.mm:519)
    const Tensor src = kNew.contiguous() ? kNew : clone(kNew, st);
    Tensor q = Tensor::empty({kvH, n, 512}, Dtype::u8);
    Tensor sc = Tensor::empty({kvH, n, 1}, Dtype::f32);
    Tensor bs = Tensor::empty({kvH, n, 1}, Dtype::f32);
    esdaCheck(esda_quantize_raw_rows(src.data, (int32_t) kvH, (int32_t) n, q.data, n * 512,
                                     static_cast<float *>(sc.data), static_cast<float *>(bs.data), n, 0, st));
    if (!kNew.contiguous()) hipCheck(hipStreamSynchronize(st), "esQuantizeRawRows");  // src copy released
    return {q, sc, bs};
}

namespace {
// A [kvH, cap, w] tensor of `dtype`, zero-filled.
Tensor zerosOf(const std::vector<int64_t> &shape, Dtype dt, hipStream_t st) {
    Tensor t = Tensor::empty(shape, dt);
    zeroFill(t.data, t.nbytes(), st);
    return t;
}
// dst[h, 0 .. n) = src[h, 0 .. n) for every head h of [kvH, rows, w] tensors of one dtype.
void copyHeads(const Tensor &dst, const Tensor &src, int n, hipStream_t st) {
    if (n <= 0) return;
    const size_t es = dtypeSize(src.dtype), row = (size_t) src.shape[2] * es;
    hipCheck(hipMemcpy2DAsync(dst.data, (size_t) dst.strides[0] * es, src.data, (size_t) src.strides[0] * es,
                              (size_t) n * row, (size_t) src.shape[0], hipMemcpyDeviceToDevice, st),
             "ESKVCache q8 copy");
}
}  // namespace

void ESKVCache::growQ8(RQ8Slot &s, int nNew, hipStream_t st) {
    const int cap = (int) s.q->shape[1];
    if (s.len + nNew <= cap) return;
    const int newCap = roundUpChunk(s.len + nNew + kGrowChunk);
    const int64_t kvH = s.q->shape[0];
    Tensor nq = zerosOf({kvH, newCap, 512}, Dtype::u8, st);
    Tensor nsc = zerosOf({kvH, newCap, 1}, Dtype::f32, st);
    Tensor nbs = zerosOf({kvH, newCap, 1}, Dtype::f32, st);
    copyHeads(nq, *s.q, s.len, st);
    copyHeads(nsc, *s.sc, s.len, st);
    copyHeads(nbs, *s.bs, s.len, st);
    hipCheck(hipStreamSynchronize(st), "ESKVCache q8 growth");  // queued reads of the old buffers
    s.q = nq;
    s.sc = nsc;
    s.bs = nbs;
}

void ESKVCache::migrateToQ8(int layer, hipStream_t st) {
    // ESKVCache.mm:522-536: a bf16 raw slot (a restored snapshot) is quantized once into a
    // q8 slot of capacity roundUp(len + kGrowChunk) and retired.
    Slot &b = slots_[layer];
    RQ8Slot &s = rq8slots_[layer];
    if (s.q || !b.k || b.v) return;
    const int live = b.len - b.start;
    const int64_t kvH = b.k->shape[0];
    const int cap = roundUpChunk(b.len + kGrowChunk);
    Tensor q = zerosOf({kvH, cap, 512}, Dtype::u8, st);
    Tensor sc = zerosOf({kvH, cap, 1}, Dtype::f32, st);
    Tensor bs = zerosOf({kvH, cap, 1}, Dtype::f32, st);
    if (live > 0) {
        const Tensor rows = clone(liveView(*b.k, b.start, b.len), st);
        esdaCheck(esda_quantize_raw_rows(rows.data, (int32_t) kvH, live, q.data, (int64_t) cap * 512,
                                         static_cast<float *>(sc.data), static_cast<float *>(bs.data), cap, 0, st));
        hipCheck(hipStreamSynchronize(st), "ESKVCache q8 migration");
    }
    s.q = q;
    s.sc = sc;
    s.bs = bs;
    s.len = live;
    b = Slot{};
}

ESKVCache::RawQ8 ESKVCache::currentRawQ8(int layer) const {
    checkLayer(layer);
    const RQ8Slot &s = rq8slots_[layer];
    if (!s.q) throw std::runtime_error("ESKVCache::currentRawQ8: layer holds no q8 rows");
    const int pitch = (int) s.q->shape[1];
    auto view = [&](const Tensor &t) { return s.len == pitch ? t : t.slice(1, 0, s.len); };
    return {view(*s.q), view(*s.sc), view(*s.bs), *s.q, *s.sc, *s.bs, s.len, pitch};
}

ESKVCache::RawQ8 ESKVCache::updateRawQ8(int layer, const Tensor &kNew, hipStream_t st) {
    lastStream_ = st;
    // ESKVCache.mm:513-556.
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::updateRawQ8 kNew");
    if (kNew.shape[2] != 512) throw std::invalid_argument("ESKVCache::updateRawQ8: expects headDim 512");
    if (slots_[layer].k && slots_[layer].v)
        throw std::runtime_error("ESKVCache::updateRawQ8: slot holds composite K/V content "
                                 "(post-norm) — not derivable as raw; re-prime the cache");
    migrateToQ8(layer, st);
    RQ8Slot &s = rq8slots_[layer];
    const int nNew = (int) kNew.shape[1];
    const Tensor src = kNew.contiguous() ? kNew : clone(kNew, st);
    if (!s.q) {
        // first store: capacity == content, as for the reference's first q8 store
        auto qsb = quantizeRawRows(src, st);
        s.q = qsb[0];
        s.sc = qsb[1];
        s.bs = qsb[2];
        s.len = nNew;
    } else {
        if (kNew.shape[0] != s.q->shape[0])
            throw std::invalid_argument("ESKVCache::updateRawQ8: kv heads differ from the slot");
        growQ8(s, nNew, st);
        const int cap = (int) s.q->shape[1];
        esdaCheck(esda_quantize_raw_rows(src.data, (int32_t) kNew.shape[0], nNew, s.q->data, (int64_t) cap * 512,
                                         static_cast<float *>(s.sc->data), static_cast<float *>(s.bs->data), cap,
                                         s.len, st));
        s.len += nNew;
    }
    if (!kNew.contiguous()) hipCheck(hipStreamSynchronize(st), "ESKVCache::updateRawQ8");
    return currentRawQ8(layer);
}

Tensor ESKVCache::decodeRawQ8(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                              const std::vector<float> &invFreq, hipStream_t st, Tensor *out) {
    lastStream_ = st;
    if (stepMode_) throw std::runtime_error("ESKVCache::decodeRawQ8: not available in compiled-step mode (beginStep .. endStep)");
    checkLayer(layer);
    checkRows(kNew, "ESKVCache::decodeRawQ8 kNew");
    if (kNew.shape[1] != 1 || kNew.shape[2] != 512)
        throw std::invalid_argument("ESKVCache::decodeRawQ8: kNew must be [kvHeads, 1, 512]");
    if (invFreq.size() < 64)
        throw std::invalid_argument("ESKVCache::decodeRawQ8: invFreq needs at least 64 entries");
    if (slots_[layer].k && slots_[layer].v)
        throw std::runtime_error("ESKVCache::decodeRawQ8: slot holds composite K/V content "
                                 "(post-norm) — not derivable as raw; re-prime the cache");
    migrateToQ8(layer, st);
    const int kvH = (int) kNew.shape[0];
    RQ8Slot &s = rq8slots_[layer];
    if (!s.q) {
        s.q = Tensor::empty({kvH, 1, 512}, Dtype::u8);
        s.sc = Tensor::empty({kvH, 1, 1}, Dtype::f32);
        s.bs = Tensor::empty({kvH, 1, 1}, Dtype::f32);
        s.len = 0;
    } else {
        if (kvH != s.q->shape[0]) throw std::invalid_argument("ESKVCache::decodeRawQ8: kv heads differ from the slot");
        growQ8(s, 1, st);
    }
    if (!invFreqDev_ || !std::equal(invFreqHost_.begin(), invFreqHost_.end(), invFreq.begin()) ||
        invFreqHost_.size() != 64) {
        if (invFreqDev_) hipCheck(hipStreamSynchronize(st), "ESKVCache rotary table");
        invFreqHost_.assign(invFreq.begin(), invFreq.begin() + 64);
        invFreqDev_ = Tensor::empty({64}, Dtype::f32);
        ropeTab_.reset();
        ropeRows_ = 0;
        hipCheck(hipMemcpyAsync(invFreqDev_->data, invFreqHost_.data(), 64 * sizeof(float),
                                hipMemcpyHostToDevice, st),
                 "ESKVCache rotary table upload");
        hipCheck(hipStreamSynchronize(st), "ESKVCache rotary table upload");
    }
    if (!q.defined() || q.dtype != Dtype::bf16 || !q.contiguous() || q.numel() % 512)
        throw std::invalid_argument("ESKVCache::decodeRawQ8: q must be contiguous bf16 [numQHeads, 512]");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != 512 || !kw.contiguous())
        throw std::invalid_argument("ESKVCache::decodeRawQ8: kw must be contiguous bf16 [512]");
    const int Hq = (int) (q.numel() / 512);
    const int cap = (int) s.q->shape[1];
    esda_raw_desc d{};
    d.batch = 1;
    d.num_q_heads = Hq;
    d.num_kv_heads = kvH;
    d.head_dim = 512;
    d.cap = cap;
    d.head_stride = (int64_t) cap * 512;
    d.seq_stride = (int64_t) kvH * cap * 512;
    d.max_visible = s.len + 1;
    d.split_rows = 0;
    d.scale = 1.0f;
    d.eps = eps;
    size_t wsBytes = 0;
    esdaCheck(esda_decode_raw_workspace_size(&d, &wsBytes));
    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) Hq * 512)
            throw std::invalid_argument("ESKVCache::decodeRawQ8: out must be contiguous bf16 [numQHeads, 512]");
        o = *out;
    } else {
        o = Tensor::empty({Hq, 512}, Dtype::bf16);
    }
    esda_raw_q8_args a{};
    a.q = q.data;
    a.k_new = kNew.data;
    a.q8_cache = s.q->data;
    a.scale = static_cast<float *>(s.sc->data);
    a.bias = static_cast<float *>(s.bs->data);
    a.sb_head_stride = cap;
    a.sb_seq_stride = (int64_t) kvH * cap;
    a.pos = positionWord(layer, s.len, st);
    a.kw = kw.data;
    a.inv_freq = static_cast<const float *>(invFreqDev_->data);
    a.rope_table = ropeTable(d.cap, st);
    a.rope_table_rows = ropeRows_;
    a.out = o.data;
    a.workspace = workspace(wsBytes, st);
    a.workspace_bytes = workspace_->nbytes();
    esdaCheck(esda_decode_raw_q8(&d, &a, st));
    s.len += 1;
    return o;
}

void ESKVCache::reset() {
    for (auto &a : k_) a.reset();
    for (auto &a : v_) a.reset();
    for (auto &s : slots_) s = Slot{};
    for (auto &s : rq8slots_) s = RQ8Slot{};
    markers_.clear();
    rewindMark_.reset();
    seqLen_ = 0;
}

}  // namespace es
