// es_capi.cpp -- the C ABI of include/esda_cache.h over es::ESKVCache and
// es::esDecodeAttnGlobal.  Exceptions are caught here and turned into status codes.
#include <exception>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "es/ESDecodeAttn.h"
#include "es/ESKVCache.h"
#include "esda_cache.h"
#include "esda_internal.h"

struct esda_cache {
    es::ESKVCache impl;
    explicit esda_cache(int n) : impl(n) {}
};

namespace {

template <class F>
int guarded(F &&f) {
    try {
        f();
        return ESDA_OK;
    } catch (const std::invalid_argument &e) {
        esda_detail::set_error(e.what());
        return ESDA_ERR_INVALID_ARGUMENT;
    } catch (const std::exception &e) {
        esda_detail::set_error(e.what());
        return ESDA_ERR_RUNTIME;
    }
}

es::Tensor rows(const void *p, int kvH, int n, int hd) {
    if (!p) throw std::invalid_argument("null tensor pointer");
    if (kvH <= 0 || n <= 0 || hd <= 0) throw std::invalid_argument("tensor sizes must be positive");
    return es::Tensor::wrap(const_cast<void *>(p), {kvH, n, hd}, es::Dtype::bf16);
}

void toView(const es::Tensor &t, esda_view *v) {
    if (!v) return;
    v->data = t.data;
    v->kv_heads = (int32_t) t.shape[0];
    v->rows = (int32_t) t.shape[1];
    v->head_dim = (int32_t) t.shape[2];
    v->head_stride = t.strides[0];
}

void needCache(const esda_cache *c) {
    if (!c) throw std::invalid_argument("null cache handle");
}

hipStream_t asStream(void *s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int esda_cache_create(int32_t num_layers, esda_cache **out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("esda_cache_create: null output");
        *out = new esda_cache(num_layers);
    });
}

void esda_cache_destroy(esda_cache *cache) { delete cache; }

int esda_cache_update(esda_cache *cache, int32_t layer, const void *k_new, const void *v_new, int32_t kv_heads,
                      int32_t n_new, int32_t head_dim, int32_t max_keep, int32_t prealloc, void *stream,
                      esda_view *k_out, esda_view *v_out) {
    return guarded([&] {
        needCache(cache);
        auto kv = cache->impl.update(layer, rows(k_new, kv_heads, n_new, head_dim),
                                     rows(v_new, kv_heads, n_new, head_dim), max_keep, prealloc != 0,
                                     asStream(stream));
        toView(kv.first, k_out);
        toView(kv.second, v_out);
    });
}

int esda_cache_update_raw(esda_cache *cache, int32_t layer, const void *k_new, int32_t kv_heads, int32_t n_new,
                          int32_t head_dim, int32_t prealloc, void *stream, esda_view *view, int32_t *len,
                          int32_t *pitch) {
    return guarded([&] {
        needCache(cache);
        auto r = cache->impl.updateRaw(layer, rows(k_new, kv_heads, n_new, head_dim), prealloc != 0,
                                       asStream(stream));
        toView(r.view, view);
        if (len) *len = r.len;
        if (pitch) *pitch = r.pitch;
    });
}

int esda_cache_current_raw(esda_cache *cache, int32_t layer, esda_view *view, int32_t *len, int32_t *pitch) {
    return guarded([&] {
        needCache(cache);
        auto r = cache->impl.currentRaw(layer);
        toView(r.view, view);
        if (len) *len = r.len;
        if (pitch) *pitch = r.pitch;
    });
}

int esda_cache_current(esda_cache *cache, int32_t layer, int32_t prealloc, esda_view *k_out, esda_view *v_out) {
    return guarded([&] {
        needCache(cache);
        auto kv = cache->impl.current(layer, prealloc != 0);
        toView(kv.first, k_out);
        toView(kv.second, v_out);
    });
}

int esda_cache_begin_step(esda_cache *cache, const int32_t *global_idx, const int32_t *sliding_idx) {
    return guarded([&] {
        needCache(cache);
        if (!global_idx || !sliding_idx) throw std::invalid_argument("esda_cache_begin_step: null index");
        cache->impl.beginStep(es::Tensor::wrap(const_cast<int32_t *>(global_idx), {1}, es::Dtype::i32),
                              es::Tensor::wrap(const_cast<int32_t *>(sliding_idx), {1}, es::Dtype::i32));
    });
}

int esda_cache_end_step(esda_cache *cache) {
    return guarded([&] {
        needCache(cache);
        cache->impl.endStep();
    });
}

int esda_cache_set_slot(esda_cache *cache, int32_t layer, void *k, void *v, int32_t kv_heads, int32_t cap,
                        int32_t head_dim) {
    return guarded([&] {
        needCache(cache);
        cache->impl.setSlot(layer, rows(k, kv_heads, cap, head_dim), rows(v, kv_heads, cap, head_dim));
    });
}

int esda_cache_slot_kv(esda_cache *cache, int32_t layer, esda_view *k_out, esda_view *v_out) {
    return guarded([&] {
        needCache(cache);
        toView(cache->impl.slotK(layer), k_out);
        toView(cache->impl.slotV(layer), v_out);
    });
}

int esda_cache_take_slot(esda_cache *cache, int32_t layer, esda_view *k_out, esda_view *v_out) {
    return guarded([&] {
        needCache(cache);
        // both present before either is taken, so a failure leaves the slot as it was
        (void) cache->impl.slotK(layer);
        (void) cache->impl.slotV(layer);
        toView(cache->impl.takeSlotK(layer), k_out);
        toView(cache->impl.takeSlotV(layer), v_out);
    });
}

int esda_cache_decode(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, const void *k_new,
                      const void *v_new, int32_t kv_heads, int32_t head_dim, int32_t max_keep, int32_t window,
                      float scale, void *out, void *stream) {
    return guarded([&] {
        needCache(cache);
        if (!q || !out || num_q_heads <= 0) throw std::invalid_argument("esda_cache_decode: null q / out");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, head_dim}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {num_q_heads, head_dim}, es::Dtype::bf16);
        cache->impl.decode(layer, qt, rows(k_new, kv_heads, 1, head_dim), rows(v_new, kv_heads, 1, head_dim),
                           max_keep, window, scale, asStream(stream), &ot);
    });
}

int esda_cache_decode_raw(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, const void *k_new,
                          int32_t kv_heads, const void *kw, float eps, const float *inv_freq, int32_t n_freq,
                          void *out, void *stream) {
    return guarded([&] {
        needCache(cache);
        if (!q || !out || !kw || !inv_freq || num_q_heads <= 0 || n_freq < 0)
            throw std::invalid_argument("esda_cache_decode_raw: null pointer");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor kwt = es::Tensor::wrap(const_cast<void *>(kw), {512}, es::Dtype::bf16);
        std::vector<float> f(inv_freq, inv_freq + n_freq);
        cache->impl.decodeRaw(layer, qt, rows(k_new, kv_heads, 1, 512), kwt, eps, f, asStream(stream), &ot);
    });
}

namespace {
void toQ8View(const es::ESKVCache::RawQ8 &r, esda_q8_view *v) {
    if (!v) return;
    v->q = r.qbuf.data;
    v->scale = static_cast<float *>(r.scbuf.data);
    v->bias = static_cast<float *>(r.bsbuf.data);
    v->kv_heads = (int32_t) r.qbuf.shape[0];
    v->len = r.len;
    v->pitch = r.pitch;
}
}  // namespace

int esda_cache_update_raw_q8(esda_cache *cache, int32_t layer, const void *k_new, int32_t kv_heads, int32_t n_new,
                             void *stream, esda_q8_view *view) {
    return guarded([&] {
        needCache(cache);
        toQ8View(cache->impl.updateRawQ8(layer, rows(k_new, kv_heads, n_new, 512), asStream(stream)), view);
    });
}

int esda_cache_current_raw_q8(esda_cache *cache, int32_t layer, esda_q8_view *view) {
    return guarded([&] {
        needCache(cache);
        toQ8View(cache->impl.currentRawQ8(layer), view);
    });
}

int esda_cache_decode_raw_q8(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads,
                             const void *k_new, int32_t kv_heads, const void *kw, float eps, const float *inv_freq,
                             int32_t n_freq, void *out, void *stream) {
    return guarded([&] {
        needCache(cache);
        if (!q || !out || !kw || !inv_freq || num_q_heads <= 0 || n_freq < 0)
            throw std::invalid_argument("esda_cache_decode_raw_q8: null pointer");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor kwt = es::Tensor::wrap(const_cast<void *>(kw), {512}, es::Dtype::bf16);
        std::vector<float> f(inv_freq, inv_freq + n_freq);
        cache->impl.decodeRawQ8(layer, qt, rows(k_new, kv_heads, 1, 512), kwt, eps, f, asStream(stream), &ot);
    });
}

int esda_cache_prefill(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, int32_t seq,
                       const void *k_new, const void *v_new, int32_t kv_heads, int32_t head_dim, int32_t max_keep,
                       int32_t window, float scale, int32_t past_len, int32_t prealloc, void *out, void *stream) {
    return guarded([&] {
        needCache(cache);
        if (!q || !out || num_q_heads <= 0 || seq <= 0 || head_dim <= 0)
            throw std::invalid_argument("esda_cache_prefill: null q / out or empty shape");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, seq, head_dim}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {seq, (int64_t) num_q_heads * head_dim}, es::Dtype::bf16);
        cache->impl.prefill(layer, qt, rows(k_new, kv_heads, seq, head_dim), rows(v_new, kv_heads, seq, head_dim),
                            max_keep, window, scale, past_len, prealloc != 0, asStream(stream), &ot);
    });
}

int esda_cache_prefill_raw(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, int32_t seq,
                           const void *k_new, int32_t kv_heads, const void *kw, float eps, const float *inv_freq,
                           int32_t n_freq, int32_t past_len, float scale, int32_t q8, void *out, void *stream) {
    return guarded([&] {
        needCache(cache);
        if (!q || !out || !kw || !inv_freq || num_q_heads <= 0 || seq <= 0 || n_freq < 0)
            throw std::invalid_argument("esda_cache_prefill_raw: null pointer or empty shape");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, seq, 512}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {seq, (int64_t) num_q_heads * 512}, es::Dtype::bf16);
        es::Tensor kwt = es::Tensor::wrap(const_cast<void *>(kw), {512}, es::Dtype::bf16);
        std::vector<float> f(inv_freq, inv_freq + n_freq);
        cache->impl.prefillRaw(layer, qt, rows(k_new, kv_heads, seq, 512), kwt, eps, f, past_len, scale, q8 != 0,
                               asStream(stream), &ot);
    });
}

int esda_cache_slot(esda_cache *cache, int32_t layer, int32_t *len, int32_t *start, int32_t *capacity,
                    int32_t *flags) {
    return guarded([&] {
        needCache(cache);
        if (len) *len = cache->impl.slotLen(layer);
        if (start) *start = cache->impl.slotStart(layer);
        if (capacity) *capacity = cache->impl.slotCapacity(layer);
        if (flags) {
            int f = 0;
            if (cache->impl.slotLost(layer)) f |= 1;
            if (cache->impl.slotShared(layer)) f |= 2;
            if (cache->impl.slotRaw(layer)) f |= 4;
            if (cache->impl.slotQ8(layer)) f |= 8;
            *flags = f;
        }
    });
}

int esda_cache_seq_len(const esda_cache *cache) { return cache ? cache->impl.seqLen() : -1; }

void esda_cache_mark_step(esda_cache *cache, int32_t n_new) {
    if (cache) cache->impl.markStep(n_new);
}

void esda_cache_reset(esda_cache *cache) {
    if (cache) cache->impl.reset();
}

int esda_cache_save_snapshot(const esda_cache *cache, const char *path, const char *fingerprint, int32_t pos) {
    if (!cache || !path || !fingerprint) return 0;
    return cache->impl.saveSnapshot(path, fingerprint, pos) ? 1 : 0;
}

int esda_cache_restore_snapshot(esda_cache *cache, const char *path, const char *fingerprint) {
    if (!cache || !path || !fingerprint) return -1;
    return cache->impl.restoreSnapshot(path, fingerprint);
}

int esda_cache_restore_snapshot_ex(esda_cache *cache, const char *path, const char *fingerprint, int32_t mode,
                                   esda_prefix_fp_fn prefix_fp, void *user) {
    if (!cache || !path || !fingerprint || mode < 0 || mode > 3) return -1;
    std::function<std::string(int)> fn;
    if (prefix_fp)
        fn = [prefix_fp, user](int pos) {
            const char *s = prefix_fp(pos, user);
            return std::string(s ? s : "");
        };
    return cache->impl.restoreSnapshot(path, fingerprint, static_cast<es::ESKVCache::RawMode>(mode), fn);
}

int esda_cache_mark_prefix(esda_cache *cache, int32_t pos, const char *fingerprint) {
    return guarded([&] {
        if (!cache || !fingerprint) throw std::invalid_argument("esda_cache_mark_prefix: null pointer");
        cache->impl.markPrefix(pos, fingerprint);
    });
}

void esda_cache_clear_rewind_mark(esda_cache *cache) {
    if (cache) cache->impl.clearRewindMark();
}

int esda_cache_mark_rewind_point(esda_cache *cache, int32_t pos) {
    return cache && cache->impl.markRewindPoint(pos) ? 1 : 0;
}

int esda_cache_rewind_to_mark(esda_cache *cache) { return cache ? cache->impl.rewindToMark() : -1; }

int esda_decode_attn_global(const void *q, int32_t num_q_heads, const void *raw_buf, int32_t num_kv_heads,
                            int32_t len, int32_t pitch, const void *kw, float eps, const float *inv_freq,
                            int32_t n_freq, void *out, void *stream) {
    return guarded([&] {
        if (!q || !raw_buf || !kw || !inv_freq || !out || n_freq < 0)
            throw std::invalid_argument("esda_decode_attn_global: null pointer");
        if (num_q_heads <= 0 || num_kv_heads <= 0 || pitch <= 0)
            throw std::invalid_argument("esda_decode_attn_global: sizes must be positive");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor rb = es::Tensor::wrap(const_cast<void *>(raw_buf), {num_kv_heads, pitch, 512}, es::Dtype::bf16);
        es::Tensor kwt = es::Tensor::wrap(const_cast<void *>(kw), {512}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {num_q_heads, 512}, es::Dtype::bf16);
        std::vector<float> f(inv_freq, inv_freq + n_freq);
        es::esDecodeAttnGlobal(qt, rb, len, pitch, kwt, eps, f, asStream(stream), &ot);
    });
}

int esda_decode_attn_global_q8(const void *q, int32_t num_q_heads, const void *q8_buf, const float *scale_buf,
                               const float *bias_buf, int32_t num_kv_heads, int32_t len, int32_t pitch,
                               const void *kw, float eps, const float *inv_freq, int32_t n_freq, void *out,
                               void *stream) {
    return guarded([&] {
        if (!q || !q8_buf || !scale_buf || !bias_buf || !kw || !inv_freq || !out || n_freq < 0)
            throw std::invalid_argument("esda_decode_attn_global_q8: null pointer");
        if (num_q_heads <= 0 || num_kv_heads <= 0 || pitch <= 0)
            throw std::invalid_argument("esda_decode_attn_global_q8: sizes must be positive");
        es::Tensor qt = es::Tensor::wrap(const_cast<void *>(q), {num_q_heads, 512}, es::Dtype::bf16);
        es::Tensor qb = es::Tensor::wrap(const_cast<void *>(q8_buf), {num_kv_heads, pitch, 512}, es::Dtype::u8);
        es::Tensor sb = es::Tensor::wrap(const_cast<float *>(scale_buf), {num_kv_heads, pitch, 1}, es::Dtype::f32);
        es::Tensor bb = es::Tensor::wrap(const_cast<float *>(bias_buf), {num_kv_heads, pitch, 1}, es::Dtype::f32);
        es::Tensor kwt = es::Tensor::wrap(const_cast<void *>(kw), {512}, es::Dtype::bf16);
        es::Tensor ot = es::Tensor::wrap(out, {num_q_heads, 512}, es::Dtype::bf16);
        std::vector<float> f(inv_freq, inv_freq + n_freq);
        es::esDecodeAttnGlobalQ8(qt, qb, sb, bb, len, pitch, kwt, eps, f, asStream(stream), &ot);
    });
}

}  // extern "C"
