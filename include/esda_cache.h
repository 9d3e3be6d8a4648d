/*
 * esda_cache.h -- C ABI over the ES* C++ layer of libesda.so (headers under include/es): the
 * reference's ESKVCache and esDecodeAttnGlobal behind an opaque handle, for FFI
 * callers (ctypes, cgo, JNI) that cannot use the C++ classes.
 *
 * Every function returns ESDA_OK or an error code from esda.h; C++ exceptions never
 * cross this boundary: std::invalid_argument becomes ESDA_ERR_INVALID_ARGUMENT and
 * std::runtime_error ESDA_ERR_RUNTIME, with the message in esda_last_error().
 * Row tensors are [kv_heads, n, head_dim] bf16 device memory with contiguous rows.
 *
 * Reference interfaces (Apertura tree):
 *   esda_cache_create / destroy    ESKVCache(int numLayers)            ESKVCache.h:46
 *   esda_cache_update              ESKVCache::update                   ESKVCache.h:57-58, ESKVCache.mm:19-110
 *   esda_cache_update_raw          ESKVCache::updateRaw                ESKVCache.h:78-79, ESKVCache.mm:458-504
 *   esda_cache_current             ESKVCache::current                  ESKVCache.h:117, ESKVCache.mm:112-119
 *   esda_cache_decode              ESKVCache::update + SDPA decode     ESAttention.mm:105, :188
 *   esda_cache_begin_step .. take_slot  compiled-step members          ESKVCache.h:93-112
 *   esda_cache_decode_raw          updateRaw + esDecodeAttnGlobal      ESAttention.mm:291-300
 *   esda_cache_update_raw_q8       ESKVCache::updateRawQ8              ESKVCache.h:81-88, ESKVCache.mm:513-556
 *   esda_cache_decode_raw_q8       updateRawQ8 + esDecodeAttnGlobalQ8  ESAttention.mm:270-277
 *   esda_cache_current_raw_q8      a q8 slot's RawQ8 record without appending (no counterpart)
 *   esda_cache_seq_len / mark_step ESKVCache::seqLen / markStep        ESKVCache.h:176-177
 *   esda_cache_reset               ESKVCache::reset                    ESKVCache.h:178, ESKVCache.mm:622-638
 *   esda_cache_save_snapshot       ESKVCache::saveSnapshot             ESKVCache.h:129, ESKVCache.mm:224-278
 *   esda_cache_restore_snapshot(_ex) ESKVCache::restoreSnapshot        ESKVCache.h:138-146, ESKVCache.mm:280-456
 *   esda_cache_mark_prefix         ESKVCache::markPrefix               ESKVCache.h:127, ESKVCache.mm:121-146
 *   esda_cache_mark_rewind_point, rewind_to_mark, clear_rewind_mark:
 *                                  ESKVCache::markRewindPoint / rewindToMark / clearRewindMark
 *                                  ESKVCache.h:160-163, ESKVCache.mm:148-222
 *   esda_cache_slot                slot bookkeeping (len, start, capacity) for callers
 *                                  and tests; the reference keeps it private (ESKVCache.h:183-192)
 *   esda_decode_attn_global        esDecodeAttnGlobal                  ESDecodeAttn.h:27-28
 *   esda_decode_attn_global_q8     esDecodeAttnGlobalQ8                ESDecodeAttn.h:30-36
 *   esda_cache_prefill             update + SDPA at seq > 1            ESAttention.mm:77-108, :168-193
 *   esda_cache_prefill_raw         updateRaw(Q8) + the raw-K prefill   ESAttention.mm:253-332
 */
#ifndef APERTURA_ESDA_CACHE_H
#define APERTURA_ESDA_CACHE_H

#include <stddef.h>
#include <stdint.h>

#include "esda.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct esda_cache esda_cache; /* opaque: one ESKVCache */

/* A non-owning view of cached rows: element (h, r, d) at data[h*head_stride + r*head_dim + d]. */
typedef struct esda_view {
    void *data;
    int32_t kv_heads;
    int32_t rows;
    int32_t head_dim;
    int64_t head_stride; /* elements */
} esda_view;

int esda_cache_create(int32_t num_layers, esda_cache **out);
void esda_cache_destroy(esda_cache *cache);

/* prealloc: 0 = legacy concat mode, 1 = preallocated chunk-grown mode. */
int esda_cache_update(esda_cache *cache, int32_t layer, const void *k_new, const void *v_new,
                      int32_t kv_heads, int32_t n_new, int32_t head_dim, int32_t max_keep,
                      int32_t prealloc, void *stream, esda_view *k_out, esda_view *v_out);

int esda_cache_update_raw(esda_cache *cache, int32_t layer, const void *k_new, int32_t kv_heads,
                          int32_t n_new, int32_t head_dim, int32_t prealloc, void *stream,
                          esda_view *view, int32_t *len, int32_t *pitch);

int esda_cache_current(esda_cache *cache, int32_t layer, int32_t prealloc, esda_view *k_out,
                       esda_view *v_out);

/* Compiled-step mode (ESKVCache::beginStep / endStep / setSlot / slotK / slotV / takeSlotK /
 * takeSlotV, ESKVCache.h:93-112; driven by ESGenerationLoop.mm:122-238).  Between begin and
 * end, esda_cache_update writes its one new row at the cache row held in the device int32
 * word global_idx (max_keep == 0) or sliding_idx (max_keep > 0) and returns the whole slot
 * buffers.  set_slot installs caller-owned [kv_heads, cap, head_dim] bf16 buffers (v == k:
 * one shared K=V buffer), which must outlive their use; slot_kv views them; take_slot views
 * and then empties the slot. */
int esda_cache_begin_step(esda_cache *cache, const int32_t *global_idx, const int32_t *sliding_idx);
int esda_cache_end_step(esda_cache *cache);
int esda_cache_set_slot(esda_cache *cache, int32_t layer, void *k, void *v, int32_t kv_heads, int32_t cap,
                        int32_t head_dim);
int esda_cache_slot_kv(esda_cache *cache, int32_t layer, esda_view *k_out, esda_view *v_out);
int esda_cache_take_slot(esda_cache *cache, int32_t layer, esda_view *k_out, esda_view *v_out);
/* A prealloc raw-K slot's live rows without appending: no counterpart in the reference,
 * whose callers see the raw view only from updateRaw; for callers and tests that inspect
 * a raw slot (e.g. after a snapshot restore or a rewind). */
int esda_cache_current_raw(esda_cache *cache, int32_t layer, esda_view *view, int32_t *len,
                           int32_t *pitch);

/* Fused decode step: append one row (v_new == k_new: one shared K=V buffer) and attend.
 * max_keep evicts as update() does; window > 0 masks all but the last `window` positions
 * (the sliding layer's mask, applied even when max_keep is 0).
 * q: [num_q_heads, head_dim] bf16; out: [num_q_heads, head_dim] bf16. */
int esda_cache_decode(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads,
                      const void *k_new, const void *v_new, int32_t kv_heads, int32_t head_dim,
                      int32_t max_keep, int32_t window, float scale, void *out, void *stream);

/* Fused raw-K decode step (head_dim 512): append one raw row and attend.  inv_freq is a
 * host array of n_freq >= 64 floats (the first 64 are used). */
int esda_cache_decode_raw(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads,
                          const void *k_new, int32_t kv_heads, const void *kw, float eps,
                          const float *inv_freq, int32_t n_freq, void *out, void *stream);

/* A q8 raw slot (ESKVCache::RawQ8): u8 rows q [kv_heads, pitch, 512] and f32 scale / bias
 * [kv_heads, pitch] (element (h, r) at h*pitch + r); rows 0 .. len-1 are live and each
 * dequantizes to x = float(q) * scale + bias.  Non-owning: valid until the slot grows. */
typedef struct esda_q8_view {
    void *q;
    float *scale;
    float *bias;
    int32_t kv_heads;
    int32_t len;
    int32_t pitch;
} esda_q8_view;

/* Quantize n_new bf16 raw rows k_new [kv_heads, n_new, 512] and append them to the layer's
 * q8 slot (a bf16 raw slot migrates first: its live rows are quantized once and retired). */
int esda_cache_update_raw_q8(esda_cache *cache, int32_t layer, const void *k_new, int32_t kv_heads,
                             int32_t n_new, void *stream, esda_q8_view *view);
int esda_cache_current_raw_q8(esda_cache *cache, int32_t layer, esda_q8_view *view);
/* Fused q8 decode step: the new raw row is quantized in the kernel into row len of the slot,
 * then rows 0 .. len are attended.  Arguments as esda_cache_decode_raw. */
int esda_cache_decode_raw_q8(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads,
                             const void *k_new, int32_t kv_heads, const void *kw, float eps,
                             const float *inv_freq, int32_t n_freq, void *out, void *stream);

/* Prefill chunk: append seq rows k_new / v_new [kv_heads, seq, head_dim] (v_new == k_new:
 * one shared K=V buffer; max_keep as esda_cache_update) and attend q [num_q_heads, seq,
 * head_dim] over the live rows with the reference's mask: past_len positions cached before
 * the chunk, window 0 (global) or the sliding window.  out [seq, num_q_heads * head_dim].
 * prealloc as esda_cache_update. */
int esda_cache_prefill(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, int32_t seq,
                       const void *k_new, const void *v_new, int32_t kv_heads, int32_t head_dim,
                       int32_t max_keep, int32_t window, float scale, int32_t past_len, int32_t prealloc,
                       void *out, void *stream);
/* Raw-K prefill chunk (head_dim 512): append the chunk's raw rows (q8 != 0: into the q8
 * stream) and attend over the whole stream, K / V rebuilt by the reference's prefill ops.
 * inv_freq: host array of n_freq floats (zero-extended to 256). */
int esda_cache_prefill_raw(esda_cache *cache, int32_t layer, const void *q, int32_t num_q_heads, int32_t seq,
                           const void *k_new, int32_t kv_heads, const void *kw, float eps, const float *inv_freq,
                           int32_t n_freq, int32_t past_len, float scale, int32_t q8, void *out, void *stream);

/* flags: bit 0 = rows before start were discarded by a compaction, bit 1 = shared K=V
 * buffer, bit 2 = raw-K content, bit 3 = q8 raw-K content (len and capacity are then the
 * q8 slot's). */
int esda_cache_slot(esda_cache *cache, int32_t layer, int32_t *len, int32_t *start,
                    int32_t *capacity, int32_t *flags);

int esda_cache_seq_len(const esda_cache *cache);
void esda_cache_mark_step(esda_cache *cache, int32_t n_new);
void esda_cache_reset(esda_cache *cache);

/* Snapshots (safetensors, the reference's layout): save returns 1 on success, 0 when a
 * layer is unprimed or the file cannot be written.  Restore returns the restored position,
 * or -1 with the cache untouched (missing / malformed file, layer-count or fingerprint
 * mismatch without a usable marker, storage-mode mismatch). */
int esda_cache_save_snapshot(const esda_cache *cache, const char *path, const char *fingerprint,
                             int32_t pos);
int esda_cache_restore_snapshot(esda_cache *cache, const char *path, const char *fingerprint);
/* The caller's prompt-prefix fingerprint at a marker position ("" or NULL: none). */
typedef const char *(*esda_prefix_fp_fn)(int32_t pos, void *user);
/* mode: 0 composite, 1 raw (q8 layers dequantize to bf16), 2 raw q8 (bf16 raw layers
 * quantize), 3 as stored (ESKVCache::RawMode); prefix_fp may be NULL. */
int esda_cache_restore_snapshot_ex(esda_cache *cache, const char *path, const char *fingerprint,
                                   int32_t mode, esda_prefix_fp_fn prefix_fp, void *user);
/* Marks position pos (>= 4096, else ESDA_ERR_INVALID_ARGUMENT) for the next snapshot. */
int esda_cache_mark_prefix(esda_cache *cache, int32_t pos, const char *fingerprint);
/* One in-memory rewind mark: 1 / 0; rewind returns the position or -1. */
int esda_cache_mark_rewind_point(esda_cache *cache, int32_t pos);
int esda_cache_rewind_to_mark(esda_cache *cache);
void esda_cache_clear_rewind_mark(esda_cache *cache);

/* esDecodeAttnGlobal: q [num_q_heads, 512], raw_buf the unsliced [num_kv_heads, pitch,
 * 512] buffer, rows 0 .. len-1 attended (already appended); out [num_q_heads, 512]. */
int esda_decode_attn_global(const void *q, int32_t num_q_heads, const void *raw_buf,
                            int32_t num_kv_heads, int32_t len, int32_t pitch, const void *kw,
                            float eps, const float *inv_freq, int32_t n_freq, void *out,
                            void *stream);

/* esDecodeAttnGlobalQ8: as esda_decode_attn_global over a q8 raw stream, q8_buf the
 * unsliced u8 [num_kv_heads, pitch, 512] buffer and scale_buf / bias_buf its f32
 * [num_kv_heads, pitch] per-row scale and bias. */
int esda_decode_attn_global_q8(const void *q, int32_t num_q_heads, const void *q8_buf,
                               const float *scale_buf, const float *bias_buf, int32_t num_kv_heads,
                               int32_t len, int32_t pitch, const void *kw, float eps,
                               const float *inv_freq, int32_t n_freq, void *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
