/*
 * oracle.h -- CPU restatement of Apertura's decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline.  The product (apertura_amd/, libesda.so) never
 * links, loads or calls it.
 *
 * What each function restates (paths relative to the Apertura tree):
 *   orc_visible          ESGemma4TextModel.mm:68-83 (buildMask) + ESAttention.mm:17-22
 *                        (alignMask) + ESKVCache.mm:102-109 (window eviction)
 *   orc_append           ESKVCache.mm:95-99 (prealloc slice_update at row len) and
 *                        ESKVCache.mm:458-504 (updateRaw); ring slot = pos mod cap
 *   orc_decode_f64       the closed form of ESAttention.mm:168-193 (SDPA decode):
 *                        O = softmax(scale * q K^T + M) V, GQA kv-major (ESOps.h:64-68)
 *   orc_decode_refround  ESAttention.mm:136-165 (the unfused composite), including its
 *                        bf16 rounding points (scores, scaling, probabilities, output)
 *   orc_decode_refround_grouped  the same, each K / V row read once per kv head and the
 *                        rows split over threads (the CPU baseline); pinned to
 *                        orc_decode_refround bit for bit with one split
 *   orc_decode_splitk    ESDecodeAttn.mm:17-117 attention loop (online softmax, m init
 *                        -3e38, fp32 accumulation, rows = ceil(L/S)) and the split merge
 *                        of ESDecodeAttn.mm:253-273, applied to plain bf16 K/V
 *   orc_rope_inv_freq    ESRotaryEmbedding.mm:8-23
 *   orc_rms_norm_rows    ESRMSNorm.mm:20-27 (manual f32 path)
 *   orc_quantize_rows    ESDecodeAttn.mm:491-539 (esQuantizeRawRows: per-row affine u8)
 *   orc_decode_raw_q8_f64 ESDecodeAttn.mm:275-369 (q8 rows dequantised, then as below)
 *   orc_prefill_f64      ESAttention.mm:168-193 at seq > 1 (SDPA over a prefill chunk with
 *                        the buildMask / alignMask additive mask), GQA kv-major
 *   orc_raw_prefill_kv   ESAttention.mm:306-326 (raw-K prefill: kNorm / vNorm by ops, RoPE
 *                        by ops with bf16 cos/sin and bf16 products and sum)
 *   orc_decode_raw_f64   ESDecodeAttn.mm:17-117 reconstruction (rinv, kw, p-RoPE pairs
 *                        (d, d+256) for d < 64, bf16 cos/sin, bf16 K, V = kraw*rinv)
 *                        + merge, evaluated in fp64 after the kernel's rounding points
 *
 * Parity pins (tests/test_oracle.py): every function above is checked against
 * closed forms, invariants, brute force and an independent library routine
 * (torch/transformers eager attention in fp64); see the test file's header.
 */
#ifndef APERTURA_ORACLE_H
#define APERTURA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float *x, uint16_t *out, size_t n);
void orc_bf16_to_f32_n(const uint16_t *x, float *out, size_t n);

/* Shape and cache-mode description of one decode step.
 *
 * Cache layout: element (b, kvh, row, d) of K lives at
 *   k[b*seq_stride + kvh*head_stride + row*D + d]   (row < cap)
 * and likewise V (v may equal k: attention_k_eq_v shared buffer).
 *
 * Per-sequence position pos[b] is the absolute position of the new token.
 *   linear (ring == 0): row of absolute position p is p - row_base[b]
 *   ring   (ring == 1): row of absolute position p is p mod cap (needs 0 < window <= cap)
 * Visible absolute positions: [lo, pos] with lo = max(0, pos - window + 1)
 * (window == 0: lo = 0), and in linear mode lo is clamped to row_base[b]. */
typedef struct orc_desc {
    int32_t B, Hq, Hkv, D;
    int32_t cap;
    int32_t window;
    int32_t ring;
    int64_t seq_stride;   /* elements between sequences  (>= Hkv*head_stride) */
    int64_t head_stride;  /* elements between kv heads   (>= cap*D)          */
    float scale;
} orc_desc;

/* Fill rows_out with the visible cache rows of sequence b in ascending absolute
 * position; returns the count (or -1 for an invalid description). */
int32_t orc_visible(const orc_desc *d, int32_t pos, int32_t row_base, int32_t *rows_out);

/* Copy k_new/v_new ([B, Hkv, D] bf16) into the cache rows of pos[b].  v_cache may
 * equal k_cache (then v_new is ignored).  row_base may be NULL (all zero). */
int32_t orc_append(const orc_desc *d, uint16_t *k_cache, uint16_t *v_cache,
                   const uint16_t *k_new, const uint16_t *v_new,
                   const int32_t *pos, const int32_t *row_base);

/* Exact attention in fp64 over the visible rows (caches already hold the new row).
 * q: [B, Hq, D] bf16; out: [B, Hq, D] fp64. */
int32_t orc_decode_f64(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                       double *out, int32_t nthreads);

/* Reference-rounding mode; out: [B, Hq, D] bf16. */
int32_t orc_decode_refround(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, const int32_t *pos,
                            const int32_t *row_base, uint16_t *out, int32_t nthreads);

/* orc_decode_refround with the query heads of a kv head sharing each K / V row read and
 * the rows of a (sequence, kv head) in nsplit splits over threads (0: as many as the
 * threads need); bit-identical to orc_decode_refround with one split, otherwise up to the
 * order in which split partial sums combine.  The CPU baseline of bench.py. */
int32_t orc_decode_refround_grouped(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                                    const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                                    int32_t nsplit, uint16_t *out, int32_t nthreads);

/* Split-K fp32 mode with nsplit splits per (sequence, kv head); out fp32. */
int32_t orc_decode_splitk(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                          const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                          int32_t nsplit, float *out, int32_t nthreads);

/* inv_freq[i] = 1 / theta^(2i/head_dim) for i < int(partial*head_dim/2), zero after;
 * length head_dim/2. */
void orc_rope_inv_freq(int32_t head_dim, float theta, float partial, float *inv_freq);

/* y = x * rsqrt(mean(x^2) + eps) [* w] per row of length n, f32 math, bf16 in/out.
 * w may be NULL (weightless). */
void orc_rms_norm_rows(const uint16_t *x, const uint16_t *w, int64_t rows, int32_t n,
                       float eps, uint16_t *y);

/* Raw-K global decode (D = 512, 8 query heads per kv head): the cache holds the
 * pre-norm kRaw rows [Hkv, pitch, 512] bf16; len rows are live.  kw: [512] bf16,
 * inv_freq: >= 64 fp32.  scale is the in-model 1.0 unless overridden.  out fp64. */
int32_t orc_decode_raw_f64(const uint16_t *q, const uint16_t *raw, int32_t Hkv, int32_t len,
                           int32_t pitch, const uint16_t *kw, float eps, const float *inv_freq,
                           float scale, double *out, int32_t nthreads);

/* Raw-K decode over a q8 raw stream: u8 rows qraw [Hkv, pitch, 512] with per-row scale and
 * bias [Hkv, pitch] f32, dequantised as float(q) * scale + bias; otherwise as
 * orc_decode_raw_f64 (esDecodeAttnGlobalQ8, ESDecodeAttn.mm:275-369, 455-489). */
int32_t orc_decode_raw_q8_f64(const uint16_t *q, const uint8_t *qraw, const float *sc, const float *bs,
                              int32_t Hkv, int32_t len, int32_t pitch, const uint16_t *kw, float eps,
                              const float *inv_freq, float scale, double *out, int32_t nthreads);

/* Per-row affine u8 quantisation of bf16 rows [rows, n] (esQuantizeRawRows,
 * ESDecodeAttn.mm:491-539): q [rows, n] u8, scale / bias [rows] f32. */
void orc_quantize_rows(const uint16_t *x, int64_t rows, int32_t n, uint8_t *q, float *scale,
                       float *bias);

/* Planted-mistake switch for the oracle's own self-tests (0 = none).  Used only by
 * tests that show a plausible mistake is caught by the pins. */
void orc_set_fault(int32_t fault);

/* Conditioning probe of orc_decode_raw_f64 / orc_decode_raw_q8_f64 (0 = off): each row's
 * rinv is moved by `ulps` fp32 ulps before K is rebuilt.  Tests use it to bound how far the
 * result moves under an ulp-level difference in the row norm. */
void orc_set_rinv_ulps(int32_t ulps);

/* Prefill attention (ESAttention.mm:168-193 at seq > 1: SDPA with the additive mask of
 * ESGemma4TextModel.mm:68-83 aligned by ESAttention.mm:17-22), fp64.
 *   q: element (h, i, d) at q[h*q_head_stride + i*q_row_stride + d], query row i < Sq at
 *      absolute position q_pos0 + i
 *   k, v: element (kvh, j, d) at k[kvh*kv_head_stride + j*D + d], key j < Sk at absolute
 *      position k_pos0 + j
 *   key j is visible to query i iff kAbs <= qAbs and (window == 0 or kAbs > qAbs - window)
 *   out: (i, h, d) at out[(i*Hq + h)*D + d]
 * Returns -1 for a query with no visible key. */
int32_t orc_prefill_f64(const uint16_t *q, int64_t q_head_stride, int64_t q_row_stride,
                        const uint16_t *k, const uint16_t *v, int64_t kv_head_stride,
                        int32_t Hq, int32_t Hkv, int32_t D, int32_t Sq, int32_t Sk,
                        int32_t q_pos0, int32_t k_pos0, int32_t window, float scale,
                        double *out, int32_t nthreads);

/* Raw-K prefill reconstruction of K and V by the reference's ops (ESAttention.mm:306-326):
 * raw, k, v [Hkv, Sk, D] bf16; key row t at absolute position pos0 + t. */
void orc_raw_prefill_kv(const uint16_t *raw, int32_t Hkv, int32_t Sk, int32_t D, const uint16_t *kw,
                        float eps, const float *inv_freq, int32_t pos0, uint16_t *k, uint16_t *v);

#ifdef __cplusplus
}
#endif
#endif
