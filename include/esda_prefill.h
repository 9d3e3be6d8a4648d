/*
 * esda_prefill.h -- C ABI of libesda.so's prefill side (MI355X, gfx950): attention of a
 * chunk of new tokens over the cache, and the raw-K stream's K / V reconstruction that
 * feeds it.  Conventions as in esda.h (plain pointers, caller-owned device memory,
 * explicit HIP stream, ESDA_OK or an error code with esda_last_error()).
 *
 * Which reference interface each entry point replaces (paths in the Apertura tree):
 *   esda_prefill            mx::fast::scaled_dot_product_attention(Q, K, V, scale, "", M) at
 *                           ESAttention.mm:188 (seq > 1) and :328 (raw-K prefill), with M
 *                           the additive mask of ESGemma4TextModel.mm:68-83 (buildMask)
 *                           aligned to the retained keys by ESAttention.mm:17-22
 *                           (alignMask); also the op-level tiled core of
 *                           ESAttention.mm:195-251 (same mathematics).  GQA kv-major
 *                           (ESOps.h:64-68).
 *   esda_raw_prefill_kv     the raw-K prefill reconstruction ESAttention.mm:306-326: K =
 *                           kNorm(raw) roped by ops at positions pos0 .. , V = vNorm(raw).
 *   esda_raw_q8_prefill_kv  the same over a q8 raw stream, rows first dequantised to
 *                           bf16(float(q) * scale + bias) (ESAttention.mm:279-281).
 */
#ifndef APERTURA_ESDA_PREFILL_H
#define APERTURA_ESDA_PREFILL_H

#include <stddef.h>
#include <stdint.h>

#include "esda.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One prefill attention call.
 *
 * q:   element (h, i, d) at q[h*q_head_stride + i*q_row_stride + d], query row i < seq_q
 *      at absolute position q_pos0 + i (the reference's pastLen + i).
 * k/v: element (kvh, j, d) at k[kvh*kv_head_stride + j*head_dim + d], key j < seq_k at
 *      absolute position k_pos0 + j (a cache view: rows dense, head stride free; with
 *      sliding eviction k_pos0 = pastLen + seq_q - seq_k, as alignMask keeps the last
 *      seq_k columns).  k == v is allowed (attention_k_eq_v): at head_dim 512 the call
 *      then streams the one buffer once and reads V from it.
 * out: element (i, h, d) at out[i*out_row_stride + h*out_head_stride + d] (bf16); the
 *      reference's [seq, numQ * headDim] is out_row_stride = numQ*headDim,
 *      out_head_stride = headDim.
 * Key j is visible to query i iff kAbs <= qAbs and (window == 0 or kAbs > qAbs - window).
 * Every query must see at least its own position: k_pos0 <= q_pos0 and
 * k_pos0 + seq_k >= q_pos0 + seq_q.
 * head_dim 128, 256 or 512; strides multiples of 8 elements; pointers 16-byte aligned. */
typedef struct esda_prefill_desc {
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t seq_q;
    int32_t seq_k;
    int32_t q_pos0;
    int32_t k_pos0;
    int32_t window;      /* 0: causal; > 0: sliding window */
    int64_t q_head_stride, q_row_stride;
    int64_t kv_head_stride;
    int64_t out_row_stride, out_head_stride;
    int32_t split_keys;  /* 0: automatic; else keys per split (a multiple of 32) */
    float scale;
} esda_prefill_desc;

typedef struct esda_prefill_args {
    const void *q, *k, *v;
    void *out;
    void *workspace;     /* split partials; esda_prefill_workspace_size bytes (may be 0) */
    size_t workspace_bytes;
} esda_prefill_args;

int esda_prefill_workspace_size(const esda_prefill_desc *desc, size_t *bytes);
int esda_prefill(const esda_prefill_desc *desc, const esda_prefill_args *args, void *stream);
/* esda_prefill's launches one at a time (for timing): stages bit 0 = the attention kernel,
 * bit 1 = the split merge (launched only when the plan splits the keys). */
int esda_prefill_stages(const esda_prefill_desc *desc, const esda_prefill_args *args, int stages,
                        void *stream);

/* Raw-K prefill reconstruction (ESAttention.mm:306-326), for kv head h and key row t at
 * absolute position pos0 + t:
 *   rinv = 1 / sqrt(mean(x^2) + eps); K0 = bf16(x * rinv * kw); V = bf16(x * rinv)
 *   c, s = bf16(cos / sin(pos * inv_freq[f])), f = d mod head_dim/2
 *   K = bf16(bf16(K0 * c) + bf16(rotateHalf(K0) * s))
 * raw element (h, t, d) at raw[h*raw_head_stride + t*head_dim + d]; k / v outputs at
 * [h*out_head_stride + t*head_dim + d]; inv_freq: head_dim/2 floats (device).
 * head_dim 128, 256 or 512. */
int esda_raw_prefill_kv(const void *raw, int64_t raw_head_stride, int32_t kv_heads, int32_t rows,
                        int32_t head_dim, const void *kw, float eps, const float *inv_freq,
                        int32_t pos0, void *k_out, void *v_out, int64_t out_head_stride,
                        void *stream);

/* The same over a q8 raw stream (head_dim 512): row (h, t) is u8 q8[h*q_head_stride +
 * t*512 ..] with scale / bias [h*sb_head_stride + t], dequantised to
 * bf16(float(q) * scale + bias) first. */
int esda_raw_q8_prefill_kv(const void *q8, int64_t q_head_stride, const float *scale,
                           const float *bias, int64_t sb_head_stride, int32_t kv_heads,
                           int32_t rows, const void *kw, float eps, const float *inv_freq,
                           int32_t pos0, void *k_out, void *v_out, int64_t out_head_stride,
                           void *stream);

/* LDS read ceiling of the prefill kernel's two operand read forms (no counterpart in the
 * reference: a measurement for the prefill kernel's roofline, like esda_stream_read for
 * the decode rings).  Each of `workgroups` workgroups of `waves` waves (4, 8 or 16) reads
 * a 64 KB LDS array for iters rounds of 8 reads per lane: 128-bit row reads
 * (transpose = 0) or 64-bit transpose reads ds_read_b64_tr_b16 (transpose != 0), 1 KB
 * (512 B) per wave per read, bank-conflict-free.  Bytes read: workgroups * waves * 64 *
 * iters * 8 * (16 or 8).  sink: workgroups * waves * 64 words (a checksum per thread). */
int esda_lds_read(int32_t waves, int32_t transpose, int32_t iters, int32_t workgroups, uint32_t *sink,
                  void *stream);

#ifdef __cplusplus
}
#endif
#endif
