/*
 * esda.h -- C ABI of the MI355X (gfx950) decode-attention library libesda.so.
 *
 * One decode step of Gemma-4 attention: append the new token's K/V row into the
 * cache and attend the single query over the visible rows, split-K across the
 * GPU, merged in fp32.  Plain pointers and sizes only; every device pointer is
 * caller-owned; every call takes an explicit HIP stream (NULL = default stream).
 * Functions return ESDA_OK or an error code; esda_last_error() gives the message
 * of the calling thread's last failure.
 *
 * Which reference interface each entry point replaces (paths in the Apertura tree):
 *   esda_decode            ESKVCache::update (ESKVCache.mm:64-109, prealloc append)
 *                          followed by mx::fast::scaled_dot_product_attention at
 *                          ESAttention.mm:188 (decode, seq == 1); the additive mask of
 *                          ESGemma4TextModel.mm:68-83 + alignMask (ESAttention.mm:17-22)
 *                          becomes in-kernel index math from (pos, window, cap).
 *   esda_kv_append         the slice_update append alone (ESKVCache.mm:97-98,
 *                          ESKVCache.mm:498 for updateRaw), for multi-row appends.
 *   esda_*_workspace_size  sizes the split partials the reference kept in MLX
 *                          temporaries (ESDecodeAttn.mm:444-452).
 */
#ifndef APERTURA_ESDA_H
#define APERTURA_ESDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ESDA_OK 0
#define ESDA_ERR_INVALID_ARGUMENT 1 /* the reference throws std::invalid_argument */
#define ESDA_ERR_RUNTIME 2          /* the reference throws std::runtime_error     */
#define ESDA_ERR_HIP 3              /* a HIP runtime call failed                   */
#define ESDA_ERR_WORKSPACE 4        /* workspace missing or too small              */
#define ESDA_ERR_DEVICE 5           /* no gfx950 device / library not usable       */

/* Shape and cache mode of one decode step.
 *
 * Cache element (b, kvh, row, d) lives at cache[b*seq_stride + kvh*head_stride +
 * row*head_dim + d] (bf16), the reference's [kvHeads, capacity, headDim] slot per
 * sequence (ESKVCache.h:183-192) with a leading sequence index.
 *
 * pos[b] is the absolute position of the new token of sequence b.
 *   ring == 0 (linear rows): the row of absolute position p is p - row_base[b]
 *             (row_base NULL = 0; after a compaction row 0 holds position row_base).
 *   ring == 1 (ring buffer): the row of absolute position p is p mod cap;
 *             requires 0 < window <= cap.
 * Visible positions (ESGemma4TextModel.mm:68-83): kj <= pos and, when window > 0,
 * kj > pos - window; in linear mode also kj >= row_base[b].
 * GQA: query head h reads kv head h / (num_q_heads / num_kv_heads) (ESOps.h:64-68). */
typedef struct esda_decode_desc {
    int32_t batch;        /* B                                              */
    int32_t num_q_heads;  /* Hq                                             */
    int32_t num_kv_heads; /* Hkv; Hq / Hkv <= 16                            */
    int32_t head_dim;     /* 128, 256 or 512                                */
    int32_t cap;          /* rows per (sequence, kv head)                   */
    int32_t window;       /* 0 = full causal, > 0 = sliding window          */
    int32_t ring;         /* 0 = linear rows, 1 = ring buffer               */
    int32_t kv_shared;    /* 1 = V aliases K (attention_k_eq_v, one buffer) */
    int64_t seq_stride;   /* elements; >= num_kv_heads * head_stride        */
    int64_t head_stride;  /* elements; >= cap * head_dim, multiple of 8     */
    int32_t max_visible;  /* expected bound on visible rows, sizes the split (0 = from
                             cap/window); rows beyond it are still attended (the last
                             split of a pair, or the balanced shares, take them) */
    int32_t split_rows;   /* rows per workgroup (0 = automatic; multiple of 16) */
    float scale;          /* softmax scale (the model uses 1.0)             */
} esda_decode_desc;

typedef struct esda_decode_args {
    const void *q;          /* [B, Hq, D] bf16, 16-byte aligned              */
    const void *k_new;      /* [B, Hkv, D] bf16                              */
    const void *v_new;      /* [B, Hkv, D] bf16; ignored when kv_shared      */
    void *k_cache;          /* bf16 cache (see layout above)                 */
    void *v_cache;          /* bf16 cache; must equal k_cache when kv_shared */
    const int32_t *pos;     /* [B] int32, device memory                      */
    const int32_t *row_base;/* [B] int32, device memory, or NULL             */
    void *out;              /* [B, Hq, D] bf16                               */
    void *workspace;        /* device scratch of esda_decode_workspace_size;
                               zero its first 256 bytes once before first use */
    size_t workspace_bytes;
} esda_decode_args;

/* Bytes of device workspace esda_decode needs for this description. */
int esda_decode_workspace_size(const esda_decode_desc *desc, size_t *bytes);

/* Append + attend + merge for one decode step (two kernel launches on `stream`).
 * Replaces ESKVCache::update + SDPA at ESAttention.mm:105 and :188. */
int esda_decode(const esda_decode_desc *desc, const esda_decode_args *args, void *stream);

/* Stage selector for esda_decode_stages (a profiling aid: the bench times the
 * split kernel alone).  esda_decode == both stages.  When the plan has one split per
 * (sequence, kv head) -- split_rows >= max_visible, or automatically when batch *
 * num_kv_heads fills the GPU -- the attend stage writes `out` itself and the merge stage
 * launches nothing. */
#define ESDA_STAGE_ATTEND 1 /* fused append + split-K partials */
#define ESDA_STAGE_MERGE 2  /* cross-split fp32 merge -> bf16 out */
int esda_decode_stages(const esda_decode_desc *desc, const esda_decode_args *args, int stages,
                       void *stream);

/* Reads (synchronously) and clears the device status word the kernels set when a
 * sequence's position is outside its cache (such a sequence is skipped: nothing is
 * written for it).  *bad_sequences receives the count flagged since the last call. */
int esda_decode_status(const esda_decode_desc *desc, void *workspace, int32_t *bad_sequences,
                       void *stream);

/* esda_decode without a workspace and without any allocation: the split partials and the
 * batch prefix table live in a static device array the library holds on every GPU it runs
 * on (32 MiB per GPU, until the process ends).  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).
 * - args->workspace is optional.  When given (device memory, >= 4 bytes, 4-byte aligned)
 *   it is only the skipped-sequence status word, read and cleared by esda_decode_status;
 *   zero it once before first use.  When NULL, skipped sequences are not reported.
 * - A step whose esda_decode_workspace_size exceeds 32 MiB is refused with
 *   ESDA_ERR_WORKSPACE (nothing is launched); such steps need esda_decode.
 * - Calls that overlap on one GPU (e.g. on two streams) share the array and race: order
 *   them on one stream, or use esda_decode with a workspace per stream.
 * The first call on a device looks up the array's address there (hipGetSymbolAddress),
 * so make that call outside graph capture.  Same kernels and results as esda_decode. */
int esda_decode_noalloc(const esda_decode_desc *desc, const esda_decode_args *args, void *stream);

/* Copy n_new rows per (sequence, kv head) into a linear cache at rows
 * row0[b] .. row0[b]+n_new-1: the reference's slice_update append
 * (ESKVCache.mm:97-98).  src: [B, Hkv, n_new, D] bf16. */
int esda_kv_append(void *cache, int64_t seq_stride, int64_t head_stride, int32_t batch,
                   int32_t num_kv_heads, int32_t head_dim, int32_t cap, const void *src,
                   int32_t n_new, const int32_t *row0, void *stream);

/* ---------------------------------------------------------------- raw-K mode
 *
 * Global layers with a raw-K cache: the cache holds only the pre-norm k_proj rows and
 * the kernel rebuilds, per streamed row (ESDecodeAttn.mm:17-117):
 *   rinv = rsqrt(mean(kraw^2) + eps)
 *   K    = bf16(rope(kraw * rinv * kw)), rotary pairs (d, d + 256) for d < 64 at
 *          rotary position = row index, cos / sin of the fp32 angle row*inv_freq[d]
 *          rounded to bf16
 *   V    = kraw * rinv (the factor is folded into the softmax weight)
 * Linear rows, full causal span: sequence b attends rows 0 .. pos[b]. */
typedef struct esda_raw_desc {
    int32_t batch;        /* B                                          */
    int32_t num_q_heads;  /* Hq                                         */
    int32_t num_kv_heads; /* Hkv; Hq / Hkv <= 16                        */
    int32_t head_dim;     /* must be 512                                */
    int32_t cap;          /* rows per (sequence, kv head): the pitch     */
    int64_t seq_stride;   /* elements; >= num_kv_heads * head_stride    */
    int64_t head_stride;  /* elements; >= cap * 512, multiple of 8      */
    int32_t max_visible;  /* upper bound on pos[b] + 1 (0 = cap)        */
    int32_t split_rows;   /* rows per split (0 = automatic; multiple of 16) */
    float scale;          /* softmax scale (the model uses 1.0)         */
    float eps;            /* k-norm epsilon                             */
} esda_raw_desc;

typedef struct esda_raw_args {
    const void *q;           /* [B, Hq, 512] bf16 (post q-norm + RoPE), 16-byte aligned */
    const void *k_new;       /* [B, Hkv, 512] bf16 raw rows written to row pos[b] before
                                attending, or NULL when the rows are already cached   */
    void *raw_cache;         /* bf16 raw-K cache (layout as esda_decode_desc)          */
    const int32_t *pos;      /* [B] int32, device memory: row of the newest token      */
    const void *kw;          /* [512] bf16 k-norm weights                              */
    const float *inv_freq;   /* [64] f32 rotary inverse frequencies                    */
    void *out;               /* [B, Hq, 512] bf16                                      */
    void *workspace;         /* esda_decode_raw_workspace_size bytes; first 256 zeroed once */
    size_t workspace_bytes;
    const void *rope_table;  /* optional, NULL: computed in the kernel.  [rope_table_rows][64]
                                u32 from esda_rope_table (cos / sin of row*inv_freq[d]);
                                read where two kv heads share a workgroup              */
    int32_t rope_table_rows; /* >= cap when rope_table is set                          */
} esda_raw_args;

int esda_decode_raw_workspace_size(const esda_raw_desc *desc, size_t *bytes);

/* Fused raw-K decode step (append + rebuild + attend + merge): replaces
 * ESKVCache::updateRaw (ESKVCache.mm:458-504) followed by esDecodeAttnGlobal
 * (ESDecodeAttn.mm:415-453) as called at ESAttention.mm:291-300. */
int esda_decode_raw(const esda_raw_desc *desc, const esda_raw_args *args, void *stream);

/* Stage-selectable form of esda_decode_raw (ESDA_STAGE_* as for esda_decode_stages). */
int esda_decode_raw_stages(const esda_raw_desc *desc, const esda_raw_args *args, int stages,
                           void *stream);

/* ------------------------------------------------------------- q8 raw-K mode
 *
 * The raw stream stored as per-row affine u8 (rawKVQ8): row x = q * scale + bias with
 * q u8 [512], scale and bias f32 (ESKVCache.h:81-91, ESKVCache.mm:506-566).  The kernel
 * widens q exactly, rebuilds K / V as in raw-K mode from x, and quantizes the new row
 * (k_new, bf16) into row pos[b] before attending (esQuantizeRawRows' arithmetic).
 * Description: esda_raw_desc, with seq_stride / head_stride counting u8 elements (bytes;
 * multiples of 16).  Workspace: esda_decode_raw_workspace_size. */
typedef struct esda_raw_q8_args {
    const void *q;             /* [B, Hq, 512] bf16 (post q-norm + RoPE)                   */
    const void *k_new;         /* [B, Hkv, 512] bf16 raw rows to quantize into row pos[b], or
                                  NULL when the rows are already cached                   */
    void *q8_cache;            /* u8 rows: (b, kvh, row, d) at b*seq_stride + kvh*head_stride
                                  + row*512 + d                                           */
    float *scale;              /* per row: (b, kvh, row) at b*sb_seq_stride + kvh*sb_head_stride + row */
    float *bias;
    int64_t sb_seq_stride;     /* elements; >= num_kv_heads * sb_head_stride              */
    int64_t sb_head_stride;    /* elements; >= cap                                        */
    const int32_t *pos;        /* [B] int32, device memory: row of the newest token       */
    const void *kw;            /* [512] bf16 k-norm weights                               */
    const float *inv_freq;     /* [64] f32 rotary inverse frequencies                     */
    void *out;                 /* [B, Hq, 512] bf16                                       */
    void *workspace;           /* esda_decode_raw_workspace_size bytes; first 256 zeroed once */
    size_t workspace_bytes;
    const void *rope_table;    /* optional; as in esda_raw_args                           */
    int32_t rope_table_rows;
} esda_raw_q8_args;

/* Fused q8 raw-K decode step (quantize-append + rebuild + attend + merge): replaces
 * ESKVCache::updateRawQ8 (ESKVCache.mm:513-556) followed by esDecodeAttnGlobalQ8
 * (ESDecodeAttn.mm:455-489) as called at ESAttention.mm:270-279. */
int esda_decode_raw_q8(const esda_raw_desc *desc, const esda_raw_q8_args *args, void *stream);
int esda_decode_raw_q8_stages(const esda_raw_desc *desc, const esda_raw_q8_args *args, int stages,
                              void *stream);

/* Quantize src [kv_heads, n_rows, 512] bf16 (contiguous) into rows row0 .. row0+n_rows-1 of
 * a q8 cache: q8 + h*q_head_stride + row*512, scale / bias + h*sb_head_stride + row
 * (esQuantizeRawRows, ESDecodeAttn.mm:491-539; ESKVCache::quantizeRawRows). */
/* Rotary table for raw-K decode: table[t*64 + d] = bf16(cos(a)) | bf16(sin(a)) << 16 with
 * a = float(t) * inv_freq[d] in fp32, t < rows -- the values the raw-K kernels otherwise
 * compute per step (the reference kernel's inline cos / sin, ESDecodeAttn.mm:51-106),
 * bit for bit.  A per-model precompute: one table serves every raw-K layer with the same
 * inv_freq.  table: rows * 256 bytes, 16-byte aligned; inv_freq: [64] f32 (device). */
int esda_rope_table(const float *inv_freq, int32_t rows, void *table, void *stream);

int esda_quantize_raw_rows(const void *src, int32_t kv_heads, int32_t n_rows, void *q8,
                           int64_t q_head_stride, float *scale, float *bias, int64_t sb_head_stride,
                           int32_t row0, void *stream);

/* dst[0 .. n-1] = value on `stream` (a kernel, so it may be captured in a graph): sets
 * the per-sequence position words that replace the host-built additive mask upload of
 * ESGemma4TextModel.mm:68-83 / ESAttention.mm:17-22. */
int esda_fill_i32(int32_t *dst, int32_t value, int32_t n, void *stream);

/* Measurement aid (no counterpart in the reference): read `bytes` (a multiple of 1024)
 * from src once, through the attend kernel's load path (LDS DMA, non-temporal, 1 KiB per
 * wave instruction), over `workgroups` workgroups of 256 threads; sink receives
 * 4 * workgroups words.  Gives the memory system's read ceiling for that path and the
 * calibration of the HBM counters on it. */
int esda_stream_read(const void *src, size_t bytes, int32_t workgroups, uint32_t *sink, void *stream);

/* Message of the calling thread's last error ("" if none). */
const char *esda_last_error(void);

/* Library version (major*10000 + minor*100 + patch). */
int esda_version(void);

#ifdef __cplusplus
}
#endif
#endif
