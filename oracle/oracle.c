/*
 * oracle.c -- CPU restatement of Apertura's decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): loaded by tests/, smoke() and the
 * cpu_baseline leg of bench.py; never by the product library.
 *
 * Parity status of each function is recorded in oracle.h and pinned by
 * tests/test_oracle.py.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static int32_t g_fault = 0;
void orc_set_fault(int32_t fault) { g_fault = fault; }

/* Conditioning probe of the raw-K restatement (0 = off): every row's rinv moved by this many
 * fp32 ulps before K is rebuilt, to measure how far the result moves under an ulp-level
 * difference in the row norm (which no implementation fixes: the reference's rsqrt and
 * summation order are its own). */
static int32_t g_rinv_ulps = 0;
void orc_set_rinv_ulps(int32_t ulps) { g_rinv_ulps = ulps; }

/* ------------------------------------------------------------------ bf16 */

uint16_t orc_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return (uint16_t) ((u >> 16) | 0x0040u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb; /* round to nearest, ties to even */
    return (uint16_t) (u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t) h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_f32_to_bf16_n(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(x[i]);
}

void orc_bf16_to_f32_n(const uint16_t *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------- visibility rule */

static int desc_ok(const orc_desc *d) {
    if (!d || d->B <= 0 || d->Hq <= 0 || d->Hkv <= 0 || d->D <= 0 || d->cap <= 0) return 0;
    if (d->Hq % d->Hkv) return 0;
    if (d->window < 0) return 0;
    if (d->ring && (d->window <= 0 || d->window > d->cap)) return 0;
    if (d->head_stride < (int64_t) d->cap * d->D) return 0;
    if (d->seq_stride < (int64_t) d->Hkv * d->head_stride) return 0;
    return 1;
}

/* Row holding absolute position p (ESKVCache.mm:97: the new row lands at row len;
 * ring mode: slot p mod cap). */
static int32_t row_of(const orc_desc *d, int32_t p, int32_t row_base) {
    return d->ring ? (p % d->cap) : (p - row_base);
}

/* Key kj is visible to query qAbs iff kj <= qAbs and, for sliding layers,
 * kj > qAbs - window (ESGemma4TextModel.mm:68-83).  Eviction keeps exactly those
 * rows (ESKVCache.mm:104), so the visible set is the contiguous absolute range
 * [lo, pos]. */
int32_t orc_visible(const orc_desc *d, int32_t pos, int32_t row_base, int32_t *rows_out) {
    if (!desc_ok(d) || pos < 0) return -1;
    int32_t lo = 0;
    if (d->window > 0) {
        lo = pos - d->window + 1;
        if (g_fault == 2) lo = pos - d->window; /* planted off-by-one */
        if (lo < 0) lo = 0;
    }
    if (!d->ring) {
        if (lo < row_base) lo = row_base;
        if (pos - row_base >= d->cap) return -1;
    } else if (d->window == 0 && pos >= d->cap) {
        return -1;
    }
    int32_t n = 0;
    for (int32_t p = lo; p <= pos; ++p) rows_out[n++] = row_of(d, p, row_base);
    return n;
}

/* ---------------------------------------------------------------- append */

int32_t orc_append(const orc_desc *d, uint16_t *k_cache, uint16_t *v_cache,
                   const uint16_t *k_new, const uint16_t *v_new,
                   const int32_t *pos, const int32_t *row_base) {
    if (!desc_ok(d)) return -1;
    if (g_fault == 4) return 0; /* planted: append dropped */
    for (int32_t b = 0; b < d->B; ++b) {
        int32_t rb = row_base ? row_base[b] : 0;
        int32_t r = row_of(d, pos[b], rb);
        if (r < 0 || r >= d->cap) return -1;
        for (int32_t h = 0; h < d->Hkv; ++h) {
            size_t dst = (size_t) b * d->seq_stride + (size_t) h * d->head_stride + (size_t) r * d->D;
            size_t src = ((size_t) b * d->Hkv + h) * d->D;
            memcpy(k_cache + dst, k_new + src, (size_t) d->D * 2);
            if (v_cache != k_cache && v_new) memcpy(v_cache + dst, v_new + src, (size_t) d->D * 2);
        }
    }
    return 0;
}

/* ------------------------------------------------------ thread fan-out */

typedef struct {
    void (*fn)(void *ctx, int64_t item);
    void *ctx;
    int64_t n_items;
    int64_t next;
    pthread_mutex_t mu;
} pool_t;

static void *pool_worker(void *arg) {
    pool_t *p = (pool_t *) arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        int64_t it = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (it >= p->n_items) break;
        p->fn(p->ctx, it);
    }
    return NULL;
}

static void run_items(void (*fn)(void *, int64_t), void *ctx, int64_t n_items, int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t) nthreads > n_items) nthreads = (int32_t) (n_items > 0 ? n_items : 1);
    pool_t p;
    p.fn = fn; p.ctx = ctx; p.n_items = n_items; p.next = 0;
    pthread_mutex_init(&p.mu, NULL);
    if (nthreads == 1) {
        pool_worker(&p);
    } else {
        pthread_t th[256];
        for (int32_t i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, pool_worker, &p);
        for (int32_t i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    }
    pthread_mutex_destroy(&p.mu);
}

/* GQA: query head h reads kv head h / (Hq/Hkv) -- kv-major contiguous groups
 * (ESOps.h:64-68, pinned by ESPrimitivesTests.mm:118-128). */
static int32_t kv_of(const orc_desc *d, int32_t h) {
    int32_t g = d->Hq / d->Hkv;
    if (g_fault == 1) return h % d->Hkv; /* planted: interleaved mapping */
    return h / g;
}

static float eff_scale(const orc_desc *d) { return g_fault == 3 ? 1.0f : d->scale; }

typedef struct {
    const orc_desc *d;
    const uint16_t *q, *k, *v;
    const int32_t *pos, *row_base;
    void *out;
    int32_t nsplit;
    int32_t status;
} job_t;

static int32_t *alloc_rows(const orc_desc *d) {
    return (int32_t *) malloc(sizeof(int32_t) * ((size_t) d->cap + 1));
}

/* ------------------------------------------------------------ fp64 mode */

static void item_f64(void *ctx, int64_t it) {
    job_t *j = (job_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t b = (int32_t) (it / d->Hq), h = (int32_t) (it % d->Hq), D = d->D;
    const int32_t kvh = kv_of(d, h);
    int32_t *rows = alloc_rows(d);
    double *out = (double *) j->out + ((size_t) b * d->Hq + h) * D;
    int32_t n = orc_visible(d, j->pos[b], j->row_base ? j->row_base[b] : 0, rows);
    if (n <= 0) { j->status = -1; free(rows); return; }
    double *qd = (double *) malloc(sizeof(double) * D);
    double *s = (double *) malloc(sizeof(double) * n);
    const uint16_t *qh = j->q + ((size_t) b * d->Hq + h) * D;
    for (int32_t i = 0; i < D; ++i) qd[i] = orc_bf16_to_f32(qh[i]);
    const size_t base = (size_t) b * d->seq_stride + (size_t) kvh * d->head_stride;
    double mx = -INFINITY;
    for (int32_t t = 0; t < n; ++t) {
        const uint16_t *kr = j->k + base + (size_t) rows[t] * D;
        double acc = 0.0;
        for (int32_t i = 0; i < D; ++i) acc += qd[i] * (double) orc_bf16_to_f32(kr[i]);
        s[t] = acc * (double) eff_scale(d);
        if (s[t] > mx) mx = s[t];
    }
    double den = 0.0;
    for (int32_t t = 0; t < n; ++t) { s[t] = exp(s[t] - mx); den += s[t]; }
    for (int32_t i = 0; i < D; ++i) out[i] = 0.0;
    for (int32_t t = 0; t < n; ++t) {
        const uint16_t *vr = j->v + base + (size_t) rows[t] * D;
        const double w = s[t] / den;
        for (int32_t i = 0; i < D; ++i) out[i] += w * (double) orc_bf16_to_f32(vr[i]);
    }
    free(qd); free(s); free(rows);
}

int32_t orc_decode_f64(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                       double *out, int32_t nthreads) {
    if (!desc_ok(d)) return -1;
    job_t j = {d, q, k_cache, v_cache, pos, row_base, out, 0, 0};
    run_items(item_f64, &j, (int64_t) d->B * d->Hq, nthreads);
    return j.status;
}

/* ------------------------------------------------- reference-rounding mode */

static float bf(float x) { return orc_bf16_to_f32(orc_f32_to_bf16(x)); }

/* ESAttention.mm:136-165, per query head:
 *   scores = bf16(q . K^T)                   (:153, bf16 matmul, f32 accumulation)
 *   scores = bf16(scores * bf16(scaling))    (:154, only when scaling != 1)
 *   sf = f32(scores) + mask                  (:156-157; masked keys contribute 0)
 *   w = bf16(softmax_precise(sf))            (:158-159)
 *   out = bf16(w . V)                        (:161, f32 accumulation)            */
static void item_refround(void *ctx, int64_t it) {
    job_t *j = (job_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t b = (int32_t) (it / d->Hq), h = (int32_t) (it % d->Hq), D = d->D;
    const int32_t kvh = kv_of(d, h);
    int32_t *rows = alloc_rows(d);
    uint16_t *out = (uint16_t *) j->out + ((size_t) b * d->Hq + h) * D;
    int32_t n = orc_visible(d, j->pos[b], j->row_base ? j->row_base[b] : 0, rows);
    if (n <= 0) { j->status = -1; free(rows); return; }
    float *qf = (float *) malloc(sizeof(float) * D);
    float *s = (float *) malloc(sizeof(float) * n);
    float *acc = (float *) malloc(sizeof(float) * D);
    const uint16_t *qh = j->q + ((size_t) b * d->Hq + h) * D;
    for (int32_t i = 0; i < D; ++i) qf[i] = orc_bf16_to_f32(qh[i]);
    const size_t base = (size_t) b * d->seq_stride + (size_t) kvh * d->head_stride;
    const float sc = eff_scale(d);
    const float scb = bf(sc);
    float mx = -INFINITY;
    for (int32_t t = 0; t < n; ++t) {
        const uint16_t *kr = j->k + base + (size_t) rows[t] * D;
        float a = 0.0f;
        for (int32_t i = 0; i < D; ++i) a += qf[i] * orc_bf16_to_f32(kr[i]);
        float sv = bf(a);
        if (sc != 1.0f) sv = bf(sv * scb);
        s[t] = sv;
        if (sv > mx) mx = sv;
    }
    float den = 0.0f;
    for (int32_t t = 0; t < n; ++t) { s[t] = expf(s[t] - mx); den += s[t]; }
    for (int32_t t = 0; t < n; ++t) s[t] = bf(s[t] / den);
    for (int32_t i = 0; i < D; ++i) acc[i] = 0.0f;
    for (int32_t t = 0; t < n; ++t) {
        const uint16_t *vr = j->v + base + (size_t) rows[t] * D;
        const float w = s[t];
        for (int32_t i = 0; i < D; ++i) acc[i] += w * orc_bf16_to_f32(vr[i]);
    }
    for (int32_t i = 0; i < D; ++i) out[i] = orc_f32_to_bf16(acc[i]);
    free(qf); free(s); free(acc); free(rows);
}

int32_t orc_decode_refround(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, const int32_t *pos,
                            const int32_t *row_base, uint16_t *out, int32_t nthreads) {
    if (!desc_ok(d)) return -1;
    job_t j = {d, q, k_cache, v_cache, pos, row_base, out, 0, 0};
    run_items(item_refround, &j, (int64_t) d->B * d->Hq, nthreads);
    return j.status;
}

/* ------------------------------------------- grouped reference rounding */

/* orc_decode_refround with each K and V row read once for the query heads of its kv head
 * and the rows of one (sequence, kv head) spread over threads: the CPU baseline that
 * bench.py times.  Same rounding points as item_refround (ESAttention.mm:136-165): f32 dot
 * products summed in dimension order, bf16 scores, bf16(scaling), a precise softmax over
 * all visible rows, bf16 weights, f32 accumulation, bf16 output.  Only the order in which
 * the splits' partial sums (softmax denominator, output accumulation) combine differs; with
 * one split per (sequence, kv head) the output is that of orc_decode_refround bit for bit.
 * The query heads of a kv head are the innermost loop (blocks of 8), so the compiler can
 * vectorise across heads without reordering any head's sums. */
#define ORC_HB 8

/* bf16 <-> fp32 as orc_bf16_to_f32 / orc_f32_to_bf16, local to this file so the compiler
 * inlines them into the loops (the exported functions are called through the PLT). */
static inline float bf2f(uint16_t h) {
    const uint32_t u = ((uint32_t) h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline float bfr(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return x;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

typedef struct {
    const orc_desc *d;
    const uint16_t *q, *k, *v;
    const int32_t *pos, *row_base;
    uint16_t *out;
    int32_t G, nsplit;
    int32_t **rows;      /* [B] visible rows */
    int32_t *nvis;       /* [B] */
    float **sc;          /* [B * Hkv] scores, then exp(s - max): [G][n] */
    float *smax, *sden;  /* [B * Hkv * nsplit][G] */
    float *pacc;         /* [B * Hkv * nsplit][D][ORC_HB * nhb] */
    int32_t status;
} gjob_t;

static void split_range(int32_t n, int32_t ns, int32_t s, int32_t *t0, int32_t *t1) {
    *t0 = (int32_t) ((int64_t) n * s / ns);
    *t1 = (int32_t) ((int64_t) n * (s + 1) / ns);
}

/* Scores of split s of (b, kvh): sc[h][t] and the split's max per head. */
__attribute__((target_clones("avx2", "default"), optimize("O3,tree-vectorize")))
static void gitem_scores(void *ctx, int64_t it) {
    gjob_t *j = (gjob_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t D = d->D, G = j->G, ns = j->nsplit;
    const int32_t pair = (int32_t) (it / ns), s = (int32_t) (it % ns);
    const int32_t b = pair / d->Hkv, kvh = pair % d->Hkv, n = j->nvis[b];
    if (n <= 0) return;
    int32_t t0, t1;
    split_range(n, ns, s, &t0, &t1);
    const size_t base = (size_t) b * d->seq_stride + (size_t) kvh * d->head_stride;
    const float sc = eff_scale(d), scb = bf(sc);
    float *qt = (float *) malloc(sizeof(float) * (size_t) D * ORC_HB);
    for (int32_t h0 = 0; h0 < G; h0 += ORC_HB) {
        for (int32_t i = 0; i < D; ++i)
            for (int32_t e = 0; e < ORC_HB; ++e) {
                const int32_t h = h0 + e;
                qt[(size_t) i * ORC_HB + e] =
                    h < G ? bf2f(j->q[((size_t) b * d->Hq + (size_t) kvh * G + h) * D + i]) : 0.0f;
            }
        float mx[ORC_HB];
        for (int32_t e = 0; e < ORC_HB; ++e) mx[e] = -INFINITY;
        for (int32_t t = t0; t < t1; ++t) {
            const uint16_t *kr = j->k + base + (size_t) j->rows[b][t] * D;
            float a[ORC_HB] = {0};
            for (int32_t i = 0; i < D; ++i) {
                const float kf = bf2f(kr[i]);
                for (int32_t e = 0; e < ORC_HB; ++e) a[e] += qt[(size_t) i * ORC_HB + e] * kf;
            }
            for (int32_t e = 0; e < ORC_HB && h0 + e < G; ++e) {
                float v = bfr(a[e]);
                if (sc != 1.0f) v = bfr(v * scb);
                j->sc[pair][(size_t) (h0 + e) * n + t] = v;
                if (v > mx[e]) mx[e] = v;
            }
        }
        for (int32_t e = 0; e < ORC_HB && h0 + e < G; ++e) j->smax[(size_t) it * G + h0 + e] = mx[e];
    }
    free(qt);
}

/* exp(s - max) in place over split s, and the split's sum per head. */
static void gitem_exp(void *ctx, int64_t it) {
    gjob_t *j = (gjob_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t G = j->G, ns = j->nsplit;
    const int32_t pair = (int32_t) (it / ns), s = (int32_t) (it % ns);
    const int32_t b = pair / d->Hkv, n = j->nvis[b];
    if (n <= 0) return;
    int32_t t0, t1;
    split_range(n, ns, s, &t0, &t1);
    for (int32_t h = 0; h < G; ++h) {
        float mx = -INFINITY;
        for (int32_t u = 0; u < ns; ++u) mx = fmaxf(mx, j->smax[((size_t) pair * ns + u) * G + h]);
        float *row = j->sc[pair] + (size_t) h * n;
        float den = 0.0f;
        for (int32_t t = t0; t < t1; ++t) { row[t] = expf(row[t] - mx); den += row[t]; }
        j->sden[(size_t) it * G + h] = den;
    }
}

/* Weights bf16(e / den) of split s and its share of the output accumulation. */
__attribute__((target_clones("avx2", "default"), optimize("O3,tree-vectorize")))
static void gitem_pv(void *ctx, int64_t it) {
    gjob_t *j = (gjob_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t D = d->D, G = j->G, ns = j->nsplit, HW = ((G + ORC_HB - 1) / ORC_HB) * ORC_HB;
    const int32_t pair = (int32_t) (it / ns), s = (int32_t) (it % ns);
    const int32_t b = pair / d->Hkv, kvh = pair % d->Hkv, n = j->nvis[b];
    float *acc = j->pacc + (size_t) it * D * HW;
    memset(acc, 0, sizeof(float) * (size_t) D * HW);
    if (n <= 0) return;
    int32_t t0, t1;
    split_range(n, ns, s, &t0, &t1);
    float *den = (float *) malloc(sizeof(float) * HW);
    for (int32_t h = 0; h < HW; ++h) {
        float v = 0.0f;
        if (h < G)
            for (int32_t u = 0; u < ns; ++u) v += j->sden[((size_t) pair * ns + u) * G + h];
        den[h] = v;
    }
    const size_t base = (size_t) b * d->seq_stride + (size_t) kvh * d->head_stride;
    for (int32_t h0 = 0; h0 < G; h0 += ORC_HB) {
        for (int32_t t = t0; t < t1; ++t) {
            const uint16_t *vr = j->v + base + (size_t) j->rows[b][t] * D;
            float w[ORC_HB];
            for (int32_t e = 0; e < ORC_HB; ++e)
                w[e] = h0 + e < G ? bfr(j->sc[pair][(size_t) (h0 + e) * n + t] / den[h0 + e]) : 0.0f;
            for (int32_t i = 0; i < D; ++i) {
                const float vf = bf2f(vr[i]);
                float *a = acc + (size_t) i * HW + h0;
                for (int32_t e = 0; e < ORC_HB; ++e) a[e] += w[e] * vf;
            }
        }
    }
    free(den);
}

/* out = bf16(sum of the splits' accumulations), splits in order. */
static void gitem_out(void *ctx, int64_t pair) {
    gjob_t *j = (gjob_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t D = d->D, G = j->G, ns = j->nsplit, HW = ((G + ORC_HB - 1) / ORC_HB) * ORC_HB;
    const int32_t b = (int32_t) pair / d->Hkv, kvh = (int32_t) pair % d->Hkv;
    if (j->nvis[b] <= 0) return;
    for (int32_t h = 0; h < G; ++h) {
        uint16_t *out = j->out + ((size_t) b * d->Hq + (size_t) kvh * G + h) * D;
        for (int32_t i = 0; i < D; ++i) {
            float v = 0.0f;
            for (int32_t u = 0; u < ns; ++u) v += j->pacc[(((size_t) pair * ns + u) * D + i) * HW + h];
            out[i] = orc_f32_to_bf16(v);
        }
    }
}

int32_t orc_decode_refround_grouped(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                                    const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                                    int32_t nsplit, uint16_t *out, int32_t nthreads) {
    if (!desc_ok(d) || nsplit < 0) return -1;
    if (g_fault == 1) return -1; /* the grouping assumes the kv-major map */
    const int32_t G = d->Hq / d->Hkv, HW = ((G + ORC_HB - 1) / ORC_HB) * ORC_HB;
    const int32_t pairs = d->B * d->Hkv;
    gjob_t j;
    memset(&j, 0, sizeof(j));
    j.d = d; j.q = q; j.k = k_cache; j.v = v_cache; j.pos = pos; j.row_base = row_base; j.out = out;
    j.G = G;
    j.rows = (int32_t **) calloc((size_t) d->B, sizeof(int32_t *));
    j.nvis = (int32_t *) calloc((size_t) d->B, sizeof(int32_t));
    int32_t nmax = 0;
    for (int32_t b = 0; b < d->B; ++b) {
        j.rows[b] = alloc_rows(d);
        j.nvis[b] = orc_visible(d, pos[b], row_base ? row_base[b] : 0, j.rows[b]);
        if (j.nvis[b] <= 0) j.status = -1;
        if (j.nvis[b] > nmax) nmax = j.nvis[b];
    }
    /* splits: enough items for the threads, at least 256 rows each */
    int32_t ns = nsplit;
    if (ns == 0) {
        const int32_t want = (4 * (nthreads > 0 ? nthreads : 1) + pairs - 1) / pairs;
        const int32_t cap = nmax / 256 > 1 ? nmax / 256 : 1;
        ns = want < cap ? want : cap;
        if (ns < 1) ns = 1;
    }
    j.nsplit = ns;
    j.sc = (float **) calloc((size_t) pairs, sizeof(float *));
    for (int32_t u = 0; u < pairs; ++u) {
        const int32_t n = j.nvis[u / d->Hkv];
        j.sc[u] = (float *) malloc(sizeof(float) * (size_t) G * (size_t) (n > 0 ? n : 1));
    }
    const int64_t items = (int64_t) pairs * ns;
    j.smax = (float *) malloc(sizeof(float) * (size_t) items * G);
    j.sden = (float *) malloc(sizeof(float) * (size_t) items * G);
    j.pacc = (float *) malloc(sizeof(float) * (size_t) items * d->D * HW);
    run_items(gitem_scores, &j, items, nthreads);
    run_items(gitem_exp, &j, items, nthreads);
    run_items(gitem_pv, &j, items, nthreads);
    run_items(gitem_out, &j, pairs, nthreads);
    for (int32_t b = 0; b < d->B; ++b) free(j.rows[b]);
    for (int32_t u = 0; u < pairs; ++u) free(j.sc[u]);
    free(j.rows); free(j.nvis); free(j.sc); free(j.smax); free(j.sden); free(j.pacc);
    return j.status;
}

/* ----------------------------------------------------------- split-K mode */

/* Online softmax per split as in ESDecodeAttn.mm:44-110 (m starts at -3e38, l at 0,
 * acc = acc*corr + e*v), then the merge of ESDecodeAttn.mm:253-273:
 *   mMax = max_s m_s;  w_s = exp(m_s - mMax);  O = sum_s acc_s w_s / sum_s l_s w_s. */
static void item_splitk(void *ctx, int64_t it) {
    job_t *j = (job_t *) ctx;
    const orc_desc *d = j->d;
    const int32_t b = (int32_t) (it / d->Hq), h = (int32_t) (it % d->Hq), D = d->D;
    const int32_t kvh = kv_of(d, h), S = j->nsplit;
    int32_t *rows = alloc_rows(d);
    float *out = (float *) j->out + ((size_t) b * d->Hq + h) * D;
    int32_t n = orc_visible(d, j->pos[b], j->row_base ? j->row_base[b] : 0, rows);
    if (n <= 0 || S <= 0) { j->status = -1; free(rows); return; }
    float *qf = (float *) malloc(sizeof(float) * D);
    float *acc = (float *) malloc(sizeof(float) * (size_t) S * D);
    float *ms = (float *) malloc(sizeof(float) * S);
    float *ls = (float *) malloc(sizeof(float) * S);
    const uint16_t *qh = j->q + ((size_t) b * d->Hq + h) * D;
    for (int32_t i = 0; i < D; ++i) qf[i] = orc_bf16_to_f32(qh[i]);
    const size_t base = (size_t) b * d->seq_stride + (size_t) kvh * d->head_stride;
    const int32_t per = (n + S - 1) / S;
    const float sc = eff_scale(d);
    for (int32_t s = 0; s < S; ++s) {
        float m = -3.0e38f, l = 0.0f;
        float *a = acc + (size_t) s * D;
        for (int32_t i = 0; i < D; ++i) a[i] = 0.0f;
        const int32_t r0 = s * per, r1 = (r0 + per < n) ? r0 + per : n;
        for (int32_t t = r0; t < r1; ++t) {
            const uint16_t *kr = j->k + base + (size_t) rows[t] * D;
            const uint16_t *vr = j->v + base + (size_t) rows[t] * D;
            float dot = 0.0f;
            for (int32_t i = 0; i < D; ++i) dot += qf[i] * orc_bf16_to_f32(kr[i]);
            const float score = dot * sc;
            const float mNew = score > m ? score : m;
            const float corr = expf(m - mNew), e = expf(score - mNew);
            l = l * corr + e;
            for (int32_t i = 0; i < D; ++i) a[i] = a[i] * corr + e * orc_bf16_to_f32(vr[i]);
            m = mNew;
        }
        ms[s] = m; ls[s] = l;
    }
    float mMax = -3.0e38f;
    for (int32_t s = 0; s < S; ++s) if (ms[s] > mMax) mMax = ms[s];
    float lTot = 0.0f;
    for (int32_t s = 0; s < S; ++s) { ms[s] = expf(ms[s] - mMax); lTot += ls[s] * ms[s]; }
    for (int32_t i = 0; i < D; ++i) {
        float a = 0.0f;
        for (int32_t s = 0; s < S; ++s) a += acc[(size_t) s * D + i] * ms[s];
        out[i] = a / lTot;
    }
    free(qf); free(acc); free(ms); free(ls); free(rows);
}

int32_t orc_decode_splitk(const orc_desc *d, const uint16_t *q, const uint16_t *k_cache,
                          const uint16_t *v_cache, const int32_t *pos, const int32_t *row_base,
                          int32_t nsplit, float *out, int32_t nthreads) {
    if (!desc_ok(d) || nsplit <= 0) return -1;
    job_t j = {d, q, k_cache, v_cache, pos, row_base, out, nsplit, 0};
    run_items(item_splitk, &j, (int64_t) d->B * d->Hq, nthreads);
    return j.status;
}

/* ------------------------------------------------------ norms and rope */

void orc_rope_inv_freq(int32_t head_dim, float theta, float partial, float *inv_freq) {
    const int32_t half = head_dim / 2;
    int32_t angles = (int32_t) ((double) partial * head_dim / 2.0);
    if (angles > half) angles = half;
    for (int32_t i = 0; i < half; ++i) inv_freq[i] = 0.0f;
    for (int32_t i = 0; i < angles; ++i)
        inv_freq[i] = (float) (1.0 / pow((double) theta, (double) (2 * i) / (double) head_dim));
}

void orc_rms_norm_rows(const uint16_t *x, const uint16_t *w, int64_t rows, int32_t n,
                       float eps, uint16_t *y) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * n;
        float ss = 0.0f;
        for (int32_t i = 0; i < n; ++i) { float v = orc_bf16_to_f32(xr[i]); ss += v * v; }
        const float inv = 1.0f / sqrtf(ss / (float) n + eps);
        for (int32_t i = 0; i < n; ++i) {
            float v = orc_bf16_to_f32(xr[i]) * inv;
            if (w) v *= orc_bf16_to_f32(w[i]);
            y[r * n + i] = orc_f32_to_bf16(v);
        }
    }
}

/* ------------------------------------------------------------ raw-K mode */

typedef struct {
    const uint16_t *q, *raw, *kw;
    const float *inv_freq;
    int32_t Hkv, len, pitch;
    float eps, scale;
    double *out;
    /* q8 raw stream (raw == NULL): u8 rows and per-row scale / bias [Hkv, pitch] */
    const uint8_t *q8;
    const float *sc, *bs;
} raw_job_t;

/* Row t of kv head kvh as fp32: the bf16 raw row, or the q8 row dequantised as
 * float(q) * scale + bias with two roundings (ESKVCache.mm:366-383; the values the q8
 * decode kernel computes on, ESDecodeAttn.mm:316-319). */
static void raw_row(const raw_job_t *j, int32_t kvh, int32_t t, float *x) {
    const size_t r = (size_t) kvh * j->pitch + t;
    if (j->raw) {
        for (int32_t i = 0; i < 512; ++i) x[i] = orc_bf16_to_f32(j->raw[r * 512 + i]);
    } else {
        const float sc = j->sc[r], bs = j->bs[r];
        for (int32_t i = 0; i < 512; ++i) {
            const float prod = (float) j->q8[r * 512 + i] * sc;
            x[i] = prod + bs;
        }
    }
}

/* One query head over all len rows of its kv head.  Reconstruction follows
 * ESDecodeAttn.mm:51-93: rinv = rsqrt(mean(kraw^2) + eps); cos/sin of the fp32
 * angle t*invfreq[f] rounded to bf16; K = bf16(rope(kraw*rinv*kw)) with pairs
 * (d, d+256) for d < 64; V = kraw*rinv (ESDecodeAttn.mm:106).  Attention in fp64. */
static void item_raw(void *ctx, int64_t it) {
    raw_job_t *j = (raw_job_t *) ctx;
    const int32_t h = (int32_t) it, kvh = h / 8, D = 512;
    double qd[512], acc[512];
    for (int32_t i = 0; i < D; ++i) { qd[i] = orc_bf16_to_f32(j->q[(size_t) h * D + i]); acc[i] = 0.0; }
    double *s = (double *) malloc(sizeof(double) * j->len);
    double *rv = (double *) malloc(sizeof(double) * j->len);
    double mx = -INFINITY;
    float xr[512];
    for (int32_t t = 0; t < j->len; ++t) {
        raw_row(j, kvh, t, xr);
        double ss = 0.0;
        for (int32_t i = 0; i < D; ++i) { double v = xr[i]; ss += v * v; }
        float rinv = 1.0f / sqrtf((float) (ss / 512.0) + j->eps);
        for (int32_t u = 0; u < g_rinv_ulps; ++u) rinv = nextafterf(rinv, INFINITY);
        for (int32_t u = 0; u > g_rinv_ulps; --u) rinv = nextafterf(rinv, -INFINITY);
        rv[t] = rinv;
        double dot = 0.0;
        for (int32_t dd = 0; dd < D; ++dd) {
            const float kn = xr[dd] * rinv * orc_bf16_to_f32(j->kw[dd]);
            float kd = kn;
            const int32_t f = dd & 255;
            if (f < 64) {
                const float a = (float) t * j->inv_freq[f];
                const float c = bf(cosf(a)), sn = bf(sinf(a));
                const int32_t pd = dd < 256 ? dd + 256 : dd - 256;
                const float kn2 = xr[pd] * rinv * orc_bf16_to_f32(j->kw[pd]);
                const float sgn = (g_fault == 5) ? -1.0f : 1.0f;
                kd = dd < 256 ? kn * c - sgn * kn2 * sn : kn * c + sgn * kn2 * sn;
            }
            dot += qd[dd] * (double) bf(kd);
        }
        s[t] = dot * (double) j->scale;
        if (s[t] > mx) mx = s[t];
    }
    double den = 0.0;
    for (int32_t t = 0; t < j->len; ++t) { s[t] = exp(s[t] - mx); den += s[t]; }
    for (int32_t t = 0; t < j->len; ++t) {
        raw_row(j, kvh, t, xr);
        const double w = s[t] / den * rv[t];
        for (int32_t i = 0; i < D; ++i) acc[i] += w * (double) xr[i];
    }
    for (int32_t i = 0; i < D; ++i) j->out[(size_t) h * D + i] = acc[i];
    free(s); free(rv);
}

int32_t orc_decode_raw_f64(const uint16_t *q, const uint16_t *raw, int32_t Hkv, int32_t len,
                           int32_t pitch, const uint16_t *kw, float eps, const float *inv_freq,
                           float scale, double *out, int32_t nthreads) {
    if (Hkv <= 0 || len <= 0 || pitch < len) return -1;
    raw_job_t j = {q, raw, kw, inv_freq, Hkv, len, pitch, eps, scale, out, NULL, NULL, NULL};
    run_items(item_raw, &j, (int64_t) Hkv * 8, nthreads);
    return 0;
}

int32_t orc_decode_raw_q8_f64(const uint16_t *q, const uint8_t *qraw, const float *sc, const float *bs,
                              int32_t Hkv, int32_t len, int32_t pitch, const uint16_t *kw, float eps,
                              const float *inv_freq, float scale, double *out, int32_t nthreads) {
    if (Hkv <= 0 || len <= 0 || pitch < len) return -1;
    raw_job_t j = {q, NULL, kw, inv_freq, Hkv, len, pitch, eps, scale, out, qraw, sc, bs};
    run_items(item_raw, &j, (int64_t) Hkv * 8, nthreads);
    return 0;
}

/* Per-row affine u8 (ESDecodeAttn.mm:491-509, ESKVCache.mm:506-511): over the row's n
 * values (bf16 -> fp32), mn = min, mx = max; scale = max((mx - mn) / 255, 1e-8);
 * q = min(round((x - mn) / scale), 255) with round half away from zero; bias = mn.
 * IEEE fp32 subtraction and division. */
void orc_quantize_rows(const uint16_t *x, int64_t rows, int32_t n, uint8_t *q, float *scale,
                       float *bias) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * n;
        float mn = INFINITY, mx = -INFINITY;
        for (int32_t i = 0; i < n; ++i) {
            const float v = orc_bf16_to_f32(xr[i]);
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        float sc = (mx - mn) / 255.0f;
        if (!(sc > 1e-8f)) sc = 1e-8f;
        if (g_fault == 6) sc = (mx - mn) / 256.0f;
        for (int32_t i = 0; i < n; ++i) {
            const float t = roundf((orc_bf16_to_f32(xr[i]) - mn) / sc);
            q[r * n + i] = (uint8_t) (t < 255.0f ? t : 255.0f);
        }
        scale[r] = sc;
        bias[r] = mn;
    }
}

/* ------------------------------------------------------------ prefill */

typedef struct {
    const uint16_t *q, *k, *v;
    int64_t q_head_stride, q_row_stride, kv_head_stride;
    int32_t Hq, Hkv, D, Sq, Sk, q_pos0, k_pos0, window;
    float scale;
    double *out;
    int32_t status;
} prefill_job_t;

/* Key j (absolute k_pos0 + j) is visible to query i (absolute q_pos0 + i) under the
 * additive mask of buildMask (ESGemma4TextModel.mm:68-83: kAbs <= qAbs, and on sliding
 * layers kAbs > qAbs - window) aligned to the retained keys by alignMask
 * (ESAttention.mm:17-22: the last Sk columns). */
static int prefill_visible(const prefill_job_t *j, int32_t i, int32_t kj) {
    const int64_t qa = (int64_t) j->q_pos0 + i, ka = (int64_t) j->k_pos0 + kj;
    if (g_fault == 7 ? ka >= qa : ka > qa) return 0; /* planted: the diagonal masked */
    if (j->window > 0 && ka <= qa - j->window) return 0;
    return 1;
}

/* One (query row, query head): O = softmax(scale * q K^T + M) V over the visible keys,
 * GQA kv-major (ESOps.h:64-68), fp64. */
static void item_prefill(void *ctx, int64_t it) {
    prefill_job_t *j = (prefill_job_t *) ctx;
    const int32_t i = (int32_t) (it / j->Hq), h = (int32_t) (it % j->Hq), D = j->D;
    const int32_t g = j->Hq / j->Hkv;
    const int32_t kvh = g_fault == 1 ? h % j->Hkv : h / g;
    const float scale = g_fault == 3 ? 1.0f : j->scale;
    double *out = j->out + ((size_t) i * j->Hq + h) * D;
    double *qd = (double *) malloc(sizeof(double) * D);
    double *s = (double *) malloc(sizeof(double) * (j->Sk > 0 ? j->Sk : 1));
    const uint16_t *qh = j->q + (size_t) h * j->q_head_stride + (size_t) i * j->q_row_stride;
    for (int32_t d = 0; d < D; ++d) qd[d] = orc_bf16_to_f32(qh[d]);
    const uint16_t *kb = j->k + (size_t) kvh * j->kv_head_stride, *vb = j->v + (size_t) kvh * j->kv_head_stride;
    double mx = -INFINITY;
    int32_t n = 0;
    for (int32_t t = 0; t < j->Sk; ++t) {
        if (!prefill_visible(j, i, t)) { s[t] = -INFINITY; continue; }
        const uint16_t *kr = kb + (size_t) t * D;
        double acc = 0.0;
        for (int32_t d = 0; d < D; ++d) acc += qd[d] * (double) orc_bf16_to_f32(kr[d]);
        s[t] = acc * (double) scale;
        if (s[t] > mx) mx = s[t];
        ++n;
    }
    for (int32_t d = 0; d < D; ++d) out[d] = 0.0;
    if (n == 0) { j->status = -1; free(qd); free(s); return; }
    double den = 0.0;
    for (int32_t t = 0; t < j->Sk; ++t) { s[t] = s[t] == -INFINITY ? 0.0 : exp(s[t] - mx); den += s[t]; }
    for (int32_t t = 0; t < j->Sk; ++t) {
        if (s[t] == 0.0) continue;
        const uint16_t *vr = vb + (size_t) t * D;
        const double w = s[t] / den;
        for (int32_t d = 0; d < D; ++d) out[d] += w * (double) orc_bf16_to_f32(vr[d]);
    }
    free(qd); free(s);
}

int32_t orc_prefill_f64(const uint16_t *q, int64_t q_head_stride, int64_t q_row_stride,
                        const uint16_t *k, const uint16_t *v, int64_t kv_head_stride,
                        int32_t Hq, int32_t Hkv, int32_t D, int32_t Sq, int32_t Sk,
                        int32_t q_pos0, int32_t k_pos0, int32_t window, float scale,
                        double *out, int32_t nthreads) {
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || Sq <= 0 || Sk <= 0 || window < 0) return -1;
    prefill_job_t j = {q, k, v, q_head_stride, q_row_stride, kv_head_stride,
                       Hq, Hkv, D, Sq, Sk, q_pos0, k_pos0, window, scale, out, 0};
    run_items(item_prefill, &j, (int64_t) Sq * Hq, nthreads);
    return j.status;
}

/* Raw-K prefill reconstruction, ESAttention.mm:306-326, per kv head h and row t (absolute
 * position pos0 + t):
 *   rinv = 1 / sqrt(mean(x^2) + eps) (ESRMSNorm, f32)
 *   K0 = bf16(x * rinv * kw), V = bf16(x * rinv)           (kNorm_, vNorm_)
 *   c, s = bf16(cos / sin(f32(pos * inv_freq[f]))), f = d mod D/2 (emb = [freqs, freqs])
 *   K = bf16(bf16(K0 * c) + bf16(rotateHalf(K0) * s)), rotateHalf(K0)[d] = -K0[d + D/2]
 *       for d < D/2 and K0[d - D/2] above (ESOps.h:58-62)
 * raw, k, v: [Hkv, Sk, D] dense; inv_freq: D/2 entries. */
void orc_raw_prefill_kv(const uint16_t *raw, int32_t Hkv, int32_t Sk, int32_t D, const uint16_t *kw,
                        float eps, const float *inv_freq, int32_t pos0, uint16_t *k, uint16_t *v) {
    const int32_t half = D / 2;
    float *x = (float *) malloc(sizeof(float) * D);
    float *k0 = (float *) malloc(sizeof(float) * D);
    for (int64_t r = 0; r < (int64_t) Hkv * Sk; ++r) {
        const int32_t t = (int32_t) (r % Sk);
        const uint16_t *xr = raw + r * D;
        float ss = 0.0f;
        for (int32_t d = 0; d < D; ++d) { x[d] = orc_bf16_to_f32(xr[d]); ss += x[d] * x[d]; }
        const float rinv = 1.0f / sqrtf(ss / (float) D + eps);
        for (int32_t d = 0; d < D; ++d) {
            k0[d] = bf(x[d] * rinv * orc_bf16_to_f32(kw[d]));
            v[r * D + d] = orc_f32_to_bf16(x[d] * rinv);
        }
        for (int32_t d = 0; d < D; ++d) {
            const float a = (float) (pos0 + t) * inv_freq[d % half];
            const float c = bf(cosf(a)), sn = bf(sinf(a));
            float rh = d < half ? -k0[d + half] : k0[d - half];
            if (g_fault == 8) rh = -rh; /* planted: rotateHalf with the wrong sign */
            k[r * D + d] = orc_f32_to_bf16(bf(k0[d] * c) + bf(rh * sn));
        }
    }
    free(x); free(k0);
}
