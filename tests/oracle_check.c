/* oracle_check.c -- runs every function of the CPU oracle (oracle/oracle.c) on small
 * seeded inputs, ragged and edge-case shapes included (rings, windows, row bases,
 * padded strides, one visible row, out-of-range positions, invalid descriptions).
 * Built by tests/test_sanitizers.py with AddressSanitizer and UndefinedBehaviorSanitizer:
 * an out-of-bounds access, overflow or leak aborts the run.  It also checks that every
 * output is finite and that the fp64, reference-rounding and split-K modes agree within
 * the parity tolerance. */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int g_fail = 0;
#define CHECK(c, msg)                                         \
    do {                                                      \
        if (!(c)) {                                           \
            printf("FAIL %s: %s\n", #c, msg);                 \
            ++g_fail;                                         \
        }                                                     \
    } while (0)

static unsigned long long g_rng = 88172645463325252ULL;
static double urand(void) {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (double) (g_rng >> 11) / 9007199254740992.0;
}
static int irand(int lo, int hi) { return lo + (int) (urand() * (hi - lo + 1)); }

static void fill_bf16(uint16_t *x, size_t n, float amp) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_f32_to_bf16((float) ((urand() * 2.0 - 1.0) * amp));
}

static void decode_case(int B, int Hq, int Hkv, int D, int cap, int window, int ring, int pad) {
    orc_desc d;
    d.B = B; d.Hq = Hq; d.Hkv = Hkv; d.D = D; d.cap = cap; d.window = window; d.ring = ring;
    d.head_stride = (int64_t) cap * D + pad;
    d.seq_stride = (int64_t) Hkv * d.head_stride + pad;
    d.scale = 1.0f / sqrtf((float) D);
    const size_t ce = (size_t) B * (size_t) d.seq_stride;
    uint16_t *q = malloc(sizeof(uint16_t) * (size_t) B * Hq * D);
    uint16_t *k = malloc(sizeof(uint16_t) * ce), *v = malloc(sizeof(uint16_t) * ce);
    uint16_t *kn = malloc(sizeof(uint16_t) * (size_t) B * Hkv * D), *vn = malloc(sizeof(uint16_t) * (size_t) B * Hkv * D);
    int32_t *pos = malloc(sizeof(int32_t) * B), *rb = malloc(sizeof(int32_t) * B);
    fill_bf16(q, (size_t) B * Hq * D, 1.5f);
    fill_bf16(k, ce, 1.5f);
    fill_bf16(v, ce, 1.5f);
    fill_bf16(kn, (size_t) B * Hkv * D, 1.5f);
    fill_bf16(vn, (size_t) B * Hkv * D, 1.5f);
    for (int b = 0; b < B; ++b) {
        pos[b] = ring ? irand(0, 4 * cap) : irand(0, cap - 1);
        rb[b] = (!ring && pos[b] > 0 && irand(0, 2) == 0) ? irand(0, pos[b]) : 0;
    }
    CHECK(orc_append(&d, k, v, kn, vn, pos, ring ? NULL : rb) == 0, "append");
    double *o64 = malloc(sizeof(double) * (size_t) B * Hq * D);
    uint16_t *orr = malloc(sizeof(uint16_t) * (size_t) B * Hq * D);
    float *osk = malloc(sizeof(float) * (size_t) B * Hq * D);
    const int32_t *r = ring ? NULL : rb;
    CHECK(orc_decode_f64(&d, q, k, v, pos, r, o64, 3) == 0, "decode_f64");
    CHECK(orc_decode_refround(&d, q, k, v, pos, r, orr, 2) == 0, "decode_refround");
    CHECK(orc_decode_splitk(&d, q, k, v, pos, r, irand(1, 9), osk, 4) == 0, "decode_splitk");
    /* the grouped restatement (the CPU baseline): one split equals refround bit for bit */
    uint16_t *og = malloc(sizeof(uint16_t) * (size_t) B * Hq * D);
    CHECK(orc_decode_refround_grouped(&d, q, k, v, pos, r, 1, og, 2) == 0, "decode_refround_grouped");
    CHECK(memcmp(og, orr, sizeof(uint16_t) * (size_t) B * Hq * D) == 0, "grouped with one split equals refround");
    CHECK(orc_decode_refround_grouped(&d, q, k, v, pos, r, irand(2, 9), og, 3) == 0, "decode_refround_grouped splits");
    free(og);
    double worst = 0.0;
    for (size_t i = 0; i < (size_t) B * Hq * D; ++i) {
        CHECK(isfinite(o64[i]) && isfinite(osk[i]), "finite output");
        const double e1 = fabs(o64[i] - (double) orc_bf16_to_f32(orr[i])), e2 = fabs(o64[i] - (double) osk[i]);
        if (e1 > worst) worst = e1;
        if (e2 > worst) worst = e2;
    }
    CHECK(worst <= 2e-2, "modes agree within tolerance");
    /* visible rows of every sequence stay inside the cache */
    int32_t *rows = malloc(sizeof(int32_t) * ((size_t) cap + 1));
    for (int b = 0; b < B; ++b) {
        const int32_t n = orc_visible(&d, pos[b], ring ? 0 : rb[b], rows);
        CHECK(n >= 1 && n <= cap, "visible count");
        for (int32_t t = 0; t < n; ++t) CHECK(rows[t] >= 0 && rows[t] < cap, "visible row in the cache");
    }
    /* a position outside a linear cache is refused, and so is a bad description */
    if (!ring) {
        CHECK(orc_visible(&d, cap, 0, rows) <= 0, "out-of-range position");
    }
    orc_desc bad = d;
    bad.head_stride = (int64_t) cap * D - 1;  /* rows would overlap: refused before any access */
    CHECK(orc_decode_f64(&bad, q, k, v, pos, r, o64, 1) != 0, "invalid description refused");
    bad = d;
    bad.window = -1;
    CHECK(orc_decode_refround(&bad, q, k, v, pos, r, orr, 1) != 0, "negative window refused");
    free(q); free(k); free(v); free(kn); free(vn); free(pos); free(rb); free(o64); free(orr); free(osk); free(rows);
}

static void raw_case(int Hkv, int len, int pitch) {
    const int D = 512;
    uint16_t *q = malloc(sizeof(uint16_t) * Hkv * 8 * D), *raw = malloc(sizeof(uint16_t) * (size_t) Hkv * pitch * D);
    uint16_t *kw = malloc(sizeof(uint16_t) * D);
    float inv[256];
    double *o = malloc(sizeof(double) * Hkv * 8 * D), *o8 = malloc(sizeof(double) * Hkv * 8 * D);
    fill_bf16(q, (size_t) Hkv * 8 * D, 1.0f);
    fill_bf16(raw, (size_t) Hkv * pitch * D, 3.0f);
    for (int i = 0; i < D; ++i) kw[i] = orc_f32_to_bf16((float) (1.0 + 0.2 * (urand() - 0.5)));
    orc_rope_inv_freq(D, 1.0e6f, 0.25f, inv);
    CHECK(orc_decode_raw_f64(q, raw, Hkv, len, pitch, kw, 1e-6f, inv, 1.0f, o, 2) == 0, "decode_raw_f64");
    uint8_t *qr = malloc((size_t) Hkv * pitch * D);
    float *sc = malloc(sizeof(float) * Hkv * pitch), *bs = malloc(sizeof(float) * Hkv * pitch);
    orc_quantize_rows(raw, (int64_t) Hkv * pitch, D, qr, sc, bs);
    CHECK(orc_decode_raw_q8_f64(q, qr, sc, bs, Hkv, len, pitch, kw, 1e-6f, inv, 1.0f, o8, 2) == 0, "decode_raw_q8_f64");
    for (int i = 0; i < Hkv * 8 * D; ++i) CHECK(isfinite(o[i]) && isfinite(o8[i]), "finite raw output");
    uint16_t *y = malloc(sizeof(uint16_t) * (size_t) Hkv * pitch * D);
    orc_rms_norm_rows(raw, kw, (int64_t) Hkv * pitch, D, 1e-6f, y);
    orc_rms_norm_rows(raw, NULL, (int64_t) Hkv * pitch, D, 1e-6f, y);
    uint16_t *kk = malloc(sizeof(uint16_t) * (size_t) Hkv * len * D), *vv = malloc(sizeof(uint16_t) * (size_t) Hkv * len * D);
    orc_raw_prefill_kv(raw, Hkv, len, D, kw, 1e-6f, inv, 3, kk, vv);
    free(q); free(raw); free(kw); free(o); free(o8); free(qr); free(sc); free(bs); free(y); free(kk); free(vv);
}

static void prefill_case(int Hq, int Hkv, int D, int Sq, int past, int window) {
    const int Sk = past + Sq;
    uint16_t *q = malloc(sizeof(uint16_t) * (size_t) Hq * Sq * D);
    uint16_t *k = malloc(sizeof(uint16_t) * (size_t) Hkv * Sk * D), *v = malloc(sizeof(uint16_t) * (size_t) Hkv * Sk * D);
    double *o = malloc(sizeof(double) * (size_t) Sq * Hq * D);
    fill_bf16(q, (size_t) Hq * Sq * D, 1.0f);
    fill_bf16(k, (size_t) Hkv * Sk * D, 1.0f);
    fill_bf16(v, (size_t) Hkv * Sk * D, 1.0f);
    CHECK(orc_prefill_f64(q, (int64_t) Sq * D, D, k, v, (int64_t) Sk * D, Hq, Hkv, D, Sq, Sk, past, 0, window,
                          1.0f / sqrtf((float) D), o, 3) == 0, "prefill_f64");
    for (size_t i = 0; i < (size_t) Sq * Hq * D; ++i) CHECK(isfinite(o[i]), "finite prefill output");
    free(q); free(k); free(v); free(o);
}

int main(void) {
    for (int it = 0; it < 60; ++it) {
        const int D = (int[]){128, 256, 512}[irand(0, 2)];
        const int Hkv = irand(1, 4), G = (int[]){1, 2, 4, 8}[irand(0, 3)];
        const int ring = irand(0, 2) == 0;
        const int cap = irand(1, 200);
        const int window = ring ? irand(1, cap) : (irand(0, 1) ? 0 : irand(1, cap));
        decode_case(irand(1, 4), Hkv * G, Hkv, D, cap, window, ring, irand(0, 1) ? 0 : 8 * irand(1, 5));
    }
    raw_case(2, 1, 1);
    raw_case(1, 37, 40);
    raw_case(3, 64, 64);
    prefill_case(8, 2, 128, 5, 0, 0);
    prefill_case(4, 4, 256, 3, 20, 8);
    prefill_case(8, 1, 512, 1, 7, 0);
    printf("%s: %d failures\n", g_fail ? "FAIL" : "OK", g_fail);
    return g_fail ? 1 : 0;
}
