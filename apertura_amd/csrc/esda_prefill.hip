// esda_prefill.hip -- Gemma-4 prefill attention for MI355X (gfx950, CDNA4).
//
// Reference behaviour (Apertura tree): a chunk of seq > 1 new tokens attends the cache
// through mx::fast::scaled_dot_product_attention (ESAttention.mm:188; raw-K layers
// :328 after the op-level reconstruction :306-326) with the additive mask of
// ESGemma4TextModel.mm:68-83 aligned by ESAttention.mm:17-22; the op-level tiled core
// (ESAttention.mm:195-251) computes the same quantity by online softmax.
//
// Kernels
//   prefill_kernel<D, QB>  one workgroup per (query tile, kv head, key split), 8 waves
//                       (two per SIMD), one workgroup per CU; QB 16-query blocks per wave
//                       (one at D = 512, one or two at D = 256, two at D = 128).  A
//                       query tile is 128 QB query rows of one kv head's GQA group,
//                       ordered position-major (row r: position r / G, group head r % G);
//                       wave w owns rows 16 QB w .. as QB blocks of 16 -- the MFMA N
//                       dimension.  The tile's visible keys (or one split of them)
//                       stream through an LDS ring of 32-key stages filled by LDS DMA,
//                       the next stage landing during this one.  Per stage each
//                       wave forms S^T[32 keys x its queries] over the whole head dim
//                       with v_mfma_f32_16x16x32_bf16 (K rows from LDS, Q^T held in
//                       registers), masks boundary stages by position, runs an fp32
//                       online softmax per query column, and accumulates O^T[D x its
//                       queries] += V^T . P^T, V^T by transpose reads from LDS and P^T
//                       straight from the score registers (the 32 keys are ordered so
//                       that the score layout is the B-operand layout).  O^T stays in
//                       registers (D/16 x QB tiles: QB * D / 16 accumulators per lane).
//   prefill_kernel<256, 1, true>  the same with 64-row tiles whose even and odd stages go
//                       to the two wave groups (waves 0-3 and 4-7 on the same query
//                       blocks), folded together through LDS at the end: short chunks
//                       at D = 256 fill the CUs with tiles instead of key splits.
//   prefill_merge_kernel  reduces split partials (m, l, acc) per (query row, head).
//   raw_prefill_kv_kernel rebuilds K and V of a raw-K (or q8 raw-K) stream by the
//                       reference's op-level rounding points.
// The C ABI (include/esda_prefill.h) is at the end of the file.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <string>

#include "esda.h"
#include "esda_device.h"
#include "esda_internal.h"
#include "esda_prefill.h"

namespace {

constexpr int kStageKeys = 32;
constexpr int kBlk = 1056;                 // LDS bytes per DMA block: 1 KB + 32 B pad
constexpr int kRingBudget = 136 * 1024;    // LDS bytes for the K / V ring
constexpr int kTargetGroups = 256;         // one workgroup per CU
// K / V stream loads without the non-temporal hint: the tiles of one kv head read the
// same keys, and the L2 keeping them for the next tile was measured 2-12% faster.
constexpr bool kStreamNT = false;

struct PrefillParams {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    float *part_acc;   // [splits][Sq * Hq][D]
    float *part_ml;    // [splits][Sq * Hq][2]
    long long q_hs, q_rs, kv_hs, o_rs, o_hs;
    int Hq, Hkv, G, Sq, Sk, q_pos0, k_pos0, window;
    int qb;                  // 16-query blocks per wave (query tile: 128 qb rows, 64 with kh)
    int tiles, splits, kps;  // query tiles per kv head, key splits, keys per split
    float scale_log2e;
    int kh;                  // 1: the two wave groups split each tile's stages (even / odd)
};

// Keys [j0, j1) that some row of query tile `tile` (QT rows) can see.
__host__ __device__ inline void tile_keys(const PrefillParams &p, int tile, int QT, int &j0, int &j1) {
    const long long rows = (long long) p.Sq * p.G;
    const long long r0 = (long long) tile * QT;
    const long long r1 = (r0 + QT < rows ? r0 + QT : rows) - 1;
    const long long qa0 = p.q_pos0 + r0 / p.G, qa1 = p.q_pos0 + r1 / p.G;
    long long lo = p.window > 0 ? qa0 - p.window + 1 - p.k_pos0 : 0;
    long long hi = qa1 - p.k_pos0 + 1;
    if (lo < 0) lo = 0;
    if (hi > p.Sk) hi = p.Sk;
    if (hi < lo) hi = lo;
    j0 = (int) lo;
    j1 = (int) hi;
}

// LDS ring geometry for head dim D: a 16-key half stage is NI DMA blocks of kBlk bytes,
// block b holding keys b + NI*q (q < 512/D) at +2D*q; a stage is the K halves then the V
// halves.  Both the 128-bit row reads (QK A operand) and the transpose reads (PV A
// operand) are bank-conflict-free in this layout (the decode kernel's measured layout).
// Eight waves per workgroup (two per SIMD) and QB 16-query blocks per wave.  O^T takes
// QB * D / 16 accumulator registers per lane beside Q^T's QB * D / 8 and 8 QB of scores,
// within the 256 registers of two waves per SIMD: QB = 1 at D = 512 (two blocks do not
// fit without spills), 1 or 2 at D = 256 (pick_qb), 2 at D = 128.  (Measured: at D = 256,
// four waves of two blocks -- one wave per SIMD -- ran 6% slower than eight waves of one
// block, and forming the next stage's scores during this stage's softmax -- a second set
// of score registers, forcing one block per wave at D = 256 -- was 5-20% slower.)
//
// KH (stage halves, D = 256 with one block per wave): waves w and w + 4 own the same query
// block and take the even and the odd stages of the tile's keys, over a ring of four
// stages per tensor (132 KB), and fold their (m, l, O^T) together through LDS at the end.
// A tile is then 64 query rows, so a chunk whose 128-row tiles would leave CUs idle gets
// twice the tiles instead of key splits -- no fp32 partials and no merge launch -- while
// each wave's work per stage and the barriers per stage stay those of the plain kernel.
constexpr int kWaves = 8;
#ifndef PV_DEPTH
#define PV_DEPTH 4
#endif
constexpr int kPairSpin = 1 << 20;  // PS: polls of the partner's flag before a wave gives up

template <int D, int NSL, int NT = 2>
struct PRing {
    static constexpr int NI = D / 32;                 // DMA blocks per 16-key half
    static constexpr int HB = NI * kBlk;              // one half stage of one tensor
    static constexpr int BYTES = 2 * NT * NSL * HB;   // NSL K stages, then NSL V stages (NT = 2)
    static constexpr int CPR = D / 8;                 // 16-byte chunks per row
    static_assert(BYTES <= kRingBudget, "the K / V slots must fit the LDS budget");
    __host__ __device__ static constexpr int off(int r) { return (r % NI) * kBlk + (r / NI) * 2 * D; }
};

// SH: V is the K buffer (attention_k_eq_v): one tensor streams, and PV reads V^T from the
// stage's K slot.  S2 (with SH, in the LDS the second tensor leaves free): every wave computes
// two stages per iteration, so the workgroup meets at one barrier per 64 keys.
//
// PS (pair split, one block per wave): waves w and w^1 (on different SIMDs) each score and
// softmax their own query block over the whole head dim, as above, but accumulate O^T for
// both blocks of the pair over half of the head dim each (wave w: dims D/2 (w & 1) on).
// Each V^T tile read from LDS then feeds two MFMAs, which halves the kernel's transpose
// reads for an exchange of P^T (1 KB per wave and stage) through LDS: the wave writes its
// P^T (and, after a rescale, its factors), then a flag, and reads its partner's once the
// partner's flag shows the stage.  The buffers alternate by stage parity: a wave rewrites a
// parity only after reading its partner's next flag, which the partner writes after reading
// this stage's P^T.  Used by the K = V kernel at D = 512 (p512gs 436 -> 422 us on one box);
// with separate K and V -- one stage per barrier -- it measured 1-3% slower and is not used.
template <int D, int QB, bool KH = false, bool SH = false, bool S2 = false, bool PS = false>
__global__ __launch_bounds__(64 * kWaves, 1) void prefill_kernel(PrefillParams p) {
    static_assert(!S2 || !KH, "two stages per iteration: all waves on both");
    static_assert(!PS || (QB == 1 && !KH), "pair split: one block per wave, every wave on every stage");
    constexpr int NQW = KH ? kWaves / 2 : kWaves;  // waves with distinct query blocks
    constexpr int NSL = KH || S2 ? 4 : 2;          // ring stages per tensor
    constexpr int SPI = KH || S2 ? 2 : 1;          // stages per iteration (KH: one per wave group)
    using R = PRing<D, NSL, SH ? 1 : 2>;
    constexpr int QT = 16 * QB * NQW;   // query rows per tile
    constexpr int KS = D / 32;          // QK k-steps
    constexpr int DT = D / 16;          // PV dim tiles
    constexpr int NB = PS ? 2 : QB;     // O^T blocks per wave
    constexpr int DW = PS ? DT / 2 : DT;  // O^T dim tiles per wave
    __shared__ __attribute__((aligned(16))) unsigned char ring[R::BYTES];
    // PS exchange, per stage parity: each wave's P^T (16 B per lane) and rescale factors
    // (4 B per lane), then one flag per wave; after both parities, each wave's row sums.
    constexpr int XP = 64 * 16 + 64 * 4;
    constexpr int XPAR = kWaves * XP + kWaves * 4;
    __shared__ __attribute__((aligned(16))) unsigned char xch[PS ? 2 * XPAR + kWaves * 16 * 4 : 16];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // Query-block wave and stage parity (both constant for the plain kernel, whose code
    // does not change: a wave-dependent parity there measured 3% slower).
    const int wq = KH ? wave % NQW : wave, kh = KH ? wave / NQW : 0;
    const int hd = PS ? (wave & 1) : 0;  // PS: this wave's half of the head dim
    // Workgroup -> (tile, kv head, split): consecutive workgroups go to consecutive XCDs
    // (dispatch is round-robin over the 8), so the (kv head, split) pair is the fastest
    // index and the workgroups on one XCD share one K / V stream in its L2; tiles run
    // heaviest (latest) first.
    const int combos = p.Hkv * p.splits;
    const int wg = (int) blockIdx.x;
    const int tile = p.tiles - 1 - wg / combos;
    const int kvh = (wg % combos) % p.Hkv, split = (wg % combos) / p.Hkv;
    const long long nrows = (long long) p.Sq * p.Hq;

    int tj0, tj1;
    tile_keys(p, tile, QT, tj0, tj1);
    const int j0 = min(tj1, tj0 + split * p.kps);
    const int j1 = min(tj1, j0 + p.kps);

    // This lane's query row in block qb: tile row wq*16*QB + 16qb + li, global row gr
    // (position gr / G, head kvh*G + gr % G); rows past the end repeat the last row and
    // are not written.
    const long long nq = (long long) p.Sq * p.G;
    auto qrow = [&](int qb) -> long long {
        const long long gr = (long long) tile * QT + wq * 16 * QB + qb * 16 + li;
        return gr < nq ? gr : nq - 1;
    };
    auto qvalid = [&](int qb) { return (long long) tile * QT + wq * 16 * QB + qb * 16 + li < nq; };

    if (j0 >= j1) {  // an empty split: no keys for this tile; the merge skips it
        if (p.splits > 1 && lg == 0 && kh == 0) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
                if (qvalid(qb)) {
                    const long long gr = qrow(qb);
                    const long long row = (gr / p.G) * p.Hq + kvh * p.G + gr % p.G;
                    *reinterpret_cast<f32x2 *>(p.part_ml + 2 * ((long long) split * nrows + row)) =
                        f32x2{-INFINITY, 0.0f};
                }
        }
        return;
    }

    // Q^T B operands: lane (li, lg) holds dims 32ks + 8lg .. +8 of its query row.
    bf16x8 qreg[QB][KS];
    int qabs[QB];  // absolute position of this lane's query in block qb
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const long long gr = qrow(qb);
        const uint16_t *qr = p.q + (size_t) (kvh * p.G + gr % p.G) * p.q_hs + (size_t) (gr / p.G) * p.q_rs + lg * 8;
        qabs[qb] = p.q_pos0 + (int) (gr / p.G);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 w = qvalid(qb) ? *reinterpret_cast<const u32x4 *>(qr + ks * 32) : u32x4{0u, 0u, 0u, 0u};
            qreg[qb][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }

    // LDS: NSL K slots then NSL V slots, each a 32-key stage (two 16-key halves).  Stage
    // s's K sits in K slot s % NSL and its V in V slot s % NSL.  Iteration i computes the
    // SPI stages SPI*i .. (one per wave group); after its barrier the stages of iteration
    // i+1 replace those of iteration i-1 (every wave is done with them) and land while
    // iteration i computes.
    //
    // DMA: K instruction t of this wave (ii = wave*KPW + t of the stage's 2 NI) fills block
    // b = ii % NI of half hh = ii / NI; lane l reads chunk l % CPR of stage row
    // r = 16hh + b + NI*(l / CPR).  V likewise.  Interior stages add the lane's byte offset
    // to a wave-uniform base; the last, partial stage clamps each row to the range.
    constexpr int KPW = 2 * R::NI / kWaves;  // DMA instructions per wave per tensor per stage
    static_assert(KPW * kWaves == 2 * R::NI, "whole DMA blocks per wave");
    const uint16_t *kvb = p.k + (size_t) kvh * p.kv_hs;
    const uint16_t *vvb = p.v + (size_t) kvh * p.kv_hs;
    const int nst = (j1 - j0 + kStageKeys - 1) / kStageKeys;
    unsigned voff[KPW];
    int vrow[KPW], ldso[KPW];
#pragma unroll
    for (int t = 0; t < KPW; ++t) {
        const int ii = wave * KPW + t, hh = ii / R::NI, b = ii % R::NI;
        vrow[t] = 16 * hh + b + R::NI * (lane / R::CPR);
        voff[t] = (unsigned) ((vrow[t] * D + (lane % R::CPR) * 8) * 2);
        ldso[t] = hh * R::HB + b * kBlk;
    }
    static_assert((NSL & (NSL - 1)) == 0, "stage slots: a power of two");
    auto kslot = [&](int s) { return ring + (s & (NSL - 1)) * 2 * R::HB; };
    auto vslot = [&](int s) { return SH ? kslot(s) : ring + 2 * NSL * R::HB + (s & (NSL - 1)) * 2 * R::HB; };
    auto issue = [&](const uint16_t *head, int s, unsigned char *slot) {
        const int jb = j0 + s * kStageKeys;
        if (jb + kStageKeys <= j1) {
            const uint16_t *base = head + (size_t) jb * D;
#pragma unroll
            for (int t = 0; t < KPW; ++t) lds_dma16_s<kStreamNT>(base, voff[t], lds_addr(slot) + ldso[t]);
        } else {
#pragma unroll
            for (int t = 0; t < KPW; ++t) {
                const int j = min(jb + vrow[t], j1 - 1);  // rows past the range repeat the last key
                lds_dma16<kStreamNT>(head + (size_t) j * D + (lane % R::CPR) * 8, lds_addr(slot) + ldso[t]);
            }
        }
    };

    const int qk_off = R::off(li) + lg * 16;                    // + 64 ks (+ HB: keys 16..31)
    const int tr_off = R::off(4 * lg + li / 4) + (li % 4) * 8;  // + 32 dt (+ HB)

    float m[QB], l[QB];
    f32x4 acc[NB][DW];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m[qb] = -INFINITY;
        l[qb] = 0.0f;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int dt = 0; dt < DW; ++dt) acc[nb][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // PS flags start at 0 (stage s shows as 2 (s + 1), plus 1 after a rescale); the loop's
    // first barrier orders these stores before any wave reads them.
    // (Flags are read and written through LDS pointers: a generic volatile access would be
    // a flat one, whose wait also drains the ring's DMAs.)
    using lds_flag = __attribute__((address_space(3))) volatile unsigned;
    if constexpr (PS) {
        if (lane < 2) *(lds_flag *) (xch + lane * XPAR + kWaves * XP + wave * 4) = 0u;
    }
    // Positions of the tile's first and last rows (the host keeps positions below 2^31).
    const int qa_min = p.q_pos0 + (int) ((long long) tile * QT / p.G);
    const int qa_max = p.q_pos0 + (int) (((long long) tile * QT + QT < nq ? (long long) tile * QT + QT : nq) - 1) / p.G;

    // S^T[keys x queries] of a stage: s[h][qb] covers keys 16h + 4lg + r of query column li.
    struct Scores {
        f32x4 s[2][QB];
    };
    auto qk = [&](const unsigned char *kb) {
        Scores sc;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sc.s[h][qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 ka0 = *reinterpret_cast<const bf16x8 *>(kb + qk_off + 64 * ks);
            const bf16x8 ka1 = *reinterpret_cast<const bf16x8 *>(kb + R::HB + qk_off + 64 * ks);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                sc.s[0][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka0, qreg[qb][ks], sc.s[0][qb], 0, 0, 0);
                sc.s[1][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka1, qreg[qb][ks], sc.s[1][qb], 0, 0, 0);
            }
        }
        return sc;
    };

    issue(kvb, 0, kslot(0));  // nst >= 1 here
    if (!SH) issue(vvb, 0, vslot(0));
    if ((KH || S2) && nst > 1) {
        issue(kvb, 1, kslot(1));
        if (!SH) issue(vvb, 1, vslot(1));
    }

    for (int s0 = 0; s0 < nst; s0 += SPI) {
        // The iteration's stages s0 .. s0+SPI-1 landed (this wave's loads; the barrier covers
        // the other waves') and every wave is done with the previous iteration
        ESDA_WAIT_VM(0);
        lds_barrier();
        // The next iteration's DMAs, spread over this iteration so that the workgroup's loads
        // do not all queue at the barrier (each slot is free once the barrier has passed):
        //  - separate K and V (plain, S2): K of the next stage at the barrier, its V after
        //    this iteration's first QK;
        //  - one K = V stream (S2): the next stage after the first QK;
        //  - S2: the stage after that once this iteration's first stage is done;
        //  - KH: all at the barrier (spreading measured slower there).
        constexpr bool kVLate = !SH && !KH;
        auto issue_k = [&]() {
            if (s0 + SPI < nst) issue(kvb, s0 + SPI, kslot(s0 + SPI));
        };
        auto issue_v = [&]() {
            if (!SH && s0 + SPI < nst) issue(vvb, s0 + SPI, vslot(s0 + SPI));
        };
        auto issue_second = [&]() {
            if (s0 + SPI + 1 < nst) {
                issue(kvb, s0 + SPI + 1, kslot(s0 + SPI + 1));
                if (!SH) issue(vvb, s0 + SPI + 1, vslot(s0 + SPI + 1));
            }
        };
        auto after_first_qk = [&]() {
            if constexpr (SH) issue_k();
            if constexpr (kVLate) issue_v();
        };
        if constexpr (!SH) issue_k();
        if constexpr (!kVLate && !SH) issue_v();
        if constexpr (KH) issue_second();
        auto stage = [&](const int s, auto after_qk) {
        const Scores cur = qk(kslot(s));
        after_qk();
        const unsigned char *vb = vslot(s);
        const int jb = j0 + s * kStageKeys;

        // Stage s's raw scores q.k; positions a boundary stage does not show to a row are
        // -inf.  A stage is fully visible to every row of the tile when its last key is at
        // or before the tile's first position, its first key is inside the window of the
        // tile's last position, and it lies inside the split.  The softmax scale (times
        // log2 e, > 0) is applied to the row maxima and inside the exponent's fma.
        const float c2 = p.scale_log2e;
        float sv[QB][8];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) sv[qb][4 * h + r] = cur.s[h][qb][r];
        const int ka_first = p.k_pos0 + jb, ka_last = ka_first + kStageKeys - 1;
        const bool full = jb + kStageKeys <= j1 && ka_last <= qa_min &&
                          (p.window == 0 || ka_first > qa_max - p.window);
        if (!full) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int qa = qabs[qb];
                const int lo = p.window > 0 ? qa - p.window : INT_MIN;  // visible: lo < ka <= qa
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int j = jb + 16 * h + 4 * lg + r;
                        const int ka = p.k_pos0 + j;
                        if (!(j < j1 && ka <= qa && ka > lo)) sv[qb][4 * h + r] = -INFINITY;
                    }
            }
        }

        // Row maxima of the stage in log2 units (scaling by c2 > 0 keeps the order).
        float mt[QB];
        bool need = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float x = sv[qb][0];
#pragma unroll
            for (int e = 1; e < 8; ++e) x = fmaxf(x, sv[qb][e]);
            mt[qb] = wave_max_across_groups(x) * c2;
            need = need || mt[qb] > m[qb] + kRescaleSlack;
        }

        // Raise the running max where a score exceeds it by the slack (rare): one
        // wave-uniform branch; lanes that do not need it scale by 1.
        unsigned char *const xs = xch + (PS ? (s & 1) * XPAR : 0);  // PS: this stage's exchange
        bool resc = false;
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(need) != 0, 0)) {
            asm volatile("" ::: "memory");  // keeps the rare rescale a branch (no if-conversion)
            resc = true;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const bool up = mt[qb] > m[qb] + kRescaleSlack;
                const float corr = up ? __builtin_amdgcn_exp2f(m[qb] - mt[qb]) : 1.0f;  // 0 while m is -inf
                l[qb] *= corr;
#pragma unroll
                for (int dt = 0; dt < DW; ++dt) acc[qb][dt] *= corr;
                m[qb] = up ? mt[qb] : m[qb];
                if constexpr (PS) *reinterpret_cast<float *>(xs + wave * XP + 1024 + lane * 4) = corr;
            }
        }

        bf16x8 pb[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float mu = m[qb] == -INFINITY ? 0.0f : m[qb];  // all keys so far masked
            bf16x8 pv;
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = (__bf16) __builtin_amdgcn_exp2f(__builtin_fmaf(sv[qb][e], c2, -mu));
            // l += the eight bf16 weights, two per v_dot2_f32_bf16 against (1, 1)
            const bf16x2 one2 = {(__bf16) 1.0f, (__bf16) 1.0f};
#pragma unroll
            for (int e = 0; e < 8; e += 2) l[qb] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pv[e], pv[e + 1]}, one2, l[qb], false);
            pb[qb] = pv;
        }
        if constexpr (PS) {  // P^T (and factors) to the partner, then the flag
            *reinterpret_cast<bf16x8 *>(xs + wave * XP + lane * 16) = pb[0];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane == 0)
                *(lds_flag *) (xs + kWaves * XP + wave * 4) = 2u * (unsigned) (s + 1) + (resc ? 1u : 0u);
        }

        // O^T += V^T . P^T: lane (li, lg) gets dim 16dt + li of keys 4lg .. 4lg+3 (first
        // half) and 16 + 4lg .. (second half): the k order of the P^T registers.
        // The V^T tiles are read PD ahead of their MFMAs (the scheduler alone kept one in flight).
        const unsigned char *const vbh = vb + 32 * DW * hd;  // PS: this wave's dims
        auto vtile = [&](int dt) {
            const short4v a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4v *) (vbh + tr_off + 32 * dt));
            const short4v a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4v *) (vbh + R::HB + tr_off + 32 * dt));
            const short8v a8 = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            return __builtin_bit_cast(bf16x8, a8);
        };
        constexpr int PD = PV_DEPTH;
        bf16x8 vf[PD];
#pragma unroll
        for (int i = 0; i < PD && i < DW; ++i) vf[i] = vtile(i);
        bf16x8 pq[NB];  // B operands: the wave's blocks (PS: its own, then its partner's)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) pq[qb] = pb[qb];
        if constexpr (PS) {
            // The partner's flag for this stage (bounded: a wave that gave up would compute
            // garbage, not hang), then its P^T and, after its rescale, its factors.
            const unsigned want = 2u * (unsigned) (s + 1);
            lds_flag *fl = (lds_flag *) (xs + kWaves * XP + (wave ^ 1) * 4);
            unsigned f = __builtin_amdgcn_readfirstlane(*fl);
            for (int it = 0; (f & ~1u) != want && it < kPairSpin; ++it) {
                __builtin_amdgcn_s_sleep(1);
                f = __builtin_amdgcn_readfirstlane(*fl);
            }
            asm volatile("" ::: "memory");
            const unsigned char *const xp = xs + (wave ^ 1) * XP;
            pq[1] = *reinterpret_cast<const bf16x8 *>(xp + lane * 16);
            if (f & 1u) {
                const float pc = *reinterpret_cast<const float *>(xp + 1024 + lane * 4);
#pragma unroll
                for (int dt = 0; dt < DW; ++dt) acc[1][dt] *= pc;
            }
        }
#pragma unroll
        for (int dt = 0; dt < DW; ++dt) {
            const bf16x8 a = vf[dt % PD];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pq[nb], acc[nb][dt], 0, 0, 0);
            if (dt + PD < DW) vf[dt % PD] = vtile(dt + PD);
            __builtin_amdgcn_sched_barrier(0);
        }
        };
        if constexpr (S2) {
            stage(s0, after_first_qk);
            issue_second();
            if (s0 + 1 < nst) stage(s0 + 1, [] {});
        } else {
            const int s = s0 + kh;  // this wave group's stage
            if (KH && s >= nst) continue;  // an odd stage count: the odd group's last iteration is empty
            stage(s, after_first_qk);
        }
    }

    if constexpr (KH) {
        // The odd-stage wave of each query block hands its (m, l, O^T) to the even-stage
        // wave through the ring's LDS (no DMA is outstanding and, after the barrier, no wave
        // reads the ring): lane-major, so each store and load of a wave is one contiguous
        // 1 KB.  A group that saw no key of a row holds m = -inf, l = 0 and adds nothing.
        constexpr int XA = QB * DT * 64 * 16;  // O^T bytes per wave
        constexpr int XW = XA + QB * 64 * 8;   // + (m, l)
        static_assert(NQW * XW <= R::BYTES, "the hand-over must fit the ring");
        unsigned char *xb = ring + wq * XW;
        lds_barrier();
        if (kh) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    *reinterpret_cast<f32x4 *>(xb + ((qb * DT + dt) * 64 + lane) * 16) = acc[qb][dt];
                *reinterpret_cast<f32x2 *>(xb + XA + (qb * 64 + lane) * 8) = f32x2{m[qb], l[qb]};
            }
        }
        lds_barrier();
        if (kh) return;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const f32x2 mlb = *reinterpret_cast<const f32x2 *>(xb + XA + (qb * 64 + lane) * 8);
            const float M = fmaxf(m[qb], mlb[0]);
            const float wa = m[qb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[qb] - M);
            const float wb = mlb[0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mlb[0] - M);
            l[qb] = l[qb] * wa + mlb[1] * wb;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                acc[qb][dt] = acc[qb][dt] * wa +
                              *reinterpret_cast<const f32x4 *>(xb + ((qb * DT + dt) * 64 + lane) * 16) * wb;
            m[qb] = M;
        }
    }

    // Row totals over the four lane groups; then the output (one split) or the partial.
    float lb[NB];  // row sums of the wave's O^T blocks
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        l[qb] += __shfl_xor(l[qb], 16);
        l[qb] += __shfl_xor(l[qb], 32);
        lb[qb] = l[qb];
    }
    if constexpr (PS) {  // the partner's row sums, through LDS past every wave's last stage
        float *xl = reinterpret_cast<float *>(xch + 2 * XPAR);
        if (lg == 0) xl[wave * 16 + li] = l[0];
        lds_barrier();
        lb[1] = xl[(wave ^ 1) * 16 + li];
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        // the block's first tile row (PS: the wave's own block, then its partner's)
        const int br = PS ? (nb == 0 ? wave : wave ^ 1) * 16 : wq * 16 * QB + nb * 16;
        const long long gr0 = (long long) tile * QT + br + li;
        if (gr0 >= nq) continue;
        const long long gr = gr0;
        const int qi = (int) (gr / p.G), qh = kvh * p.G + (int) (gr % p.G);
        const long long row = (long long) qi * p.Hq + qh;
        const int d0 = 16 * DW * hd;  // the wave's first O^T dim
        if (p.splits == 1) {
            const float inv = 1.0f / lb[nb];
            uint16_t *o = p.out + (size_t) qi * p.o_rs + (size_t) qh * p.o_hs + d0 + 4 * lg;
#pragma unroll
            for (int dt = 0; dt < DW; ++dt) {
                const f32x4 v4 = acc[nb][dt] * inv;
                bf16x4 b4 = {(__bf16) v4[0], (__bf16) v4[1], (__bf16) v4[2], (__bf16) v4[3]};
                *reinterpret_cast<bf16x4 *>(o + 16 * dt) = b4;
            }
        } else {
            float *pa = p.part_acc + ((long long) split * nrows + row) * D + d0 + 4 * lg;
#pragma unroll
            for (int dt = 0; dt < DW; ++dt) *reinterpret_cast<f32x4 *>(pa + 16 * dt) = acc[nb][dt];
            if (lg == 0 && nb < QB)  // (m, l) from the block's owner
                *reinterpret_cast<f32x2 *>(p.part_ml + 2 * ((long long) split * nrows + row)) = f32x2{m[nb < QB ? nb : 0], l[nb < QB ? nb : 0]};
        }
    }
}

// out(i, h, 4 dims) = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) over the splits
// with l_s > 0 (one thread per (row, 4 dims)).
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
    const long long nrows = (long long) p.Sq * p.Hq;
    const long long t = (long long) blockIdx.x * 256 + threadIdx.x;
    if (t >= nrows * (D / 4)) return;
    const long long row = t / (D / 4);
    const int d4 = (int) (t % (D / 4));
    float M = -INFINITY;
    for (int s = 0; s < p.splits; ++s) {
        const f32x2 ml = *reinterpret_cast<const f32x2 *>(p.part_ml + 2 * ((long long) s * nrows + row));
        if (ml[1] > 0.0f) M = fmaxf(M, ml[0]);
    }
    float den = 0.0f;
    f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < p.splits; ++s) {
        const f32x2 ml = *reinterpret_cast<const f32x2 *>(p.part_ml + 2 * ((long long) s * nrows + row));
        if (!(ml[1] > 0.0f)) continue;
        const float w = __builtin_amdgcn_exp2f(ml[0] - M);
        den += ml[1] * w;
        num += w * *reinterpret_cast<const f32x4 *>(p.part_acc + ((long long) s * nrows + row) * D + 4 * d4);
    }
    const f32x4 v4 = num * (1.0f / den);
    const int i = (int) (row / p.Hq), h = (int) (row % p.Hq);
    bf16x4 b4 = {(__bf16) v4[0], (__bf16) v4[1], (__bf16) v4[2], (__bf16) v4[3]};
    *reinterpret_cast<bf16x4 *>(p.out + (size_t) i * p.o_rs + (size_t) h * p.o_hs + 4 * d4) = b4;
}

// ------------------------------------------------------------ raw-K reconstruction
//
// One wave per key row.  Lane l holds dims HP*l .. +HP of each half (HP = D/128), so each
// rotary pair (d, d + D/2) sits in one lane.  The sum of squares is an fp32 wave
// reduction; rinv = 1 / sqrt(mean + eps) with IEEE division and square root.
struct RawKvParams {
    const uint16_t *raw;        // bf16 rows, or NULL with q8 / scale / bias
    const unsigned char *q8;
    const float *sc, *bs;
    long long raw_hs, sb_hs, out_hs;
    const uint16_t *kw;
    const float *inv_freq;
    float eps;
    int Hkv, rows, pos0;
    uint16_t *k, *v;
};

__device__ __forceinline__ float bf16r(float x) { return (float) (__bf16) x; }

template <int D, bool Q8>
__global__ __launch_bounds__(256) void raw_prefill_kv_kernel(RawKvParams p) {
#pragma clang fp contract(off)  // every rounding point as written (no fused multiply-add)
    constexpr int HP = D / 128, HALF = D / 2;
    const int lane = threadIdx.x & 63;
    const long long gw = (long long) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= (long long) p.Hkv * p.rows) return;
    const int h = (int) (gw / p.rows), t = (int) (gw % p.rows);
    float x[2][HP];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < HP; ++e) {
            const int d = half * HALF + HP * lane + e;
            if constexpr (Q8) {
                const size_t r = (size_t) h * p.sb_hs + t;
                const float prod = (float) p.q8[(size_t) h * p.raw_hs + (size_t) t * D + d] * p.sc[r];
                x[half][e] = bf16r(prod + p.bs[r]);  // the bf16 raw view of the q8 row
            } else {
                x[half][e] = __builtin_bit_cast(float, (unsigned) p.raw[(size_t) h * p.raw_hs + (size_t) t * D + d] << 16);
            }
        }
    float ss = 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < HP; ++e) ss += x[half][e] * x[half][e];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const float rinv = 1.0f / sqrtf(ss / (float) D + p.eps);
    uint16_t *ko = p.k + (size_t) h * p.out_hs + (size_t) t * D;
    uint16_t *vo = p.v + (size_t) h * p.out_hs + (size_t) t * D;
    const float pos = (float) (p.pos0 + t);
#pragma unroll
    for (int e = 0; e < HP; ++e) {
        const int d = HP * lane + e;
        const float k0a = bf16r(x[0][e] * rinv * __builtin_bit_cast(float, (unsigned) p.kw[d] << 16));
        const float k0b = bf16r(x[1][e] * rinv * __builtin_bit_cast(float, (unsigned) p.kw[d + HALF] << 16));
        float sn, cs;
        sincos_f32(pos * p.inv_freq[d], sn, cs);
        const float c = bf16r(cs), s = bf16r(sn);
        ko[d] = __builtin_bit_cast(uint16_t, (__bf16) (bf16r(k0a * c) + bf16r(-k0b * s)));
        ko[d + HALF] = __builtin_bit_cast(uint16_t, (__bf16) (bf16r(k0b * c) + bf16r(k0a * s)));
        vo[d] = __builtin_bit_cast(uint16_t, (__bf16) (x[0][e] * rinv));
        vo[d + HALF] = __builtin_bit_cast(uint16_t, (__bf16) (x[1][e] * rinv));
    }
}

// ------------------------------------------------------------ LDS read ceiling
//
// The read rate of the LDS on the prefill kernel's two read forms, for its roofline: each
// wave of W reads its 4 KB share of a 64 KB array, 8 reads in flight per round, with the
// QK operand's 128-bit row reads (TR = false) or the PV operand's 64-bit transpose reads
// ds_read_b64_tr_b16 (TR = true), every lane group of a read on consecutive addresses
// (bank-conflict-free).  Every address is masked into the array.
template <int W, bool TR>
__global__ __launch_bounds__(64 * W, 1) void lds_read_kernel(int iters, unsigned *sink) {
    __shared__ __attribute__((aligned(16))) unsigned char buf[65536];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 65536 / 4; i += 64 * W) reinterpret_cast<unsigned *>(buf)[i] = (unsigned) i * 2654435761u;
    __syncthreads();
    const unsigned base = lds_addr(buf);
    constexpr unsigned kStep = TR ? 512u : 1024u, kLane = TR ? 8u : 16u;
    unsigned acc = 0u;
    // The wait names the read registers as operands, so that no use of them is scheduled
    // above it (the compiler does not count the assembly reads).
    for (int it = 0; it < iters; ++it) {
        unsigned a[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            a[u] = base + (((unsigned) (it * 8 + u) * kStep + (unsigned) wave * 4096u + (unsigned) lane * kLane) & 65535u);
        if constexpr (TR) {
            u32x2 y[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(y[u]) : "v"(a[u]));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]), "+v"(y[6]), "+v"(y[7])
                         :: "memory");
#pragma unroll
            for (int u = 0; u < 8; ++u) acc ^= y[u][0] ^ y[u][1];
        } else {
            u32x4 x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) asm volatile("ds_read_b128 %0, %1" : "=v"(x[u]) : "v"(a[u]));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])
                         :: "memory");
#pragma unroll
            for (int u = 0; u < 8; ++u) acc ^= x[u][0] ^ x[u][1] ^ x[u][2] ^ x[u][3];
        }
    }
    sink[(size_t) blockIdx.x * 64 * W + tid] = acc;
}

// ------------------------------------------------------------ host side

int fail(int code, const std::string &msg) {
    esda_detail::set_error(msg);
    return code;
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// 16-query blocks per wave: two where they fit the registers (D <= 256), except at
// D = 256 when the two-block tiles would leave CUs idle without key splits -- a split's
// partials cost 4 D bytes per query row written and read again.
int pick_qb(int D, long long rows, int Hkv) {
    if (D == 512) return 1;
    if (D == 128) return 2;
    const long long tiles2 = (rows + 16 * 2 * kWaves - 1) / (16 * 2 * kWaves);
    return tiles2 * Hkv >= kTargetGroups ? 2 : 1;
}

// Stage halves (the KH kernel, 64-row tiles) at D = 256 with one block per wave, when the
// 128-row tiles alone would leave CUs idle: twice the tiles instead of key splits.
bool pick_kh(int D, int qb, long long rows, int Hkv) {
    if (D != 256 || qb != 1) return false;
    const long long tiles1 = (rows + 16 * kWaves - 1) / (16 * kWaves);
    return tiles1 * Hkv < kTargetGroups;
}

// Validates a description and fills the kernel parameters' shape fields and plan.
int plan_prefill(const esda_prefill_desc *d, PrefillParams *p) {
    if (!d) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: null description");
    const int D = d->head_dim;
    if (D != 128 && D != 256 && D != 512)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: head_dim must be 128, 256 or 512");
    if (d->num_q_heads <= 0 || d->num_kv_heads <= 0 || d->num_q_heads % d->num_kv_heads)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: num_q_heads must be a multiple of num_kv_heads");
    if (d->seq_q <= 0 || d->seq_k <= 0 || d->window < 0 || d->q_pos0 < 0 || d->k_pos0 < 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: sizes, positions and window must be non-negative");
    if ((long long) d->q_pos0 + d->seq_q > INT_MAX || (long long) d->k_pos0 + d->seq_k > INT_MAX)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: positions must stay below 2^31");
    if (d->k_pos0 > d->q_pos0 || (long long) d->k_pos0 + d->seq_k < (long long) d->q_pos0 + d->seq_q)
        return fail(ESDA_ERR_INVALID_ARGUMENT,
                    "esda_prefill: the keys must hold every query's own position (k_pos0 <= q_pos0, "
                    "k_pos0 + seq_k >= q_pos0 + seq_q)");
    for (long long st : {d->q_head_stride, d->q_row_stride, d->kv_head_stride, d->out_row_stride, d->out_head_stride})
        if (st < 0 || st % 8)
            return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: strides must be non-negative multiples of 8");
    if (d->kv_head_stride < (long long) d->seq_k * D && d->num_kv_heads > 1)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: kv_head_stride smaller than a head's rows");
    if (d->split_keys < 0 || d->split_keys % kStageKeys)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: split_keys must be a multiple of 32");
    if (!(d->scale > 0.0f) || !std::isfinite(d->scale))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: scale must be positive and finite");
    *p = PrefillParams{};
    p->Hq = d->num_q_heads;
    p->Hkv = d->num_kv_heads;
    p->G = d->num_q_heads / d->num_kv_heads;
    p->Sq = d->seq_q;
    p->Sk = d->seq_k;
    p->q_pos0 = d->q_pos0;
    p->k_pos0 = d->k_pos0;
    p->window = d->window;
    p->q_hs = d->q_head_stride;
    p->q_rs = d->q_row_stride;
    p->kv_hs = d->kv_head_stride;
    p->o_rs = d->out_row_stride;
    p->o_hs = d->out_head_stride;
    p->scale_log2e = d->scale * 1.4426950408889634f;
    p->qb = pick_qb(D, (long long) d->seq_q * p->G, d->num_kv_heads);
    p->kh = pick_kh(D, p->qb, (long long) d->seq_q * p->G, d->num_kv_heads) ? 1 : 0;
    const int QT = 16 * p->qb * (p->kh ? kWaves / 2 : kWaves);
    const long long tiles = ((long long) d->seq_q * p->G + QT - 1) / QT;
    if (tiles * d->num_kv_heads > (1LL << 24))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: too many query tiles");
    p->tiles = (int) tiles;
    // The widest key range of any tile (the last one under a causal mask).
    int maxn = 0;
    for (int t = 0; t < p->tiles; ++t) {
        int a, b;
        tile_keys(*p, t, QT, a, b);
        maxn = std::max(maxn, b - a);
    }
    int kps;
    if (d->split_keys > 0) {
        kps = d->split_keys;
    } else {
        // enough workgroups to cover the CUs, each with at least 8 stages
        const long long groups = tiles * d->num_kv_heads;
        long long s = (kTargetGroups + groups - 1) / groups;
        const long long smax = std::max<long long>(1, maxn / (8 * kStageKeys));
        s = std::min(s, smax);
        kps = (int) (((maxn + s - 1) / s + kStageKeys - 1) / kStageKeys * kStageKeys);
    }
    if (kps <= 0) kps = kStageKeys;
    const long long splits = (maxn + kps - 1) / kps;
    if (splits > 65535 || tiles * d->num_kv_heads * splits > INT_MAX)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: too many key splits");
    p->kps = kps;
    p->splits = (int) std::max<long long>(1, splits);
    return ESDA_OK;
}

size_t workspace_of(const PrefillParams &p, int D) {
    if (p.splits <= 1) return 0;
    const size_t rows = (size_t) p.Sq * p.Hq;
    return (size_t) p.splits * rows * ((size_t) D * 4 + 8) + 256;
}

template <int D>
void launch_prefill(const PrefillParams &p, int stages, hipStream_t st) {
    if (stages & 1) {
        const dim3 grid(p.tiles * p.Hkv * p.splits), block(64 * kWaves);
        if constexpr (D == 512) {
            if (p.k == p.v) hipLaunchKernelGGL((prefill_kernel<512, 1, false, true, true, true>), grid, block, 0, st, p);
            else hipLaunchKernelGGL((prefill_kernel<512, 1>), grid, block, 0, st, p);
        }
        else if constexpr (D == 128)
            hipLaunchKernelGGL((prefill_kernel<128, 2>), grid, block, 0, st, p);
        else if (p.qb == 2)
            hipLaunchKernelGGL((prefill_kernel<256, 2, false, false, true>), grid, block, 0, st, p);
        else if (p.kh)
            hipLaunchKernelGGL((prefill_kernel<256, 1, true>), grid, block, 0, st, p);
        else
            hipLaunchKernelGGL((prefill_kernel<256, 1>), grid, block, 0, st, p);
    }
    if ((stages & 2) && p.splits > 1) {
        const long long n = (long long) p.Sq * p.Hq * (D / 4);
        hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, p);
    }
}

int run_raw_kv(const RawKvParams &p, int D, bool q8, hipStream_t st) {
    int rc = esda_detail::check_device();
    if (rc != ESDA_OK) return rc;
    const long long waves = (long long) p.Hkv * p.rows;
    if (waves == 0) return ESDA_OK;
    const dim3 grid((unsigned) ((waves + 3) / 4)), block(256);
    if (q8) {
        hipLaunchKernelGGL((raw_prefill_kv_kernel<512, true>), grid, block, 0, st, p);
    } else if (D == 512) {
        hipLaunchKernelGGL((raw_prefill_kv_kernel<512, false>), grid, block, 0, st, p);
    } else if (D == 256) {
        hipLaunchKernelGGL((raw_prefill_kv_kernel<256, false>), grid, block, 0, st, p);
    } else {
        hipLaunchKernelGGL((raw_prefill_kv_kernel<128, false>), grid, block, 0, st, p);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ESDA_ERR_HIP, std::string("raw_prefill_kv launch: ") + hipGetErrorString(e));
    return ESDA_OK;
}

}  // namespace

extern "C" {

int esda_prefill_workspace_size(const esda_prefill_desc *desc, size_t *bytes) {
    if (!bytes) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill_workspace_size: null output");
    PrefillParams p;
    const int rc = plan_prefill(desc, &p);
    if (rc != ESDA_OK) return rc;
    *bytes = workspace_of(p, desc->head_dim);
    return ESDA_OK;
}

int esda_prefill_stages(const esda_prefill_desc *desc, const esda_prefill_args *a, int stages, void *stream) {
    PrefillParams p;
    int rc = plan_prefill(desc, &p);
    if (rc != ESDA_OK) return rc;
    if (!a || !a->q || !a->k || !a->v || !a->out) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: null pointer");
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_prefill: tensors must be 16-byte aligned");
    const int D = desc->head_dim;
    const size_t need = workspace_of(p, D);
    if (need) {
        if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
            return fail(ESDA_ERR_WORKSPACE, "esda_prefill: workspace missing or smaller than "
                                            "esda_prefill_workspace_size");
        const size_t rows = (size_t) p.Sq * p.Hq;
        p.part_acc = static_cast<float *>(a->workspace);
        p.part_ml = reinterpret_cast<float *>(static_cast<char *>(a->workspace) + (size_t) p.splits * rows * D * 4);
    }
    rc = esda_detail::check_device();
    if (rc != ESDA_OK) return rc;
    p.q = static_cast<const uint16_t *>(a->q);
    p.k = static_cast<const uint16_t *>(a->k);
    p.v = static_cast<const uint16_t *>(a->v);
    p.out = static_cast<uint16_t *>(a->out);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (D == 512) launch_prefill<512>(p, stages, st);
    else if (D == 256) launch_prefill<256>(p, stages, st);
    else launch_prefill<128>(p, stages, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ESDA_ERR_HIP, std::string("esda_prefill launch: ") + hipGetErrorString(e));
    return ESDA_OK;
}

int esda_prefill(const esda_prefill_desc *desc, const esda_prefill_args *a, void *stream) {
    return esda_prefill_stages(desc, a, 3, stream);
}

int esda_raw_prefill_kv(const void *raw, int64_t raw_head_stride, int32_t kv_heads, int32_t rows, int32_t head_dim,
                        const void *kw, float eps, const float *inv_freq, int32_t pos0, void *k_out, void *v_out,
                        int64_t out_head_stride, void *stream) {
    if (head_dim != 128 && head_dim != 256 && head_dim != 512)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_raw_prefill_kv: head_dim must be 128, 256 or 512");
    if (!raw || !kw || !inv_freq || !k_out || !v_out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_raw_prefill_kv: null pointer");
    if (kv_heads <= 0 || rows < 0 || pos0 < 0 || !(eps >= 0.0f) ||
        (kv_heads > 1 && (raw_head_stride < (int64_t) rows * head_dim || out_head_stride < (int64_t) rows * head_dim)))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_raw_prefill_kv: invalid sizes or strides");
    RawKvParams p{};
    p.raw = static_cast<const uint16_t *>(raw);
    p.raw_hs = raw_head_stride;
    p.out_hs = out_head_stride;
    p.kw = static_cast<const uint16_t *>(kw);
    p.inv_freq = inv_freq;
    p.eps = eps;
    p.Hkv = kv_heads;
    p.rows = rows;
    p.pos0 = pos0;
    p.k = static_cast<uint16_t *>(k_out);
    p.v = static_cast<uint16_t *>(v_out);
    return run_raw_kv(p, head_dim, false, static_cast<hipStream_t>(stream));
}

int esda_raw_q8_prefill_kv(const void *q8, int64_t q_head_stride, const float *scale, const float *bias,
                           int64_t sb_head_stride, int32_t kv_heads, int32_t rows, const void *kw, float eps,
                           const float *inv_freq, int32_t pos0, void *k_out, void *v_out, int64_t out_head_stride,
                           void *stream) {
    if (!q8 || !scale || !bias || !kw || !inv_freq || !k_out || !v_out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_raw_q8_prefill_kv: null pointer");
    if (kv_heads <= 0 || rows < 0 || pos0 < 0 || !(eps >= 0.0f) ||
        (kv_heads > 1 && (q_head_stride < (int64_t) rows * 512 || sb_head_stride < rows ||
                          out_head_stride < (int64_t) rows * 512)))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_raw_q8_prefill_kv: invalid sizes or strides");
    RawKvParams p{};
    p.q8 = static_cast<const unsigned char *>(q8);
    p.sc = scale;
    p.bs = bias;
    p.raw_hs = q_head_stride;
    p.sb_hs = sb_head_stride;
    p.out_hs = out_head_stride;
    p.kw = static_cast<const uint16_t *>(kw);
    p.inv_freq = inv_freq;
    p.eps = eps;
    p.Hkv = kv_heads;
    p.rows = rows;
    p.pos0 = pos0;
    p.k = static_cast<uint16_t *>(k_out);
    p.v = static_cast<uint16_t *>(v_out);
    return run_raw_kv(p, 512, true, static_cast<hipStream_t>(stream));
}

int esda_lds_read(int32_t waves, int32_t transpose, int32_t iters, int32_t workgroups, uint32_t *sink,
                  void *stream) {
    if (!sink) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_lds_read: null sink");
    if (iters <= 0 || workgroups <= 0 || workgroups > 65535)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_lds_read: iters must be positive, workgroups in 1 .. 65535");
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(workgroups);
    const bool tr = transpose != 0;
    if (waves != 4 && waves != 8 && waves != 16)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_lds_read: waves must be 4, 8 or 16");
    if (waves == 4 && tr) hipLaunchKernelGGL((lds_read_kernel<4, true>), grid, dim3(256), 0, st, iters, sink);
    if (waves == 4 && !tr) hipLaunchKernelGGL((lds_read_kernel<4, false>), grid, dim3(256), 0, st, iters, sink);
    if (waves == 8 && tr) hipLaunchKernelGGL((lds_read_kernel<8, true>), grid, dim3(512), 0, st, iters, sink);
    if (waves == 8 && !tr) hipLaunchKernelGGL((lds_read_kernel<8, false>), grid, dim3(512), 0, st, iters, sink);
    if (waves == 16 && tr) hipLaunchKernelGGL((lds_read_kernel<16, true>), grid, dim3(1024), 0, st, iters, sink);
    if (waves == 16 && !tr) hipLaunchKernelGGL((lds_read_kernel<16, false>), grid, dim3(1024), 0, st, iters, sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? ESDA_OK : fail(ESDA_ERR_HIP, std::string("lds_read_kernel launch: ") + hipGetErrorString(e));
}

}  // extern "C"
