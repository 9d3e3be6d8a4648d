// esda_decode.hip -- Gemma-4 decode attention for MI355X (gfx950, CDNA4).
//
// One decode step = fused KV append + split-K single-query attention + fp32 merge.
// Reference behaviour (Apertura tree): ESKVCache::update prealloc append
// (ESKVCache.mm:64-109) followed by mx::fast::scaled_dot_product_attention at
// ESAttention.mm:188, with the visibility rule of ESGemma4TextModel.mm:68-83 and the
// split merge of ESDecodeAttn.mm:253-273; in raw-K mode, ESKVCache::updateRaw
// (ESKVCache.mm:458-504) followed by esDecodeAttnGlobal (ESDecodeAttn.mm:17-117, 415-453).
//
// Kernels
//   attend_kernel  grid (splits, kv heads, sequences) or balanced shares of a ragged
//                  batch; 4 or 8 waves, one workgroup per CU (two at D = 256), the
//                  ring in the whole LDS or in half of it.  A workgroup streams
//                  visible rows of one (sequence, kv head) -- or of 2 or 4 kv heads
//                  packed together -- through an LDS ring filled by LDS DMA, splits the head dim across its
//                  waves for the QK and PV MFMAs (the GQA group is the MFMA N dimension),
//                  runs an fp32 online softmax and writes (m, l, acc) partials.  The
//                  workgroup whose split ends at the new token also copies its row into
//                  the cache.  Details at the kernel.
//   merge_kernel   reduces the partials of all splits per (sequence, query head).
//   append_kernel  multi-row append (slice_update) for prefill-style callers.
// The C ABI (include/esda.h) is at the end of the file.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

#include "esda.h"
#include "esda_device.h"
#include "esda_internal.h"
#include "esda_plan.h"

namespace {

constexpr int kTile = 16;          // MFMA row block; split sizes are multiples of it
constexpr int kMaxGroup = 16;
constexpr int kTargetGroups = 256;  // one workgroup per MI355X CU; plans of two per CU aim at twice that
constexpr int kWaves256 = 4;        // waves per workgroup of the plain kernels at D = 256
constexpr int kOcc256 = 2;          // and their workgroups per CU
// The 512-dim shared stream's kernel is built with its ring in half the LDS (4 stages) although
// its plans place one workgroup per CU: see dispatch_attend.
constexpr int kOcc512Shared = 2;
constexpr int kMinRows = 64;        // fewest rows per workgroup the automatic plan gives
constexpr int kMinRowsOcc2 = 32;    // the same for grids of two workgroups per CU (C1: step
                                    // 8.3 -> 7.8 us with 32-row splits; 16 rows: 8.0)
constexpr int kMaxGroups = 16384;   // workgroups per launch
constexpr int kMaxBatch = 256;      // sequences per call (one per thread of the prefix scan)

// Per-sequence views, the prefix table, shares, segments and merge owners: the integer
// arithmetic of esda_plan.h (shared with the host tests).
using esda_plan::SeqView;
using esda_plan::seq_view;

struct AttendParams {
    const uint16_t *q, *k_new, *v_new;
    uint16_t *k_cache, *v_cache;
    const int *pos, *row_base;
    float *part_acc, *part_ml;
    int *status;
    long long seq_stride, head_stride;
    // Hkv and G count packed kv heads: a workgroup serves pk consecutive kv heads of one
    // sequence (gk query heads each) as one group of G = pk * gk query heads.
    int B, Hq, Hkv, G, cap, window, ring;
    int pk, gk;
    int balanced;      // 1: W balanced shares of all rows; 0: grid (S, Hkv, B) of chunk-row splits
    int W, S, chunk;
    float scale_log2e;
    long long *table;  // balanced: prefix sums of visible rows per sequence, for the merge
    uint16_t *out;     // written directly for (sequence, kv head) pairs of one segment
    // raw-K mode only
    const uint16_t *kw;
    const float *inv_freq;
    const unsigned *rope_tab;  // optional [rows][64] cos/sin pairs (esda_rope_table), row = cache row
    float eps;
    // q8 raw-K mode: u8 rows at q8 (strides as for k_cache, in bytes) and per-row scale /
    // bias at qsc / qbs[b * sb_seq_stride + kv head * sb_head_stride + row]
    unsigned char *q8;
    float *qsc, *qbs;
    long long sb_seq_stride, sb_head_stride;
};



// ---------------------------------------------------------------- LDS ring layout
//
// A workgroup streams its rows through a ring of NS stages of 16 rows in LDS.  Rows
// arrive by LDS DMA (global_load_lds_dwordx4: 64 lanes x 16 B land contiguously at
// M0 + 16*lane), non-temporal, so in-flight data costs no registers and each
// instruction reads 1 KB of contiguous HBM.  One instruction carries RPI = 512/D rows:
// instruction i of a stage holds rows i + q*NI (q < RPI) in a 1056-byte block (1 KB +
// 32 B pad), sub-row q at +2D*q bytes.  The 32-byte pad (a measured choice: 16 B leaves
// both the 128-bit row reads and the transpose reads 2-way bank-conflicted on gfx950)
// makes both read patterns conflict-free with every address a base plus an immediate.
// EXTRA: LDS bytes the kernel variant needs beside the ring and the score exchange; PSX:
// LDS bytes it keeps per ring stage beside the rows.
template <int D, bool SHARED, int NW, int EXTRA = 0, int PSX = 0, int LDSB = 160 * 1024>
struct Ring {
    static constexpr int RPI = 512 / D;                     // rows per DMA instruction
    static constexpr int NI = 16 / RPI;                     // DMA instructions per stage
    static constexpr int CPR = D / 8;                       // 16-byte chunks per row
    static constexpr int BLK = 1056;                        // LDS bytes per DMA block
    static constexpr int TB = NI * BLK;                     // one tensor's stage
    static constexpr int SB = (SHARED ? 1 : 2) * TB;        // stage bytes (K [+ V])
    static constexpr int DW = D / NW;                       // dims per wave
    static constexpr int SL = DW / 8;                       // chunks per wave slice
    static constexpr int KKW = DW / 32;                     // QK k-steps per wave
    static constexpr int DTW = DW / 16;                     // PV dim tiles per wave
    static constexpr int DPT = NI / NW;                     // DMA per wave per tensor
    static constexpr int DPW = DPT * (SHARED ? 1 : 2);      // DMA per wave per stage
    static constexpr int XB = 2 * NW * 64 * 16;             // score-exchange bytes
    // reserve: kernel arguments' spill room (256 B) and the batch prefix scan (int64 per
    // sequence + one per wave)
    static constexpr int NS_ = (LDSB - XB - 256 - ((kMaxBatch + 1) + NW) * 8 - EXTRA) / (SB + PSX);
    static constexpr int NS = NS_ > 16 ? 16 : NS_;          // stages in the ring
    static_assert(DW % 32 == 0 && NI % NW == 0, "wave slices must cover whole MFMA steps");
    static_assert(NS >= 4, "the ring needs at least 4 stages");
    static_assert((NS - 3) * DPW <= 60, "vmcnt holds at most 63 outstanding loads");
    // Byte offset of (row r, chunk cin of wave slice ws) inside a tensor stage.
    __device__ static __forceinline__ int off(int r, int ws, int cin) {
        return (r % NI) * BLK + (r / NI) * 2 * D + (ws * SL + cin) * 16;
    }
};


// ------------------------------------------------------------ raw-K reconstruction
//
// Raw mode (ESDecodeAttn.mm:51-106): the cache holds pre-norm k_proj rows.  Per row,
// rinv = rsqrt(mean(kraw^2) + eps); K = bf16(rope(kraw * rinv * kw)) with rotary pairs
// (d, d + 256) for d < 64, whose cos / sin are those of the fp32 angle t * inv_freq[d]
// rounded to bf16; V = kraw * rinv, with rinv folded into the softmax weight.

constexpr int kRawDim = 512;
constexpr int kRopePairs = 64;
constexpr int kTabStride = 68;  // words per cos/sin table row: 64 + 4 (conflict-free 128-bit reads)
// LDS of the raw-mode exchanges for NW waves, in this order: row sums of squares
// [3][16][NW], the row factors [2][3][16], (q8) the row sums [3][16][NW], and the cos/sin
// tables [2][16][kTabStride] computed in the kernel.
constexpr int raw_extra_lds(int nw, bool q8 = false) {
    return 3 * 16 * nw * 4 + 2 * 3 * 16 * 4 + (q8 ? 3 * 16 * nw * 4 : 0) + 2 * 16 * kTabStride * 4;
}
// q8 raw-K mode: u8 stages are widened into bf16 staging slots laid out as the D = 512
// ring (16 rows of 1056-byte blocks), four deep; per-row scale / bias ride beside each
// u8 stage.
constexpr int kQ8Stage = 16 * 1056;
constexpr int kQ8Slots = 4;
constexpr int kQ8SbStages = 16;
constexpr int q8_extra_lds(int nw) {
    return raw_extra_lds(nw, true) + kQ8Slots * kQ8Stage + kQ8SbStages * 2 * 16 * 4;
}


// The segments of one launch's workgroup: grid plans give workgroup (split, kv head,
// sequence) rows [split * chunk, ...) of its pair; balanced plans give workgroup w its share
// of all visible rows of the batch, walked pair by pair (esda_plan.h).  segment(b, kvh, j0,
// j1, view, slot, direct) runs each; the ring is free again when it returns (the walk puts
// a barrier between segments).  NW: waves per workgroup.
template <int NW, class Seg>
__device__ __forceinline__ void walk_segments(const AttendParams &p, Seg &&segment) {
    const int wg = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (!p.balanced) {
        // Fixed splits (uniform lengths: one sequence, or windowed local layers): workgroup
        // (split, kvh, b) takes rows [split * chunk, (split + 1) * chunk) of its pair.
        const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
        const SeqView sv = seq_view(p.pos[b], p.row_base ? p.row_base[b] : 0, p.cap, p.window, p.ring);
        if (!sv.ok) {
            if (split == 0 && kvh == 0 && tid == 0) atomicAdd(p.status, 1);
            return;
        }
        int j0, j1;
        if (!esda_plan::grid_split(split, p.S, p.chunk, sv.nvis, &j0, &j1)) return;
        segment(b, kvh, j0, j1, sv, ((size_t) b * p.Hkv + kvh) * p.S + split, j0 == 0 && j1 == sv.nvis);
        return;
    }

    // Balanced shares (ragged batches).
    // Visible rows of every sequence and their exclusive prefix sums (the rows that
    // precede sequence b in the linearised order).  Up to 64 sequences every wave scans
    // the batch in its own lanes (no LDS, no barrier); larger batches (up to 256, one per
    // thread) go through LDS.
    __shared__ long long s_pref[kMaxBatch + 1];
    __shared__ long long s_wtot[NW];
    const bool single = p.B == 1;
    const bool wave_scan = p.B <= 64;
    long long w_incl = 0, w_nv = 0;  // wave scan: lane t's inclusive sum and rows of sequence t
    SeqView w_view{0, 0, 0, 0};
    long long rows_seq = 0;          // sum of visible rows over the batch
    if (single) {
        // one sequence: its view straight from the (wave-uniform) position word
        w_view = seq_view(p.pos[0], p.row_base ? p.row_base[0] : 0, p.cap, p.window, p.ring);
        rows_seq = w_view.ok ? w_view.nvis : 0;
        if (wg == 0 && tid == 0) {
            if (!w_view.ok) atomicAdd(p.status, 1);
            esda_plan::write_prefix_entry(p.table, 0, 1, 0, rows_seq);
        }
    } else {
        const int t = wave_scan ? lane : tid;
        SeqView v{0, 0, 0, 0};
        if (t < p.B) v = seq_view(p.pos[t], p.row_base ? p.row_base[t] : 0, p.cap, p.window, p.ring);
        const long long nv = v.ok ? v.nvis : 0;
        long long x = nv;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const long long y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (wave_scan) {
            w_incl = x;
            w_nv = nv;
            w_view = v;
            rows_seq = __shfl(x, 63);
            if (wg == 0 && wave == 0) {
                if (t < p.B && !v.ok) atomicAdd(p.status, 1);
                esda_plan::write_prefix_entry(p.table, t, p.B, x - nv, rows_seq);
            }
        } else {
            if (lane == 63) s_wtot[wave] = x;
            __syncthreads();  // no DMA is in flight yet
            long long off = 0;
            for (int i = 0; i < wave; ++i) off += s_wtot[i];
            if (tid < p.B) s_pref[tid + 1] = off + x;
            if (tid == 0) s_pref[0] = 0;
            if (wg == 0 && tid < p.B && !v.ok) atomicAdd(p.status, 1);
            __syncthreads();
            // B + 1 entries (B may be 256 = one per thread): the total goes in separately
            if (wg == 0) esda_plan::write_prefix_entry(p.table, tid, p.B, tid < p.B ? s_pref[tid] : 0, s_pref[p.B]);
            rows_seq = s_pref[p.B];
        }
    }
    const long long rows_total = rows_seq * p.Hkv;
    // Rows before sequence b (b <= B) and its view; the same in every lane.
    auto lane64 = [](long long v, int l) {
        const unsigned lo = __builtin_amdgcn_readlane((unsigned) v, l);
        const unsigned hi = __builtin_amdgcn_readlane((unsigned) ((unsigned long long) v >> 32), l);
        return (long long) (((unsigned long long) hi << 32) | lo);
    };
    auto pref_at = [&](int b) -> long long {
        if (single) return b == 0 ? 0 : rows_seq;
        if (!wave_scan) return s_pref[b];
        return b >= p.B ? rows_seq : lane64(w_incl - w_nv, b);
    };
    auto view_at = [&](int b) -> SeqView {
        if (single) return w_view;
        if (!wave_scan) return seq_view(p.pos[b], p.row_base ? p.row_base[b] : 0, p.cap, p.window, p.ring);
        return SeqView{__builtin_amdgcn_readlane(w_view.nvis, b), __builtin_amdgcn_readlane(w_view.first, b),
                       __builtin_amdgcn_readlane(w_view.newrow, b), __builtin_amdgcn_readlane(w_view.ok, b)};
    };

    // This workgroup's share of all visible rows, linearised as (sequence, kv head, row):
    // [rows_total * wg / Wr, rows_total * (wg + 1) / Wr) with Wr = min(W, rows_total), so
    // that every share holds at least one row (W is sized from the bound on rows; early in
    // a long cache fewer rows are visible) and workgroups wg >= Wr have nothing to do.  A
    // share covers one or more segments; the partial of workgroup wg for pair
    // u = b * Hkv + kvh goes to slot u + wg, so the slots of one pair are consecutive and
    // distinct pairs never share a slot.
    const int Wr = esda_plan::active_shares(rows_total, p.W);
    if (wg >= Wr) return;
    const long long lo = esda_plan::share_begin(rows_total, Wr, wg), hi = esda_plan::share_begin(rows_total, Wr, wg + 1);
    long long x = lo;
    int b = 0;
    while (x < hi) {
        // the sequence holding row x (x < rows_total): the count of sequences that end at
        // or before it
        if (single) {
            b = 0;
        } else if (wave_scan) {
            b = __popcll(__ballot(lane < p.B && w_incl * p.Hkv <= x));
        } else {
            while (pref_at(b + 1) * p.Hkv <= x) ++b;
        }
        const long long pb = pref_at(b);
        const int n = (int) (pref_at(b + 1) - pb);
        const esda_plan::Segment sg = esda_plan::segment_at(x, hi, pb * p.Hkv, n);
        const int kvh = sg.kvh, j0 = sg.j0, j1 = sg.j1;
        const long long seg_end = sg.end;
        const SeqView v = view_at(b);
        // Every value of the segment is the same in all lanes (computed from LDS and kernel
        // arguments); saying so keeps the ring's control flow and addresses scalar.
        const SeqView sv{uniform(v.nvis), uniform(v.first), uniform(v.newrow), uniform(v.ok)};
        const int ub = uniform(b), ukvh = uniform(kvh), uj0 = uniform(j0), uj1 = uniform(j1);
        segment(ub, ukvh, uj0, uj1, sv, (size_t) esda_plan::share_slot((long long) ub * p.Hkv + ukvh, wg),
                uj0 == 0 && uj1 == n);
        lds_barrier();  // every wave is done with the ring before the next segment refills it
        x = seg_end;
    }
}

// --------------------------------------------------------------------- attend kernel
//
// grid (splits, kv heads, sequences), NW = 4 or 8 waves per workgroup, the ring in 1/OCC of
// the LDS (so that OCC workgroups fit per CU).  A workgroup owns `chunk` consecutive visible rows
// of one (sequence, kv head) and streams them through the LDS ring in 16-row stages.
// When each pair needs one split and pairs are plentiful, pk = 2 or 4 kv heads of a
// sequence share a workgroup:
// a stage then holds 16 / pk rows of each, their query heads fill the MFMA N dimension
// side by side, and scores of a head against another kv head's rows are masked.
// Ragged batches use balanced shares instead: workgroup w takes rows
// [total * w / W, total * (w + 1) / W) of all visible rows linearised by (sequence, kv
// head, row), one segment per pair it touches.  The head dim is split
// across the waves: per stage, each wave forms partial scores S^T[16 rows x 16 heads]
// over its dims with v_mfma_f32_16x16x32_bf16 (the GQA group is the MFMA N dimension,
// zero-padded to 16, so each K/V byte is read from HBM once per group), the partials
// are summed through LDS, every wave runs the same online softmax, and each wave
// accumulates O^T for its own dims with v_mfma_f32_16x16x16_bf16 (V^T from LDS by
// transpose reads).  One barrier per stage: the scores of stage s+1 are formed while
// stage s is accumulated.  With attention_k_eq_v the V rows are the K rows in LDS.
//
// RAW (D = 512, one tensor): the QK operand is rebuilt from raw rows in registers.  The
// row norms need all four waves' dims, so each stage's partial sums of squares (and its
// cos/sin table) are published two stages ahead: in iteration s the waves publish
// stage s+2's sums and table, form stage s+1's scores and accumulate stage s.
//
// The new token's row is copied from k_new/v_new into the cache by the workgroup whose
// split ends at it (bit-exact copy); that workgroup's own loads read the row from
// k_new/v_new and no other workgroup reads it, so the copy needs no ordering.
//
// Q8 (raw mode over a q8 raw stream, esDecodeAttnGlobalQ8, ESDecodeAttn.mm:275-369): rows
// are u8 with a per-row scale and bias, x = q * scale + bias.  The u8 ring (512-byte rows)
// is widened into bf16 staging slots three stages ahead, where q is exact, so the raw
// pipeline runs on q itself: the Gram diagonal and a row sum give sum(q^2) and sum(q)
// exactly, hence sum(x^2); K = bf16(rope(fma(q, scale*rinv, bias*rinv) * kw)); V enters
// as q with the weight P = bf16(e * scale * rinv) and the bias as sum P * bias / scale.
// The workgroup holding a sequence's new row quantizes it into the cache first.
template <int D, bool SHARED, int NW, bool RAW, bool Q8 = false, int OCC = 1>
// The LDS ring allows OCC workgroups per CU, i.e. OCC * NW/4 waves per SIMD: telling the
// compiler so lifts the register limit it would otherwise keep for higher occupancy,
// which it meets by serialising LDS reads behind their uses.  (Plans may still place one
// workgroup per CU on a kernel built with OCC = 2: its shallower ring is what they want.)
__global__ __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW), amdgpu_waves_per_eu(OCC * NW / 4, OCC * NW / 4)))
void attend_kernel(AttendParams p) {
    static_assert(!RAW || (D == kRawDim && SHARED && (NW == 4 || NW == 8)), "raw mode: one 512-dim stream, 4 or 8 waves");
    static_assert(!Q8 || (RAW && NW == 8), "q8 mode is raw mode with 8 waves");
    // R: the compute layout of a stage (and, outside q8 mode, the DMA ring); RD: the DMA ring.
    using R = Ring<D, SHARED, NW, RAW && !Q8 ? raw_extra_lds(NW) : 0, 0, 160 * 1024 / OCC>;
    using RD = std::conditional_t<Q8, Ring<256, true, NW, q8_extra_lds(NW)>, R>;
    static_assert(OCC == 1 || !RAW, "raw mode holds one workgroup per CU");
    // D = 512 exchanges only the live heads' partial scores (the padding columns are zero)
    constexpr bool kLiveX = D == 512 && !RAW;
    constexpr int NS = RD::NS, DW = R::DW, KKW = R::KKW, DTW = R::DTW;
    // DMA instructions per wave per stage (q8: the u8 rows plus one scale / bias piece)
    constexpr int DPW = Q8 ? RD::DPT + 1 : RD::DPW;
    // Stages between the one being accumulated and the newest one that must have landed.
    constexpr int AHEAD = Q8 ? 3 : RAW ? 2 : 1;
    static_assert(NS >= AHEAD + 3, "the ring must hold the look-ahead stages and one in flight");
    static_assert(!Q8 || NS <= kQ8SbStages, "one scale / bias area per ring stage");
    // Distinct arrays per stage: the compiler tracks DMA completion per LDS object, so a
    // read of stage u only waits for stage u's DMA, never for the stages behind it.
    __shared__ __attribute__((aligned(16))) unsigned char r0[RD::SB], r1[RD::SB], r2[RD::SB], r3[RD::SB],
        r4[RD::SB], r5[RD::SB], r6[RD::SB], r7[RD::SB], r8[RD::SB], r9[RD::SB], r10[RD::SB], r11[RD::SB],
        r12[RD::SB], r13[RD::SB], r14[RD::SB], r15[RD::SB];
    // Stage buffer u (a compile-time index).
    auto ring = [&](auto uc) -> unsigned char * {
        constexpr int u = decltype(uc)::value % NS;
        if constexpr (u == 0) return r0;
        else if constexpr (u == 1) return r1;
        else if constexpr (u == 2) return r2;
        else if constexpr (u == 3) return r3;
        else if constexpr (u == 4) return r4;
        else if constexpr (u == 5) return r5;
        else if constexpr (u == 6) return r6;
        else if constexpr (u == 7) return r7;
        else if constexpr (u == 8) return r8;
        else if constexpr (u == 9) return r9;
        else if constexpr (u == 10) return r10;
        else if constexpr (u == 11) return r11;
        else if constexpr (u == 12) return r12;
        else if constexpr (u == 13) return r13;
        else if constexpr (u == 14) return r14;
        else return r15;
    };
    __shared__ f32x4 xch[2][NW][64];  // partial scores, double-buffered by stage parity
    // Raw mode: per-row partial sums of squares xss[stage % 3][row][wave], the per-row
    // norm factors xr, and the cos/sin table xtab[stage % 2][row][pair] (bf16 cos in the low
    // half, sin in the high half) when the kernel computes it.
    __shared__ __attribute__((aligned(16))) unsigned char rawlds[RAW ? raw_extra_lds(NW, Q8) : 16];
    auto *xss = reinterpret_cast<float (*)[16][NW]>(rawlds);
    // xr[stage % 2][0][row] = the weight factor (rinv; q8: scale * rinv), [1] its inverse,
    // [2] (q8) bias / scale
    auto *xr = reinterpret_cast<float (*)[3][16]>(rawlds + 3 * 16 * NW * 4);
    // q8: row sums of q [stage % 3][row][wave]
    auto *xsq = reinterpret_cast<float (*)[16][NW]>(rawlds + 3 * 16 * NW * 4 + 2 * 3 * 16 * 4);
    auto *xtab = reinterpret_cast<unsigned (*)[16][kTabStride]>(rawlds + 3 * 16 * NW * 4 + 2 * 3 * 16 * 4 +
                                                                (Q8 ? 3 * 16 * NW * 4 : 0));
    // q8: bf16 staging slots and the per-stage scale / bias rows
    __shared__ __attribute__((aligned(16))) unsigned char q8stg[Q8 ? kQ8Slots * kQ8Stage : 16];
    __shared__ __attribute__((aligned(16))) float q8sb[Q8 ? kQ8SbStages : 1][2][16];
    // cos/sin table of a stage: TR rows (one per position) x 64 pairs over 64*NW threads
    constexpr int TR = 16;
    constexpr int EPT = TR * 64 / (64 * NW);
    static_assert(EPT >= 1, "every thread computes at least one table entry");
    constexpr int TPR = 64 / EPT;  // threads per table row

    const int wg = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;

    // Packed kv heads: a stage holds RPP = 16 / pk rows of each of the pk kv heads (stage
    // row r belongs to kv head r / RPP, row r % RPP of the stage's row range).  pk is 1, 2
    // or 4 and the same in every lane.
    const int pk = uniform(p.pk);
    const int lrpp = 4 - __builtin_ctz(pk), RPP = 1 << lrpp;
    // Query head li belongs to kv head li / gk of the group (padding heads li >= G take
    // the last); the C rows 4lg .. 4lg+3 of this lane come from one kv head (RPP >= 4).
    const bool hmatch = ((4 * lg) >> lrpp) == min(li / p.gk, pk - 1);
    const int jl = (4 * lg) & (RPP - 1);

    // One segment: rows [j0, j1) of (sequence b, packed kv head kvh).  `slot` indexes its
    // partial; `direct` means the segment is the whole pair and writes the output itself.
    auto segment = [&](const int b, const int kvh, const int j0, const int j1, const SeqView sv,
                       const size_t slot, const bool direct) {
    const bool append = p.k_new != nullptr;

    // kv head kvh * pk + i of sequence b sits at head_off + i * head_stride
    const size_t head_off = (size_t) b * p.seq_stride + (size_t) kvh * pk * p.head_stride;
    uint16_t *kbase = p.k_cache + head_off;
    uint16_t *vbase = p.v_cache + head_off;
    const uint16_t *knew = append ? p.k_new + ((size_t) b * p.Hkv + kvh) * pk * D : nullptr;
    const uint16_t *vnew = SHARED ? knew : p.v_new + ((size_t) b * p.Hkv + kvh) * pk * D;
    // q8: the u8 rows (same element strides, in bytes) and the scale / bias rows
    unsigned char *q8base = Q8 ? p.q8 + head_off : nullptr;
    const size_t sb_off = Q8 ? (size_t) b * p.sb_seq_stride + (size_t) kvh * pk * p.sb_head_stride : 0;

    // 32-dim chunk of the QK k-step kk of this wave.  Raw mode interleaves the waves so
    // that each rotary pair (d, d + 256), d < 64, sits in one lane of wave 0 or 1.
    auto qk_chunk = [&](int kk) { return RAW ? wave + NW * kk : wave * KKW + kk; };
    // k-step holding the rotary partners (chunk + 8) of the chunk at k-step 0
    constexpr int KP = 8 / NW;

    // Q^T operand for this wave's dims: lane (li, lg) = head li, dims 32*chunk + 8lg .. +8
    // (zero for heads >= G).
    bf16x8 qv[KKW];
    {
        const bool qok = li < p.G;
        const uint16_t *qrow = p.q + ((size_t) b * p.Hq + (size_t) kvh * p.G + (qok ? li : 0)) * D + lg * 8;
#pragma unroll
        for (int kk = 0; kk < KKW; ++kk) {
            const u32x4 t = qok ? *reinterpret_cast<const u32x4 *>(qrow + 32 * qk_chunk(kk)) : u32x4{0u, 0u, 0u, 0u};
            qv[kk] = __builtin_bit_cast(bf16x8, t);
        }
    }
    // Raw mode: k-norm weights of the lane's QK dims, and the rotary frequencies of the
    // four table entries this thread computes per stage (row tid/16, pairs 4(tid%16)..+4).
    float kwf[RAW ? KKW : 1][8];
    float invf[RAW ? EPT : 1] = {};
    if constexpr (RAW) {
#pragma unroll
        for (int kk = 0; kk < KKW; ++kk) {
            const u32x4 t = *reinterpret_cast<const u32x4 *>(p.kw + 32 * qk_chunk(kk) + 8 * lg);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kwf[kk][2 * e] = bf16_lo(t[e]);
                kwf[kk][2 * e + 1] = bf16_hi(t[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < EPT; ++e) invf[e] = p.inv_freq[EPT * (tid % TPR) + e];
    }
    if constexpr (Q8) {
        // The new row of each kv head of the group is quantized into the cache before the
        // ring starts (wave pr: kv head pr), esQuantizeRawRows' arithmetic
        // (ESDecodeAttn.mm:491-509): min / max over the row, scale = max((max - min) / 255,
        // 1e-8), q = min(round((x - min) / scale), 255) rounding half away from zero, IEEE
        // division.  The ring then reads it like every other row.
        if (append && j1 == sv.nvis) {
            for (int pr = wave; pr < pk; pr += NW) {
                const u32x4 t = *reinterpret_cast<const u32x4 *>(knew + pr * D + lane * 8);
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[2 * e] = bf16_lo(t[e]);
                    x[2 * e + 1] = bf16_hi(t[e]);
                }
                float mn = x[0], mx = x[0];
#pragma unroll
                for (int e = 1; e < 8; ++e) {
                    mn = fminf(mn, x[e]);
                    mx = fmaxf(mx, x[e]);
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    mn = fminf(mn, __shfl_xor(mn, o));
                    mx = fmaxf(mx, __shfl_xor(mx, o));
                }
                float scl = (mx - mn) / 255.0f;
                if (!(scl > 1e-8f)) scl = 1e-8f;
                unsigned lo = 0u, hi = 0u;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned qi = (unsigned) fminf(roundf((x[e] - mn) / scl), 255.0f);
                    if (e < 4) lo |= qi << (8 * e);
                    else hi |= qi << (8 * (e - 4));
                }
                unsigned char *row = q8base + (size_t) pr * p.head_stride + (size_t) sv.newrow * kRawDim;
                *reinterpret_cast<uint2 *>(row + lane * 8) = uint2{lo, hi};
                if (lane == 0) {
                    const size_t at = sb_off + (size_t) pr * p.sb_head_stride + (size_t) sv.newrow;
                    p.qsc[at] = scl;
                    p.qbs[at] = mn;
                }
            }
        }
    }
    ESDA_WAIT_VM(0);  // operands are in registers before the ring starts counting its own loads
    if constexpr (Q8) lds_barrier();  // and the new row's stores are done before any wave's DMA

    // DMA source slot of this lane: sub-row dq, chunk dchunk of the row.
    const int dq = lane / RD::CPR, dchunk = lane % RD::CPR;
    const int nst = (j1 - j0 + RPP - 1) >> lrpp;
    constexpr int EB = Q8 ? 1 : 2;                // bytes per cache element (strides count elements)
    constexpr int ROWB = Q8 ? kRawDim : D * 2;    // bytes per cache row
    // Per-lane byte offsets of this wave's DMA slots inside a stage's row range (stage row
    // r: kv head r / RPP of the group, row r % RPP; below 2^31 bytes, checked by the host).
    unsigned dvoff[RD::DPT];
#pragma unroll
    for (int t = 0; t < RD::DPT; ++t) {
        const int r = wave * RD::DPT + t + dq * RD::NI;
        dvoff[t] = (unsigned) ((size_t) (r >> lrpp) * p.head_stride * EB + (size_t) (r & (RPP - 1)) * ROWB + dchunk * 16);
    }
    // DMA of stage st into ring buffer `buf` (ring slot `slot`).
    auto dma = [&](int st, unsigned char *buf, int slot) {
        const int jst = j0 + st * RPP;
        if constexpr (Q8) {
            // scale / bias of the stage's rows: wave w loads the scales (w < 4) or biases of
            // stage rows 4(w % 4) .. +3, one row per lane
            if (lane < 4) {
                const int sr = 4 * (wave & 3) + lane, pr = sr >> lrpp;
                const int j = jst + (sr & (RPP - 1)), jj = j < j1 ? j : j1 - 1;
                const float *src = (wave < 4 ? p.qsc : p.qbs) + sb_off + (size_t) pr * p.sb_head_stride +
                                   (size_t) (sv.first + jj);
                lds_dma4(src, lds_addr(&q8sb[slot][wave >> 2][4 * (wave & 3)]));
            }
        }
        if (jst + RPP < j1 && sv.first + jst + RPP <= p.cap) {
            // Interior stage: RPP consecutive cache rows per kv head, none clamped or new.
            if constexpr (Q8) {
                const unsigned char *qb = q8base + (size_t) (sv.first + jst) * kRawDim;
#pragma unroll
                for (int t = 0; t < RD::DPT; ++t) lds_dma16_s(qb, dvoff[t], lds_addr(buf) + (wave * RD::DPT + t) * RD::BLK);
                return;
            }
            const uint16_t *kb = kbase + (size_t) (sv.first + jst) * D;
            const uint16_t *vb = vbase + (size_t) (sv.first + jst) * D;
#pragma unroll
            for (int t = 0; t < RD::DPT; ++t) {
                const int i = wave * RD::DPT + t;
                lds_dma16_s(kb, dvoff[t], lds_addr(buf) + i * RD::BLK);
                if constexpr (!SHARED) lds_dma16_s(vb, dvoff[t], lds_addr(buf) + RD::TB + i * RD::BLK);
            }
            return;
        }
#pragma unroll
        for (int t = 0; t < RD::DPT; ++t) {
            const int i = wave * RD::DPT + t;           // DMA block of this stage
            const int sr = i + dq * RD::NI;             // stage row this lane feeds
            const int pr = sr >> lrpp;                  // its kv head within the group
            const int j = jst + (sr & (RPP - 1));       // its logical row
            const int jj = j < j1 ? j : j1 - 1;          // clamp: masked rows read a visible row
            int r = sv.first + jj;
            if (r >= p.cap) r -= p.cap;
            if constexpr (Q8) {
                // the new row was quantized into the cache before the ring started
                lds_dma16(q8base + (size_t) pr * p.head_stride + (size_t) r * kRawDim + dchunk * 16,
                          lds_addr(buf) + i * RD::BLK);
                continue;
            }
            const bool from_new = append && (jj == sv.nvis - 1);
            const size_t hoff = (size_t) pr * p.head_stride + (size_t) r * D;
            const uint16_t *ks = (from_new ? knew + pr * D : kbase + hoff) + dchunk * 8;
            lds_dma16(ks, lds_addr(buf) + i * RD::BLK);
            if constexpr (!SHARED) {
                const uint16_t *vs = (from_new ? vnew + pr * D : vbase + hoff) + dchunk * 8;
                lds_dma16(vs, lds_addr(buf) + RD::TB + i * RD::BLK);
            }
        }
    };
    // q8: bf16 staging slot of stage s, and the widening of u8 stage s (ring buffer u8buf)
    // into it: thread t takes row t / 32, bytes 16 (t % 32) .. +16; a byte's bf16 is the
    // upper half of its fp32 (exact for 0 .. 255).
    auto stg = [&](int s) -> unsigned char * { return q8stg + (s & (kQ8Slots - 1)) * kQ8Stage; };
    auto convert = [&](int s, const unsigned char *u8buf) {
        if constexpr (Q8) {
            const int r = tid >> 5, c16 = tid & 31;
            const u32x4 w = *reinterpret_cast<const u32x4 *>(u8buf + (r & 7) * RD::BLK + (r >> 3) * kRawDim + c16 * 16);
            unsigned o[8];
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const unsigned lo = __builtin_bit_cast(unsigned, (float) ((w[e] >> (16 * h)) & 255u));
                    const unsigned hi = __builtin_bit_cast(unsigned, (float) ((w[e] >> (16 * h + 8)) & 255u));
                    o[2 * e + h] = __builtin_amdgcn_perm(hi, lo, 0x07060302u);
                }
            unsigned char *dst = stg(s) + r * R::BLK + c16 * 32;
            *reinterpret_cast<u32x4 *>(dst) = u32x4{o[0], o[1], o[2], o[3]};
            *reinterpret_cast<u32x4 *>(dst + 16) = u32x4{o[4], o[5], o[6], o[7]};
        }
    };

    // Per-lane LDS offsets: the QK A operand (row li, chunk qk_chunk(kk), 16 bytes at
    // 8lg dims) and the V^T transpose read (lane (li, lg) supplies row 4lg + li/4, dims
    // wave*DW + 16dt + 4(li%4) .. +4; ds_read_b64_tr_b16 hands lane li of the group dim
    // 16dt + li of rows 4lg .. 4lg+3, the PV A operand).
    const int qk_off = R::off(li, 0, 0) + lg * 16;                     // + 64*qk_chunk(kk)
    const int tr_off = R::off(4 * lg + li / 4, wave, 0) + (li % 4) * 8;  // + 32*dt
    constexpr int VOFF = SHARED ? 0 : R::TB;

    float m = -INFINITY, l = 0.0f;
    float bt = 0.0f;  // q8: sum of P * bias / scale of this lane's head (the bias part of PV)
    f32x4 acc[DTW];
#pragma unroll
    for (int dt = 0; dt < DTW; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Partial scores of a stage over this wave's dims, published for the other waves.
    auto qk_partial = [&](const unsigned char *kb, int par) {
        f32x4 sp = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KKW; ++kk) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(kb + qk_off + 64 * qk_chunk(kk));
            sp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qv[kk], sp, 0, 0, 0);
        }
        // D = 512: only the live heads' columns (lanes li < G) are exchanged; the padding
        // heads' partials are zero (their Q^T operand is)
        if (!kLiveX || li < p.G) xch[par][wave][lane] = sp;
    };

    // ---- raw mode helpers
    u32x4 araw[RAW ? KKW : 1];  // raw QK operand of the next stage to score
    auto load_raw = [&](const unsigned char *kb) {
#pragma unroll
        for (int kk = 0; kk < (RAW ? KKW : 1); ++kk)
            araw[kk] = *reinterpret_cast<const u32x4 *>(kb + qk_off + 64 * qk_chunk(kk));
    };
    // Partial sum of squares of row li over this wave's dims -> xss[buf][li][wave]: the
    // diagonal of the stage's 16x16 Gram matrix over those dims.  The A and B operands of
    // v_mfma_f32_16x16x32_bf16 take the same lane data (row li, dims 8lg..+8 of each
    // chunk), and products of bf16 values are exact in the fp32 accumulation.
    // q8: the operand is q itself, so the diagonal is sum(q^2), and an MFMA against ones
    // gives sum(q) -> xsq; both are exact integers (per wave at most 64 * 255^2 < 2^24).
    auto publish_ss = [&](int buf) {
        if constexpr (RAW) {
            f32x4 g = {0.0f, 0.0f, 0.0f, 0.0f}, g1 = {0.0f, 0.0f, 0.0f, 0.0f};
            bf16x8 ones;
#pragma unroll
            for (int e = 0; e < 8; ++e) ones[e] = (__bf16) 1.0f;
#pragma unroll
            for (int kk = 0; kk < KKW; ++kk) {
                const bf16x8 a = __builtin_bit_cast(bf16x8, araw[kk]);
                g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, a, g, 0, 0, 0);
                if constexpr (Q8) g1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, g1, 0, 0, 0);
            }
            // C layout: lane (li, lg) holds C[4lg + i][li]; row li's diagonal entry is
            // register li - 4lg of the lanes with lg == li / 4.
            const int i = li - 4 * lg;
            if (i >= 0 && i < 4) {
                xss[buf][li][wave] = i == 0 ? g[0] : i == 1 ? g[1] : i == 2 ? g[2] : g[3];
                if constexpr (Q8) xsq[buf][li][wave] = i == 0 ? g1[0] : i == 1 ? g1[1] : i == 2 ? g1[2] : g1[3];
            }
        }
    };
    // cos/sin table of stage st: this thread's row tid / TPR, pairs EPT*(tid % TPR) .. +EPT.
    auto publish_tab = [&](int st, int buf) {
        if constexpr (RAW) {
            const int row = tid / TPR;
            const float t = (float) (sv.first + j0 + st * TR + row);
            unsigned w[EPT];
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                float s, c;
                sincos_f32(t * invf[e], s, c);
                w[e] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{c, s}, bf16x2));
            }
            unsigned *dst = &xtab[buf][row][EPT * (tid % TPR)];
            static_assert(EPT == 1 || EPT == 2 || EPT == 4, "table entries per thread");
            if constexpr (EPT == 4) {
                *reinterpret_cast<u32x4 *>(dst) = u32x4{w[0], w[1], w[2], w[3]};
            } else if constexpr (EPT == 2) {
                *reinterpret_cast<uint2 *>(dst) = uint2{w[0], w[1]};
            } else {
                *dst = w[0];
            }
        }
    };
    // mean(kraw^2) + eps of a row; rinv = rsqrt of it.
    auto row_ms = [&](int buf, int row) {
        float sum = 0.0f;
#pragma unroll
        for (int q4 = 0; q4 < NW; q4 += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&xss[buf][row][q4]);
            sum += (v[0] + v[1]) + (v[2] + v[3]);
        }
        return sum * (1.0f / kRawDim) + p.eps;
    };
    // q8: mean(x^2) + eps of a row from its sums, x = q * scale + bias: mean(x^2) =
    // scale^2 var(q) + mean(x)^2, 512^2 var(q) = 512 sum(q^2) - sum(q)^2.  sum(q) < 2^24 is
    // exact in fp32; sum(q^2) may round by a few units in 3.3e7, which moves var(q) by
    // ~1e-5 of its size at most and mean(x^2) far less (the mean term carries no such error).
    auto q8_ms = [&](int buf, int row, float scl, float bias) {
        float s2 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int q4 = 0; q4 < NW; q4 += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(&xss[buf][row][q4]);
            const f32x4 c = *reinterpret_cast<const f32x4 *>(&xsq[buf][row][q4]);
            s2 += (a[0] + a[1]) + (a[2] + a[3]);
            s1 += (c[0] + c[1]) + (c[2] + c[3]);
        }
        const float var = fmaxf(__builtin_fmaf(512.0f, s2, -s1 * s1), 0.0f);
        const float mean = __builtin_fmaf(scl, s1 * (1.0f / kRawDim), bias);
        return scl * scl * var * (1.0f / (kRawDim * kRawDim)) + __builtin_fmaf(mean, mean, p.eps);
    };
    // Scores of the stage held in araw: rebuild K in registers, then MFMA.  sbslot: the
    // ring slot of the stage (q8: its scale / bias rows).
    auto qk_raw = [&](int ssbuf, int tabbuf, int par, int sbslot) {
        if constexpr (RAW) {
            float kn[KKW][8];
            if constexpr (Q8) {
                const float scl = q8sb[sbslot][0][li], bias = q8sb[sbslot][1][li];
                const float rinv = __builtin_amdgcn_rsqf(q8_ms(ssbuf, li, scl, bias));
                const float alpha = scl * rinv, beta = bias * rinv;
                // the weight factor scale * rinv, its inverse, and bias / scale (two IEEE
                // divisions: written by wave 2, whose SIMD has no rotary work)
                if (wave == 2 && lg == 0) {
                    xr[par][0][li] = alpha;
                    xr[par][1][li] = 1.0f / alpha;
                    xr[par][2][li] = bias / scl;
                }
    #pragma unroll
                for (int kk = 0; kk < KKW; ++kk)
    #pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kn[kk][2 * e] = __builtin_fmaf(bf16_lo(araw[kk][e]), alpha, beta) * kwf[kk][2 * e];
                        kn[kk][2 * e + 1] = __builtin_fmaf(bf16_hi(araw[kk][e]), alpha, beta) * kwf[kk][2 * e + 1];
                    }
            } else {
                (void) sbslot;
                const float ms = row_ms(ssbuf, li);
                const float rinv = __builtin_amdgcn_rsqf(ms);
                // rinv and 1/rinv (= ms * rinv) of the row, for the stage's softmax weights.
                if (wave == 0 && lg == 0) {
                    xr[par][0][li] = rinv;
                    xr[par][1][li] = ms * rinv;
                }
    #pragma unroll
                for (int kk = 0; kk < KKW; ++kk)
    #pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kn[kk][2 * e] = bf16_lo(araw[kk][e]) * rinv * kwf[kk][2 * e];
                        kn[kk][2 * e + 1] = bf16_hi(araw[kk][e]) * rinv * kwf[kk][2 * e + 1];
                    }
            }
            if (wave < 2) {
                // chunk `wave` (k-step 0) holds dims d = 32*wave + 8lg + e < 64; chunk wave + 8
                // (k-step KP) their rotary partners.
                const unsigned *tb = &xtab[tabbuf][li][32 * wave + 8 * lg];
                const u32x4 t0 = *reinterpret_cast<const u32x4 *>(tb);
                const u32x4 t1 = *reinterpret_cast<const u32x4 *>(tb + 4);
    #pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned w = e < 4 ? t0[e] : t1[e - 4];
                    const float c = bf16_lo(w), s = bf16_hi(w);
                    const float lo = kn[0][e], hi = kn[KP][e];
                    kn[0][e] = lo * c - hi * s;
                    kn[KP][e] = hi * c + lo * s;
                }
            }
            f32x4 sp = {0.0f, 0.0f, 0.0f, 0.0f};
    #pragma unroll
            for (int kk = 0; kk < KKW; ++kk) {
                bf16x8 a;
    #pragma unroll
                for (int e = 0; e < 8; ++e) a[e] = (__bf16) kn[kk][e];
                sp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qv[kk], sp, 0, 0, 0);
            }
            xch[par][wave][lane] = sp;
        }
    };

    // The buffer the compute reads for stage s held in ring slot uc: the ring itself, or
    // (q8) the stage's bf16 staging slot.
    auto cbuf = [&](int s, auto uc) -> unsigned char * {
        if constexpr (Q8) return stg(s);
        else return ring(uc);
    };
    // Prologue: fill NS-1 stages; publish what iteration 0 needs.
    unroll<NS - 1>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (u < nst) dma(u, ring(uc), u);
    });
    if constexpr (RAW) {
        // stages 0..2 landed (stage 2 for the first iteration's sums of squares; q8: the
        // stages widened here)
        if (nst - 1 >= NS - 2) {
            ESDA_WAIT_VM((NS - 4) * DPW);
        } else {
            ESDA_WAIT_VM(0);
        }
        lds_barrier();
        if constexpr (Q8) {
            convert(0, ring(std::integral_constant<int, 0>{}));
            if (nst > 1) convert(1, ring(std::integral_constant<int, 1>{}));
            if (nst > 2) convert(2, ring(std::integral_constant<int, 2>{}));
            lds_barrier();
        }
        load_raw(cbuf(0, std::integral_constant<int, 0>{}));
        publish_ss(0);
        publish_tab(0, 0);
        if (nst > 1) {
            load_raw(cbuf(1, std::integral_constant<int, 1>{}));
            publish_ss(1);
            publish_tab(1, 1);
        }
        lds_barrier();
        // scores of stage 0 (its raw operand is read again; araw keeps stage 1's)
        {
            u32x4 keep[KKW];
#pragma unroll
            for (int kk = 0; kk < KKW; ++kk) keep[kk] = araw[kk];
            load_raw(cbuf(0, std::integral_constant<int, 0>{}));
            qk_raw(0, 0, 0, 0);
#pragma unroll
            for (int kk = 0; kk < KKW; ++kk) araw[kk] = keep[kk];
        }
    } else {
        if (nst - 1 >= NS - 2) {
            ESDA_WAIT_VM((NS - 2) * DPW);
        } else {
            ESDA_WAIT_VM(0);
        }
        lds_barrier();
        qk_partial(ring(std::integral_constant<int, 0>{}), 0);
    }

    // Iteration st: one barrier, after which (a) every wave's stage-st partial scores
    // are in xch, (b) stage st+AHEAD has landed from every wave's DMA, and (c) every wave
    // is done with stage st-1's buffer, which is refilled at once.  The scores of stage
    // st+1 are computed alongside stage st's PV, so the two dependency chains overlap.
    auto stage = [&](int s0, auto uc) {
        constexpr int u = decltype(uc)::value;
        const int st = s0 + u;
        if (st >= nst) return;
        if (st + AHEAD < nst) {
            // own DMA for stage st+AHEAD done; the stages behind it may stay in flight --
            // except at D = 256, whose two workgroups per CU then keep twice the 512-dim
            // kernel's bytes in flight (16.8 MB over the GPU, past the 6-15 MB at which the
            // read probe peaks): waiting for every issued stage there took C5 7.50 -> 7.44 ms
            if (D != 256 && nst - st - AHEAD - 1 >= NS - 2 - AHEAD) {
                ESDA_WAIT_VM((NS - 2 - AHEAD) * DPW);
            } else {
                ESDA_WAIT_VM(0);
            }
        }
        lds_barrier();
        if (st + NS - 1 < nst) dma(st + NS - 1, ring(std::integral_constant<int, (u + NS - 1) % NS>{}), (u + NS - 1) % NS);
        // q8: widen stage st+3 (landed: this iteration's wait) for the next iterations
        if constexpr (Q8) {
            if (st + 3 < nst) convert(st + 3, ring(std::integral_constant<int, (u + 3) % NS>{}));
        }
        f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (RAW || !kLiveX || li < p.G) {
            sc = xch[st & 1][0][lane];
#pragma unroll
            for (int w = 1; w < NW; ++w) sc += xch[st & 1][w][lane];
        }
        // V^T operands of this stage (plain kernels), read behind the exchange so that
        // their latency hides under the softmax instead of following it
        const unsigned char *vb = cbuf(st, uc) + VOFF;
        short4v va[RAW ? 1 : DTW];
        if constexpr (!RAW) {
#pragma unroll
            for (int dt = 0; dt < DTW; ++dt)
                va[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) short4v *) (vb + tr_off + 32 * dt));
        }
        // The look-ahead work runs unconditionally (one basic block with the softmax, so
        // the two interleave): past the last stage it reads stale but in-bounds LDS and
        // writes exchange slots that are never read again.
        if constexpr (RAW) {
            qk_raw((st + 1) % 3, (st + 1) & 1, (st + 1) & 1, (u + 1) % NS);
            load_raw(cbuf(st + 2, std::integral_constant<int, (u + 2) % NS>{}));
            publish_ss((st + 2) % 3);
            publish_tab(st + 2, st & 1);
        } else {
            qk_partial(ring(std::integral_constant<int, (u + 1) % NS>{}), (st + 1) & 1);
        }
        // Online softmax (log2 domain), identical in every wave; rows past the split
        // end (last stage only) and rows of another kv head of the group are masked.
        const int jt = j0 + st * RPP + jl;
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = hmatch && (jt + r) < j1 ? sc[r] * p.scale_log2e : -INFINITY;
        const float tmax = wave_max_across_groups(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        if (__any(tmax > m + kRescaleSlack)) {
            const float mnew = fmaxf(m, tmax);
            const float corr = __builtin_amdgcn_exp2f(m - mnew);
            l *= corr;
            if constexpr (Q8) bt *= corr;
#pragma unroll
            for (int dt = 0; dt < DTW; ++dt) acc[dt] *= corr;
            m = mnew;
        }
        short4v pbs;
        if constexpr (RAW) {
            // V = kraw * rinv enters through the weight: P = bf16(e * rinv).  l adds the
            // same rounded weight divided by rinv (ms * rinv = 1 / rinv), so numerator and
            // denominator carry identical rounding and a dominant row is reproduced exactly.
            // q8: the factor is scale * rinv (V enters as q) and the bias adds P * bias / scale.
            const f32x4 ri = *reinterpret_cast<const f32x4 *>(&xr[st & 1][0][4 * lg]);
            const f32x4 rn = *reinterpret_cast<const f32x4 *>(&xr[st & 1][1][4 * lg]);
            f32x4 gm = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (Q8) gm = *reinterpret_cast<const f32x4 *>(&xr[st & 1][2][4 * lg]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(sc[r] - m);
                const __bf16 pw = (__bf16) (e * ri[r]);
                l += (float) pw * rn[r];
                if constexpr (Q8) bt += (float) pw * gm[r];
                pbs[r] = __builtin_bit_cast(short, pw);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const __bf16 pr = (__bf16) __builtin_amdgcn_exp2f(sc[r] - m);
                l += (float) pr;
                pbs[r] = __builtin_bit_cast(short, pr);
            }
        }
        // O^T (this wave's dims) += V^T . P^T
#pragma unroll
        for (int dt = 0; dt < DTW; ++dt) {
            if constexpr (RAW) {
                const short4v a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) short4v *) (vb + tr_off + 32 * dt));
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pbs, acc[dt], 0, 0, 0);
            } else {
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[dt], pbs, acc[dt], 0, 0, 0);
            }
        }
    };
    for (int s0 = 0; s0 < nst; s0 += NS) unroll<NS>([&](auto uc) { stage(s0, uc); });

    // Fused append: the workgroup whose rows end at the new token copies k_new / v_new
    // into its cache row (bit-exact).  Its own DMA reads that row from k_new / v_new and
    // no other workgroup reads it; the copy runs after this workgroup's ring has
    // drained, so no outstanding load is counted against the ring's waits.
    if (!Q8 && append && j1 == sv.nvis) {
        for (int pr = wave; pr < pk; pr += NW) {  // wave pr copies kv head pr of the group
            const size_t row = (size_t) pr * p.head_stride + (size_t) sv.newrow * D;
            for (int c = lane; c < D / 8; c += 64) {
                *reinterpret_cast<u32x4 *>(kbase + row + c * 8) =
                    *reinterpret_cast<const u32x4 *>(knew + pr * D + c * 8);
                if constexpr (!SHARED)
                    *reinterpret_cast<u32x4 *>(vbase + row + c * 8) =
                        *reinterpret_cast<const u32x4 *>(vnew + pr * D + c * 8);
            }
        }
    }

    // Partial of this split: every wave holds the same (m, l) and its own dim slice.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if constexpr (Q8) {
        // the bias part of PV is the same for every dim of a head
        bt += __shfl_xor(bt, 16);
        bt += __shfl_xor(bt, 32);
#pragma unroll
        for (int dt = 0; dt < DTW; ++dt) acc[dt] += bt;
    }
    if (direct) {
        // The only segment of this (sequence, kv head): normalise here, with the merge's
        // arithmetic (acc * (1 / l), then bf16); the merge skips this pair.
        if (li < p.G) {
            const float inv = 1.0f / l;
            uint16_t *dst = p.out + ((size_t) b * p.Hq + (size_t) kvh * p.G + li) * D + wave * DW;
#pragma unroll
            for (int dt = 0; dt < DTW; ++dt) {
                bf16x4 r;
#pragma unroll
                for (int e = 0; e < 4; ++e) r[e] = (__bf16) (acc[dt][e] * inv);
                *reinterpret_cast<uint2 *>(dst + 16 * dt + 4 * lg) = __builtin_bit_cast(uint2, r);
            }
        }
        return;
    }
    if (li < p.G) {
        const size_t pidx = slot * p.G + li;
        float *dst = p.part_acc + pidx * D + wave * DW;
        // D = 512: the partials are stored non-temporal (the merge reads them from another
        // XCD; C4 step 82.2 -> 81.2 us, C2 14.7 -> 14.2).  The short D = 256 launches finish
        // sooner with write-back stores (C1 attend 5.4 against 5.8 us).
        if constexpr (D == 512) {
#pragma unroll
            for (int dt = 0; dt < DTW; ++dt) __builtin_nontemporal_store(acc[dt], reinterpret_cast<f32x4 *>(dst + 16 * dt + 4 * lg));
            if (wave == 0 && lg == 0) __builtin_nontemporal_store(f32x2{m, l}, reinterpret_cast<f32x2 *>(p.part_ml + pidx * 2));
        } else {
#pragma unroll
            for (int dt = 0; dt < DTW; ++dt) *reinterpret_cast<f32x4 *>(dst + 16 * dt + 4 * lg) = acc[dt];
            if (wave == 0 && lg == 0) *reinterpret_cast<f32x2 *>(p.part_ml + pidx * 2) = f32x2{m, l};
        }
    }
    };

    walk_segments<NW>(p, segment);
}

// ------------------------------------------------- raw-K attend with wave-private rings
//
// Raw-K decode (ESDecodeAttn.mm:17-117) when the caller passes the precomputed rotary table
// -- the ES layer's path.  A workgroup serves one kv head (a contiguous run of its rows, as
// the composite kernel's) with four waves, one per SIMD.  Each wave owns whole 16-row stages
// (16 consecutive positions) over the full 512-dim head, in turn: wave w takes stages w,
// w + 4, w + 8, ... of a segment.  It streams their rows through two LDS slots of its own and
// their cos / sin table rows through a table buffer of its own, filled by its own LDS DMA and
// waited on with its own vmcnt, so the main loop has no barrier and no exchange between
// waves.  Per stage a wave:
//   - reads the 16 raw rows as MFMA A operands (lane (li, lg): row li, dims kdim(kk, lg)
//     of k-step kk);
//   - forms their 16x16 Gram matrix with 16 MFMAs: the diagonal is each row's sum of
//     squares (exact bf16 products, fp32 sums), hence rinv = rsqrt(mean + eps);
//   - rebuilds K = bf16(rope(kraw * rinv * kw)), rounded where the reference rounds it:
//     kraw * kw comes exactly (a product of two bf16 values fits fp32) from MFMAs of the
//     lane's own rows against diag(kw) operands built once per kernel, whose C layout
//     hands every lane the dims it supplied; one multiply by rinv, the rotation and the
//     bf16 rounding remain per element.  The rotary partners (d, d + 256), d < 64, sit in
//     one lane (k-steps 0, 1 and 8, 9); their bf16 cos / sin come from the table rows,
//     whose buffer takes the next stage's table rows once the rotary k-steps have read it;
//   - scores the kv head's query heads (up to 16: the MFMA's N dimension, zero-padded) with
//     16 MFMAs, runs its own online softmax, and accumulates O^T[512 x 16 heads] with 32
//     MFMAs over V = kraw read back by transpose reads, rinv folded into the weight:
//     P = bf16(e * rinv), l += P / rinv.
// Q8 (esDecodeAttnGlobalQ8, ESDecodeAttn.mm:275-369): rows are u8 with a per-row scale and
// bias (x = q * scale + bias).  sum(q^2) and sum(q) of each row are exact integer dot products
// of the u8 bytes (v_dot4_u32_u8, summed over the four lane groups), hence mean(x^2), and every
// lane computes its own row's factors;
// K = bf16(rope(fma(q, scale * rinv, bias * rinv) * kw)); q is also written to a bf16 tile
// of the wave's that the transpose reads use as V, with P = bf16(e * scale * rinv) and the
// bias entering as sum(P * bias / scale) per head.
// At the end of a segment the four waves' (m, l, O) merge through LDS into one partial.

constexpr int kWaves = 4;                  // waves of the wave-private-ring kernels
constexpr int kBlk = 1056;                 // LDS bytes per 1 KiB DMA block (1 KiB + 32 B pad)

// Dims of k-step kk held by lane group lg: 8 consecutive dims, the four lane groups side by
// side (32 kk + 8 lg), so that a row's lane groups read (and the q8 V tile's writes write)
// adjacent 16-byte pieces, without LDS bank conflicts; the rotary partners of k-steps 0, 1 are
// k-steps 8, 9 of the same lane.
__device__ __forceinline__ int kdim(int kk, int lg) { return 32 * kk + 8 * lg; }
// The rotary k-steps: dims 0 .. 63 (k-steps 0, 1) and their partners 256 .. 319 (8, 9).
__device__ __forceinline__ constexpr bool rot_step(int kk) { return (kk & 7) < 2; }

// Lazy-rescale threshold of the raw kernels (log2 units).  Their V rows are RMS-normalised
// (|v_d| <= sqrt(512)), so with probabilities up to 2^64 before normalisation the partial
// sums stay below rows * 2^64 * 2^6 < 2^101 for any row count under 2^31, far from fp32's
// limit.  The in-model scale of these layers is 1.0, which spreads the scores widely:
// with the generic threshold of 8 about half of all stages would rescale.
constexpr float kRawRescaleSlack = 64.0f;

template <bool Q8>
struct WRing {
    static constexpr int ROWS = Q8 ? 8 * kBlk : 16 * kBlk;  // a stage's 16 rows (q8: two per block)
    static constexpr int SB = Q8 ? 128 : 0;                  // q8: 16 scales, 16 biases
    static constexpr int SLOT = ROWS + SB;
    static constexpr int STG = Q8 ? 16 * kBlk : 0;           // q8: the bf16 V tile
    static constexpr int TAB = 4 * kBlk;                     // the stage's 16 cos/sin table rows (swizzled)
    static constexpr int WAVE = 2 * SLOT + STG + TAB;        // one wave's LDS: two slots, the V tile, the table
    static constexpr int MERGE = kWaves * 16 * 516 * 4;      // end-of-segment merge area (aliases the rings)
    static_assert(kWaves * WAVE >= MERGE, "the merge area fits in the rings");
};

// DMA of LDS blocks I .. N-1 of an interior stage: block i is 1 KiB of memory at
// base[i / 4] + (i % 4) KiB and lands at LDS block i (lds + i * kBlk), so four blocks share
// one scalar base (immediate offsets) and each costs one scalar instruction beside its DMA.
template <int I, int N>
__device__ __forceinline__ void ring_blocks(const uint64_t *base, unsigned voff, unsigned lds) {
    if constexpr (I < N) {
        constexpr int k = I & 3;
        lds_dma16_o<k * 1024, 4 * (I >> 2) * kBlk + k * (kBlk - 1024)>(base[I >> 2], voff, lds);
        ring_blocks<I + 1, N>(base, voff, lds);
    }
}

template <bool Q8>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kWaves, 64 * kWaves), amdgpu_waves_per_eu(1, 1)))
void raw_attend_kernel(AttendParams p) {
    using W = WRing<Q8>;
    __shared__ __attribute__((aligned(16))) unsigned char wlds[kWaves * W::WAVE];
    // per-wave row factors of the stage being computed (the softmax's rows 4lg .. 4lg + 3):
    // [0] rinv (q8: scale * rinv), [1] its inverse, [2] (q8) bias / scale
    __shared__ __attribute__((aligned(16))) float xf[kWaves][3][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;
    unsigned char *const wl = wlds + wave * W::WAVE;

    // q8: the k-norm weights in fp32, read per k-step (the lanes of a lane group read the
    // same 32 bytes); 128 of them per lane would not fit in registers beside O^T and Q^T.
    __shared__ __attribute__((aligned(16))) float kwl[Q8 ? kRawDim : 1];
    if constexpr (Q8) {
        const unsigned t = reinterpret_cast<const unsigned *>(p.kw)[tid];
        kwl[2 * tid] = bf16_lo(t);
        kwl[2 * tid + 1] = bf16_hi(t);
        __syncthreads();
    }
    // Raw: the A operands of the x * kw products, diag(kw) over 16 dims.  For k-step kk and half
    // hh the B operand is the lane's own dims kdim(kk, lg) + 4hh .. + 3 of row li; lane
    // (li, lg) then holds kw of dim kdim(kk, lg) + 4hh + (li & 3) at slot li & 3 when
    // lg == li / 4 and zeros elsewhere, and the product's C layout hands every lane x * kw
    // of the same dims it supplied.
    short4v dg[Q8 ? 1 : 16][2];
    if constexpr (!Q8) {
        const short *kwb = reinterpret_cast<const short *>(p.kw);
        const int s = li & 3;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const short w = (li >> 2) == lg ? kwb[kdim(kk, lg) + 4 * hh + s] : (short) 0;
                dg[kk][hh] = short4v{s == 0 ? w : (short) 0, s == 1 ? w : (short) 0, s == 2 ? w : (short) 0,
                                     s == 3 ? w : (short) 0};
            }
    }

    auto segment = [&](const int b, const int kvh, const int j0, const int j1, const SeqView sv, const size_t slot,
                       const bool direct) {
        const bool append = p.k_new != nullptr;
        const size_t head_off = (size_t) b * p.seq_stride + (size_t) kvh * p.head_stride;
        uint16_t *const kbase = p.k_cache + head_off;
        const uint16_t *const knew = append ? p.k_new + ((size_t) b * p.Hkv + kvh) * kRawDim : nullptr;
        unsigned char *const q8base = Q8 ? p.q8 + head_off : nullptr;
        const size_t sb_off = Q8 ? (size_t) b * p.sb_seq_stride + (size_t) kvh * p.sb_head_stride : 0;

        // Q^T operand: head li of the packed pair (zero for padding heads li >= G)
        bf16x8 qv[16];
        {
            const bool qok = li < p.G;
            const uint16_t *qrow = p.q + ((size_t) b * p.Hq + (size_t) kvh * p.G + (qok ? li : 0)) * kRawDim;
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                const u32x4 t = qok ? *reinterpret_cast<const u32x4 *>(qrow + kdim(kk, lg)) : u32x4{0u, 0u, 0u, 0u};
                qv[kk] = __builtin_bit_cast(bf16x8, t);
            }
        }
        if constexpr (Q8) {
            // The new row is quantized into the cache before any DMA (wave 0),
            // esQuantizeRawRows' arithmetic (ESDecodeAttn.mm:491-509).
            if (append && j1 == sv.nvis && wave == 0) {
                const u32x4 t = *reinterpret_cast<const u32x4 *>(knew + lane * 8);
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[2 * e] = bf16_lo(t[e]);
                    x[2 * e + 1] = bf16_hi(t[e]);
                }
                float mn = x[0], mx = x[0];
#pragma unroll
                for (int e = 1; e < 8; ++e) {
                    mn = fminf(mn, x[e]);
                    mx = fmaxf(mx, x[e]);
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    mn = fminf(mn, __shfl_xor(mn, o));
                    mx = fmaxf(mx, __shfl_xor(mx, o));
                }
                float scl = (mx - mn) / 255.0f;
                if (!(scl > 1e-8f)) scl = 1e-8f;
                unsigned lo = 0u, hi = 0u;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned qi = (unsigned) fminf(roundf((x[e] - mn) / scl), 255.0f);
                    if (e < 4) lo |= qi << (8 * e);
                    else hi |= qi << (8 * (e - 4));
                }
                unsigned char *row = q8base + (size_t) sv.newrow * kRawDim;
                *reinterpret_cast<uint2 *>(row + lane * 8) = uint2{lo, hi};
                if (lane == 0) {
                    const size_t at = sb_off + (size_t) sv.newrow;
                    p.qsc[at] = scl;
                    p.qbs[at] = mn;
                }
            }
        }
        ESDA_WAIT_VM(0);  // operands in registers (and the q8 row stored) before the ring counts its loads
        if constexpr (Q8) {
            if (append && j1 == sv.nvis) lds_barrier();  // the quantized row is in memory before any DMA
        }

        const int nst = (j1 - j0 + 15) >> 4;  // 16-row stages: 16 positions
        // DMA of stage st's rows into slot sl.  Rows past the segment end repeat its last row
        // (their scores are masked); the new token's raw row comes from k_new.
        auto dma_rows = [&](int st, unsigned char *sl) {
            const int jst = j0 + 16 * st;
            const unsigned lb = lds_addr(sl);
            // q8 block i: rows 2i, 2i + 1; lane l loads row 2i + (l & 1), 16-byte piece l >> 1
            const int h = lane & 1, pc = lane >> 1;
            if (jst + 16 < j1) {
                // Interior stage: all sixteen positions exist (the segment's last row is in the
                // last stage).  Four consecutive 1 KiB blocks of memory (raw rows; pairs of q8
                // rows) share one scalar base through the DMA's immediate offset (ring_blocks).
                if constexpr (Q8) {
                    const unsigned char *r0 = q8base + (size_t) (sv.first + jst) * kRawDim;
                    const uint64_t base[2] = {sbase64(r0), sbase64(r0 + 4096)};
                    const unsigned v = (unsigned) (h * kRawDim + pc * 16);
                    ring_blocks<0, 8>(base, v, lb);
                } else {
                    const unsigned char *r0 = reinterpret_cast<const unsigned char *>(kbase + (size_t) (sv.first + jst) * kRawDim);
                    const uint64_t base[4] = {sbase64(r0), sbase64(r0 + 4096), sbase64(r0 + 8192), sbase64(r0 + 12288)};
                    ring_blocks<0, 16>(base, (unsigned) (lane * 16), lb);
                }
            } else {
                if constexpr (Q8) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int j = min(jst + 2 * i + h, j1 - 1);
                        lds_dma16(q8base + (size_t) (sv.first + j) * kRawDim + pc * 16, lb + i * kBlk);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int j = min(jst + r, j1 - 1);
                        const uint16_t *src = (append && j == sv.nvis - 1) ? knew : kbase + (size_t) (sv.first + j) * kRawDim;
                        lds_dma16(src + lane * 8, lb + r * kBlk);
                    }
                }
            }
            if constexpr (Q8) {
                // scales (lanes 0..15) and biases (16..31) of the stage's rows
                if (lane < 32) {
                    const int j = min(jst + (lane & 15), j1 - 1);
                    lds_dma4((lane < 16 ? p.qsc : p.qbs) + sb_off + (size_t) (sv.first + j), lb + W::ROWS);
                }
            }
        };
        // raw: chunk c (of 4) of stage st's row DMAs, rows 4c .. 4c + 3.  The next stage's rows
        // go out in four chunks over the iteration (at the top, after the Gram pass, beside the
        // table rows, after the scores) rather than sixteen DMAs at once, which stalled their
        // issue behind the other waves' loads (c4raw attend 91.3 -> 90.8 us).
        auto dma_rows_part = [&](int st, unsigned char *sl, auto cc) {
            constexpr int c = decltype(cc)::value;
            const int jst = j0 + 16 * st;
            const unsigned lb = lds_addr(sl);
            if (jst + 16 < j1) {
                const unsigned char *r0 = reinterpret_cast<const unsigned char *>(kbase + (size_t) (sv.first + jst) * kRawDim);
                const uint64_t base[4] = {sbase64(r0), sbase64(r0 + 4096), sbase64(r0 + 8192), sbase64(r0 + 12288)};
                ring_blocks<4 * c, 4 * c + 4>(base, (unsigned) (lane * 16), lb);
            } else {
#pragma unroll
                for (int r = 4 * c; r < 4 * c + 4; ++r) {
                    const int j = min(jst + r, j1 - 1);
                    const uint16_t *src = (append && j == sv.nvis - 1) ? knew : kbase + (size_t) (sv.first + j) * kRawDim;
                    lds_dma16(src + lane * 8, lb + r * kBlk);
                }
            }
        };
        // DMA of stage st's 16 table rows into the wave's table buffer: block bt holds positions
        // 4bt .. 4bt + 3, piece c of position rib at 16 * (16 rib + (c + 4 rib) mod 16).  Loaded
        // temporal (the rows non-temporal): the workgroups of the other kv heads at the same
        // positions run on the same XCD and read them from the L2.
        auto dma_tab = [&](int st) {
            const int jst = j0 + 16 * st;
            const int rib = lane >> 4, c = (lane - 4 * rib) & 15;
            const unsigned tdst = lds_addr(wl + 2 * W::SLOT + W::STG);
            if (jst + 16 <= j1) {
                const uint64_t tb = sbase64(p.rope_tab + (size_t) (sv.first + jst) * kRopePairs);
                const unsigned tvoff = (unsigned) (rib * 256 + c * 16);
                lds_dma16_o<0, 0, false>(tb, tvoff, tdst);
                lds_dma16_o<1024, kBlk - 1024, false>(tb, tvoff, tdst);
                lds_dma16_o<2048, 2 * kBlk - 2048, false>(tb, tvoff, tdst);
                lds_dma16_o<3072, 3 * kBlk - 3072, false>(tb, tvoff, tdst);
            } else {
#pragma unroll
                for (int bt = 0; bt < 4; ++bt) {
                    const int j = min(jst + 4 * bt + rib, j1 - 1);
                    lds_dma16<false>(p.rope_tab + (size_t) (sv.first + j) * kRopePairs + c * 4, tdst + bt * kBlk);
                }
            }
        };

        // This wave's stages: w, w + 4, ...; local index i uses slot i & 1.  One stage is in
        // flight at a time: the next one's DMA is issued as soon as the current one has
        // landed (the other slot was consumed by the previous iteration).  Two in flight
        // while waiting measured slower (c4raw attend 96.4 against 94.5 us, c4q8 110.1
        // against 108.5): the loads of all waves together then oversubscribe the memory system.
        const int st0 = wave;
        if (st0 < nst) {
            dma_rows(st0, wl);
            dma_tab(st0);
        }

        float m = -INFINITY, l = 0.0f;
        float bt = 0.0f;  // q8: sum of P * bias / scale of this lane's head
        f32x4 acc[32];
#pragma unroll
        for (int dt = 0; dt < 32; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float *const xfw = &xf[wave][0][0];

        for (int st = st0, it = 0; st < nst; st += kWaves, ++it) {
            unsigned char *const sl = wl + (it & 1) * W::SLOT;
            ESDA_WAIT_VM(0);  // this stage's rows and table rows landed
            unsigned char *const nsl = wl + ((it + 1) & 1) * W::SLOT;
            const bool more = st + kWaves < nst;
            if (more) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the other slot's reads are done
                if constexpr (Q8) dma_rows(st + kWaves, nsl);
                else dma_rows_part(st + kWaves, nsl, std::integral_constant<int, 0>{});
            }
            // Scores S^T[16 rows x 16 heads] of K = bf16(rope(x * rinv * kw)) (q8: x = q * scale
            // + bias), rounded where ESDecodeAttn.mm:51-93 rounds it.
            f32x4 sp0 = {0.0f, 0.0f, 0.0f, 0.0f}, sp1 = {0.0f, 0.0f, 0.0f, 0.0f};
            // cos / sin of row li's position for the rotary pairs this lane holds
            auto load_tab = [&](u32x4 (&tab)[4]) {
                const int bt2 = li >> 2, rib = li & 3;  // row li: position li of the stage
#pragma unroll
                for (int c4 = 0; c4 < 4; ++c4) {
                    // the pieces (4 frequencies each) of the lane's rotary dims kdim(kr, lg) .. + 7
                    const int c = 8 * (c4 >> 1) + 2 * lg + (c4 & 1);
                    tab[c4] = *reinterpret_cast<const u32x4 *>(wl + 2 * W::SLOT + W::STG + bt2 * kBlk +
                                                               16 * (16 * rib + ((c + 4 * rib) & 15)));
                }
            };
            auto pack = [](const float (&v)[8]) -> bf16x8 {
                bf16x8 r;
#pragma unroll
                for (int e = 0; e < 8; ++e) r[e] = (__bf16) v[e];
                return r;
            };
            // rope over rotary k-steps kr, kr + 8 (dims kdim(kr, lg) + e and their partners + 256)
            auto rotate = [](const u32x4 (&tab)[4], int kr, float (&lo)[8], float (&hi)[8]) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned w = tab[2 * kr + e / 4][e & 3];
                    const float c = bf16_lo(w), s = bf16_hi(w);
                    const float x0 = lo[e], x1 = hi[e];
                    lo[e] = x0 * c - x1 * s;
                    hi[e] = x1 * c + x0 * s;
                }
            };
            // Pass 1: the row norms.  Raw: from Gram products of the rows as stored.  q8: from
            // integer sums of the u8 bytes (the rebuild below widens them to bf16 for the V tile).
            uint2 w8[Q8 ? 16 : 1];  // q8: the lane's 8 u8 values of row li for k-step kk
            u32x4 xr[Q8 ? 1 : 16];  // raw: the lane's row pieces, k-step kk (pass 1, kept for the rebuild)
            float rq = 0.0f, fq = 0.0f;  // q8: scale * rinv and bias * rinv of row li
            {
                if constexpr (Q8) {
                    // All sixteen u8 reads go out before the first V-tile write: LDS accesses
                    // complete in order, so a read issued after a write would wait for it.
                    // Row r's 16-byte piece pc (dims 16 pc ..) sits at (r / 2) * kBlk + 32 pc +
                    // 16 (r % 2) (two rows interleaved per DMA block); the lane's dims kdim(kk, lg)
                    // are half of piece 2kk + lg / 2.
#pragma unroll
                    for (int kk = 0; kk < 16; ++kk)
                        w8[kk] = *reinterpret_cast<const uint2 *>(sl + (li >> 1) * kBlk + 32 * (2 * kk + (lg >> 1)) +
                                                                  16 * (li & 1) + 8 * (lg & 1));
                    const float scl = reinterpret_cast<const float *>(sl + W::ROWS)[li];
                    const float bias = reinterpret_cast<const float *>(sl + W::ROWS)[16 + li];
                    __builtin_amdgcn_sched_barrier(0);
                    // sum(q^2) and sum(q) of the lane's quarter of row li, exact in integers
                    unsigned s2 = 0u, s1 = 0u;
#pragma unroll
                    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
                        for (int w = 0; w < 2; ++w) {
                            const unsigned x = w ? w8[kk].y : w8[kk].x;
                            s2 = __builtin_amdgcn_udot4(x, x, s2, false);
                            s1 = __builtin_amdgcn_udot4(x, 0x01010101u, s1, false);
                        }
                    // whole-row sums in every lane of row li's column (lanes li + 16 lg)
                    s2 = wave_sum_across_groups(s2);
                    s1 = wave_sum_across_groups(s1);
                    // mean(x^2) = scale^2 var(q) + mean(x)^2 with 512^2 var(q) = 512 sum(q^2) - sum(q)^2,
                    // formed exactly in fp64 (below 2^35) and rounded once
                    const float var = (float) (512.0 * (double) s2 - (double) s1 * (double) s1);
                    const float mean = __builtin_fmaf(scl, (float) s1 * (1.0f / kRawDim), bias);
                    const float ms = scl * scl * var * (1.0f / (kRawDim * kRawDim)) + __builtin_fmaf(mean, mean, p.eps);
                    const float rinv = __builtin_amdgcn_rsqf(ms);
                    rq = scl * rinv;
                    fq = bias * rinv;
                    if (lg == 0) {
                        xfw[0 * 16 + li] = rq;
                        xfw[1 * 16 + li] = __builtin_amdgcn_rcpf(rq);
                        xfw[2 * 16 + li] = bias * __builtin_amdgcn_rcpf(scl);
                    }
                } else {
                    f32x4 g = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int kk = 0; kk < 16; ++kk) {
                        xr[kk] = *reinterpret_cast<const u32x4 *>(sl + li * kBlk + 2 * kdim(kk, lg));
                        const bf16x8 x = __builtin_bit_cast(bf16x8, xr[kk]);
                        g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, x, g, 0, 0, 0);
                    }
                    // Row factors (C layout: lane (li, lg) holds C[4lg + i][li]; row li's diagonal
                    // is register li - 4lg of the lanes with lg == li / 4, which publish them).
                    const int i = li - 4 * lg;
                    if (i >= 0 && i < 4) {
                        const float s2 = i == 0 ? g[0] : i == 1 ? g[1] : i == 2 ? g[2] : g[3];
                        const float ms = s2 * (1.0f / kRawDim) + p.eps;
                        const float rinv = __builtin_amdgcn_rsqf(ms);
                        xfw[0 * 16 + li] = rinv;
                        xfw[1 * 16 + li] = ms * rinv;
                    }
                }
            }
            // q8: the u8 values are converted once, in pass 2; this keeps the compiler from
            // hoisting the conversions above the row-factor exchange, which would hold 128 floats
            // live across it (it parks such values in accumulation registers)
            if constexpr (Q8) {
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) asm volatile("" : "+v"(w8[kk]));
            }
            if constexpr (!Q8) {
                if (more) dma_rows_part(st + kWaves, nsl, std::integral_constant<int, 1>{});
            }
            // Other lanes read the factors back: a compiler memory barrier keeps those loads
            // after the stores above (the lanes' LDS accesses then run in order).
            asm volatile("" ::: "memory");
            u32x4 tab[4];
            load_tab(tab);
            const float rk = Q8 ? rq : xfw[0 * 16 + li];  // rinv of row li (q8: scale * rinv)
            // Pass 2: x * rinv * kw of k-step kk, dims kdim(kk, lg) .. + 7 of row li.
            auto xkw = [&](int kk, float (&v)[8]) {
                if constexpr (Q8) {
                    // fma(q, scale * rinv, bias * rinv) * kw, per element; the same floats of q,
                    // packed to bf16 (exact), are the k-step's part of the V tile
                    float q[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) q[e] = (float) ((((e >> 2) ? w8[kk].y : w8[kk].x) >> (8 * (e & 3))) & 255u);
                    unsigned o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        o[e] = __builtin_amdgcn_perm(__builtin_bit_cast(unsigned, q[2 * e + 1]), __builtin_bit_cast(unsigned, q[2 * e]),
                                                     0x07060302u);
                    *reinterpret_cast<u32x4 *>(wl + 2 * W::SLOT + li * kBlk + 2 * kdim(kk, lg)) = u32x4{o[0], o[1], o[2], o[3]};
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(q[e], rk, fq) * kwl[kdim(kk, lg) + e];
                } else {
                    // x * kw exactly (a product of two bf16 values fits fp32) by MFMAs against
                    // the diagonal kw operands, then times rinv
                    const u32x4 t = xr[kk];
                    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                    const f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        dg[kk][0], __builtin_bit_cast(short4v, uint2{t[0], t[1]}), z, 0, 0, 0);
                    const f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        dg[kk][1], __builtin_bit_cast(short4v, uint2{t[2], t[3]}), z, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = d0[e] * rk;
                        v[4 + e] = d1[e] * rk;
                    }
                }
            };
#pragma unroll
            for (int kr = 0; kr < 2; ++kr) {
                float lo[8], hi[8];
                xkw(kr, lo);
                xkw(kr + 8, hi);
                rotate(tab, kr, lo, hi);
                sp0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack(lo), qv[kr], sp0, 0, 0, 0);
                sp1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack(hi), qv[kr + 8], sp1, 0, 0, 0);
            }
            // the table buffer is read (the rotary k-steps above): the next stage's rows may land
            if (st + kWaves < nst) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                dma_tab(st + kWaves);
                if constexpr (!Q8) dma_rows_part(st + kWaves, nsl, std::integral_constant<int, 2>{});
            }
#pragma unroll
            for (int kk = 2; kk < 16; ++kk) {
                if (rot_step(kk)) continue;
                float v[8];
                xkw(kk, v);
                if (kk & 1) sp1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack(v), qv[kk], sp1, 0, 0, 0);
                else sp0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack(v), qv[kk], sp0, 0, 0, 0);
            }
            f32x4 sc = sp0 + sp1;
            if constexpr (!Q8) {
                if (more) dma_rows_part(st + kWaves, nsl, std::integral_constant<int, 3>{});
            }
            // Online softmax (log2 domain) over stage rows 4lg .. 4lg + 3: rows past the
            // segment end are masked.
            const int jt = j0 + 16 * st + 4 * lg;
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[r] = (jt + r) < j1 ? sc[r] * p.scale_log2e : -INFINITY;
            const float tmax = wave_max_across_groups(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
            m = m == -INFINITY ? tmax : m;  // first stage: nothing accumulated to rescale
            if (__builtin_expect(__any(tmax > m + kRawRescaleSlack), 0)) {
                const float mnew = fmaxf(m, tmax);
                const float corr = __builtin_amdgcn_exp2f(m - mnew);
                l *= corr;
                if constexpr (Q8) bt *= corr;
#pragma unroll
                for (int dt = 0; dt < 32; ++dt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float x = acc[dt][e];
                        acc_scale(x, corr);
                        acc[dt][e] = x;
                    }
                m = mnew;
            }
            short4v pbs;
            {
                const f32x4 ri = *reinterpret_cast<const f32x4 *>(xfw + 0 * 16 + 4 * lg);
                const f32x4 rn = *reinterpret_cast<const f32x4 *>(xfw + 1 * 16 + 4 * lg);
                f32x4 gm = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (Q8) gm = *reinterpret_cast<const f32x4 *>(xfw + 2 * 16 + 4 * lg);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(sc[r] - m);
                    const __bf16 pw = (__bf16) (e * ri[r]);
                    l += (float) pw * rn[r];
                    if constexpr (Q8) bt += (float) pw * gm[r];
                    pbs[r] = __builtin_bit_cast(short, pw);
                }
            }
            // O^T += V^T . P^T over all 512 dims (V^T by transpose reads: lane (li, lg)
            // supplies row 4lg + li/4, dims 16dt + 4(li % 4) .. + 4)
            const unsigned char *vb = Q8 ? wl + 2 * W::SLOT : sl;
            const int tr_off = (4 * lg + li / 4) * kBlk + (li % 4) * 8;
#pragma unroll
            for (int dt = 0; dt < 32; ++dt) {
                const short4v av = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) short4v *) (vb + tr_off + 32 * dt));
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, pbs, acc[dt], 0, 0, 0);
                if ((dt & 7) == 7) __builtin_amdgcn_sched_barrier(0);  // at most 8 reads in flight
            }
        }

        // Fused append (raw): the workgroup whose rows end at the new token copies k_new
        // into its cache row (its DMA read the row from k_new; no other workgroup reads it).
        if (!Q8 && append && j1 == sv.nvis && wave == 0) {
            const size_t row = (size_t) sv.newrow * kRawDim;
            *reinterpret_cast<u32x4 *>(kbase + row + lane * 8) = *reinterpret_cast<const u32x4 *>(knew + lane * 8);
        }

        // This wave's (m, l, O): l and (q8) the bias term summed over the lane groups.
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if constexpr (Q8) {
            bt += __shfl_xor(bt, 16);
            bt += __shfl_xor(bt, 32);
#pragma unroll
            for (int dt = 0; dt < 32; ++dt) acc[dt] += bt;
        }
        // Merge the four waves through LDS (aliasing the rings, which are all consumed).
        ESDA_WAIT_VM(0);
        lds_barrier();
        float *const accb = reinterpret_cast<float *>(wlds);          // [wave][head][516]
        float *const mlb = &xf[0][0][0];                               // [wave][2][16] (m, l)
#pragma unroll
        for (int dt = 0; dt < 32; ++dt)
            *reinterpret_cast<f32x4 *>(accb + (wave * 16 + li) * 516 + 16 * dt + 4 * lg) = acc[dt];
        if (lg == 0) {
            mlb[wave * 32 + li] = m;
            mlb[wave * 32 + 16 + li] = l;
        }
        lds_barrier();
        {
            const int h = tid >> 4, d4 = tid & 15;  // head h, dims 4 d4 + 64 k
            float mw[kWaves], M = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                mw[w] = mlb[w * 32 + h];
                M = fmaxf(M, mw[w]);
            }
            float cw[kWaves], L = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                cw[w] = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - M);
                L += cw[w] * mlb[w * 32 + 16 + h];
            }
            if (h < p.G) {
                const size_t hq = (size_t) b * p.Hq + (size_t) kvh * p.G + h;
                const size_t pidx = slot * p.G + h;
                const float inv = 1.0f / L;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int d = 4 * d4 + 64 * k;
                    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) o += *reinterpret_cast<const f32x4 *>(accb + (w * 16 + h) * 516 + d) * cw[w];
                    if (direct) {
                        bf16x4 r;
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = (__bf16) (o[e] * inv);
                        *reinterpret_cast<uint2 *>(p.out + hq * kRawDim + d) = __builtin_bit_cast(uint2, r);
                    } else {
                        // non-temporal, as the 512-dim attend kernel's partials
                        __builtin_nontemporal_store(o, reinterpret_cast<f32x4 *>(p.part_acc + pidx * kRawDim + d));
                    }
                }
                if (!direct && d4 == 0) {
                    __builtin_nontemporal_store(f32x2{M, L}, reinterpret_cast<f32x2 *>(p.part_ml + pidx * 2));
                }
            }
        }
        lds_barrier();  // the merge area is read before the next segment's DMA overwrites it
    };
    walk_segments<kWaves>(p, segment);
}

struct MergeParams {
    const float *part_acc, *part_ml;
    const long long *table;
    const int *pos, *row_base;
    uint16_t *out;
    int B, Hq, Hkv, G, D, cap, window, ring;
    int balanced, W, S, chunk;
};

constexpr int kMergeThreads = 256;
constexpr int kMergeDims = 64;      // output dims per merge workgroup (16 lanes x float4)
constexpr int kMergeGroups = kMergeThreads / (kMergeDims / 4);  // split groups reduced in parallel (16)

// Cross-split merge (ESDecodeAttn.mm:253-273 restated in the log2 domain):
// M = max_s m_s; O = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// One workgroup per (sequence, query head, 64 output dims); 16 split groups x 16 float4
// lanes.  Each thread issues its partial loads together with the (m, l) loads, so the
// whole merge is one memory round trip; each split group weighs its splits against its
// own max, and the final sum over the groups rescales them to the largest (no block-wide
// reduction before the weights).  (Against 128 dims x 8 groups, the narrower workgroups and one 8-byte
// (m, l) load per split took 1.8 us off the C4 step and 1.2 us off C2's.)
// REGS: splits per thread held in registers (S <= 16 * REGS in one pass): 4, or 16 for
// more splits (the raw-K C4 shape packs two kv heads into 128 splits).

// The splits that hold partials of pair (b, kvh): their count ns (0 when the sequence
// is skipped) and the slot of the first, as the attend kernel laid them out.
__device__ __forceinline__ int pair_splits(const MergeParams &p, int b, int kvh, size_t &pbase) {
    int ns;
    if (p.balanced) {
        // The attend workgroups w0 .. w1 that covered pair (b, kvh) (every one of them holds
        // rows of the pair and wrote its slot); an inconsistent table reads nothing.
        int w0 = 0;
        ns = esda_plan::pair_owners(p.table[b], p.table[b + 1], p.table[p.B], p.Hkv, kvh, p.W, &w0);
        if (ns == 0) return 0;
        pbase = (size_t) esda_plan::share_slot((long long) b * p.Hkv + kvh, w0);
    } else {
        const SeqView sv = seq_view(p.pos[b], p.row_base ? p.row_base[b] : 0, p.cap, p.window, p.ring);
        if (!sv.ok) return 0;
        ns = esda_plan::grid_splits(sv.nvis, p.chunk, p.S);
        pbase = ((size_t) b * p.Hkv + kvh) * p.S;
    }
    return ns;
}

template <int REGS>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(MergeParams p) {
    __shared__ f32x4 part[kMergeGroups][kMergeDims / 4];
    __shared__ float lsum[kMergeGroups], gmax[kMergeGroups];
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / p.G, g = h % p.G;
    const int tid = threadIdx.x;
    size_t pbase;
    const int ns = pair_splits(p, b, kvh, pbase);
    if (ns <= 1) return;  // one workgroup covered the pair and wrote the output itself
    const int dq = tid % (kMergeDims / 4), sg = tid / (kMergeDims / 4);
    const int d0 = blockIdx.x * kMergeDims + dq * 4;

    float mloc = -INFINITY;
    float ms[REGS], ls[REGS];
    f32x4 av[REGS];
    // Fast path: every split this thread owns fits in registers.
    const bool in_regs = ns <= kMergeGroups * REGS;
    if (in_regs) {
#pragma unroll
        for (int u = 0; u < REGS; ++u) {
            const int s = sg + u * kMergeGroups;
            if (s < ns) {
                const size_t ix = (pbase + s) * p.G + g;
                av[u] = *reinterpret_cast<const f32x4 *>(p.part_acc + ix * p.D + d0);
                const f32x2 ml = *reinterpret_cast<const f32x2 *>(p.part_ml + ix * 2);
                ms[u] = ml[0];
                ls[u] = ml[1];
            } else {
                av[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                ms[u] = -INFINITY;
                ls[u] = 0.0f;
            }
            mloc = fmaxf(mloc, ms[u]);
        }
    } else {
        for (int s = sg; s < ns; s += kMergeGroups) mloc = fmaxf(mloc, p.part_ml[((pbase + s) * p.G + g) * 2]);
    }
    // Each split group combines its splits against its own max (the same in the group's 16
    // lanes: m is per split); the groups are rescaled to their common max in the final sum.
    const float mx = mloc == -INFINITY ? 0.0f : mloc;  // a group without splits: weights 0

    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float lt = 0.0f;
    if (in_regs) {
#pragma unroll
        for (int u = 0; u < REGS; ++u) {
            const float w = __builtin_amdgcn_exp2f(ms[u] - mx);  // 0 for absent splits
            o += av[u] * w;
            lt += ls[u] * w;
        }
    } else {
        for (int s = sg; s < ns; s += kMergeGroups) {
            const size_t ix = (pbase + s) * p.G + g;
            const float w = __builtin_amdgcn_exp2f(p.part_ml[ix * 2] - mx);
            o += *reinterpret_cast<const f32x4 *>(p.part_acc + ix * p.D + d0) * w;
            lt += p.part_ml[ix * 2 + 1] * w;
        }
    }
    part[sg][dq] = o;
    if (dq == 0) {
        lsum[sg] = lt;
        gmax[sg] = mloc;
    }
    __syncthreads();
    if (tid < kMergeDims / 4) {
        float M = gmax[0];
#pragma unroll
        for (int u = 1; u < kMergeGroups; ++u) M = fmaxf(M, gmax[u]);
        f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
        float l = 0.0f;
#pragma unroll
        for (int u = 0; u < kMergeGroups; ++u) {
            // a group with no split (its max -inf) adds nothing
            const float c = gmax[u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(gmax[u] - M);
            t += part[u][tid] * c;
            l += lsum[u] * c;
        }
        const float inv = 1.0f / l;
        uint16_t *dst = p.out + ((size_t) b * p.Hq + h) * p.D + blockIdx.x * kMergeDims + tid * 4;
        bf16x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (__bf16) (t[e] * inv);
        *reinterpret_cast<uint2 *>(dst) = __builtin_bit_cast(uint2, r);
    }
}

// Merge for pairs of few splits (balanced shares): one thread per (sequence,
// query head, 4 output dims), no barriers.  Splits are read 8 at a time -- the loads of
// a chunk issue together, so up to 8 splits cost one memory round trip -- with the
// running max raised per chunk (same result as merge_kernel up to summation order).
constexpr int kMergeRowsThreads = 256;
constexpr int kMergeRowsChunk = 8;

__global__ __launch_bounds__(kMergeRowsThreads) void merge_rows_kernel(MergeParams p) {
    const int D4 = p.D / 4;
    const int t = blockIdx.x * kMergeRowsThreads + threadIdx.x;
    const int b = blockIdx.y;
    if (t >= p.Hq * D4) return;
    const int h = t / D4, d4 = t - (t / D4) * D4;
    const int kvh = h / p.G, g = h % p.G;
    size_t pbase;
    const int ns = pair_splits(p, b, kvh, pbase);
    if (ns <= 1) return;  // written by the attend kernel, or skipped
    float mx = -INFINITY, lt = 0.0f;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < ns; s0 += kMergeRowsChunk) {
        float mv[kMergeRowsChunk], lv[kMergeRowsChunk];
        f32x4 av[kMergeRowsChunk];
#pragma unroll
        for (int u = 0; u < kMergeRowsChunk; ++u) {
            mv[u] = -INFINITY;
            lv[u] = 0.0f;
            av[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (s0 + u < ns) {
                const size_t ix = (pbase + s0 + u) * p.G + g;
                mv[u] = p.part_ml[ix * 2];
                lv[u] = p.part_ml[ix * 2 + 1];
                av[u] = *reinterpret_cast<const f32x4 *>(p.part_acc + ix * p.D + d4 * 4);
            }
        }
        float cm = mv[0];
#pragma unroll
        for (int u = 1; u < kMergeRowsChunk; ++u) cm = fmaxf(cm, mv[u]);
        const float mn = fmaxf(mx, cm);
        const float c = __builtin_amdgcn_exp2f(mx - mn);  // 0 on the first chunk
        o *= c;
        lt *= c;
#pragma unroll
        for (int u = 0; u < kMergeRowsChunk; ++u) {
            const float w = __builtin_amdgcn_exp2f(mv[u] - mn);  // 0 for absent splits
            o += av[u] * w;
            lt += lv[u] * w;
        }
        mx = mn;
    }
    const float inv = 1.0f / lt;
    bf16x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (__bf16) (o[e] * inv);
    *reinterpret_cast<uint2 *>(p.out + ((size_t) b * p.Hq + h) * p.D + d4 * 4) = __builtin_bit_cast(uint2, r);
}

// Per-row affine u8 of raw rows (esQuantizeRawRows, ESDecodeAttn.mm:491-539): one wave
// per row of src [kv heads, n, 512] bf16; row (h, i) -> q8[h * q_head_stride + (row0 + i)
// * 512 ..], scale / bias at [h * sb_head_stride + row0 + i].  The attend kernel's q8 mode
// quantizes the decode step's new row with the same arithmetic.
__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint16_t *src, int n, long long rows,
                                                            unsigned char *q8, long long q_head_stride,
                                                            float *scale, float *bias, long long sb_head_stride,
                                                            int row0) {
    const long long r = (long long) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const long long h = r / n, i = r - (r / n) * n;
    const u32x4 t = *reinterpret_cast<const u32x4 *>(src + r * kRawDim + lane * 8);
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = bf16_lo(t[e]);
        x[2 * e + 1] = bf16_hi(t[e]);
    }
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) {
        mn = fminf(mn, x[e]);
        mx = fmaxf(mx, x[e]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o));
        mx = fmaxf(mx, __shfl_xor(mx, o));
    }
    float scl = (mx - mn) / 255.0f;
    if (!(scl > 1e-8f)) scl = 1e-8f;
    unsigned lo = 0u, hi = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const unsigned qi = (unsigned) fminf(roundf((x[e] - mn) / scl), 255.0f);
        if (e < 4) lo |= qi << (8 * e);
        else hi |= qi << (8 * (e - 4));
    }
    *reinterpret_cast<uint2 *>(q8 + h * q_head_stride + (row0 + i) * kRawDim + lane * 8) = uint2{lo, hi};
    if (lane == 0) {
        scale[h * sb_head_stride + row0 + i] = scl;
        bias[h * sb_head_stride + row0 + i] = mn;
    }
}

// Rotary cos/sin table for raw-K decode: entry (t, f) = bf16 cos | bf16 sin << 16 of the
// fp32 angle t * inv_freq[f], t < rows, f < 64 -- publish_tab's arithmetic.
__global__ __launch_bounds__(256) void rope_table_kernel(const float *inv_freq, long long n, unsigned *tab) {
    const long long i = (long long) blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int t = (int) (i / kRopePairs), f = (int) (i % kRopePairs);
    float s, c;
    sincos_f32((float) t * inv_freq[f], s, c);
    tab[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{c, s}, bf16x2));
}

__global__ void fill_i32_kernel(int *dst, int value, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = value;
}

// Plain row copy for multi-row appends (slice_update at rows row0 .. row0 + n - 1).
__global__ __launch_bounds__(256) void append_kernel(uint16_t *cache, long long seq_stride,
                                                      long long head_stride, int Hkv, int D,
                                                      int cap, const uint16_t *src, int n_new,
                                                      const int *row0, int *status) {
    const int b = blockIdx.z, h = blockIdx.y;
    const int r0 = row0[b];
    if (r0 < 0 || r0 + n_new > cap) {
        if (h == 0 && blockIdx.x == 0 && threadIdx.x == 0 && status) atomicAdd(status, 1);
        return;
    }
    const int chunks = D / 8;
    const size_t total = (size_t) n_new * chunks;
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t) gridDim.x * blockDim.x) {
        const int r = (int) (i / chunks), c = (int) (i % chunks);
        const uint4 v = *reinterpret_cast<const uint4 *>(src + (((size_t) b * Hkv + h) * n_new + r) * D + c * 8);
        *reinterpret_cast<uint4 *>(cache + (size_t) b * seq_stride + (size_t) h * head_stride +
                                   (size_t) (r0 + r) * D + c * 8) = v;
    }
}

// Read-only stream over `blocks` 1 KiB blocks through the attend kernel's load path
// (global_load_lds_dwordx4 ... nt into LDS, 64 lanes x 16 B = 1 KiB per instruction,
// up to 15 in flight per wave): the memory system's ceiling for that path, and the
// reference point of the HBM counters for it.  Workgroup w reads blocks [blocks * w / G,
// blocks * (w + 1) / G) round-robin over its 4 waves; each wave keeps one word of what it
// read, so the loads feed an output (sink[4 * w + wave]).
__global__ __launch_bounds__(256) void stream_read_kernel(const unsigned char *src, long long blocks, unsigned *sink) {
    __shared__ __attribute__((aligned(16))) unsigned char buf[4][16][1024];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const long long b0 = blocks * blockIdx.x / gridDim.x, b1 = blocks * (blockIdx.x + 1) / gridDim.x;
    int i = 0;
    for (long long b = b0 + wave; b < b1; b += 4, ++i) {
        // at most 14 outstanding before this one: the load that last filled slot i % 16
        // (16 loads ago) has landed
        ESDA_WAIT_VM(14);
        lds_dma16(src + b * 1024 + lane * 16, lds_addr(&buf[wave][i & 15][0]));
    }
    ESDA_WAIT_VM(0);
    lds_barrier();
    const unsigned x = reinterpret_cast<const unsigned *>(&buf[wave][lane & 15][0])[lane];
    unsigned s = x;
    for (int o = 32; o > 0; o >>= 1) s ^= __shfl_xor(s, o);
    if (lane == 0) sink[4 * blockIdx.x + wave] = s;
}

// ------------------------------------------------------------------------ host side

thread_local std::string g_err;

}  // namespace

void esda_detail::set_error(const std::string &msg) { g_err = msg; }

namespace {

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(ESDA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The library is built for gfx950 only: refuse other devices loudly.
int check_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    static std::mutex mu;
    static int checked[64] = {0};
    std::lock_guard<std::mutex> lk(mu);
    if (dev < 0 || dev >= 64) return fail(ESDA_ERR_DEVICE, "device index out of range");
    if (checked[dev] == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        checked[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    }
    if (checked[dev] < 0) return fail(ESDA_ERR_DEVICE, "libesda.so is built for gfx950 only");
    return ESDA_OK;
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

int esda_detail::check_device() { return ::check_device(); }

namespace {

struct Plan {
    int G, maxvis, balanced, W, S, chunk;
    int pk;   // kv heads packed per workgroup (the kernels see Hkv / pk heads of G * pk)
    int per_cu;  // attend workgroups per CU the plan is sized for (1 or 2)
    size_t off_table, off_ml, off_acc, bytes;
};

// Kv heads per workgroup for a grid of one split per (sequence, kv head): with several
// workgroups' worth of pairs per CU, packing pk kv heads (pk * G <= 16 query heads, the
// MFMA's N dimension) gives each workgroup one pk-times longer stream instead of pk short
// ones, each of which would pay the ring's fill and drain.  Local layers (G = 2) at C5's
// batch: 512 pairs -> 256 workgroups of two kv heads.
int choose_pack(const esda_decode_desc *d, int G, long long S, int target) {
    const long long pairs = (long long) d->batch * d->num_kv_heads;
    int pk = 1;
    while (pk < 4 && S == 1 && G * pk * 2 <= kMaxGroup && d->num_kv_heads % (pk * 2) == 0 &&
           pairs / (pk * 2) >= target &&
           (long long) d->head_stride * 2 * (pk * 2) + 16LL * d->head_dim * 2 < (1LL << 31))
        pk *= 2;
    return pk;
}

// raw: the raw-K kernels take one kv head per workgroup.
int make_plan(const esda_decode_desc *d, Plan *pl, bool raw = false) {
    if (!d) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null description");
    if (d->batch <= 0 || d->num_q_heads <= 0 || d->num_kv_heads <= 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: batch and head counts must be positive");
    if (d->batch > kMaxBatch)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: at most 256 sequences per call");
    if (d->head_dim != 128 && d->head_dim != 256 && d->head_dim != 512)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: head_dim must be 128, 256 or 512");
    if (d->num_q_heads % d->num_kv_heads)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: num_q_heads must be a multiple of num_kv_heads");
    const int G = d->num_q_heads / d->num_kv_heads;
    if (G > kMaxGroup)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: at most 16 query heads per kv head");
    if (d->cap <= 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: cap must be positive");
    if (d->window < 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: window must be >= 0");
    if (d->ring && (d->window <= 0 || d->window > d->cap))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: ring mode needs 0 < window <= cap");
    if (d->head_stride < (int64_t) d->cap * d->head_dim || (d->head_stride % 8) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: head_stride must be >= cap*head_dim and a multiple of 8");
    if (d->seq_stride < (int64_t) d->num_kv_heads * d->head_stride || (d->seq_stride % 8) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: seq_stride must be >= num_kv_heads*head_stride and a multiple of 8");
    if (d->split_rows < 0 || (d->split_rows % kTile) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: split_rows must be a multiple of 16");
    int bound = d->ring ? d->window : (d->window > 0 ? std::min(d->window, d->cap) : d->cap);
    int maxvis = d->max_visible > 0 ? std::min(d->max_visible, bound) : bound;
    // Several full-causal sequences have ragged lengths: workgroups then take balanced
    // shares of all rows (the kernel scans the lengths).  Otherwise (one sequence, or
    // windowed local layers whose lengths are nearly equal) a plain grid of fixed splits
    // per (sequence, kv head) starts faster.
    pl->balanced = d->batch > 1 && !d->ring;
    // Workgroups per CU: two at D = 256 (C5 step 7.47 ms against 7.58 with plans of one per
    // CU), else one.  At D = 512 two per CU measured slower on grid plans (twice the splits
    // cost more in the merge than they gain: C4 step 82.7 -> 85.1 us) and on balanced shares
    // (C5 7.64 against 7.52 ms with 256 shares).
    pl->per_cu = (!raw && d->head_dim == 256) ? kOcc256 : 1;
    const int target = pl->per_cu * kTargetGroups;  // workgroups that fill the GPU
    pl->pk = 1;
    // Work split.  Sizing uses the upper bound on rows (the kernels see the real ones),
    // counted per packed kv head (a row of a pk-packed head is pk cache rows).
    // Automatic: about one workgroup per CU, no fewer than 64 rows each; split_rows > 0
    // asks for that many rows per workgroup.
    const long long rows_max = (long long) maxvis * d->batch * (d->num_kv_heads / pl->pk);
    const long long per = d->split_rows > 0 ? d->split_rows : kMinRows;
    pl->G = G;
    pl->maxvis = maxvis;
    size_t slots;
    if (pl->balanced) {
        long long W = (rows_max + per - 1) / per;
        if (d->split_rows == 0 && W > target) W = target;
        if (W > kMaxGroups) W = kMaxGroups;
        if (W < 1) W = 1;
        pl->W = (int) W;
        pl->S = pl->chunk = 0;
        slots = (size_t) d->batch * (d->num_kv_heads / pl->pk) + (size_t) W;  // pair u's partial from workgroup w at u + w
    } else {
        long long chunk = d->split_rows;
        if (chunk == 0) {
            // The fewest rows per split that keep the grid within one workgroup per CU, in
            // whole 16-row tiles (C2, 4 pairs of 8193 rows: 64-row rounding gave 192-row
            // splits and 176 workgroups, 11.4 us; 16-row rounding gives 144 and 228, 10.3).
            const long long pairs = (long long) d->batch * (d->num_kv_heads / pl->pk);
            const long long per_pair = std::max(1LL, target / pairs);
            chunk = (maxvis + per_pair - 1) / per_pair;
            chunk = (chunk + kTile - 1) / kTile * kTile;
            const int min_rows = pl->per_cu == 2 ? kMinRowsOcc2 : kMinRows;
            if (chunk < min_rows) chunk = min_rows;
            if (chunk > 8192) chunk = 8192;
        }
        long long S = (maxvis + chunk - 1) / chunk;
        if (S > kMaxGroups) {
            chunk = (maxvis + kMaxGroups - 1) / kMaxGroups;
            chunk = (chunk + kTile - 1) / kTile * kTile;
            S = (maxvis + chunk - 1) / chunk;
        }
        pl->W = 0;
        pl->S = (int) S;
        pl->chunk = (int) chunk;
        if (!raw && d->split_rows == 0) pl->pk = choose_pack(d, G, S, target);
        slots = (size_t) d->batch * (d->num_kv_heads / pl->pk) * S;
    }
    const size_t parts = slots * G * pl->pk;
    pl->off_table = 256;
    pl->off_ml = pl->off_table + (((size_t) (d->batch + 1) * sizeof(long long) + 255) / 256) * 256;
    pl->off_acc = pl->off_ml + ((parts * 2 * sizeof(float) + 255) / 256) * 256;
    pl->bytes = pl->off_acc + parts * d->head_dim * sizeof(float);
    return ESDA_OK;
}

// Waves per workgroup (the head dim is split across them); workgroups per CU: Plan::per_cu.  D = 256:
// two workgroups of 4 waves per CU, each with half the LDS for its ring (4 stages of 16
// rows), so each SIMD runs two waves of independent workgroups that never wait on each
// other's barriers.  Against one workgroup of 8 waves (two per SIMD in barrier lockstep,
// the softmax repeated by all 8): C3 attend 23.9 -> 22.3 us, C5 step 7.80 -> 7.61 ms, C1
// 5.7 -> 5.3 us.  D = 512 keeps 4 waves (its 8-wave form loses a ring stage to the larger
// score exchange and runs C4 ~6% slower).  D = 128 has too few dims for 8 waves of 32-dim MFMA
// steps.
template <int D>
constexpr int ring_waves() { return D == 256 ? kWaves256 : 4; }

// Raw mode: 8 waves, two per SIMD, so one wave's dependency stalls overlap the other's
// reconstruction work.
constexpr int kRawWaves = 8;

template <int D, bool SHARED, bool RAW = false, bool Q8 = false, int OCC = 1>
hipError_t launch_attend(const AttendParams &ap, dim3 grid, hipStream_t st) {
    constexpr int NW = RAW ? kRawWaves : ring_waves<D>();
    hipLaunchKernelGGL((attend_kernel<D, SHARED, NW, RAW, Q8, OCC>), grid, dim3(64 * NW), 0, st, ap);
    return hipGetLastError();
}

// The 512-dim shared stream (C2, C4, C5's global layers) runs the kernel whose ring takes half
// the LDS -- 4 stages of 16 rows, two of them in flight (32 KB) -- at one workgroup per CU.
// Shallower rings measured faster there, the register budget of two waves per SIMD making no
// difference: C4 step 78.8-79.1 us at 4 stages (80 KB budget), 79.9-80.1 at 5, 80.4-80.6 at 6,
// 81.5-81.9 at 9 (the full LDS), 108.6 at 3; C2 13.4 against 14.2 us at 9.  Over 256
// workgroups two stages each keep ~8.4 MB in flight, enough to saturate HBM (a read probe reads
// 7.1-7.3 TB/s with 6-15 MB in flight, less with ~30 MB), where 9 stages keep ~29 MB.  A
// separate 512-dim V needs the whole LDS for 4 stages; D = 128 stages are 4 KB.
hipError_t dispatch_attend(int D, bool shared, const AttendParams &ap, dim3 grid, hipStream_t st) {
    constexpr int O256 = kOcc256, O512 = kOcc512Shared;
    switch (D) {
        case 128: return shared ? launch_attend<128, true>(ap, grid, st) : launch_attend<128, false>(ap, grid, st);
        case 256:
            return shared ? launch_attend<256, true, false, false, O256>(ap, grid, st)
                          : launch_attend<256, false, false, false, O256>(ap, grid, st);
        default:
            return shared ? launch_attend<512, true, false, false, O512>(ap, grid, st)
                          : launch_attend<512, false>(ap, grid, st);
    }
}

// The raw-mode step as a plain decode description: linear rows, full causal span, one
// shared stream of 512-dim rows.
int raw_as_decode(const esda_raw_desc *r, esda_decode_desc *d) {
    if (!r) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: null description");
    if (r->head_dim != kRawDim) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: head_dim must be 512");
    if (!(r->eps >= 0.0f)) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: eps must be >= 0");
    std::memset(d, 0, sizeof(*d));
    d->batch = r->batch;
    d->num_q_heads = r->num_q_heads;
    d->num_kv_heads = r->num_kv_heads;
    d->head_dim = r->head_dim;
    d->cap = r->cap;
    d->window = 0;
    d->ring = 0;
    d->kv_shared = 1;
    d->seq_stride = r->seq_stride;
    d->head_stride = r->head_stride;
    d->max_visible = r->max_visible;
    d->split_rows = r->split_rows;
    d->scale = r->scale;
    return ESDA_OK;
}

// Launches the requested stages of one decode step (raw: the raw-K attend kernel).
// mode: 0 composite, 1 raw-K, 2 q8 raw-K.  status: the skipped-sequence counter (null =
// the workspace's first word).
int run_stages(const esda_decode_desc *d, const Plan &pl, const AttendParams &ap_in, uint16_t *out,
               void *workspace, int stages, int mode, hipStream_t st, int *status = nullptr) {
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    long long *table = reinterpret_cast<long long *>(ws + pl.off_table);
    float *part_ml = reinterpret_cast<float *>(ws + pl.off_ml);
    float *part_acc = reinterpret_cast<float *>(ws + pl.off_acc);
    if (stages & ESDA_STAGE_ATTEND) {
        AttendParams ap = ap_in;
        ap.part_acc = part_acc;
        ap.part_ml = part_ml;
        ap.status = status ? status : reinterpret_cast<int *>(ws);
        ap.seq_stride = d->seq_stride;
        ap.head_stride = d->head_stride;
        ap.B = d->batch;
        ap.Hq = d->num_q_heads;
        ap.Hkv = d->num_kv_heads / pl.pk;
        ap.G = pl.G * pl.pk;
        ap.pk = pl.pk;
        ap.gk = pl.G;
        ap.cap = d->cap;
        ap.window = d->window;
        ap.ring = d->ring;
        ap.balanced = pl.balanced;
        ap.W = pl.W;
        ap.S = pl.S;
        ap.chunk = pl.chunk;
        ap.table = table;
        ap.scale_log2e = d->scale * kLog2e;
        ap.out = out;
        const dim3 grid = pl.balanced ? dim3(pl.W) : dim3(pl.S, d->num_kv_heads / pl.pk, d->batch);
        hipError_t e;
        if (mode == 0) {
            e = dispatch_attend(d->head_dim, d->kv_shared != 0, ap, grid, st);
        } else if (ap.rope_tab) {
            // with the precomputed cos/sin table (the ES layer's form): the wave-private-ring
            // kernel, one kv head per workgroup
            if (mode == 1) hipLaunchKernelGGL(raw_attend_kernel<false>, grid, dim3(64 * kWaves), 0, st, ap);
            else hipLaunchKernelGGL(raw_attend_kernel<true>, grid, dim3(64 * kWaves), 0, st, ap);
            e = hipGetLastError();
        } else if (mode == 1) {
            // without a table the 8-wave kernel computes its cos/sin per stage
            e = launch_attend<kRawDim, true, true>(ap, grid, st);
        } else {
            e = launch_attend<kRawDim, true, true, true>(ap, grid, st);
        }
        if (e != hipSuccess) return hip_fail(e, "attend_kernel launch");
    }
    // One split per pair: the attend workgroups wrote every output themselves.
    if ((stages & ESDA_STAGE_MERGE) && !(!pl.balanced && pl.S == 1)) {
        MergeParams mp;
        mp.part_acc = part_acc;
        mp.part_ml = part_ml;
        mp.table = table;
        mp.pos = ap_in.pos;
        mp.row_base = ap_in.row_base;
        mp.out = out;
        mp.B = d->batch;
        mp.Hq = d->num_q_heads;
        mp.Hkv = d->num_kv_heads / pl.pk;
        mp.G = pl.G * pl.pk;
        mp.D = d->head_dim;
        mp.cap = d->cap;
        mp.window = d->window;
        mp.ring = d->ring;
        mp.balanced = pl.balanced;
        mp.W = pl.W;
        mp.S = pl.S;
        mp.chunk = pl.chunk;
        if (pl.balanced || pl.S <= kMergeRowsChunk) {
            // Balanced shares give each pair a few splits: thread-per-output merge (C5's
            // global layers: 11 -> 4.4 us), as do grids of at most kMergeRowsChunk splits
            // (one memory round trip per thread).  Larger grids keep merge_kernel, whose
            // workgroups reduce 16 split groups side by side (at C1's 16 splits over 8 pairs
            // the rows kernel would run 4 workgroups and two round trips: 9.0 -> 11.8 us a step).
            const int threads = d->num_q_heads * (d->head_dim / 4);
            dim3 grid((threads + kMergeRowsThreads - 1) / kMergeRowsThreads, d->batch);
            hipLaunchKernelGGL(merge_rows_kernel, grid, dim3(kMergeRowsThreads), 0, st, mp);
        } else {
            dim3 grid(d->head_dim / kMergeDims, d->num_q_heads, d->batch);
            if (pl.S <= kMergeGroups * 4)
                hipLaunchKernelGGL(merge_kernel<4>, grid, dim3(kMergeThreads), 0, st, mp);
            else
                hipLaunchKernelGGL(merge_kernel<16>, grid, dim3(kMergeThreads), 0, st, mp);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "merge_kernel launch");
    }
    return ESDA_OK;
}

// Argument checks shared by esda_decode_stages and esda_decode_noalloc (everything but
// the workspace).
int check_decode_args(const esda_decode_desc *d, const esda_decode_args *a) {
    if (!a) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null arguments");
    if (!a->q || !a->k_new || !a->k_cache || !a->v_cache || !a->pos || !a->out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null device pointer");
    if (!d->kv_shared && !a->v_new)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: v_new is required unless kv_shared");
    if (d->kv_shared && a->v_cache != a->k_cache)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: kv_shared needs v_cache == k_cache");
    if (!d->kv_shared && a->v_cache == a->k_cache)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: separate K/V need distinct caches");
    if (!aligned16(a->q) || !aligned16(a->k_new) || (a->v_new && !aligned16(a->v_new)) ||
        !aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->out))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: tensors must be 16-byte aligned");
    return ESDA_OK;
}

AttendParams decode_params(const esda_decode_desc *d, const esda_decode_args *a) {
    AttendParams ap{};
    ap.q = static_cast<const uint16_t *>(a->q);
    ap.k_new = static_cast<const uint16_t *>(a->k_new);
    ap.v_new = static_cast<const uint16_t *>(d->kv_shared ? a->k_new : a->v_new);
    ap.k_cache = static_cast<uint16_t *>(a->k_cache);
    ap.v_cache = static_cast<uint16_t *>(a->v_cache);
    ap.pos = a->pos;
    ap.row_base = a->row_base;
    return ap;
}

}  // namespace

// ------------------------------------------------ static scratch of esda_decode_noalloc
//
// The split partials, the batch prefix table and (when the caller passes no status word)
// the skipped-sequence counter of esda_decode_noalloc live here instead of in a caller
// workspace.  Every GPU the library runs on holds its own copy for the life of the
// process.  In host code `scratch` names a host-side stand-in, never the device memory:
// kernels get the address hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// Device address of `scratch` on the current device, looked up once per device.
int scratch_address(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(ESDA_ERR_DEVICE, "device index out of range");
    static std::mutex mu;
    static void *addr[64] = {nullptr};
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(ESDA_ERR_RUNTIME, "hipGetSymbolAddress(scratch) returned null");
        addr[dev] = p;
    }
    *out = addr[dev];
    return ESDA_OK;
}

}  // namespace

extern "C" {

const char *esda_last_error(void) { return g_err.c_str(); }

int esda_version(void) { return 100; }

int esda_decode_workspace_size(const esda_decode_desc *desc, size_t *bytes) {
    Plan pl;
    int rc = make_plan(desc, &pl);
    if (rc) return rc;
    if (!bytes) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_workspace_size: null output");
    *bytes = pl.bytes;
    return ESDA_OK;
}

int esda_decode_stages(const esda_decode_desc *d, const esda_decode_args *a, int stages,
                       void *stream) {
    Plan pl;
    int rc = make_plan(d, &pl);
    if (rc) return rc;
    rc = check_decode_args(d, a);
    if (rc) return rc;
    if (!a->workspace || a->workspace_bytes < pl.bytes || !aligned16(a->workspace))
        return fail(ESDA_ERR_WORKSPACE, "esda_decode: workspace missing or smaller than esda_decode_workspace_size");
    if ((stages & (ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE)) == 0 || (stages & ~3))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_stages: bad stage mask");
    rc = check_device();
    if (rc) return rc;
    return run_stages(d, pl, decode_params(d, a), static_cast<uint16_t *>(a->out), a->workspace, stages, 0,
                      reinterpret_cast<hipStream_t>(stream));
}

int esda_decode_noalloc(const esda_decode_desc *d, const esda_decode_args *a, void *stream) {
    Plan pl;
    int rc = make_plan(d, &pl);
    if (rc) return rc;
    rc = check_decode_args(d, a);
    if (rc) return rc;
    // The workspace argument is optional here and only ever the status word.
    if (a->workspace && (a->workspace_bytes < sizeof(int32_t) || (reinterpret_cast<uintptr_t>(a->workspace) & 3u)))
        return fail(ESDA_ERR_WORKSPACE, "esda_decode_noalloc: a status word needs >= 4 bytes, 4-byte aligned");
    if (pl.bytes > kScratchBytes)
        return fail(ESDA_ERR_WORKSPACE, "esda_decode_noalloc: this step needs " + std::to_string(pl.bytes) +
                                            " bytes of scratch; the library's static scratch holds " +
                                            std::to_string(kScratchBytes) + " (use esda_decode with a workspace)");
    rc = check_device();
    if (rc) return rc;
    void *ws = nullptr;
    rc = scratch_address(&ws);
    if (rc) return rc;
    int *status = a->workspace ? static_cast<int *>(a->workspace) : static_cast<int *>(ws);
    return run_stages(d, pl, decode_params(d, a), static_cast<uint16_t *>(a->out), ws,
                      ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE, 0, reinterpret_cast<hipStream_t>(stream), status);
}

int esda_decode(const esda_decode_desc *desc, const esda_decode_args *args, void *stream) {
    return esda_decode_stages(desc, args, ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE, stream);
}

int esda_decode_raw_workspace_size(const esda_raw_desc *desc, size_t *bytes) {
    esda_decode_desc d;
    int rc = raw_as_decode(desc, &d);
    if (rc) return rc;
    Plan pl;
    rc = make_plan(&d, &pl, /*raw=*/true);
    if (rc) return rc;
    if (!bytes) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_workspace_size: null output");
    *bytes = pl.bytes;
    return ESDA_OK;
}

int esda_decode_raw_stages(const esda_raw_desc *desc, const esda_raw_args *a, int stages, void *stream) {
    esda_decode_desc d;
    int rc = raw_as_decode(desc, &d);
    if (rc) return rc;
    Plan pl;
    rc = make_plan(&d, &pl, /*raw=*/true);
    if (rc) return rc;
    if (!a) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: null arguments");
    if (!a->q || !a->raw_cache || !a->pos || !a->kw || !a->inv_freq || !a->out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: null device pointer");
    if (!aligned16(a->q) || (a->k_new && !aligned16(a->k_new)) || !aligned16(a->raw_cache) ||
        !aligned16(a->kw) || !aligned16(a->inv_freq) || !aligned16(a->out))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: tensors must be 16-byte aligned");
    if (a->rope_table && (a->rope_table_rows < d.cap || !aligned16(a->rope_table)))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw: rope_table needs >= cap rows, 16-byte aligned");
    if (!a->workspace || a->workspace_bytes < pl.bytes || !aligned16(a->workspace))
        return fail(ESDA_ERR_WORKSPACE, "esda_decode_raw: workspace missing or smaller than esda_decode_raw_workspace_size");
    if ((stages & (ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE)) == 0 || (stages & ~3))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_stages: bad stage mask");
    rc = check_device();
    if (rc) return rc;
    AttendParams ap{};
    ap.q = static_cast<const uint16_t *>(a->q);
    ap.k_new = static_cast<const uint16_t *>(a->k_new);
    ap.v_new = ap.k_new;
    ap.k_cache = static_cast<uint16_t *>(a->raw_cache);
    ap.v_cache = ap.k_cache;
    ap.pos = a->pos;
    ap.row_base = nullptr;
    ap.kw = static_cast<const uint16_t *>(a->kw);
    ap.inv_freq = a->inv_freq;
    ap.rope_tab = static_cast<const unsigned *>(a->rope_table);
    ap.eps = desc->eps;
    return run_stages(&d, pl, ap, static_cast<uint16_t *>(a->out), a->workspace, stages, 1,
                      reinterpret_cast<hipStream_t>(stream));
}

int esda_decode_raw(const esda_raw_desc *desc, const esda_raw_args *args, void *stream) {
    return esda_decode_raw_stages(desc, args, ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE, stream);
}

int esda_decode_raw_q8_stages(const esda_raw_desc *desc, const esda_raw_q8_args *a, int stages, void *stream) {
    esda_decode_desc d;
    int rc = raw_as_decode(desc, &d);
    if (rc) return rc;
    if ((d.head_stride % 16) || (d.seq_stride % 16))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: u8 strides must be multiples of 16 bytes");
    Plan pl;
    rc = make_plan(&d, &pl, /*raw=*/true);
    if (rc) return rc;
    if (!a) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: null arguments");
    if (!a->q || !a->q8_cache || !a->scale || !a->bias || !a->pos || !a->kw || !a->inv_freq || !a->out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: null device pointer");
    if (!aligned16(a->q) || (a->k_new && !aligned16(a->k_new)) || !aligned16(a->q8_cache) ||
        !aligned16(a->kw) || !aligned16(a->inv_freq) || !aligned16(a->out) ||
        (reinterpret_cast<uintptr_t>(a->scale) & 3u) || (reinterpret_cast<uintptr_t>(a->bias) & 3u))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: tensors must be 16-byte aligned (scale / bias 4)");
    if (a->rope_table && (a->rope_table_rows < d.cap || !aligned16(a->rope_table)))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: rope_table needs >= cap rows, 16-byte aligned");
    if (a->sb_head_stride < d.cap || a->sb_seq_stride < (int64_t) d.num_kv_heads * a->sb_head_stride)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8: scale / bias strides smaller than the cache");
    if (!a->workspace || a->workspace_bytes < pl.bytes || !aligned16(a->workspace))
        return fail(ESDA_ERR_WORKSPACE, "esda_decode_raw_q8: workspace missing or smaller than esda_decode_raw_workspace_size");
    if ((stages & (ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE)) == 0 || (stages & ~3))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_raw_q8_stages: bad stage mask");
    rc = check_device();
    if (rc) return rc;
    AttendParams ap{};
    ap.q = static_cast<const uint16_t *>(a->q);
    ap.k_new = static_cast<const uint16_t *>(a->k_new);
    ap.v_new = ap.k_new;
    ap.k_cache = static_cast<uint16_t *>(a->q8_cache);  // not read in q8 mode
    ap.v_cache = ap.k_cache;
    ap.q8 = static_cast<unsigned char *>(a->q8_cache);
    ap.qsc = a->scale;
    ap.qbs = a->bias;
    ap.sb_seq_stride = a->sb_seq_stride;
    ap.sb_head_stride = a->sb_head_stride;
    ap.pos = a->pos;
    ap.row_base = nullptr;
    ap.kw = static_cast<const uint16_t *>(a->kw);
    ap.inv_freq = a->inv_freq;
    ap.rope_tab = static_cast<const unsigned *>(a->rope_table);
    ap.eps = desc->eps;
    return run_stages(&d, pl, ap, static_cast<uint16_t *>(a->out), a->workspace, stages, 2,
                      reinterpret_cast<hipStream_t>(stream));
}

int esda_decode_raw_q8(const esda_raw_desc *desc, const esda_raw_q8_args *args, void *stream) {
    return esda_decode_raw_q8_stages(desc, args, ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE, stream);
}

int esda_rope_table(const float *inv_freq, int32_t rows, void *table, void *stream) {
    if (!inv_freq || !table) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_rope_table: null pointer");
    if (rows < 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_rope_table: rows must be >= 0");
    if (!aligned16(table) || (reinterpret_cast<uintptr_t>(inv_freq) & 3u))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_rope_table: table 16-byte, inv_freq 4-byte aligned");
    int rc = check_device();
    if (rc) return rc;
    const long long n = (long long) rows * kRopePairs;
    if (n == 0) return ESDA_OK;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), inv_freq, n, static_cast<unsigned *>(table));
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ESDA_OK : hip_fail(e, "rope_table_kernel launch");
}

int esda_quantize_raw_rows(const void *src, int32_t kv_heads, int32_t n_rows, void *q8, int64_t q_head_stride,
                           float *scale, float *bias, int64_t sb_head_stride, int32_t row0, void *stream) {
    if (!src || !q8 || !scale || !bias)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_quantize_raw_rows: null pointer");
    if (kv_heads <= 0 || n_rows < 0 || row0 < 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_quantize_raw_rows: bad sizes");
    if (!aligned16(src) || (reinterpret_cast<uintptr_t>(q8) & 7u) || (q_head_stride % 8))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_quantize_raw_rows: src 16-byte, q8 rows 8-byte aligned");
    if (q_head_stride < (int64_t) (row0 + n_rows) * kRawDim || sb_head_stride < row0 + n_rows)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_quantize_raw_rows: head strides smaller than the rows written");
    if (n_rows == 0) return ESDA_OK;
    int rc = check_device();
    if (rc) return rc;
    const long long rows = (long long) kv_heads * n_rows;
    const unsigned blocks = (unsigned) ((rows + 3) / 4);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const uint16_t *>(src), n_rows, rows, static_cast<unsigned char *>(q8),
                       q_head_stride, scale, bias, sb_head_stride, row0);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ESDA_OK : hip_fail(e, "quantize_rows_kernel launch");
}

int esda_decode_status(const esda_decode_desc *desc, void *workspace, int32_t *bad_sequences,
                       void *stream) {
    if (!workspace || !bad_sequences)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_status: null pointer");
    (void) desc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, workspace, sizeof(v), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "esda_decode_status read");
    const int32_t zero = 0;
    e = hipMemcpyAsync(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "esda_decode_status clear");
    *bad_sequences = v;
    return ESDA_OK;
}

int esda_kv_append(void *cache, int64_t seq_stride, int64_t head_stride, int32_t batch,
                   int32_t num_kv_heads, int32_t head_dim, int32_t cap, const void *src,
                   int32_t n_new, const int32_t *row0, void *stream) {
    if (!cache || !src || !row0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: null pointer");
    if (batch <= 0 || num_kv_heads <= 0 || n_new <= 0 || cap <= 0 || head_dim <= 0 || (head_dim % 8))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: bad sizes");
    if (head_stride < (int64_t) cap * head_dim || seq_stride < (int64_t) num_kv_heads * head_stride ||
        (head_stride % 8) || (seq_stride % 8))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: bad strides");
    if (!aligned16(cache) || !aligned16(src))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: tensors must be 16-byte aligned");
    int rc = check_device();
    if (rc) return rc;
    const size_t total = (size_t) n_new * (head_dim / 8);
    int gx = (int) std::min<size_t>((total + 255) / 256, 1024);
    dim3 grid(gx, num_kv_heads, batch);
    hipLaunchKernelGGL(append_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<uint16_t *>(cache), (long long) seq_stride, (long long) head_stride,
                       num_kv_heads, head_dim, cap, static_cast<const uint16_t *>(src), n_new, row0,
                       nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "append_kernel launch");
    return ESDA_OK;
}

int esda_stream_read(const void *src, size_t bytes, int32_t workgroups, uint32_t *sink, void *stream) {
    if (!src || !sink) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_stream_read: null pointer");
    if (bytes == 0 || (bytes % 1024) || !aligned16(src))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_stream_read: bytes must be a positive multiple of 1024, src 16-byte aligned");
    if (workgroups < 1 || workgroups > 65535)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_stream_read: workgroups must be in 1 .. 65535");
    int rc = check_device();
    if (rc) return rc;
    hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const unsigned char *>(src), (long long) (bytes / 1024), sink);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ESDA_OK : hip_fail(e, "stream_read_kernel launch");
}

int esda_fill_i32(int32_t *dst, int32_t value, int32_t n, void *stream) {
    if (!dst || n < 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_fill_i32: null pointer or negative count");
    if (n == 0) return ESDA_OK;
    int rc = check_device();
    if (rc) return rc;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), dst, value, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "fill_i32_kernel launch");
    return ESDA_OK;
}

}  // extern "C"
