// plan_check.cpp -- host check of the work-placement arithmetic in
// apertura_amd/csrc/esda_plan.h, the functions the attend and merge kernels call.
// Built and run by tests/test_plan_arithmetic.py with g++.
//
// For each random batch: the visible rows of every sequence (seq_view), the prefix table
// as the kernel's threads write it (one thread per sequence over a 64-lane wave or a
// 256-thread workgroup), every workgroup's share and its walk over (sequence, kv head)
// segments, the partial slots they write, and the owners the merge derives per pair.
// Checked: the table is complete and table[B] is the total; every active share is
// non-empty; the segments of a pair cover its rows exactly once, in order; the merge's
// owners w0 .. w1 are exactly the workgroups that wrote the pair's slots, and those slots
// are distinct across pairs; a pair covered by one workgroup is the one written directly.
// Grid splits: the splits of a pair cover [0, nvis) exactly once and the merge's count
// matches.  PLANT_TABLE_BUG: the prefix table's total is written by thread B (which a
// 256-sequence batch does not have) -- the checker must report it.
#include "esda_plan.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

using namespace esda_plan;

static int g_fail = 0;
#define CHECK(c, ...)                                   \
    do {                                                \
        if (!(c)) {                                     \
            if (g_fail < 20) {                          \
                std::printf("FAIL %s: ", #c);           \
                std::printf(__VA_ARGS__);               \
                std::printf("\n");                      \
            }                                           \
            ++g_fail;                                   \
        }                                               \
    } while (0)

struct Batch {
    int B, Hkv, W, cap, window, ring;
    std::vector<int> pos, base;
};

// The table as the kernel writes it: threads 0 .. threads-1 of workgroup 0, one per sequence.
static void write_table(const std::vector<long long> &nv, int threads, std::vector<long long> &table) {
    const int B = (int) nv.size();
    long long total = 0;
    for (long long v : nv) total += v;
    long long run = 0;
    for (int t = 0; t < threads; ++t) {
        const long long excl = run;
        if (t < B) run += nv[t];
#ifdef PLANT_TABLE_BUG
        if (t <= B) table[t] = t < B ? excl : total;
#else
        write_prefix_entry(table.data(), t, B, excl, total);
#endif
    }
}

static void check_balanced(const Batch &bt) {
    const int B = bt.B, Hkv = bt.Hkv;
    std::vector<long long> nv(B);
    long long rows_seq = 0;
    for (int b = 0; b < B; ++b) {
        const SeqView v = seq_view(bt.pos[b], bt.base[b], bt.cap, bt.window, bt.ring);
        nv[b] = v.ok ? v.nvis : 0;
        rows_seq += nv[b];
    }
    const int threads = B <= 64 ? 64 : 256;  // the wave scan, or the workgroup's LDS scan
    std::vector<long long> table(B + 1, -1);
    write_table(nv, threads, table);
    for (int b = 0; b <= B; ++b) CHECK(table[b] >= 0, "B=%d: table[%d] never written", B, b);
    CHECK(table[B] == rows_seq, "B=%d: table[B]=%lld total=%lld", B, table[B], rows_seq);
    if (table[B] != rows_seq) return;
    const long long rows_total = rows_seq * Hkv;
    const int Wr = active_shares(rows_total, bt.W);
    // segments per pair: (j0, j1, workgroup)
    struct Seg { int j0, j1, w; long long slot; bool direct; };
    std::vector<std::vector<Seg>> segs((size_t) B * Hkv);
    for (int w = 0; w < bt.W; ++w) {
        if (w >= Wr) continue;  // the kernel returns: no rows for it
        const long long lo = share_begin(rows_total, Wr, w), hi = share_begin(rows_total, Wr, w + 1);
        CHECK(lo < hi, "B=%d W=%d: share %d empty [%lld, %lld)", B, bt.W, w, lo, hi);
        long long x = lo;
        int guard = 0;
        while (x < hi && ++guard < 100000) {
            // the kernel's rule: b = the number of sequences whose rows end at or before x
            int b = 0;
            while (b < B && (table[b + 1]) * Hkv <= x) ++b;
            CHECK(b < B, "row %lld past the last sequence", x);
            if (b >= B) return;
            const int n = (int) (table[b + 1] - table[b]);
            const Segment sg = segment_at(x, hi, table[b] * Hkv, n);
            CHECK(sg.kvh >= 0 && sg.kvh < Hkv && sg.j0 >= 0 && sg.j1 <= n && sg.j0 < sg.j1,
                  "bad segment kvh=%d j0=%d j1=%d n=%d", sg.kvh, sg.j0, sg.j1, n);
            const long long u = (long long) b * Hkv + sg.kvh;
            segs[u].push_back({sg.j0, sg.j1, w, share_slot(u, w), sg.j0 == 0 && sg.j1 == n});
            CHECK(sg.end > x, "no progress");
            x = sg.end;
        }
    }
    std::vector<char> slot_used((size_t) B * Hkv + bt.W, 0);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hkv; ++h) {
            auto &s = segs[(size_t) b * Hkv + h];
            std::sort(s.begin(), s.end(), [](const Seg &a, const Seg &c) { return a.j0 < c.j0; });
            int at = 0;
            for (const Seg &g : s) {
                CHECK(g.j0 == at, "B=%d pair (%d,%d): gap or overlap at %d (segment starts %d)", B, b, h, at, g.j0);
                at = g.j1;
                CHECK(g.slot >= 0 && g.slot < (long long) slot_used.size(), "slot %lld out of range", g.slot);
                if (g.slot >= 0 && g.slot < (long long) slot_used.size()) {
                    CHECK(!slot_used[g.slot], "slot %lld written twice", g.slot);
                    slot_used[g.slot] = 1;
                }
            }
            CHECK(at == nv[b], "pair (%d,%d): covered %d of %lld rows", b, h, at, nv[b]);
            int w0 = -1;
            const int ns = pair_owners(table[b], table[b + 1], table[B], Hkv, h, bt.W, &w0);
            CHECK(ns == (int) s.size(), "pair (%d,%d): merge reads %d splits, %zu written", b, h, ns, s.size());
            for (int i = 0; i < (int) s.size() && i < ns; ++i)
                CHECK(s[i].w == w0 + i, "pair (%d,%d): owner %d is workgroup %d, merge expects %d", b, h, i, s[i].w,
                      w0 + i);
            if (s.size() == 1) CHECK(s[0].direct, "pair (%d,%d) in one share not written directly", b, h);
            for (const Seg &g : s)
                if (s.size() > 1) CHECK(!g.direct, "pair (%d,%d) split but written directly", b, h);
        }
}

static void check_grid(std::mt19937_64 &rng) {
    std::uniform_int_distribution<int> dn(0, 300000), dc(1, 600), ds(1, 300);
    const int nvis = dn(rng), chunk = 16 * dc(rng), S = ds(rng);
    int at = 0, written = 0;
    for (int s = 0; s < S; ++s) {
        int j0, j1;
        if (!grid_split(s, S, chunk, nvis, &j0, &j1)) continue;
        CHECK(j0 == at && j1 > j0, "grid nvis=%d chunk=%d S=%d: split %d [%d,%d) at %d", nvis, chunk, S, s, j0, j1, at);
        at = j1;
        ++written;
    }
    CHECK(at == nvis, "grid nvis=%d chunk=%d S=%d: covered %d", nvis, chunk, S, at);
    CHECK(written == (nvis ? grid_splits(nvis, chunk, S) : 0), "grid: %d splits written, merge reads %d", written,
          grid_splits(nvis, chunk, S));
}

int main(int argc, char **argv) {
    const int n = argc > 1 ? std::atoi(argv[1]) : 3000;
    std::mt19937_64 rng(20260101);
    auto U = [&](int a, int b) { return std::uniform_int_distribution<int>(a, b)(rng); };
    int done = 0;
    for (int it = 0; it < n; ++it) {
        Batch bt;
        // every 16th batch at the limits: 256 sequences, 16 kv heads, 16384 workgroups
        const bool limit = it % 16 == 0;
        bt.B = limit ? 256 : (it % 5 == 0 ? U(65, 256) : U(1, 64));
        bt.Hkv = limit ? 16 : U(1, 16);
        bt.W = limit ? 16384 : (U(0, 3) == 0 ? U(1, 16384) : U(1, 512));
        bt.ring = U(0, 3) == 0;
        bt.cap = limit ? U(1 << 16, 1 << 20) : U(1, 40000);
        bt.window = bt.ring ? U(1, bt.cap) : (U(0, 1) ? 0 : U(1, bt.cap));
        const bool tiny = U(0, 4) == 0;  // fewer rows than workgroups (T < W)
        for (int b = 0; b < bt.B; ++b) {
            int p;
            if (bt.ring) p = U(0, 4 * bt.cap);
            else p = tiny ? U(0, 3) : U(-1, bt.cap);  // -1 and cap: out of range, skipped
            const int base = bt.ring ? 0 : (U(0, 3) == 0 && p > 0 ? U(0, p) : 0);
            bt.pos.push_back(p);
            bt.base.push_back(base);
        }
        check_balanced(bt);
        check_grid(rng);
        ++done;
    }
    std::printf("%s: %d batches, %d failures\n", g_fail ? "FAIL" : "OK", done, g_fail);
    return g_fail ? 1 : 0;
}
