// esda_plan.h -- the integer arithmetic that places decode work: which cache rows a
// sequence attends, the batch prefix table, each workgroup's share of the rows of a
// balanced plan, the (sequence, kv head, rows) segments a share covers, and which
// workgroups' partials the merge reads for a pair.  The attend and merge kernels call
// these functions on the device; tests/test_plan_arithmetic.py compiles them with g++
// and checks them over thousands of random batches on the host.
//
// Reference behaviour: the visibility rule is ESGemma4TextModel.mm:68-83 (kj <= pos and,
// on sliding layers, kj > pos - window), over the row layout of ESKVCache.mm:64-109
// (linear rows after compaction) or a ring of `cap` rows.
#pragma once

#if defined(__HIP__)
#define ESDA_HD __host__ __device__ __forceinline__
#else
#define ESDA_HD inline
#endif

namespace esda_plan {

// a / b for a >= 0, b > 0: 32-bit division when both fit (the common case on the device,
// far shorter than the 64-bit sequence); the same quotient either way.
ESDA_HD long long div_nonneg(long long a, long long b) {
    if (((unsigned long long) a | (unsigned long long) b) >> 32 == 0) return (long long) ((unsigned) a / (unsigned) b);
    return (long long) ((unsigned long long) a / (unsigned long long) b);
}

struct SeqView {
    int nvis;    // visible rows
    int first;   // cache row of the oldest visible position
    int newrow;  // cache row receiving the new token
    int ok;
};

// Visible absolute positions are [lo, pos] with lo = max(0, pos - window + 1) for a
// sliding layer; rows hold p - base (linear) or p mod cap (ring).  Logical row j (0 =
// oldest) lives at cache row first + j (mod cap).  A position outside a linear cache
// (or negative) gives ok = 0 and no rows.
ESDA_HD SeqView seq_view(int pos, int base, int cap, int window, int ring) {
    SeqView v{0, 0, 0, 0};
    if (pos < 0) return v;
    int lo = window > 0 ? (pos - window + 1 > 0 ? pos - window + 1 : 0) : 0;
    if (ring) {
        v.newrow = pos % cap;
        v.first = lo % cap;
    } else {
        if (lo < base) lo = base;
        v.newrow = pos - base;
        if (v.newrow < 0 || v.newrow >= cap) return v;
        v.first = lo - base;
    }
    v.nvis = pos - lo + 1;
    v.ok = 1;
    return v;
}

// The prefix table of a balanced plan, table[0 .. B]: table[b] = visible rows of the
// sequences before b, table[B] = all of them.  Written by the threads t of one
// workgroup, one sequence each (B <= threads): thread t < B writes its entry, thread 0
// also the total (there may be no thread B).
ESDA_HD void write_prefix_entry(long long *table, int t, int B, long long exclusive, long long total) {
    if (t < B) table[t] = exclusive;
    if (t == 0) table[B] = total;
}

// Grid plans: split s of a pair with nvis visible rows covers logical rows [j0, j1) with
// j0 = s * chunk; the last of the S splits takes every remaining row, so a max_visible
// hint below the real length makes that split longer instead of dropping rows.  Returns
// false for a split with no rows.
ESDA_HD bool grid_split(int s, int S, int chunk, int nvis, int *j0, int *j1) {
    *j0 = s * chunk;
    if (*j0 >= nvis) return false;
    *j1 = (s == S - 1 || nvis - *j0 < chunk) ? nvis : *j0 + chunk;
    return true;
}

// Splits of a grid pair that wrote partials (the merge reads these).
ESDA_HD int grid_splits(int nvis, int chunk, int S) {
    const int n = (nvis + chunk - 1) / chunk;
    return n < S ? n : S;
}

// Workgroups that hold rows: every share must hold at least one, and fewer rows may be
// visible than the plan sized its W workgroups for.
ESDA_HD int active_shares(long long rows_total, int W) { return (int) (rows_total < W ? rows_total : W); }

// Share of workgroup w < Wr over all rows linearised as (sequence, kv head, row):
// [share_begin(w), share_begin(w + 1)).
ESDA_HD long long share_begin(long long rows_total, int Wr, int w) { return div_nonneg(rows_total * w, Wr); }

// The segment of a share that starts at linear row x, inside sequence b whose rows begin
// at linear row sb = rows_before_b * Hkv and number n per kv head: kv head kvh, rows
// [j0, j0 + (end - x)) of it, where end = min(the pair's end, the share's end hi).
struct Segment {
    int kvh, j0, j1;
    long long end;
};
ESDA_HD Segment segment_at(long long x, long long hi, long long sb, int n) {
    Segment s;
    s.kvh = (int) div_nonneg(x - sb, n);
    s.j0 = (int) (x - sb - (long long) s.kvh * n);
    const long long pair_end = sb + (long long) (s.kvh + 1) * n;
    s.end = pair_end < hi ? pair_end : hi;
    s.j1 = s.j0 + (int) (s.end - x);
    return s;
}

// Partial slot of workgroup w's segment of pair u = b * Hkv + kvh: the slots of one pair
// are consecutive and two pairs never share one (B * Hkv + W slots in all).
ESDA_HD long long share_slot(long long u, int w) { return u + w; }

// The workgroups w0 .. w1 whose shares hold rows of pair (b, kvh) -- those holding its
// first and last rows -- for the merge, from the prefix table entries table_b = table[b],
// table_b1 = table[b + 1] and table_total = table[B].  Returns their count (0 for a
// sequence with no rows or an inconsistent table) and sets *w0.
ESDA_HD int pair_owners(long long table_b, long long table_b1, long long table_total, int Hkv, int kvh, int W,
                        int *w0) {
    const long long n = table_b1 - table_b;
    const long long rows_total = table_total * Hkv;
    if (n <= 0 || rows_total <= 0) return 0;
    const long long first = table_b * Hkv + (long long) kvh * n, last = first + n - 1;
    if (first < 0 || last >= rows_total) return 0;
    const long long Wr = rows_total < W ? rows_total : W;
    // workgroup w holds row r iff share_begin(w) <= r < share_begin(w + 1), i.e. the
    // largest w with rows_total * w / Wr <= r: w = ((r + 1) * Wr - 1) / rows_total
    const int a = (int) div_nonneg((first + 1) * Wr - 1, rows_total);
    const int z = (int) div_nonneg((last + 1) * Wr - 1, rows_total);
    if (a < 0 || z >= Wr || a > z) return 0;
    *w0 = a;
    return z - a + 1;
}

}  // namespace esda_plan
