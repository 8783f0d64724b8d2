// Work schedule of the persistent attention-forward kernels (bf16 and fp32 modes).
//
// An item is 128 queries (one query tile) of one (batch, head). A persistent grid of at most one
// workgroup per CU walks a list of work units in "snake" order (unit k of round j: j*G + w on even
// rounds, (j+1)*G-1-w' on odd ones, w' defined below), so a workgroup pairs an expensive unit with a
// cheap one. A unit is an item, or, when an item's causal cost exceeds a workgroup's fair share of the
// launch (total cost / G), one part of it: S consecutive 64-key tiles, the last part taking the rest.
// The parts of one item run on different workgroups; each writes its partial (m, l, O) to a workspace
// slot and the workgroup that finishes last merges them, in part order, with the reference's rescale.
//
// The unit list is built on the host as "kinds" sorted by decreasing cost: a kind is one (query tile,
// part) pair, and its units are that tile's items, one per (sequence, head) whose sequence reaches the
// tile (every sequence when the batch is not ragged), sequences by decreasing length, heads fastest.
// Padding tiles (past a sequence's end, which only write the empty rows) come last.
//
// Folded units. A causal launch that fits one round (at most one unit per workgroup, no split, full
// sequences, T a multiple of 128) has nothing for the snake to pair, so its longest query tile sets the
// launch time while the average costs half as much. Such a launch folds instead: a unit is the 64-query
// tiles p and n-1-p (n = T / 64) of one (batch, head), which together cost n + 1 64-query key steps for
// every p. The kernel runs a folded unit as a 128-query item whose rows 0-63 are tile p and rows 64-127
// tile n-1-p, over the key tiles of the upper one; the waves of tile p skip the key tiles past it.
#pragma once

#include "dt_internal.h"

#include <algorithm>

namespace dt {

constexpr int kItemRows = 128;  // queries per item
constexpr int kMaxQTiles = 64;  // T <= 8192
constexpr int kMaxKinds = 256;
constexpr int kMaxParts = 3;
constexpr int kMinPartTiles = 16;  // 64-key tiles

// Kernel argument (3.6 KB).
struct Schedule {
    int n_kinds;
    int n_units;
    int dense;    // 1: no padding and nothing split, so kind j is query tile n_qt-1-j with B*H units
    int fold;     // 1 (dense only): unit kind j is the folded pair of 64-query tiles j and 2*n_qt-1-j
    int n_qt;
    int S;        // 64-key tiles per part of a split item (0: nothing is split)
    int n_slots;  // split items: one counter and kMaxParts partial results each
    int cum[kMaxKinds + 1];     // units in kinds 0 .. j-1
    int kind[kMaxKinds];        // query tile | part << 8 | parts << 12 | padding << 16
    int split_base[kMaxQTiles]; // slot of the first split item of a query tile (its units' order)
    int nb[kMaxQTiles];         // sequences with rows in a query tile
    int seq[kMaxRaggedBatch];   // i-th longest sequence (stable) | its length << 16
};

struct Unit {
    int b, h, qt, L;    // sequence, head, query tile, the sequence's length
    int qa, qb;         // first query of the item's rows 0-63 and of its rows 64-127 (qa + 64 unless folded)
    int part, parts;    // parts == 1: a whole item
    int slot;           // split items: workspace slot
    bool pad;           // a padding tile
};

// The unit index a workgroup takes in round `round` of the snake walk. Workgroup w runs on XCD w % 8
// (workgroups are dealt to the eight XCDs in turn). In even rounds it takes unit round*G + w; in odd
// rounds the unit mirrored across the round of the partner w ^ 7 (same position within its group of 8).
// When every kind holds a multiple of 8 units (H a multiple of 8) and G is one too, unit k's head is
// congruent to k mod 8, so every unit of one head runs on one XCD and its K/V rows pass through one L2.
__host__ __device__ inline int snake_item(int round, int G, int w) {
    const int wo = (G & 7) == 0 ? (w ^ 7) : w;
    return (round & 1) ? (round + 1) * G - 1 - wo : round * G + w;
}

// cum: the schedule's cum[] (kernel argument, or a copy of it in LDS, which a workgroup loads in one step
// instead of a chain of dependent scalar loads)
__host__ __device__ inline Unit decode_unit(int k, const Schedule& sc, int H, const int* cum) {
    if (sc.dense) {  // arithmetic only (the table search is a chain of dependent scalar loads)
        const int BH = sc.cum[1];
        const int r = k % BH;
        Unit u;
        if (sc.fold) {
            u.qt = k / BH;
            u.qa = 64 * u.qt;
            u.qb = 64 * (2 * sc.n_qt - 1 - u.qt);
        } else {
            u.qt = sc.n_qt - 1 - k / BH;
            u.qa = u.qt * kItemRows;
            u.qb = u.qa + 64;
        }
        u.part = 0;
        u.parts = 1;
        u.pad = false;
        u.b = r / H;
        u.h = r % H;
        u.L = sc.seq[0] >> 16;
        u.slot = 0;
        return u;
    }
    int lo = 0, hi = sc.n_kinds - 1;  // the kind j with cum[j] <= k < cum[j+1]
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cum[mid] <= k) lo = mid;
        else hi = mid - 1;
    }
    const int info = sc.kind[lo];
    const int r = k - cum[lo];
    Unit u;
    u.qt = info & 0xff;
    u.qa = u.qt * kItemRows;
    u.qb = u.qa + 64;
    u.part = (info >> 8) & 0xf;
    u.parts = (info >> 12) & 0xf;
    u.pad = (info >> 16) & 1;
    const int s = sc.seq[(u.pad ? sc.nb[u.qt] : 0) + r / H];
    u.b = s & 0xffff;
    u.L = s >> 16;
    u.h = r % H;
    u.slot = sc.split_base[u.qt] + r;
    return u;
}

// Host side. Causal cost of a query tile in 64-key tiles, for a sequence of length L (0: padding tile).
inline int tile_cost(int qt, int L, int causal) {
    const int q0 = qt * kItemRows;
    if (q0 >= L) return 0;
    const int k_end = causal ? std::min(q0 + kItemRows, L) : L;
    return (k_end + 63) / 64;
}

// Builds the schedule of one launch on G workgroups; split = 0 keeps every item whole; fold = 0 never
// folds (a kernel that cannot run folded units).
inline void build_schedule(const FlashArgs& a, const SeqLens& sl, int G, bool split, Schedule* sc, bool fold = false) {
    *sc = Schedule{};
    const int n_qt = (a.T + kItemRows - 1) / kItemRows;
    int idx[kMaxRaggedBatch];
    for (int b = 0; b < a.B; ++b) idx[b] = b;
    if (a.ragged) std::stable_sort(idx, idx + a.B, [&](int x, int y) { return sl.len[x] > sl.len[y]; });
    for (int i = 0; i < a.B; ++i) sc->seq[i] = idx[i] | ((a.ragged ? sl.len[idx[i]] : a.T) << 16);
    // per query tile: sequences reaching it and their nominal cost (that of the longest one)
    int64_t total = 0;
    int cmax = 0, cost[kMaxQTiles];
    for (int qt = 0; qt < n_qt; ++qt) {
        int nb = 0;
        for (int b = 0; b < a.B; ++b) nb += (a.ragged ? sl.len[b] : a.T) > qt * kItemRows;
        sc->nb[qt] = nb;
        cost[qt] = nb > 0 ? tile_cost(qt, a.ragged ? sl.len[idx[0]] : a.T, a.causal) : 0;
        for (int i = 0; i < nb; ++i) total += (int64_t)a.H * tile_cost(qt, sc->seq[i] >> 16, a.causal);
        cmax = std::max(cmax, cost[qt]);
    }
    // Part size: the fair share of a workgroup, at least a third of the largest item. Items are split only
    // when the largest costs at least twice the fair share: a split part pays a second item boundary (its
    // partial result goes through the workspace), which measured as costly as the imbalance it removes at
    // B*H = 16, T = 2048 (largest item 1.9x the share), while few heads (a tensor-parallel shard) leave most
    // CUs idle without it.
    // A part is at least kMinPartTiles tiles: its end (partial stores, counter, merge through memory) costs
    // about three steps, too much for small items (B=1, T=512, H=16 split into 3-tile parts took 14.7 µs
    // against 5 whole).
    int S = 0;
    if (split && a.causal && G > 0) {
        const int64_t fair = (total + G - 1) / G;
        if (cmax >= 2 * fair)
            S = (int)std::max<int64_t>(std::max<int64_t>(fair, kMinPartTiles), (cmax + kMaxParts - 1) / kMaxParts);
        if (S >= cmax) S = 0;
    }
    sc->S = S;
    // a launch that splits nothing and fits one round folds (see the top of this file)
    if (fold && S == 0 && a.causal && !a.ragged && a.T % kItemRows == 0 && n_qt >= 2 && G > 0 &&
        (int64_t)a.B * a.H * n_qt <= G) {
        // kind j: the pair (j, 2*n_qt-1-j) of 64-query tiles; every pair costs 2*n_qt+1 tile steps of 64 queries
        for (int j = 0; j < n_qt; ++j) {
            sc->kind[j] = j;
            sc->cum[j + 1] = sc->cum[j] + a.B * a.H;
            sc->nb[j] = a.B;
        }
        sc->n_kinds = n_qt;
        sc->n_units = sc->cum[n_qt];
        sc->n_qt = n_qt;
        sc->dense = 1;
        sc->fold = 1;
        return;
    }
    struct K {
        int cost, qt, part, parts, pad, count;
    };
    K ks[kMaxKinds];
    int nk = 0, slots = 0;
    for (int qt = 0; qt < n_qt; ++qt) {
        const int count = sc->nb[qt] * a.H;
        if (count == 0) continue;
        const int parts = S > 0 && cost[qt] > S ? (cost[qt] + S - 1) / S : 1;
        sc->split_base[qt] = parts > 1 ? slots : 0;
        if (parts > 1) slots += count;
        for (int p = 0; p < parts; ++p)
            ks[nk++] = K{parts == 1 ? cost[qt] : std::min(S, cost[qt] - p * S), qt, p, parts, 0, count};
    }
    std::stable_sort(ks, ks + nk, [](const K& x, const K& y) {
        if (x.cost != y.cost) return x.cost > y.cost;
        return x.qt > y.qt;
    });
    for (int qt = 0; qt < n_qt; ++qt) {  // padding tiles, in query-tile order
        const int count = (a.B - sc->nb[qt]) * a.H;
        if (count > 0) ks[nk++] = K{0, qt, 0, 1, 1, count};
    }
    for (int j = 0; j < nk; ++j) {
        sc->kind[j] = ks[j].qt | (ks[j].part << 8) | (ks[j].parts << 12) | (ks[j].pad << 16);
        sc->cum[j + 1] = sc->cum[j] + ks[j].count;
    }
    sc->n_kinds = nk;
    sc->n_units = sc->cum[nk];
    sc->n_slots = slots;
    sc->n_qt = n_qt;
    sc->dense = !a.ragged && slots == 0;
}

// Workspace of split items: per slot a counter and kMaxParts partial results of 128 rows (128 O values and
// (m_s, m_t, l, -) per row, 132 floats, in the kernel's register order). Fewer than G items are ever split
// (each costs more than total / G).
constexpr size_t kPartialFloats = (size_t)kItemRows * 136;

}  // namespace dt
