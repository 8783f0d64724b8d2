// Work items of the persistent attention-forward kernels (bf16 and fp32 modes).
//
// An item is 128 queries (one query tile) of one (batch, head). A persistent grid of at most one
// workgroup per CU walks the items in "snake" order over a list sorted by decreasing causal cost
// (item k of round j: j*G + w on even rounds, (j+1)*G-1-w on odd ones), so a workgroup pairs a long
// query tile with a short one. In a ragged batch the list holds only the tiles that start before
// their sequence's end, in the same cost order, followed by the padding tiles.
#pragma once

#include "dt_internal.h"

#include <algorithm>

namespace dt {

constexpr int kItemRows = 128;  // queries per item

struct Item {
    int b, h, qt;
};

// Item order of a ragged batch, built on the host: the items that compute (query tiles that start
// before their sequence's end) sorted by decreasing causal cost, i.e. query tile from the last to the
// first and, within a tile, the sequences long enough to reach it; then the padding items (tiles past
// a sequence's end, which only write the empty rows).
struct RaggedOrder {
    int n_valid;             // computing items
    int cum_valid[65];       // cum_valid[j]: computing items in the tiles n_qt-1 .. n_qt-j
    int cum_pad[65];         // the same for padding items
    int nb[64];              // nb[qt]: sequences with rows in tile qt
    uint16_t order[kMaxRaggedBatch];  // sequences by decreasing length (stable)
};

// The item index a workgroup takes in round `round` of the snake walk. Workgroup w runs on XCD w % 8
// (workgroups are dealt to the eight XCDs in turn). In even rounds it takes item round*G + w, whose
// (batch, head) index is congruent to w mod 8 when B*H and G are multiples of 8; in odd rounds it takes
// the item mirrored across the round, of the partner w ^ 7 (same cost rank: w ^ 7 differs from w only in
// its low three bits), whose (batch, head) index is again congruent to w mod 8. So every item of one head
// runs on one XCD and the head's K/V rows pass through one L2.
__device__ __forceinline__ int snake_item(int round, int G, int w) {
    const int wo = (G & 7) == 0 ? (w ^ 7) : w;
    return (round & 1) ? (round + 1) * G - 1 - wo : round * G + w;
}

__device__ __forceinline__ Item decode_item(int k, int n_qt, int BH, int H) {
    Item it;
    it.qt = n_qt - 1 - k / BH;  // items sorted by decreasing causal cost
    const int r = k % BH;
    it.b = r / H;
    it.h = r % H;
    return it;
}

__device__ __forceinline__ Item decode_item_ragged(int k, int n_qt, int H, const RaggedOrder& ro) {
    const bool pad = k >= ro.n_valid;
    const int* cum = pad ? ro.cum_pad : ro.cum_valid;
    const int kk = pad ? k - ro.n_valid : k;
    int j = 0;
    while (j + 1 < n_qt && cum[j + 1] <= kk) ++j;
    Item it;
    it.qt = n_qt - 1 - j;
    const int r = kk - cum[j];
    it.b = ro.order[(pad ? ro.nb[it.qt] : 0) + r / H];
    it.h = r % H;
    return it;
}

// Host side: the ragged order (a.ragged only; T <= 8192, so at most 64 query tiles).
inline void build_ragged_order(const FlashArgs& a, const SeqLens& sl, RaggedOrder* ro) {
    *ro = RaggedOrder{};
    if (!a.ragged) return;
    const int n_qt = (a.T + kItemRows - 1) / kItemRows;
    int idx[kMaxRaggedBatch];
    for (int b = 0; b < a.B; ++b) idx[b] = b;
    std::stable_sort(idx, idx + a.B, [&](int x, int y) { return sl.len[x] > sl.len[y]; });
    for (int b = 0; b < a.B; ++b) ro->order[b] = (uint16_t)idx[b];
    for (int qt = 0; qt < n_qt; ++qt) {
        int nb = 0;
        for (int b = 0; b < a.B; ++b) nb += sl.len[b] > qt * kItemRows;
        ro->nb[qt] = nb;
    }
    for (int j = 0; j < n_qt; ++j) {
        const int qt = n_qt - 1 - j;
        ro->cum_valid[j + 1] = ro->cum_valid[j] + ro->nb[qt] * a.H;
        ro->cum_pad[j + 1] = ro->cum_pad[j] + (a.B - ro->nb[qt]) * a.H;
    }
    ro->n_valid = ro->cum_valid[n_qt];
}

// Persistent grid size: one workgroup per CU of the current device (at most the item count).
int persistent_grid(int64_t n_items, int* grid);

}  // namespace dt
