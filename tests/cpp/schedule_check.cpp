// Host-side check of the attention-forward work schedule (dirktensor_amd/csrc/flash_items.h): for each
// shape, walks the snake order on the grid the launcher would use and verifies that every computing
// item's key tiles are covered exactly once by its parts, every padding tile appears once, split items
// have one workspace slot shared by their parts and distinct from all others, and the kernel arguments
// fit in 4 KB. Prints one line per shape and exits non-zero on any failure.
#include "../../dirktensor_amd/csrc/flash_items.h"

#include <algorithm>
#include <cstdio>
#include <map>
#include <random>
#include <set>
#include <tuple>
#include <vector>

using namespace dt;

static int check(int B, int T, int H, int causal, const std::vector<int>& lens, int cus) {
    FlashArgs a{};
    a.B = B;
    a.T = T;
    a.H = H;
    a.causal = causal;
    a.ragged = !lens.empty();
    SeqLens sl{};
    for (int b = 0; b < B; ++b) sl.len[b] = lens.empty() ? T : lens[b];
    Schedule sc;
    build_schedule(a, sl, cus, true, &sc);
    const int grid = std::min(cus, sc.n_units);
    const int n_qt = (T + kItemRows - 1) / kItemRows;
    std::map<std::tuple<int, int, int>, std::vector<int>> tiles;
    std::map<std::tuple<int, int, int>, int> pads, slot_of;
    std::set<int> slots;
    int bad = 0, max_parts = 1;
    for (int round = 0;; ++round) {
        bool any = false;
        for (int w = 0; w < grid; ++w) {
            const int k = snake_item(round, grid, w);
            if (k >= sc.n_units) continue;
            any = true;
            const Unit u = decode_unit(k, sc, H, sc.cum);
            if (u.b < 0 || u.b >= B || u.h < 0 || u.h >= H || u.qt < 0 || u.qt >= n_qt || u.L != sl.len[u.b]) {
                ++bad;
                continue;
            }
            const auto key = std::make_tuple(u.b, u.h, u.qt);
            if (u.pad != (u.qt * kItemRows >= u.L)) ++bad;
            if (u.pad) {
                pads[key]++;
                continue;
            }
            const int n = tile_cost(u.qt, u.L, causal);
            const int t0 = u.parts > 1 ? u.part * sc.S : 0;
            const int t1 = u.parts > 1 ? std::min(t0 + sc.S, n) : n;
            for (int t = t0; t < t1; ++t) tiles[key].push_back(t);
            max_parts = std::max(max_parts, u.parts);
            if (u.parts > 1) {
                if (u.slot < 0 || u.slot >= sc.n_slots || u.parts > kMaxParts) ++bad;
                const auto it = slot_of.find(key);
                if (it == slot_of.end()) {
                    if (!slots.insert(u.slot).second) ++bad;
                    slot_of[key] = u.slot;
                } else if (it->second != u.slot) {
                    ++bad;
                }
            }
        }
        if (!any) break;
    }
    int missing = 0;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int qt = 0; qt < n_qt; ++qt) {
                const auto key = std::make_tuple(b, h, qt);
                if (qt * kItemRows >= sl.len[b]) {
                    missing += pads[key] != 1;
                    continue;
                }
                std::vector<int> v = tiles[key];
                std::sort(v.begin(), v.end());
                const int n = tile_cost(qt, sl.len[b], causal);
                bool ok = (int)v.size() == n;
                for (int t = 0; ok && t < n; ++t) ok = v[t] == t;
                missing += !ok;
            }
    const size_t args = sizeof(FlashArgs) + sizeof(Schedule);
    bad += args > 4096;
    std::printf("B=%d T=%d H=%d causal=%d %s cus=%d: units %d, S %d, split items %d, parts <= %d, grid %d: %s\n", B, T, H,
                causal, lens.empty() ? "dense" : "ragged", cus, sc.n_units, sc.S, sc.n_slots, max_parts, grid,
                bad + missing ? "FAIL" : "ok");
    return bad + missing;
}

int main() {
    int fails = 0;
    std::mt19937 rng(4001);
    std::vector<int> r8(8), r256(256);
    for (int& x : r8) x = 64 + (int)(rng() % 1985);
    for (int& x : r256) x = 1 + (int)(rng() % 8192);
    for (int cus : {256, 80, 7}) {
        fails += check(1, 2048, 16, 1, {}, cus);
        fails += check(1, 4096, 16, 1, {}, cus);
        fails += check(1, 6144, 16, 1, {}, cus);
        fails += check(1, 8192, 2, 1, {}, cus);
        fails += check(1, 4096, 2, 1, {}, cus);
        fails += check(1, 2048, 4, 1, {}, cus);
        fails += check(8, 2048, 16, 1, r8, cus);
        fails += check(3, 1000, 5, 1, {}, cus);
        fails += check(3, 1000, 5, 1, {1000, 7, 129}, cus);
        fails += check(2, 3000, 3, 1, {3000, 2900}, cus);
        fails += check(2, 64, 16, 1, {}, cus);
        fails += check(1, 1, 1, 1, {}, cus);
        fails += check(1, 2048, 16, 0, {}, cus);
        fails += check(4, 777, 3, 0, {777, 1, 300, 500}, cus);
        fails += check(256, 8192, 1, 1, r256, cus);
        fails += check(3, 4096, 2, 1, {4096, 2500, 129}, cus);
    }
    return fails != 0;
}
