// Host-side check of the attention-forward work schedule (dirktensor_amd/csrc/flash_items.h): for each
// shape, walks the snake order on the grid the launcher would use and verifies, per 64-query tile of
// every (batch, head), that its rows are written by exactly one unit and that the key tiles its rows see
// are covered exactly once by its unit's parts (whole, split or folded units alike), that split items
// have one workspace slot shared by their parts and distinct from all others, and that the kernel
// arguments fit in 4 KB. Prints one line per shape and exits non-zero on any failure.
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
    build_schedule(a, sl, cus, true, &sc, true);
    const int grid = std::min(cus, sc.n_units);
    const int n_qt = (T + kItemRows - 1) / kItemRows;
    const int n_h = (T + 63) / 64;  // 64-query tiles
    // per (b, h, 64-query tile): the key tiles it is computed over, and how often its rows are written
    std::map<std::tuple<int, int, int>, std::vector<int>> tiles;
    std::map<std::tuple<int, int, int>, int> written, slot_of;
    std::set<int> slots;
    int bad = 0, max_parts = 1;
    for (int round = 0;; ++round) {
        bool any = false;
        for (int w = 0; w < grid; ++w) {
            const int k = snake_item(round, grid, w);
            if (k >= sc.n_units) continue;
            any = true;
            const Unit u = decode_unit(k, sc, H, sc.cum);
            if (u.b < 0 || u.b >= B || u.h < 0 || u.h >= H || u.qt < 0 || u.qt >= n_qt || u.L != sl.len[u.b] ||
                u.qa < 0 || u.qa % 64 || u.qb % 64 || u.qb <= u.qa || (!sc.fold && u.qb != u.qa + 64)) {
                ++bad;
                continue;
            }
            if (u.pad != (u.qa >= u.L)) ++bad;
            // the kernel's key range: up to the upper half's last query (causal), split into parts
            const int n = u.pad ? 0 : ((causal ? std::min(u.qb + 64, u.L) : u.L) + 63) / 64;
            const int t0 = u.parts > 1 ? u.part * sc.S : 0;
            const int t1 = u.parts > 1 ? std::min(t0 + sc.S, n) : n;
            max_parts = std::max(max_parts, u.parts);
            for (int half = 0; half < 2; ++half) {
                const int q = half ? u.qb : u.qa;
                if (q >= T) continue;
                const auto key = std::make_tuple(u.b, u.h, q / 64);
                if (u.part == 0) written[key]++;
                if (q >= u.L) continue;  // rows past the sequence: the empty row, no keys
                const int need = causal ? std::min(q + 64, u.L) : u.L;  // keys the half's last row sees
                for (int t = t0; t < t1; ++t)
                    if (t * 64 < need) tiles[key].push_back(t);
            }
            if (u.parts > 1) {
                if (u.slot < 0 || u.slot >= sc.n_slots || u.parts > kMaxParts || sc.fold) ++bad;
                const auto key = std::make_tuple(u.b, u.h, u.qt);
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
            for (int j = 0; j < n_h; ++j) {
                const auto key = std::make_tuple(b, h, j);
                missing += written[key] != 1;
                if (j * 64 >= sl.len[b]) continue;
                std::vector<int> v = tiles[key];
                std::sort(v.begin(), v.end());
                const int n = ((causal ? std::min(64 * j + 64, sl.len[b]) : sl.len[b]) + 63) / 64;
                bool ok = (int)v.size() == n;
                for (int t = 0; ok && t < n; ++t) ok = v[t] == t;
                missing += !ok;
            }
    const size_t args = sizeof(FlashArgs) + sizeof(Schedule);
    bad += args > 4096;
    std::printf("B=%d T=%d H=%d causal=%d %s cus=%d: units %d, fold %d, S %d, split items %d, parts <= %d, grid %d: %s\n",
                B, T, H, causal, lens.empty() ? "dense" : "ragged", cus, sc.n_units, sc.fold, sc.S, sc.n_slots,
                max_parts, grid, bad + missing ? "FAIL" : "ok");
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
        fails += check(1, 1024, 16, 1, {}, cus);
        fails += check(2, 2048, 8, 1, {}, cus);
        fails += check(1, 256, 3, 1, {}, cus);
        fails += check(1, 2112, 16, 1, {}, cus);
    }
    return fails != 0;
}
