// Host-side check of the stream-K schedule in mfma_tile.h: for many tile /
// slice / slot counts, every (tile, slice) is computed exactly once, each
// workgroup uses each partial slot at most once, and the fixup's partial
// list for a shared tile is exactly the segments written for it, in
// workgroup order. Prints "ok <cases>" or the first violation.
#include <cstdio>
#include <vector>

#include "mfma_tile.h"

using namespace nnc;

static int check(int tiles, int iters, int slots, int fixup) {
    const StreamK sk = plan_streamk(tiles, iters, slots, fixup);
    if (sk.G < 1 || sk.G > slots || sk.sk_tiles < 0 || sk.sk_tiles > tiles) return 1;
    std::vector<int> cover((size_t)tiles * iters, 0);
    // per tile: workgroups that wrote a partial, with their slot
    std::vector<std::vector<std::pair<int, int>>> parts(tiles);
    std::vector<int> whole(tiles, 0);
    for (int g = 0; g < sk.G; ++g) {
        SegmentWalker w(sk, g);
        Segment s;
        int used[2] = {0, 0};
        while (w.next(sk, s)) {
            if (s.tile < 0 || s.tile >= tiles || s.kb < 0 || s.ke > iters || s.kb >= s.ke) return 2;
            for (int k = s.kb; k < s.ke; ++k) cover[(size_t)s.tile * iters + k]++;
            if (s.slot < 0) {
                if (s.kb != 0 || s.ke != iters) return 3;
                whole[s.tile]++;
            } else {
                if (s.slot > 1 || used[s.slot]++) return 4;
                if (s.tile >= sk.sk_tiles) return 5;
                parts[s.tile].push_back({g, s.slot});
            }
        }
    }
    for (size_t i = 0; i < cover.size(); ++i)
        if (cover[i] != 1) return 6;
    bool any_shared = false;
    for (int t = 0; t < tiles; ++t) {
        if (whole[t] + (parts[t].empty() ? 0 : 1) != 1) return 7;
        if (t >= sk.sk_tiles) continue;
        int g0 = -1, g1 = -1, first = -1;
        const bool shared = tile_partials(sk, t, g0, g1, first);
        if (shared != !parts[t].empty()) return 8;
        if (!shared) continue;
        any_shared = true;
        if ((int)parts[t].size() != g1 - g0 + 1) return 9;
        for (int i = 0; i < (int)parts[t].size(); ++i) {
            if (parts[t][i].first != g0 + i) return 10;
            if (parts[t][i].second != (i == 0 ? first : 0)) return 11;
        }
    }
    if (any_shared != sk.needs_fixup()) return 12;
    return 0;
}

int main() {
    int cases = 0;
    const int slots_list[] = {1, 7, 64, 256, 512, 768};
    for (int slots : slots_list)
        for (int tiles = 1; tiles <= 1200; tiles += (tiles < 40 ? 1 : 37))
            for (int iters = 1; iters <= 160; iters += (iters < 12 ? 1 : 19))
                for (int fixup : {0, 4, 16}) {
                    const int r = check(tiles, iters, slots, fixup);
                    ++cases;
                    if (r) {
                        printf("FAIL code %d tiles %d iters %d slots %d fixup %d\n", r, tiles, iters, slots, fixup);
                        return 1;
                    }
                }
    printf("ok %d\n", cases);
    return 0;
}
