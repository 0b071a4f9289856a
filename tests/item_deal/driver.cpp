// Brute-force check of item_deal.h: for every case on stdin
// ("m_tiles per_m nxcd sh_m" per line), every item index in
// [0, m_tiles * per_m) is drawn by exactly one (XCD, draw) pair, each XCD's
// shared-group draws come first and cover its own N block of the last sh_m M
// tiles, M tiles fastest, the blocks of consecutive XCDs consecutive and
// differing in size by at most one N tile, and its other draws are its own
// whole M tiles.
// Prints "ok <cases>" or the first violation.
#include <cstdio>
#include <vector>

#include "item_deal.h"

int main() {
    int cases = 0;
    hf::XcdDeal d{};
    while (std::scanf("%d %d %d %d", &d.m_tiles, &d.per_m, &d.nxcd, &d.sh_m) == 4) {
        ++cases;
        for (int x = 0; x < d.nxcd; ++x) {
            const int w = hf::xcd_sh_n0(d, x + 1) - hf::xcd_sh_n0(d, x);
            if (hf::xcd_sh_n0(d, 0) != 0 || hf::xcd_sh_n0(d, d.nxcd) != d.per_m || w < d.per_m / d.nxcd ||
                w > (d.per_m + d.nxcd - 1) / d.nxcd) {
                std::printf("case %d: xcd %d shared block of %d N tiles\n", cases, x, w);
                return 1;
            }
        }
        const int total = d.m_tiles * d.per_m;
        std::vector<int> seen(total, 0);
        for (int x = 0; x < d.nxcd; ++x) {
            const int n = hf::xcd_items(d, x);
            for (int li = 0; li < n; ++li) {
                const int it = hf::xcd_item(d, x, li);
                if (it < 0 || it >= total) {
                    std::printf("case %d: xcd %d draw %d -> item %d outside [0, %d)\n", cases, x, li, it, total);
                    return 1;
                }
                ++seen[it];
                const int mt = it / d.per_m, nt = it % d.per_m;
                const bool shared_tile = mt >= d.m_tiles - d.sh_m;
                const int n0 = hf::xcd_sh_n0(d, x), n1 = hf::xcd_sh_n0(d, x + 1);
                if (li < (n1 - n0) * d.sh_m) {
                    if (!shared_tile || nt < n0 || nt >= n1 || mt != d.m_tiles - d.sh_m + li % d.sh_m ||
                        nt != n0 + li / d.sh_m) {
                        std::printf("case %d: xcd %d shared draw %d -> (%d, %d)\n", cases, x, li, mt, nt);
                        return 1;
                    }
                } else if (shared_tile || mt % d.nxcd != x) {
                    std::printf("case %d: xcd %d draw %d -> M tile %d not its own\n", cases, x, li, mt);
                    return 1;
                }
            }
        }
        for (int i = 0; i < total; ++i)
            if (seen[i] != 1) {
                std::printf("case %d: item %d drawn %d times\n", cases, i, seen[i]);
                return 1;
            }
    }
    std::printf("ok %d\n", cases);
    return 0;
}
