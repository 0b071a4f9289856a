// item_deal.h -- which items of a prefill grouped GEMM each XCD takes when
// workgroups draw items from per-XCD counters (grouped_gemm.hip,
// dynamic_items).  Plain constexpr C++ so a host build can check that every
// item is dealt exactly once (tests/item_deal).
//
// Items are (M tile, N tile) pairs numbered mt * per_m + nt (one K split).
// XCD x takes, in this order:
//   1. when sh_m > 0: the last sh_m M tiles (one group whose rows share one
//      weight matrix, the shared expert's) over its own block of N tiles
//      [xcd_sh_n0(x), xcd_sh_n0(x + 1)) -- the per_m N tiles split into nxcd
//      consecutive blocks as evenly as whole tiles allow -- M tiles fastest,
//      so that its workgroups stream each of those weight tiles together
//      through the XCD's L2;
//   2. its whole M tiles x, x + nxcd, x + 2 nxcd, ... of the others, N tiles
//      fastest (an M tile's N tiles share its activation rows in the XCD's L2).
// (Workgroups whose counter is spent go on to the other XCDs' counters, so
// blocks of unequal size even out at the end.)
#pragma once

namespace hf {

struct XcdDeal {
    int m_tiles;  // M tiles in the launch (the shared group's last)
    int per_m;    // N tiles per M tile
    int nxcd;     // XCDs dealt to
    int sh_m;     // M tiles of the shared group dealt by N blocks (0: none)
};

// First N tile of XCD x's block of the shared group (x = nxcd: per_m).
constexpr int xcd_sh_n0(const XcdDeal& d, int x) { return x * d.per_m / d.nxcd; }

// Items of XCD x.
constexpr int xcd_items(const XcdDeal& d, int x) {
    return (d.m_tiles - d.sh_m - x + d.nxcd - 1) / d.nxcd * d.per_m +
           (xcd_sh_n0(d, x + 1) - xcd_sh_n0(d, x)) * d.sh_m;
}

// The item of XCD x's li-th draw, li < xcd_items(d, x).
constexpr int xcd_item(const XcdDeal& d, int x, int li) {
    const int n0 = xcd_sh_n0(d, x);
    const int ns = (xcd_sh_n0(d, x + 1) - n0) * d.sh_m;
    if (li < ns) return (d.m_tiles - d.sh_m + li % d.sh_m) * d.per_m + n0 + li / d.sh_m;
    li -= ns;
    return (x + d.nxcd * (li / d.per_m)) * d.per_m + li % d.per_m;
}

}  // namespace hf
