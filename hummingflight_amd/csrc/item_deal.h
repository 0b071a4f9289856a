// item_deal.h -- which items of a prefill grouped GEMM each XCD takes when
// workgroups draw items from per-XCD counters (grouped_gemm.hip,
// dynamic_items).  Plain constexpr C++ so a host build can check that every
// item is dealt exactly once (tests/item_deal).
//
// Items are (M tile, N tile) pairs numbered mt * per_m + nt (one K split).
// XCD x takes, in this order:
//   1. when sh_m > 0: the last sh_m M tiles (one group whose rows share one
//      weight matrix, the shared expert's) over its own block of sh_nl N tiles
//      [x * sh_nl, (x + 1) * sh_nl), M tiles fastest, so that its workgroups
//      stream each of those weight tiles together through the XCD's L2;
//   2. its whole M tiles x, x + nxcd, x + 2 nxcd, ... of the others, N tiles
//      fastest (an M tile's N tiles share its activation rows in the XCD's L2).
// sh_nl * nxcd must equal per_m when sh_m > 0.
#pragma once

namespace hf {

struct XcdDeal {
    int m_tiles;  // M tiles in the launch (the shared group's last)
    int per_m;    // N tiles per M tile
    int nxcd;     // XCDs dealt to
    int sh_m;     // M tiles of the shared group dealt by N blocks (0: none)
    int sh_nl;    // N tiles per XCD block of the shared group
};

// Items of XCD x.
constexpr int xcd_items(const XcdDeal& d, int x) {
    return (d.m_tiles - d.sh_m - x + d.nxcd - 1) / d.nxcd * d.per_m + d.sh_nl * d.sh_m;
}

// The item of XCD x's li-th draw, li < xcd_items(d, x).
constexpr int xcd_item(const XcdDeal& d, int x, int li) {
    const int ns = d.sh_nl * d.sh_m;
    if (li < ns) return (d.m_tiles - d.sh_m + li % d.sh_m) * d.per_m + x * d.sh_nl + li / d.sh_m;
    li -= ns;
    return (x + d.nxcd * (li / d.per_m)) * d.per_m + li % d.per_m;
}

}  // namespace hf
