// split_pipeline.h -- prefetch depths, LDS sizes and wait counts of the
// prefill grouped GEMMs' DMA rings (grouped_gemm_split_kernel, and the wait
// counts of grouped_gemm_wide_kernel at the end).  Plain constexpr C++ so a
// host build can check the wait counts against a brute-force count of the
// issue sequence.
//
// Per item, sub-step j = H * s + half multiplies A half `half` (H = 2 when the
// activations carry a lo half) of K stage s against B stage s.  A is DA
// sub-steps and B is DB K stages ahead; the rings hold DA + 1 A stages
// (ROWS x 64 BF16 each) and DB + 1 B stages (64 * CB weight rows x 64 BF16).
#pragma once

#include <cstddef>

namespace hf {

// Column blocks per wavefront: 256-row tiles 4; 192-row tiles 6 for outputs
// of plain rows (384 weight rows) and 4 for gate/up, which leaves LDS for
// weights two stages ahead.
constexpr int split_cb(bool swiglu, int rows) { return rows == 256 || swiglu ? 4 : 6; }
constexpr int split_da(int rows, int cb, int h) { return rows == 256 && h == 2 ? 2 : 1; }
constexpr int split_db(int rows, int cb, int h) { return cb == 6 || (rows == 256 && h == 2) ? 1 : 2; }
constexpr size_t split_lds(int rows, int cb, int h) {
    return 2 * ((size_t)(split_da(rows, cb, h) + 1) * rows * 64 + (size_t)(split_db(rows, cb, h) + 1) * 64 * cb * 64);
}
constexpr size_t split_lds_max(int rows, int cb) {
    return split_lds(rows, cb, 1) > split_lds(rows, cb, 2) ? split_lds(rows, cb, 1) : split_lds(rows, cb, 2);
}

// DMA instructions a wavefront may leave outstanding at sub-step j (half =
// j % H) once A(j) and B(j / H) have landed, in the steady issue pattern
// "sub-step q issues A(q + DA), then B(q / H + DB) when q % H == 0" (loads
// complete in issue order): those issued after the later of the two.  NAD /
// NBD: DMA instructions per A / B stage per wavefront.
constexpr int split_after(int H, int DA, int DB, int half, int NAD, int NBD) {
    const int s0 = 16;  // any stage past the prologue
    const int j = s0 * H + half;
    const int pa = j - DA;         // A(j): first op of sub-step pa
    const int pb = H * (s0 - DB);  // B(s0): second op of sub-step pb
    int n = 0, p = 0;
    if (pa > pb) {
        p = pa;
        if (p % H == 0) n += NBD;  // that sub-step's B follows A(j)
    } else {
        p = pb;
    }
    for (int q = p + 1; q < j; ++q) n += NAD + (q % H == 0 ? NBD : 0);
    return n;
}

// True when no wait count includes A instructions: then a wavefront may issue
// fewer than NAD per A stage (the tile's unused rows) and every wait still
// covers the loads it guards.
constexpr bool split_a_may_skip(int H, int DA, int DB, int NAD, int NBD) {
    for (int half = 0; half < H; ++half)
        if (split_after(H, DA, DB, half, NAD, NBD) != split_after(H, DA, DB, half, 0, NBD)) return false;
    return true;
}

// Wide gate/up tiles (grouped_gemm_wide_kernel): per wavefront, a prologue
// issues A(0) and weight half-stages 0, 1, 2; sub-step j = H*s + half waits,
// meets the workgroup at a barrier, issues A(j + 1) (0 .. NAD DMA
// instructions: the item's used rows) and weight half-stages
// 2s + 3 + half, ... (wide_w_per_substep(H) of them, NWH DMAs each: both on a
// one-half stage, one per sub-step of a two-half stage); loads past the item
// issue nothing.  The first sub-step of stage s needs A(j) and half-stages 2s
// and 2s + 1, whose fragments it keeps in registers for a second sub-step,
// which needs A(j) only.  Steady count of DMA instructions a sub-step may
// leave outstanding (the last weight half-stage issued before it):
constexpr int wide_after(int nwh) { return nwh; }
constexpr int wide_w_per_substep(int halves) { return 2 / halves; }
// ... valid while the loads it assumes were issued (half-stage 2s + 2, or
// 2s + 3 for a second sub-step, exists); otherwise the sub-step waits for
// everything.
constexpr bool wide_steady(int s, int nk) { return s + 1 < nk; }

}  // namespace hf
