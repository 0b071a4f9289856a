// Prints the prefill GEMM pipeline parameters (split_pipeline.h) for every
// configuration the library instantiates: rows swiglu halves cb da db nad nbd
// after_half0 after_half1 lds_bytes a_may_skip; then the wide gate/up tiles'
// line: "wide" nad nwh after w_per_substep(1) w_per_substep(2).
#include <cstdio>

#include "split_pipeline.h"

int main() {
    using namespace hf;
    const int rows_list[] = {192, 256};
    for (int rows : rows_list)
        for (int swiglu = 0; swiglu < 2; ++swiglu)
            for (int h = 1; h <= 2; ++h) {
                const int cb = split_cb(swiglu != 0, rows);
                const int da = split_da(rows, cb, h), db = split_db(rows, cb, h);
                const int nad = rows / 64, nbd = cb;
                std::printf("%d %d %d %d %d %d %d %d %d %d %zu %d\n", rows, swiglu, h, cb, da, db, nad, nbd,
                            split_after(h, da, db, 0, nad, nbd), h == 2 ? split_after(h, da, db, 1, nad, nbd) : -1,
                            split_lds_max(rows, cb), split_a_may_skip(h, da, db, nad, nbd) ? 1 : 0);
            }
    // wide gate/up tiles (160-row M tiles, 32-row weight half-stages):
    // "wide nad nwh after w_per_substep(1) w_per_substep(2)"
    std::printf("wide %d %d %d %d %d\n", (160 / 8 + 7) / 8, 32 / 8, wide_after(32 / 8), wide_w_per_substep(1),
                wide_w_per_substep(2));
    return 0;
}
