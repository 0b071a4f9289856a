// hf_grouped.h -- multi-token MoE: dispatch and the BF16 MFMA grouped GEMM.
#pragma once

#include "hf_common.h"

namespace hf {

constexpr int kGemmTileRows = 128;  // M rows per grouped-GEMM tile (kPrefillTileRows at prefill sizes)
// Prefill tiles: 192 rows (a routed expert's rows at T = 4096 in one tile);
// one-group GEMMs (dense layers, LM head) with T >= 192: 256 rows.
constexpr int kPrefillTileRows = 192, kDenseTileRows = 256;
constexpr int kGemmTileK = 64;      // K per pipeline stage (K % (64 * ksplit) == 0)

enum GemmEpi { EPI_PARTIAL = 0, EPI_SWIGLU = 1, EPI_SCATTER = 2 };

// Weight rows per tile of the wide prefill kernel (eight wavefronts of 64
// weight rows, 32 gate + 32 up or 64 down rows, each over all rows of an M
// tile), and the rows of its M tiles when A has a lo half: x in the gate/up
// GEMM (GemmArgs::lo_tiles), h in the down projection.
constexpr int kWideTileCols = 512, kWideTileRows = 160;

// Weight rows per tile for M tiles of tile_rows rows (MoE prefill: gate/up
// 512 with wide = true when the N outputs of h divide into whole wide tiles,
// else 256, i.e. 128 gate + 128 up rows; otherwise 384; one-group GEMMs with
// 256-row tiles: 256), and the N tiles that cover N output columns (a SWIGLU
// tile's weight rows are half gate, half up).
inline int gemm_tile_cols(int tile_rows, int epi, int N = 0, bool wide = false) {
    if (tile_rows == kPrefillTileRows) {
        if (epi == EPI_SWIGLU) return wide && N > 0 && N % (kWideTileCols / 2) == 0 ? kWideTileCols : 256;
        return 384;
    }
    return tile_rows == kDenseTileRows ? 256 : 128;
}
inline int gemm_n_tiles(int epi, int N, int tile_cols) {
    const int cols = epi == EPI_SWIGLU ? tile_cols / 2 : tile_cols;
    return (N + cols - 1) / cols;
}

// Arguments of one grouped GEMM launch (see grouped_gemm.hip).
struct GemmArgs {
    int K;                      // reduction length (multiple of 64 * ksplit)
    int N;                      // output columns (SWIGLU: intermediate rows per matrix)
    int n_tiles;                // ceil(N / output columns per tile); SWIGLU: tile_cols / 2 per tile
    int tile_rows;              // M rows per tile: kGemmTileRows, kPrefillTileRows or kDenseTileRows
    int tile_cols;              // B rows (weight rows) per tile: gemm_tile_cols(tile_rows, epilogue)
    // M tiling: tile i covers rows [tile_row0[i], min(+tile_rows, group_end[tile_group[i]]))
    const int* tile_group;      // null: one group, rows [0, rows_total) in tile_rows-row tiles
    const int* tile_row0;
    const int* ntiles_dev;      // device count of M tiles (null: m_tiles)
    int m_tiles;
    const int* group_end;       // rows of group g end at group_end[g] (null: rows_total)
    int rows_total;
    // A: BF16 rows of length K; row r reads row a_rowmap[r] (or r) of a_hi / a_lo
    const uint16_t* a_hi;
    const uint16_t* a_lo;       // null: no lo half
    const unsigned* a_lo_flag;  // device flag: lo half present (null: use a_lo when given)
    const int* a_rowmap;
    // B: [N, K] rows of group g at b_tab[3g + b_which] (and +1: up for SWIGLU), else fixed
    const uint16_t* const* b_tab;
    int b_which;
    const uint16_t* b_fixed0;
    const uint16_t* b_fixed1;
    int b_ld;                   // B row stride in elements
    // PARTIAL with fixed B on the split kernel's tiles (tile_rows
    // kPrefillTileRows or kDenseTileRows): output columns [b_split, N)
    // multiply rows (column - b_split) of b_fixed1, the columns before them
    // b_fixed0's (a gate / up pair as one [2 I, K] matrix; b_split a multiple
    // of the tile's columns).  0: b_fixed0 only.
    int b_split;
    // epilogue operands
    float* out_f32;             // PARTIAL [ksplit][rows][N]; SCATTER y rows
    uint16_t* h_hi;             // SWIGLU h [rows][N] hi / lo
    uint16_t* h_lo;
    const int* scatter_rows;    // SCATTER: y row of GEMM row r
    int ksplit;                 // split-K factor (PARTIAL only; 1 otherwise)
    unsigned* item_ctr;         // 8 zeroed per-XCD work counters (null: static items; see dynamic_items)
    // Nonzero (one group, statically dealt items): the XCDs split the tiles
    // into by_ntile N groups x (XCDs / by_ntile) M groups, one block each,
    // and walk their block's items with M tiles fastest, so the workgroups of
    // an XCD that share a weight tile stream it together through that XCD's
    // L2.  Groups must divide evenly; else (XCDs) N groups and one M group,
    // when the N tiles divide; else the usual dealing.
    int by_ntile;
    // M tiles of the last group (the shared expert's rows), when the prefill
    // kernel takes dynamic items (item_ctr) with ksplit 1 and n_tiles a
    // multiple of the XCD count: each XCD then takes the items of its block
    // of n_tiles / 8 N tiles over all of these M tiles first, M tiles fastest,
    // so that its workgroups stream each shared weight tile together through
    // the XCD's L2 rather than once per M tile.  0: no such group.
    int shared_mtiles;
    // Wide gate/up tiles (tile_cols kWideTileCols): the M tiles the kernel
    // takes instead when the a_lo_flag is set, kWideTileRows rows each (same
    // groups; shared_mtiles of them the shared expert's).
    struct {
        const int* group;
        const int* row0;
        const int* count;
        int shared_mtiles;
    } lo_tiles;
};

// Groups whose b_tab entry (3g + b_which) is null are skipped.
hipError_t launch_grouped_gemm(int epi, const GemmArgs& a, int blocks, hipStream_t s);
// p[0, n) = 0 by a kernel (graph-capture safe, unlike a memset node).
hipError_t launch_clear_u32(unsigned* p, int n, hipStream_t s);
// out[i] = sum over k < ks of part[k * n + i], in k order (n a multiple of 4).
hipError_t launch_sum_splits(const float* part, int ks, size_t n, float* out, hipStream_t s);
// The SWIGLU epilogue after a gate/up GEMM split over K: part is
// [ks][T][2 I] FP32 (gate columns [0, I), up [I, 2 I)); g and u are the sums
// over the splits in split order, h = silu(g) * u goes out as BF16 hi / lo
// [T][I] (I a multiple of 4).
hipError_t launch_swiglu_splits(const float* part, int ks, int T, int I, uint16_t* h_hi, uint16_t* h_lo,
                                hipStream_t s);
hipError_t launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, size_t n, unsigned* flag,
                             hipStream_t s);
// out[t] = sum_r wts[t, r] * y[t*k + r] (+ y[shared_row0 + t] when shared_row0 >= 0); d % 4 == 0.
hipError_t launch_combine(const float* wts, const float* y, int T, int k, int d, int shared_row0,
                          float* out, hipStream_t s);
hipError_t launch_router_reduce(const float* part, int ksplit, int T, int E, const float* bias,
                                float* logits, float2* scores, hipStream_t s);
// Stable counting sort of the T*k (token, rank) pairs by expert plus the M-tile
// list (tile_rows rows per tile) of the grouped GEMM.  With shared_rows > 0 a
// group E of shared_rows rows (sorted rows T*k + t <- token t) follows the
// experts: the shared expert multiplied in the same launches.  chunk_hist
// ([kDispatchMaxChunks, E] ints, or null) lets large batches count and
// scatter in several workgroups.
// The dispatch also zeroes item_ctr[kItemCounters] (or nothing when null):
// the per-XCD work counters of the gate/up (first 8) and down (last 8)
// grouped GEMMs that follow it.
constexpr int kDispatchMaxChunks = 64;
constexpr int kItemCounters = 16;
// An M-tile list: tile i covers sorted rows [row0[i], +rows) of group
// expert[i] (clipped to the group's end); count[0] tiles in use.
struct TileList {
    int rows = 0;  // rows per tile (0: no list)
    int* expert = nullptr;
    int* row0 = nullptr;
    int* count = nullptr;
};
// tl0: the M tiles of both grouped GEMMs; tl1 (when tl1.rows > 0): a second
// list of the same groups, the wide kernel's tiles for the down projection
// and, when x has a lo half, for the gate/up GEMM (GemmArgs::lo_tiles).
hipError_t launch_dispatch(const int* idx, int T, int k, int E, const TileList& tl0, const TileList& tl1,
                           int shared_rows, int* counts, int* offsets, int* perm, int* row_token, int* chunk_hist,
                           unsigned* item_ctr, hipStream_t s);

}  // namespace hf
