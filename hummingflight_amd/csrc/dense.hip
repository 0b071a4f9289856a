// dense.hip -- the dense MLP layers (GLMForward::denseMlp, glm_forward.cpp:410-432).
//
// out = Wd . (silu(Wg . x) * (Wu . x)) with the dense intermediate size
// (intermediateSize, config.h:16; 12288 at GLM-5.2 against 2048 per routed
// expert).  The matrices are the same [out, in] BF16 layout as an expert's,
// so
//   T = 1:  the decode GEMVs multiply them as a "shared expert" of
//           inter / slice slices (the down GEMV sums the slices' partial
//           products in a fixed order), no routed slots;
//   T > 1:  the grouped GEMM multiplies every token row by the one weight set
//           (one group, no dispatch): gate/up with the SwiGLU epilogue into
//           h (BF16 hi + lo) -- for a short prompt split over K into FP32
//           gate / up partials, the SwiGLU then applied to their sums by a
//           small kernel -- then down straight into out.  h stays exact to
//           ~16 bits, as in the MoE layer: the dense down projection sums
//           12288 terms with weight 1, and an FP16 h moves its outputs by up
//           to ~4e-3 at hidden 6144, past the 2e-3 absolute tolerance.
#include "hf_api_internal.h"
#include "hf_grouped.h"

namespace hf {

void dense_workspace_free() {
    DenseWorkspace& w = g.dws;
    for (void* p : {(void*)w.h1, (void*)w.hh, (void*)w.hl, (void*)w.part, (void*)w.gu_part})
        if (p) hipFree(p);
    w = DenseWorkspace{};
}

// K splits of a short prompt's gate/up GEMM on the 256-row tiles (FP32 gate
// and up partials, then the SwiGLU in swiglu_splits_kernel).  One M tile has
// only 2 I / 256 items (96 at GLM-5.2's 12288) for 256 workgroups; two
// splits measured at 6144 x 12288 (two MI355X machines): T = 256 0.283-0.293 ->
// 0.234-0.246 ms, 192 0.241 -> 0.209, 160 0.221 -> 0.190, 128 0.180-0.188 ->
// 0.175-0.181, 64 0.130-0.140 -> 0.128-0.130 (the 128-row kernel unsplit
// before); at T <= 32 even or slower (-3 % to +8 % by machine), from two M tiles
// (T = 384, 512) 6-7 % slower; three, four or eight splits slower than two
// (288 / 384 / 768 items take two or three rounds of 256 workgroups).
static int dense_gu_ksplit_auto(int T) { return T >= 64 && T <= kDenseTileRows ? 2 : 1; }

static int dense_workspace_reserve(int inter) {
    DenseWorkspace& w = g.dws;
    const int tokens = g.max_tokens > 1 && g.gws.xh ? g.max_tokens : 0;
    if (inter <= w.inter && tokens <= w.tokens) return HFMOE_OK;
    dense_workspace_free();
    hipError_t e = hipMalloc(&w.h1, sizeof(float) * (size_t)inter);
    if (e == hipSuccess && tokens) e = hipMalloc(&w.hh, 2 * (size_t)tokens * inter);
    if (e == hipSuccess && tokens) e = hipMalloc(&w.hl, 2 * (size_t)tokens * inter);
    // Partials for up to 8 K splits of a short prompt (one M tile leaves the
    // down projection 24 items), 2 of a long one.
    const int part_rows = std::max(2 * tokens, std::min(8 * tokens, 4096));
    if (e == hipSuccess && tokens) e = hipMalloc(&w.part, sizeof(float) * (size_t)part_rows * g.cfg.d);
    int gu_part_rows = 0;
    for (int t = 2; t <= tokens; ++t) gu_part_rows = std::max(gu_part_rows, t * dense_gu_ksplit_auto(t));
    if (e == hipSuccess && gu_part_rows > 0)
        e = hipMalloc(&w.gu_part, sizeof(float) * (size_t)gu_part_rows * 2 * inter);
    if (e != hipSuccess) {
        dense_workspace_free();
        return fail(HFMOE_ERR_OUT_OF_MEMORY, "dense MLP workspace (inter %d, %d tokens): %s", inter, tokens,
                    hipGetErrorString(e));
    }
    w.inter = inter;
    w.tokens = tokens;
    w.part_rows = tokens ? part_rows : 0;
    w.gu_part_rows = gu_part_rows;
    return HFMOE_OK;
}

// HFMOE_DENSE_GU_KSPLIT (1..8) overrides the choice; either only within the
// partials' workspace (sized for the automatic choice at every T up to
// max_tokens), with whole 64-wide K stages per split and tiles that do not
// straddle the gate / up boundary.
static int dense_gu_ksplit(int T, int I, int stages) {
    const DenseWorkspace& w = g.dws;
    const int want = env_int("HFMOE_DENSE_GU_KSPLIT", dense_gu_ksplit_auto(T));
    if (want <= 1 || want > 8 || (size_t)want * T > (size_t)w.gu_part_rows || stages % want ||
        I % gemm_tile_cols(kDenseTileRows, EPI_PARTIAL))
        return 1;
    return want;
}

// Slice rows for the decode kernels: the routed expert size when it divides
// inter, else the largest divisor of inter that is a multiple of 8 and at
// most 4096, with at most kMaxSlots slices.
static int dense_slice(int inter) {
    const int I = g.cfg.I;
    if (inter % I == 0 && inter / I <= kMaxSlots) return I;
    for (int n = (inter + 4095) / 4096; n <= kMaxSlots; ++n)
        if (inter % n == 0 && (inter / n) % 8 == 0) return inter / n;
    return 0;
}

// K splits of the down projection (both tile kinds take their items
// statically here): the fewest splits that minimise the rounds of items
// per workgroup, counted in whole-K item times (384 items on 256 workgroups:
// two rounds of whole items, against three of half items with two splits),
// each split a whole number of 64-wide K stages and the partials
// ([splits, T, hidden] FP32) within the workspace's part_rows.
static int dense_down_ksplit(int items, int stages, int T, int blocks) {
    int best = 1;
    double best_rounds = (double)((items + blocks - 1) / blocks);
    for (int k = 2; k <= 8; ++k) {
        if (stages % k || (size_t)k * T > (size_t)g.dws.part_rows) continue;
        const double rounds = (double)(((size_t)items * k + blocks - 1) / blocks) / k;
        if (rounds < best_rounds - 1e-9) {
            best = k;
            best_rounds = rounds;
        }
    }
    return best;
}

#define HF_CHECK_LAUNCH(expr, what)                      \
    do {                                                 \
        hipError_t e_ = (expr);                          \
        prof_end(p, s);                                  \
        if (e_ != hipSuccess) return fail_hip(e_, what); \
    } while (0)

int dense_forward(LayerState& L, const float* x, int T, float* out, hipStream_t s) {
    const Cfg& c = g.cfg;
    DenseWorkspace& w = g.dws;
    Pending p;
    const bool gemm = T > 1 && w.hh && c.d % kGemmTileK == 0 && L.dense_inter % kGemmTileK == 0;
    if (!gemm) {
        Cfg cd = c;
        cd.k = 0;
        cd.I = L.dense_slice;
        cd.n_shared = L.dense_inter / L.dense_slice;
        for (int t = 0; t < T; ++t) {
            const float* xt = x + (size_t)t * c.d;
            float* ot = out + (size_t)t * c.d;
            prof_begin(p, "dense_gateup", s);
            HF_CHECK_LAUNCH(launch_gateup_t1(xt, L.dev, cd, nullptr, nullptr, nullptr, w.h1, cd.n_shared,
                                             gu_blocks(), s),
                            "dense gate/up launch");
            prof_begin(p, "dense_down", s);
            HF_CHECK_LAUNCH(launch_down_t1(w.h1, L.dev, cd, nullptr, nullptr, nullptr, ot, cd.n_shared,
                                           dn_blocks(), s),
                            "dense down launch");
        }
        return HFMOE_OK;
    }
    GroupedWorkspace& gw = g.gws;
    // Past one 128-row M tile, the 256-row tiles (HFMOE_DENSE_MIN_TOKENS): a
    // second 128-row M tile streams all the weights again (at 6144 x 12288:
    // T = 129 0.320 against 0.206 ms, 191 0.325 against 0.246), and the
    // 256-row tiles were faster at every T from 256 to 1024; up to 128 tokens
    // the 128-row kernel is (T = 128: 0.188 against 0.201 ms).
    const int TR = T >= env_int("HFMOE_DENSE_MIN_TOKENS", kGemmTileRows + 1) ? kDenseTileRows : kGemmTileRows;
    const int I = L.dense_inter;
    prof_begin(p, "split_x", s);
    HF_CHECK_LAUNCH(launch_split_bf16(x, gw.xh, gw.xl, (size_t)T * c.d, gw.lo_flag, s), "split x");
    GemmArgs gu{};
    gu.K = c.d;
    gu.N = I;
    gu.tile_rows = TR;
    gu.tile_cols = gemm_tile_cols(TR, EPI_SWIGLU);
    gu.n_tiles = gemm_n_tiles(EPI_SWIGLU, I, gu.tile_cols);
    gu.m_tiles = (T + TR - 1) / TR;
    gu.rows_total = T;
    gu.a_hi = gw.xh;
    gu.a_lo = gw.xl;
    gu.a_lo_flag = gw.lo_flag;
    gu.b_fixed0 = L.dev.sg;
    gu.b_fixed1 = L.dev.su;
    gu.b_ld = c.d;
    gu.h_hi = w.hh;
    gu.h_lo = w.hl;
    gu.ksplit = 1;
    // Every M tile multiplies the same weights: the XCDs take blocks of 4 N
    // groups x 2 M groups and walk M fastest, so a weight tile is read once
    // per XCD and round rather than once per M tile, and an activation tile
    // once per round of the XCD's N tiles (measured at T = 4096 against 8 x 1
    // and 2 x 4 blocks).  Items are independent: results are unchanged.
    // HFMOE_DENSE_BY_NTILE=0 deals whole M tiles per XCD instead.  (128-row
    // tiles, at most two M tiles, measured the same either way: 8 x 1 blocks
    // at T = 150 and 191 took gate/up 169-172 us like contiguous ranges.)
    const int by_ntile = TR == kDenseTileRows && env_int("HFMOE_DENSE_BY_NTILE", 1) != 0 ? 4 : 0;
    gu.by_ntile = by_ntile;
    const int gu_ks = dense_gu_ksplit(T, I, c.d / kGemmTileK);
    if (gu_ks > 1) {
        // Gate and up as one [2 I, d] matrix (b_split) on 256-row tiles,
        // FP32 partials per K split, then silu(g) * u and the h split from
        // their sums.
        gu.tile_rows = kDenseTileRows;
        gu.m_tiles = (T + kDenseTileRows - 1) / kDenseTileRows;
        gu.by_ntile = env_int("HFMOE_DENSE_BY_NTILE", 1) != 0 ? 4 : 0;
        gu.N = 2 * I;
        gu.tile_cols = gemm_tile_cols(kDenseTileRows, EPI_PARTIAL);
        gu.n_tiles = gemm_n_tiles(EPI_PARTIAL, 2 * I, gu.tile_cols);
        gu.b_split = I;
        gu.out_f32 = w.gu_part;
        gu.ksplit = gu_ks;
        prof_begin(p, "dense_gateup_gemm", s);
        HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_PARTIAL, gu, gemm_blocks(kDenseTileRows), s), "dense gate/up gemm");
        prof_begin(p, "dense_swiglu", s);
        HF_CHECK_LAUNCH(launch_swiglu_splits(w.gu_part, gu_ks, T, I, w.hh, w.hl, s), "dense gate/up split sum");
    } else {
        prof_begin(p, "dense_gateup_gemm", s);
        HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SWIGLU, gu, gemm_blocks(TR), s), "dense gate/up gemm");
    }
    GemmArgs dn{};
    dn.K = I;
    dn.N = c.d;
    dn.tile_rows = TR;
    dn.tile_cols = gemm_tile_cols(TR, EPI_PARTIAL);
    dn.n_tiles = gemm_n_tiles(EPI_PARTIAL, c.d, dn.tile_cols);
    dn.m_tiles = (T + TR - 1) / TR;
    dn.rows_total = T;
    dn.a_hi = w.hh;
    dn.a_lo = w.hl;
    dn.b_fixed0 = L.dev.sd;
    dn.b_ld = I;
    dn.out_f32 = out;
    // K splits for both tile kinds: one M tile gives the down projection only
    // hidden / 128 (128-row tiles) or hidden / 256 items.
    dn.ksplit = dense_down_ksplit(dn.m_tiles * dn.n_tiles, I / kGemmTileK, T, gemm_blocks(TR));
    if (dn.ksplit > 1) dn.out_f32 = w.part;
    dn.by_ntile = by_ntile;
    prof_begin(p, "dense_down_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_PARTIAL, dn, gemm_blocks(TR), s), "dense down gemm");
    if (dn.ksplit > 1) {
        prof_begin(p, "dense_down_sum", s);
        HF_CHECK_LAUNCH(launch_sum_splits(w.part, dn.ksplit, (size_t)T * c.d, out, s), "dense down split sum");
    }
    return HFMOE_OK;
}

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_register_dense_layer(int layer, const hfmoe_dense_weights* w) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!w || !w->gate_dev || !w->up_dev || !w->down_dev)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: dense gate, up and down weights are required", layer);
    // 16-byte vector and LDS-DMA loads read the three matrices; the norm weight is read per element.
    rc = check_align(layer, "dense gate", w->gate_dev, 16);
    if (!rc) rc = check_align(layer, "dense up", w->up_dev, 16);
    if (!rc) rc = check_align(layer, "dense down", w->down_dev, 16);
    if (!rc) rc = check_align(layer, "post_attention_norm", w->post_attention_norm_dev, 2);
    if (rc) return rc;
    const int inter = w->intermediate;
    const int slice = inter > 0 && inter % 8 == 0 ? dense_slice(inter) : 0;
    if (!slice)
        return fail(HFMOE_ERR_UNSUPPORTED, "layer %d: dense intermediate %d must be a positive multiple of 8 "
                    "splitting into at most %d slices of at most 4096 rows", layer, inter, kMaxSlots);
    if ((size_t)inter * sizeof(float) > 160 * 1024)
        return fail(HFMOE_ERR_UNSUPPORTED, "layer %d: dense intermediate %d FP32 activations exceed LDS", layer, inter);
    rc = dense_workspace_reserve(inter);
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it != g.layers.end() && it->second.etab_dev) hipFree(it->second.etab_dev);
    LayerState st;
    st.dense = true;
    st.dense_inter = inter;
    st.dense_slice = slice;
    st.dev.sg = w->gate_dev;
    st.dev.su = w->up_dev;
    st.dev.sd = w->down_dev;
    st.norm_w = w->post_attention_norm_dev;
    g.layers[layer] = st;
    return HFMOE_OK;
}

int hfmoe_dense_mlp_forward(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream) {
    int rc = require_cfg();
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it == g.layers.end() || !it->second.dense)
        return fail(HFMOE_ERR_NOT_REGISTERED, "layer %d is not a registered dense layer", layer);
    if (T < 0 || T > g.max_tokens)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "T=%d outside 0..max_tokens=%d", T, g.max_tokens);
    if (T == 0) return HFMOE_OK;
    if (!x_dev || !out_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null activation pointer");
    if ((reinterpret_cast<uintptr_t>(x_dev) | reinterpret_cast<uintptr_t>(out_dev)) & 15)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "activations must be 16-byte aligned");
    return dense_forward(it->second, x_dev, T, out_dev, pick_stream(stream));
}

}  // extern "C"
