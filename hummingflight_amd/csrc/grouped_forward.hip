// grouped_forward.hip -- multi-token MoE layer (batched decode and prefill).
//
// The reference runs one token at a time (glm_forward.cpp:755-811); here all
// T tokens go through the layer together, each expert's weights read once:
//   1. x -> BF16 hi/lo halves (+ a device flag when any lo half is nonzero)
//   2. router logits [T, E] by grouped GEMM with split-K, reduced in fixed order,
//      then score pairs (sigmoid, sigmoid + bias)
//   3. per-token selection (hf_select.h), one block per token
//   4. dispatch: stable counting sort of (token, rank) pairs by expert
//   5. gate/up grouped GEMM over the routed groups plus the shared expert as
//      one more group -> h (BF16 hi/lo, sorted rows)
//   6. down grouped GEMM -> y at each pair's slot [T*k, d], shared rows after
//   7. combine: out[t] = (sum_r w[t,r] * y[t*k + r]) + y[T*k + t]
#include "hf_api_internal.h"
#include "hf_grouped.h"

namespace hf {

static bool grouped_supported() {
    const Cfg& c = g.cfg;
    return c.d % kGemmTileK == 0 && c.I % kGemmTileK == 0 && c.n_shared <= 1;
}

// Split-K factor of the router GEMM: about one (tile, split) item per CU,
// each split at least 4 K stages long.  (At d = 6144, E = 256: T = 4096 in
// 4 splits, router GEMM + split sum 58-61 -> 45-47 us against 8, which gave
// two items per CU; T = 1024 in 16 against 24, 31-32 -> 25-26 us; FP32 x
// alike.)
static int router_ksplit(int T) {
    const Cfg& c = g.cfg;
    const int tiles = ((T + kGemmTileRows - 1) / kGemmTileRows) * ((c.E + 127) / 128);
    const int kmax = c.d / kGemmTileK;
    const int want = (g.num_cus + tiles - 1) / tiles;
    int best = 1;
    for (int ks = 1; ks <= kmax / 4 && ks <= want; ++ks)
        if (kmax % ks == 0) best = ks;
    return best;
}

// Persistent grid: two 4-wave workgroups per CU (128-row tiles) or one
// workgroup per CU (larger tiles).
int gemm_blocks(int tile_rows) {
    return env_int("HFMOE_GEMM_BLOCKS", tile_rows == kGemmTileRows ? g.num_cus * 2 : g.num_cus);
}

// Prefill tiles (192 rows; the wide tiles' own list 160) once experts
// average 4+ rows (HFMOE_PREFILL_MIN_ROWS): an expert's rows then mostly fit
// one tile, its weights stream through the memory system once, and each
// activation row is requested once per 512 weight rows (the wide tiles; 256
// or 384 on the split tiles).  Measured at full shape (256 experts top-8,
// near-uniform routing): from 3 to 6 rows per expert the 128-row kernel
// (whose wavefronts skip the row blocks a group does not fill) and the
// prefill tiles are even; from 7 on the prefill tiles win by more the more
// rows an expert has (T = 224: +4.5 %, 512: +15 %, 1024: +30 %, 2048: +39 %,
// 2560: +34 % tokens/s).  Batched decode with skewed popularity (T = 64,
// Zipf) stays on the 128-row kernel.
static int expert_tile_rows(int T) {
    const Cfg& c = g.cfg;
    const int min_rows = env_int("HFMOE_PREFILL_MIN_ROWS", 4);
    return (size_t)T * c.k >= (size_t)min_rows * c.E ? kPrefillTileRows : kGemmTileRows;
}

void grouped_workspace_free() {
    GroupedWorkspace& w = g.gws;
    void* ptrs[] = {w.counts, w.offsets, w.perm, w.row_token, w.tile_expert, w.tile_row0, w.ntiles,
                    w.tile_expert_gu, w.tile_row0_gu, w.chunk_hist, w.item_ctr, w.lo_flag, w.xh, w.xl, w.hh, w.hl, w.y, w.part};
    for (void* p : ptrs)
        if (p) hipFree(p);
    w = GroupedWorkspace{};
}

int grouped_workspace_alloc() {
    grouped_workspace_free();
    const Cfg& c = g.cfg;
    const int T = g.max_tokens;
    if (T <= 1 || !grouped_supported()) return HFMOE_OK;
    GroupedWorkspace& w = g.gws;
    // Sorted rows: T*k routed (token, rank) pairs, then T shared-expert rows.
    const size_t R = (size_t)T * c.k + (size_t)T * c.n_shared;
    w.max_tiles = c.E + 1 + (int)(((size_t)T * c.k + kGemmTileRows - 1) / kGemmTileRows) +
                  (T + kGemmTileRows - 1) / kGemmTileRows;
    size_t tks = 0;
    for (int t = 2; t <= T; ++t) tks = std::max(tks, (size_t)t * router_ksplit(t));
    struct A {
        void** p;
        size_t bytes;
    } list[] = {
        {(void**)&w.counts, sizeof(int) * c.E},
        {(void**)&w.offsets, sizeof(int) * (c.E + 2)},
        {(void**)&w.perm, sizeof(int) * R},
        {(void**)&w.row_token, sizeof(int) * R},
        {(void**)&w.tile_expert, sizeof(int) * w.max_tiles},
        {(void**)&w.tile_row0, sizeof(int) * w.max_tiles},
        {(void**)&w.ntiles, 256},
        {(void**)&w.tile_expert_gu, sizeof(int) * w.max_tiles},
        {(void**)&w.tile_row0_gu, sizeof(int) * w.max_tiles},
        {(void**)&w.chunk_hist, sizeof(int) * (size_t)kDispatchMaxChunks * c.E},
        {(void**)&w.item_ctr, sizeof(unsigned) * kItemCounters},
        {(void**)&w.lo_flag, 256},
        {(void**)&w.xh, 2 * (size_t)T * c.d},
        {(void**)&w.xl, 2 * (size_t)T * c.d},
        {(void**)&w.hh, 2 * R * c.I},
        {(void**)&w.hl, 2 * R * c.I},
        {(void**)&w.y, 4 * R * c.d},
        {(void**)&w.part, 4 * tks * c.E},
    };
    for (auto& a : list) {
        hipError_t e = hipMalloc(a.p, a.bytes);
        if (e != hipSuccess) {
            grouped_workspace_free();
            return fail(HFMOE_ERR_OUT_OF_MEMORY, "multi-token workspace (%zu bytes): %s", a.bytes,
                        hipGetErrorString(e));
        }
    }
    return HFMOE_OK;
}

#define HF_CHECK_LAUNCH(expr, what)                      \
    do {                                                 \
        hipError_t e_ = (expr);                          \
        prof_end(p, s);                                  \
        if (e_ != hipSuccess) return fail_hip(e_, what); \
    } while (0)

int grouped_tile_rows(int T) { return expert_tile_rows(T); }

// The prefill gate/up GEMM takes the wide tiles (512 weight rows, 256
// outputs of h; 192 rows, or 160 from a second tile list when x has a lo
// half) when the intermediate size is a multiple of 256, unless
// HFMOE_PREFILL_WIDE=0 (192 x 256 tiles, and 192 x 384 for the down
// projection, which otherwise takes 160 x 512 tiles from the second list
// when hidden is a multiple of 512).
static bool prefill_wide(int TR) {
    return TR == kPrefillTileRows && g.cfg.I % (kWideTileCols / 2) == 0 && env_int("HFMOE_PREFILL_WIDE", 1) != 0;
}

int grouped_route(LayerState& L, const float* x, int T, hipStream_t s) {
    const Cfg& c = g.cfg;
    GroupedWorkspace& w = g.gws;
    const int shared_rows = c.n_shared > 0 ? T : 0;
    const int TR = expert_tile_rows(T);
    Pending p;

    prof_begin(p, "split_x", s);
    HF_CHECK_LAUNCH(launch_split_bf16(x, w.xh, w.xl, (size_t)T * c.d, w.lo_flag, s), "split x");

    const int ks = router_ksplit(T);
    GemmArgs r{};
    r.K = c.d;
    r.N = c.E;
    r.tile_rows = kGemmTileRows;
    r.tile_cols = 128;
    r.n_tiles = (c.E + 127) / 128;
    r.m_tiles = (T + kGemmTileRows - 1) / kGemmTileRows;
    r.rows_total = T;
    r.a_hi = w.xh;
    r.a_lo = w.xl;
    r.a_lo_flag = w.lo_flag;
    r.b_fixed0 = L.dev.router;
    r.b_ld = c.d;
    r.out_f32 = w.part;
    r.ksplit = ks;
    prof_begin(p, "router_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_PARTIAL, r, gemm_blocks(kGemmTileRows), s), "router gemm");
    prof_begin(p, "router_reduce", s);
    HF_CHECK_LAUNCH(launch_router_reduce(w.part, ks, T, c.E, L.dev.bias, g.ws.logits, g.ws.scores, s),
                    "router reduce");
    prof_begin(p, "select", s);
    HF_CHECK_LAUNCH(launch_select(g.ws.scores, T, c, g.ws.idx, g.ws.wts, s), "select");
    prof_begin(p, "dispatch", s);
    TileList tl{TR, w.tile_expert, w.tile_row0, w.ntiles}, tl_gu{};
    w.wide = prefill_wide(TR);
    if (w.wide) tl_gu = TileList{kWideTileRows, w.tile_expert_gu, w.tile_row0_gu, w.ntiles_wide()};
    HF_CHECK_LAUNCH(launch_dispatch(g.ws.idx, T, c.k, c.E, tl, tl_gu, shared_rows, w.counts, w.offsets, w.perm,
                                    w.row_token, w.chunk_hist, TR == kPrefillTileRows ? w.item_ctr : nullptr, s),
                    "dispatch");
    return HFMOE_OK;
}

int grouped_experts(const uint16_t* const* etab, int T, hipStream_t s) {
    const Cfg& c = g.cfg;
    GroupedWorkspace& w = g.gws;
    const int P = T * c.k;
    const int shared_rows = c.n_shared > 0 ? T : 0;
    const int TR = expert_tile_rows(T);
    Pending p;

    // Gate/up of every group: the routed experts' (token, rank) rows and the
    // shared expert's token rows (group E), one launch.  The wide tiles when
    // the dispatch of this batch wrote their tile list.
    const bool wide = w.wide && TR == kPrefillTileRows;
    GemmArgs gu{};
    gu.K = c.d;
    gu.N = c.I;
    gu.tile_rows = TR;
    gu.tile_cols = gemm_tile_cols(TR, EPI_SWIGLU, c.I, wide);
    gu.n_tiles = gemm_n_tiles(EPI_SWIGLU, c.I, gu.tile_cols);
    gu.tile_group = w.tile_expert;
    gu.tile_row0 = w.tile_row0;
    gu.ntiles_dev = w.ntiles;
    if (wide) {  // x with a lo half: the 160-row tiles
        gu.lo_tiles.group = w.tile_expert_gu;
        gu.lo_tiles.row0 = w.tile_row0_gu;
        gu.lo_tiles.count = w.ntiles_wide();
        gu.lo_tiles.shared_mtiles = (shared_rows + kWideTileRows - 1) / kWideTileRows;
    }
    gu.group_end = w.offsets + 1;
    gu.rows_total = P + shared_rows;
    gu.a_hi = w.xh;
    gu.a_lo = w.xl;
    gu.a_lo_flag = w.lo_flag;
    gu.a_rowmap = w.row_token;
    gu.b_tab = etab;
    gu.b_which = 0;
    gu.b_ld = c.d;
    gu.h_hi = w.hh;
    gu.h_lo = w.hl;
    gu.ksplit = 1;
    gu.item_ctr = TR == kPrefillTileRows ? w.item_ctr : nullptr;  // short batched items: static
    gu.shared_mtiles = (shared_rows + TR - 1) / TR;
    // h goes to the down projection exact, as BF16 hi + lo halves (about 16
    // significand bits).  FP16 h (11 bits) was measured at 0.61 of the
    // 2e-3 + 1e-2 tolerance over a full-shape prefill with near-uniform
    // routing weights and past it (1.1-1.7) with a trained router's spread of
    // weights or larger activations; the hi / lo halves stay at ~0.01-0.03.
    prof_begin(p, "expert_gateup_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SWIGLU, gu, gemm_blocks(TR), s), "gate/up gemm");

    // Down projections of every group; row r's output lands at row perm[r] of
    // y: pair slot t*k + r for routed rows, T*k + t for the shared expert.
    // The wide down tiles (160 rows x 512 weight rows, on the gate/up's
    // 160-row list) when hidden is a multiple of 512, unless
    // HFMOE_DOWN_WIDE=0 (192 x 384).
    const bool dn_wide = wide && c.d % kWideTileCols == 0 && env_int("HFMOE_DOWN_WIDE", 1) != 0;
    GemmArgs dn{};
    dn.K = c.I;
    dn.N = c.d;
    dn.tile_rows = dn_wide ? kWideTileRows : TR;
    dn.tile_cols = dn_wide ? kWideTileCols : gemm_tile_cols(TR, EPI_SCATTER);
    dn.n_tiles = gemm_n_tiles(EPI_SCATTER, c.d, dn.tile_cols);
    dn.tile_group = dn_wide ? w.tile_expert_gu : w.tile_expert;
    dn.tile_row0 = dn_wide ? w.tile_row0_gu : w.tile_row0;
    dn.ntiles_dev = dn_wide ? w.ntiles_wide() : w.ntiles;
    dn.group_end = w.offsets + 1;
    dn.rows_total = P + shared_rows;
    dn.a_hi = w.hh;
    dn.a_lo = w.hl;
    dn.b_tab = etab;
    dn.b_which = 2;
    dn.b_ld = c.I;
    dn.out_f32 = w.y;
    dn.scatter_rows = w.perm;
    dn.ksplit = 1;
    dn.item_ctr = TR == kPrefillTileRows ? w.item_ctr + kItemCounters / 2 : nullptr;
    dn.shared_mtiles = dn_wide ? (shared_rows + kWideTileRows - 1) / kWideTileRows : gu.shared_mtiles;
    prof_begin(p, "expert_down_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SCATTER, dn, gemm_blocks(TR), s), "down gemm");
    return HFMOE_OK;
}

int grouped_combine(int T, float* out, hipStream_t s) {
    const Cfg& c = g.cfg;
    const int P = T * c.k;
    Pending p;
    prof_begin(p, "combine", s);
    HF_CHECK_LAUNCH(launch_combine(g.ws.wts, g.gws.y, T, c.k, c.d, c.n_shared > 0 ? P : -1, out, s), "combine");
    return HFMOE_OK;
}

int forward_grouped(LayerState& L, const float* x, int T, float* out, hipStream_t s,
                    const hfmoe_route_debug* dbg) {
    if (!g.gws.xh) return forward_tokenwise(L, x, T, out, s, dbg);
    int rc = grouped_route(L, x, T, s);
    if (!rc) rc = grouped_experts(L.dev.etab, T, s);
    if (!rc) rc = grouped_combine(T, out, s);
    return rc ? rc : copy_debug(dbg, T, s);
}

}  // namespace hf
