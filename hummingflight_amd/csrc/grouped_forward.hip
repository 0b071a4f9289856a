// grouped_forward.hip -- multi-token MoE layer (batched decode and prefill).
//
// The reference runs one token at a time (glm_forward.cpp:755-811); here all
// T tokens go through the layer together, each expert's weights read once:
//   1. x -> BF16 hi/lo halves (+ a device flag when any lo half is nonzero)
//   2. router logits [T, E] by grouped GEMM with split-K, reduced in fixed order,
//      then score pairs (sigmoid, sigmoid + bias)
//   3. per-token selection (hf_select.h), one block per token
//   4. dispatch: stable counting sort of (token, rank) pairs by expert
//   5. routed gate/up grouped GEMM -> h (BF16 hi/lo, sorted rows)
//   6. shared-expert gate/up GEMM over all tokens -> shared h
//   7. routed down grouped GEMM -> y at each pair's slot [T*k, d]
//   8. shared down GEMM fused with the combine: out[t] = sum_r w*y + shared
#include "hf_api_internal.h"
#include "hf_grouped.h"

namespace hf {

static bool grouped_supported() {
    const Cfg& c = g.cfg;
    return c.d % 32 == 0 && c.I % 32 == 0;
}

// Split-K factor of the router GEMM: enough (tile, split) items for every CU.
static int router_ksplit(int T) {
    const Cfg& c = g.cfg;
    const int tiles = ((T + kGemmTileRows - 1) / kGemmTileRows) * ((c.E + 127) / 128);
    const int kmax = c.d / 32;
    const int want = (2 * g.num_cus + tiles - 1) / tiles;
    int best = 1;
    for (int ks = 1; ks <= kmax && ks <= want; ++ks)
        if (kmax % ks == 0) best = ks;
    return best;
}

static int gemm_blocks() { return env_int("HFMOE_GEMM_BLOCKS", g.num_cus * 2); }

void grouped_workspace_free() {
    GroupedWorkspace& w = g.gws;
    void* ptrs[] = {w.counts, w.offsets, w.perm, w.row_token, w.tile_expert, w.tile_row0, w.ntiles,
                    w.lo_flag, w.xh, w.xl, w.hh, w.hl, w.y, w.shh, w.shl, w.part};
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
    const size_t P = (size_t)T * c.k;
    const size_t Is = (size_t)c.n_shared * c.I;
    w.max_tiles = c.E + (int)((P + kGemmTileRows - 1) / kGemmTileRows);
    size_t tks = 0;
    for (int t = 2; t <= T; ++t) tks = std::max(tks, (size_t)t * router_ksplit(t));
    struct A {
        void** p;
        size_t bytes;
    } list[] = {
        {(void**)&w.counts, sizeof(int) * c.E},
        {(void**)&w.offsets, sizeof(int) * (c.E + 1)},
        {(void**)&w.perm, sizeof(int) * P},
        {(void**)&w.row_token, sizeof(int) * P},
        {(void**)&w.tile_expert, sizeof(int) * w.max_tiles},
        {(void**)&w.tile_row0, sizeof(int) * w.max_tiles},
        {(void**)&w.ntiles, 256},
        {(void**)&w.lo_flag, 256},
        {(void**)&w.xh, 2 * (size_t)T * c.d},
        {(void**)&w.xl, 2 * (size_t)T * c.d},
        {(void**)&w.hh, 2 * P * c.I},
        {(void**)&w.hl, 2 * P * c.I},
        {(void**)&w.y, 4 * P * c.d},
        {(void**)&w.shh, 2 * (size_t)T * (Is ? Is : 1)},
        {(void**)&w.shl, 2 * (size_t)T * (Is ? Is : 1)},
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

// out[t] = sum_r w[t, r] * y[t*k + r] when there is no shared expert to fuse with.
__global__ void combine_kernel(const float* __restrict__ wts, const float* __restrict__ y, int T,
                               int k, int d, float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * d) return;
    const size_t t = i / d, n = i % d;
    float moe = 0.0f;
    for (int r = 0; r < k; ++r) moe += wts[t * k + r] * y[(t * k + r) * d + n];
    out[i] = moe;
}

#define HF_CHECK_LAUNCH(expr, what)                  \
    do {                                             \
        hipError_t e_ = (expr);                      \
        prof_end(p, s);                              \
        if (e_ != hipSuccess) return fail_hip(e_, what); \
    } while (0)

int forward_grouped(LayerState& L, const float* x, int T, float* out, hipStream_t s,
                    const hfmoe_route_debug* dbg) {
    if (!g.gws.xh) return forward_tokenwise(L, x, T, out, s, dbg);
    const Cfg& c = g.cfg;
    GroupedWorkspace& w = g.gws;
    const int Is = c.n_shared * c.I;
    const int blocks = gemm_blocks();
    Pending p;

    prof_begin(p, "split_x", s);
    HF_CHECK_LAUNCH(launch_split_bf16(x, w.xh, w.xl, (size_t)T * c.d, w.lo_flag, s), "split x");

    const int ks = router_ksplit(T);
    GemmArgs r{};
    r.K = c.d;
    r.N = c.E;
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
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_PARTIAL, r, blocks, s), "router gemm");
    prof_begin(p, "router_reduce", s);
    HF_CHECK_LAUNCH(launch_router_reduce(w.part, ks, T, c.E, L.dev.bias, g.ws.logits, g.ws.scores, s),
                    "router reduce");
    prof_begin(p, "select", s);
    HF_CHECK_LAUNCH(launch_select(g.ws.scores, T, c, g.ws.idx, g.ws.wts, s), "select");
    prof_begin(p, "dispatch", s);
    HF_CHECK_LAUNCH(launch_dispatch(g.ws.idx, T, c.k, c.E, kGemmTileRows, w.counts, w.offsets, w.perm,
                                    w.row_token, w.tile_expert, w.tile_row0, w.ntiles, s),
                    "dispatch");

    GemmArgs gu{};
    gu.K = c.d;
    gu.N = c.I;
    gu.n_tiles = (c.I + 63) / 64;
    gu.tile_group = w.tile_expert;
    gu.tile_row0 = w.tile_row0;
    gu.ntiles_dev = w.ntiles;
    gu.group_end = w.offsets + 1;
    gu.rows_total = T * c.k;
    gu.a_hi = w.xh;
    gu.a_lo = w.xl;
    gu.a_lo_flag = w.lo_flag;
    gu.a_rowmap = w.row_token;
    gu.b_tab = L.dev.etab;
    gu.b_which = 0;
    gu.b_ld = c.d;
    gu.h_hi = w.hh;
    gu.h_lo = w.hl;
    gu.ksplit = 1;
    prof_begin(p, "expert_gateup_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SWIGLU, gu, blocks, s), "routed gate/up gemm");

    if (c.n_shared > 0) {
        GemmArgs sg{};
        sg.K = c.d;
        sg.N = Is;
        sg.n_tiles = (Is + 63) / 64;
        sg.m_tiles = (T + kGemmTileRows - 1) / kGemmTileRows;
        sg.rows_total = T;
        sg.a_hi = w.xh;
        sg.a_lo = w.xl;
        sg.a_lo_flag = w.lo_flag;
        sg.b_fixed0 = L.dev.sg;
        sg.b_fixed1 = L.dev.su;
        sg.b_ld = c.d;
        sg.h_hi = w.shh;
        sg.h_lo = w.shl;
        sg.ksplit = 1;
        prof_begin(p, "shared_gateup_gemm", s);
        HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SWIGLU, sg, blocks, s), "shared gate/up gemm");
    }

    GemmArgs dn{};
    dn.K = c.I;
    dn.N = c.d;
    dn.n_tiles = (c.d + 127) / 128;
    dn.tile_group = w.tile_expert;
    dn.tile_row0 = w.tile_row0;
    dn.ntiles_dev = w.ntiles;
    dn.group_end = w.offsets + 1;
    dn.rows_total = T * c.k;
    dn.a_hi = w.hh;
    dn.a_lo = w.hl;
    dn.b_tab = L.dev.etab;
    dn.b_which = 2;
    dn.b_ld = c.I;
    dn.out_f32 = w.y;
    dn.scatter_rows = w.perm;
    dn.ksplit = 1;
    prof_begin(p, "expert_down_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_SCATTER, dn, blocks, s), "routed down gemm");

    if (c.n_shared > 0) {
        GemmArgs sd{};
        sd.K = Is;
        sd.N = c.d;
        sd.n_tiles = (c.d + 127) / 128;
        sd.m_tiles = (T + kGemmTileRows - 1) / kGemmTileRows;
        sd.rows_total = T;
        sd.a_hi = w.shh;
        sd.a_lo = w.shl;
        sd.b_fixed0 = L.dev.sd;
        sd.b_ld = Is;
        sd.out_f32 = out;
        sd.comb_w = g.ws.wts;
        sd.comb_y = w.y;
        sd.comb_k = c.k;
        sd.ksplit = 1;
        prof_begin(p, "shared_down_combine_gemm", s);
        HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_COMBINE, sd, blocks, s), "shared down + combine gemm");
    } else {
        const size_t n = (size_t)T * c.d;
        prof_begin(p, "combine", s);
        HF_CHECK_LAUNCH(launch(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                               g.ws.wts, w.y, T, c.k, c.d, out),
                        "combine");
    }
    return copy_debug(dbg, T, s);
}

}  // namespace hf
