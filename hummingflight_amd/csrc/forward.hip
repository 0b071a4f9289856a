// forward.hip -- MoE-layer orchestration on the device (GLMForward::moeLayer,
// glm_forward.cpp:509-661): router -> selection -> expert SwiGLU -> weighted
// combine + shared expert, all on one stream with no host round trip.
#include "hf_api_internal.h"
#include "hf_select.h"

namespace hf {

// Three 4-wave blocks per CU: at d = 6144 every wavefront owns exactly 6 rows.
int gu_blocks() { return env_int("HFMOE_GU_BLOCKS", g.num_cus * 3); }
// One block (a band of output rows) per CU.
int dn_blocks() { return env_int("HFMOE_DN_BLOCKS", g.num_cus); }

int copy_debug(const hfmoe_route_debug* dbg, int T, hipStream_t s) {
    if (!dbg) return HFMOE_OK;
    const Cfg& c = g.cfg;
    hipError_t e = hipSuccess;
    if (dbg->logits_dev && e == hipSuccess)
        e = hipMemcpyAsync(dbg->logits_dev, g.ws.logits, sizeof(float) * (size_t)T * c.E,
                           hipMemcpyDeviceToDevice, s);
    if (dbg->idx_dev && e == hipSuccess)
        e = hipMemcpyAsync(dbg->idx_dev, g.ws.idx, sizeof(int) * (size_t)T * c.k,
                           hipMemcpyDeviceToDevice, s);
    if (dbg->weight_dev && e == hipSuccess)
        e = hipMemcpyAsync(dbg->weight_dev, g.ws.wts, sizeof(float) * (size_t)T * c.k,
                           hipMemcpyDeviceToDevice, s);
    if (T > 1 && g.gws.offsets) {
        if (dbg->offsets_dev && e == hipSuccess)
            e = hipMemcpyAsync(dbg->offsets_dev, g.gws.offsets, sizeof(int) * (size_t)(c.E + 1),
                               hipMemcpyDeviceToDevice, s);
        if (dbg->perm_dev && e == hipSuccess)
            e = hipMemcpyAsync(dbg->perm_dev, g.gws.perm, sizeof(int) * (size_t)T * c.k,
                               hipMemcpyDeviceToDevice, s);
    }
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "debug copies");
}

int forward_t1_on(LayerState& L, const float* x, float* out, hipStream_t s, const T1Buffers& b, bool profile) {
    const Cfg& c = g.cfg;
    const int nslots = c.k + c.n_shared;
    Pending p;
    auto begin = [&](const char* name) {
        if (profile) prof_begin(p, name, s);
    };
    auto end = [&]() {
        if (profile) prof_end(p, s);
    };
    begin("router");
    hipError_t e = launch_router_logits_t1(x, L.dev, c, b.logits, b.scores, s);
    end();
    if (e != hipSuccess) return fail_hip(e, "router launch");
    // The gate/up kernel routes in place, overlapped with the loads of the
    // shared expert's first rows (HFMOE_FUSE_SELECT=0 runs selection as its own
    // kernel first, for comparison).
    const bool fused = env_int("HFMOE_FUSE_SELECT", 1) != 0;
    if (!fused) {
        begin("select");
        e = launch_select(b.scores, 1, c, b.idx, b.wts, s);
        end();
        if (e != hipSuccess) return fail_hip(e, "select launch");
    }
    begin("expert_gateup");
    e = launch_gateup_t1(x, L.dev, c, fused ? b.scores : nullptr, b.idx, b.wts, b.h, nslots, gu_blocks(), s);
    end();
    if (e != hipSuccess) return fail_hip(e, "gate/up launch");
    begin("expert_down");
    e = launch_down_t1(b.h, L.dev, c, b.idx, b.wts, nullptr, out, nslots, dn_blocks(), s);
    end();
    if (e != hipSuccess) return fail_hip(e, "down launch");
    return HFMOE_OK;
}

int forward_t1(LayerState& L, const float* x, float* out, hipStream_t s, const hfmoe_route_debug* dbg) {
    const T1Buffers b{g.ws.logits, g.ws.scores, g.ws.idx, g.ws.wts, g.ws.h};
    int rc = forward_t1_on(L, x, out, s, b, true);
    return rc ? rc : copy_debug(dbg, 1, s);
}

}  // namespace hf

namespace hf {

// Multi-token forward, token by token over the decode kernels (every token
// re-streams its experts' weights): used for shapes the grouped GEMM does not
// tile (hidden or intermediate not a multiple of 64).
int forward_tokenwise(LayerState& L, const float* x, int T, float* out, hipStream_t s,
                      const hfmoe_route_debug* dbg) {
    const Cfg& c = g.cfg;
    const int nslots = c.k + c.n_shared;
    Pending p;
    prof_begin(p, "router", s);
    hipError_t e = launch_router_logits(x, T, L.dev, c, g.ws.logits, g.ws.scores, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "router launch");
    prof_begin(p, "select", s);
    e = launch_select(g.ws.scores, T, c, g.ws.idx, g.ws.wts, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "select launch");
    for (int t = 0; t < T; ++t) {
        e = launch_gateup_t1(x + (size_t)t * c.d, L.dev, c, nullptr, g.ws.idx + (size_t)t * c.k,
                             nullptr, g.ws.h, nslots, gu_blocks(), s);
        if (e != hipSuccess) return fail_hip(e, "gate/up launch");
        e = launch_down_t1(g.ws.h, L.dev, c, g.ws.idx + (size_t)t * c.k, g.ws.wts + (size_t)t * c.k,
                           nullptr, out + (size_t)t * c.d, nslots, dn_blocks(), s);
        if (e != hipSuccess) return fail_hip(e, "down launch");
    }
    return copy_debug(dbg, T, s);
}

}  // namespace hf
