// streamed.hip -- decode with routed experts resident in pinned host RAM.
//
// The on-device counterpart of the reference's scheduler + GPU staging window
// (Scheduler::getExpertPtr scheduler.cpp:646-741 feeding gpuExpertStage,
// cuda_backend.cpp:395-428, from moeLayer glm_forward.cpp:562-602): only the k
// experts the router selects cross PCIe, into an HBM slot pool that caches
// them (LRU) and, once a layer has routed, receives the experts predicted for
// the next layer ahead of time (Scheduler::onLayerRouterDone,
// scheduler.cpp:238-388).  Slot and prediction decisions: expert_stream_policy.h.
//
// Per call (T = 1), on the caller's stream s and the library's copy stream:
//   s:    router -> D2H of the k selected ids (pinned) -> event `routed`
//   s:    shared expert gate/up + down into shared_out (overlaps the copies)
//   host: wait `routed`; look up each selected expert: a resident slot (or one
//         already being filled by a copy-ahead) is reused, a miss queues three
//         hipMemcpyAsync (gate, up, down) on the copy stream after the slot's
//         previous reader finished, then records `copied`
//   copy: then the copies of the next layer's predicted experts
//   s:    wait every used slot's `copied`, upload the 3k slot pointers, run
//         the routed gate/up and down GEMVs with out = routed sum + shared_out,
//         record each slot's `consumed`.
#include "hf_api_internal.h"

#include <cstring>

namespace hf {

void stream_pool_release() {
    StreamPool& P = g.pool;
    for (auto ev : P.copied)
        if (ev) hipEventDestroy(ev);
    for (auto ev : P.consumed)
        if (ev) hipEventDestroy(ev);
    if (P.routed) hipEventDestroy(P.routed);
    if (P.base) hipFree(P.base);
    if (P.idx_host) hipHostFree(P.idx_host);
    if (P.w_host) hipHostFree(P.w_host);
    if (P.etab_host) hipHostFree(P.etab_host);
    if (P.etab_dev) hipFree(P.etab_dev);
    if (P.iota_dev) hipFree(P.iota_dev);
    if (P.shared_out) hipFree(P.shared_out);
    P = StreamPool{};
}

static int pool_init() {
    StreamPool& P = g.pool;
    if (P.base) return HFMOE_OK;
    const Cfg& c = g.cfg;
    P.slot_bytes = (size_t)6 * c.d * c.I;
    // Slots: the VRAM budget (AdaptiveConfig::vramBudgetBytes) when given,
    // else two layers' worth of selected experts; never fewer than 2k (one
    // layer's selection plus the next layer's copy-ahead).
    int slots = 2 * c.k;
    if (g.vram_budget) slots = (int)std::min<uint64_t>(g.vram_budget / P.slot_bytes, 1 << 20);
    if (slots < 2 * c.k) slots = 2 * c.k;
    hipError_t e = hipMalloc(&P.base, P.slot_bytes * (size_t)slots);
    if (e != hipSuccess)
        return fail(HFMOE_ERR_OUT_OF_MEMORY, "expert staging pool (%d x %zu bytes): %s", slots,
                    P.slot_bytes, hipGetErrorString(e));
    P.slots = slots;
    P.policy.reset(slots);
    P.policy.opt = g.stream_opt;
    P.copied.assign(slots, nullptr);
    P.consumed.assign(slots, nullptr);
    for (int i = 0; i < slots && e == hipSuccess; ++i) {
        e = hipEventCreateWithFlags(&P.copied[i], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&P.consumed[i], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&P.routed, hipEventDisableTiming);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&P.idx_host), sizeof(int) * kMaxTopK, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&P.w_host), sizeof(float) * kMaxTopK, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&P.etab_host), sizeof(void*) * 3 * kMaxTopK, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&P.etab_dev, sizeof(void*) * 3 * kMaxTopK);
    if (e == hipSuccess) e = hipMalloc(&P.iota_dev, sizeof(int) * kMaxTopK);
    if (e == hipSuccess) e = hipMalloc(&P.shared_out, sizeof(float) * c.d);
    if (e == hipSuccess) {
        int iota[kMaxTopK];
        for (int i = 0; i < kMaxTopK; ++i) iota[i] = i;
        e = hipMemcpy(P.iota_dev, iota, sizeof iota, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        stream_pool_release();
        return fail_hip(e, "expert staging pool setup");
    }
    return HFMOE_OK;
}

// Queues expert eid's [gate | up | down] (host) into slot on the copy stream,
// after the last kernel that read the slot.
static int copy_expert(const LayerState& L, int eid, int slot) {
    StreamPool& P = g.pool;
    const size_t proj = (size_t)g.cfg.I * g.cfg.d;
    uint16_t* dst = P.base + (size_t)slot * (P.slot_bytes / 2);
    hipError_t e = hipStreamWaitEvent(g.copy_stream, P.consumed[slot], 0);
    for (int q = 0; q < 3 && e == hipSuccess; ++q)
        e = hipMemcpyAsync(dst + q * proj, L.host_experts[3 * eid + q], proj * 2, hipMemcpyHostToDevice,
                           g.copy_stream);
    if (e == hipSuccess) e = hipEventRecord(P.copied[slot], g.copy_stream);
    if (e != hipSuccess) return fail_hip(e, "expert H2D");
    g.pcie_bytes += 3 * proj * 2;
    return HFMOE_OK;
}

int streamed_forward_t1(int layer, LayerState& L, const float* x, float* out, hipStream_t s,
                        const hfmoe_route_debug* dbg) {
    int rc = pool_init();
    if (rc) return rc;
    StreamPool& P = g.pool;
    const Cfg& c = g.cfg;

    Pending p;
    prof_begin(p, "router", s);
    hipError_t e = launch_router_logits_t1(x, L.dev, c, g.ws.logits, g.ws.scores, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "router launch");
    prof_begin(p, "select", s);
    e = launch_select(g.ws.scores, 1, c, g.ws.idx, g.ws.wts, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "select launch");
    e = hipMemcpyAsync(P.idx_host, g.ws.idx, sizeof(int) * c.k, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipEventRecord(P.routed, s);
    if (e != hipSuccess) return fail_hip(e, "routing readback");

    // Shared expert while the selected experts cross PCIe.
    const float* addend = nullptr;
    if (c.n_shared > 0) {
        Cfg cs = c;
        cs.k = 0;
        float* hs = g.ws.h + (size_t)c.k * c.I;
        prof_begin(p, "shared_gateup", s);
        e = launch_gateup_t1(x, L.dev, cs, nullptr, nullptr, nullptr, hs, c.n_shared, gu_blocks(), s);
        prof_end(p, s);
        if (e != hipSuccess) return fail_hip(e, "shared gate/up launch");
        prof_begin(p, "shared_down", s);
        e = launch_down_t1(hs, L.dev, cs, nullptr, nullptr, nullptr, P.shared_out, c.n_shared,
                           dn_blocks(), s);
        prof_end(p, s);
        if (e != hipSuccess) return fail_hip(e, "shared down launch");
        addend = P.shared_out;
    }

    e = hipEventSynchronize(P.routed);
    if (e != hipSuccess) return fail_hip(e, "wait for routing");

    int used[2 * kMaxTopK];
    const size_t proj = (size_t)c.I * c.d;
    for (int r = 0; r < c.k; ++r) {
        const int eid = P.idx_host[r];
        if (eid < 0 || eid >= c.E) return fail(HFMOE_ERR_HIP, "router produced expert id %d", eid);
        bool copy = false;
        const int slot = P.policy.lookup(layer, eid, used, r, &copy);
        if (slot < 0) return fail(HFMOE_ERR_HIP, "expert slot pool exhausted");
        if (copy) {
            int rc2 = copy_expert(L, eid, slot);
            if (rc2) return rc2;
        }
        used[r] = slot;
        const uint16_t* base = P.base + (size_t)slot * (P.slot_bytes / 2);
        P.etab_host[3 * r] = base;
        P.etab_host[3 * r + 1] = base + proj;
        P.etab_host[3 * r + 2] = base + 2 * proj;
        e = hipStreamWaitEvent(s, P.copied[slot], 0);
        if (e != hipSuccess) return fail_hip(e, "wait for expert H2D");
    }
    // Copy-ahead of the next layer's predicted experts, queued behind this
    // layer's copies; slots this call uses (and earlier copy-aheads of the
    // batch) are not victims.
    auto nx = g.layers.find(layer + 1);
    const bool next_streamed = nx != g.layers.end() && nx->second.location == HFMOE_EXPERTS_HOST_PINNED;
    const std::vector<int> guess = P.policy.route_done(layer, P.idx_host, c.k, next_streamed);
    int nclaimed = c.k;
    for (int eid : guess) {
        if (eid < 0 || eid >= c.E || nclaimed >= 2 * kMaxTopK) continue;
        const int slot = P.policy.stage(layer + 1, eid, used, nclaimed);
        if (slot < 0) continue;
        int rc2 = copy_expert(nx->second, eid, slot);
        if (rc2) return rc2;
        used[nclaimed++] = slot;
    }
    e = hipMemcpyAsync(P.etab_dev, P.etab_host, sizeof(void*) * 3 * c.k, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return fail_hip(e, "slot table upload");

    Cfg cr = c;
    cr.n_shared = 0;
    LayerDev Lr = L.dev;
    Lr.etab = P.etab_dev;
    prof_begin(p, "expert_gateup", s);
    e = launch_gateup_t1(x, Lr, cr, nullptr, P.iota_dev, nullptr, g.ws.h, c.k, gu_blocks(), s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "routed gate/up launch");
    prof_begin(p, "expert_down", s);
    e = launch_down_t1(g.ws.h, Lr, cr, P.iota_dev, g.ws.wts, addend, out, c.k, dn_blocks(), s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "routed down launch");
    for (int r = 0; r < c.k && e == hipSuccess; ++r) e = hipEventRecord(P.consumed[used[r]], s);
    if (e != hipSuccess) return fail_hip(e, "slot release");

    if (dbg) {
        if (dbg->logits_dev && e == hipSuccess)
            e = hipMemcpyAsync(dbg->logits_dev, g.ws.logits, sizeof(float) * c.E, hipMemcpyDeviceToDevice, s);
        if (dbg->idx_dev && e == hipSuccess)
            e = hipMemcpyAsync(dbg->idx_dev, g.ws.idx, sizeof(int) * c.k, hipMemcpyDeviceToDevice, s);
        if (dbg->weight_dev && e == hipSuccess)
            e = hipMemcpyAsync(dbg->weight_dev, g.ws.wts, sizeof(float) * c.k, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail_hip(e, "debug copies");
    }
    return HFMOE_OK;
}

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_stream_set_options(const hfmoe_stream_options* o) {
    int rc = require_init();
    if (rc) return rc;
    if (!o) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null options");
    if (!(o->ema_alpha > 0.0f && o->ema_alpha <= 1.0f) || !(o->overlap_alpha >= 0.0f && o->overlap_alpha <= 1.0f))
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "ema_alpha must be in (0, 1] and overlap_alpha in [0, 1]");
    StreamPolicyOptions& so = g.stream_opt;
    so.prefetch = o->prefetch_next_layer != 0;
    so.ema_predictor = o->ema_predictor != 0;
    so.ema_alpha = o->ema_alpha;
    so.overlap_floor = o->overlap_floor;
    so.overlap_alpha = o->overlap_alpha;
    g.pool.policy.opt = so;
    return HFMOE_OK;
}

int hfmoe_stream_get_options(hfmoe_stream_options* o) {
    int rc = require_init();
    if (rc) return rc;
    if (!o) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null options");
    *o = hfmoe_stream_options{};
    const StreamPolicyOptions& so = g.stream_opt;
    o->prefetch_next_layer = so.prefetch;
    o->ema_predictor = so.ema_predictor;
    o->ema_alpha = so.ema_alpha;
    o->overlap_floor = so.overlap_floor;
    o->overlap_alpha = so.overlap_alpha;
    return HFMOE_OK;
}

int hfmoe_stream_read_counters(hfmoe_stream_counters* out) {
    int rc = require_init();
    if (rc) return rc;
    if (!out) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null counters");
    const StreamPolicyCounters& n = g.pool.policy.n;
    *out = hfmoe_stream_counters{};
    out->lookups = n.lookups;
    out->hits = n.hits;
    out->misses = n.misses;
    out->pred_staged = n.pred_staged;
    out->pred_consumed = n.pred_consumed;
    out->pred_wasted = n.pred_wasted;
    out->pred_resident = n.pred_resident;
    out->copies = n.copies;
    out->slots = g.pool.slots;
    return HFMOE_OK;
}

int hfmoe_stream_reset(void) {
    int rc = require_init();
    if (rc) return rc;
    // Host bookkeeping only: copies still queued land in slots that are now
    // empty, and any later copy into a slot is ordered after them on the copy
    // stream and after the slot's last reader.
    g.pool.policy.reset(g.pool.slots);
    g.pool.policy.opt = g.stream_opt;
    return HFMOE_OK;
}

}  // extern "C"
