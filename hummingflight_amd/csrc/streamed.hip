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
#include "hf_grouped.h"

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
    if (P.idx_batch_host) hipHostFree(P.idx_batch_host);
    if (P.w_batch_host) hipHostFree(P.w_batch_host);
    if (P.wave_tabs) hipHostFree(P.wave_tabs);
    P = StreamPool{};
}

// Experts per wave of a multi-token call that needs `distinct` experts: all of
// them when they fit the pool, else half the pool, so one wave's copies land
// in the slots the wave before last released while the last wave computes.
static int wave_size(int slots, int distinct) {
    return distinct <= slots ? distinct : std::max(1, slots / 2);
}

// Coherent pinned host memory a kernel can read and write, and its device address.
template <typename Ptr>
static hipError_t mapped_alloc(Ptr* host, Ptr* dev, size_t bytes) {
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(host), bytes, hipHostMallocCoherent | hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(dev), (void*)*host, 0);
    return e;
}

// Routing of n pairs (ids, weights) from the workspace to mapped host memory,
// by a kernel on s; then `routed` is recorded on s.
static hipError_t routing_to_host(int* idx_dev_view, float* w_dev_view, size_t n, hipStream_t s) {
    hipError_t e = launch_copy_u32(reinterpret_cast<const uint32_t*>(g.ws.idx),
                                   reinterpret_cast<uint32_t*>(idx_dev_view), n, s);
    if (e == hipSuccess)
        e = launch_copy_u32(reinterpret_cast<const uint32_t*>(g.ws.wts), reinterpret_cast<uint32_t*>(w_dev_view), n, s);
    if (e == hipSuccess) e = hipEventRecord(g.pool.routed, s);
    return e;
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
    if (e == hipSuccess) e = mapped_alloc(&P.idx_host, &P.idx_host_dev, sizeof(int) * kMaxTopK);
    if (e == hipSuccess) e = mapped_alloc(&P.w_host, &P.w_host_dev, sizeof(float) * kMaxTopK);
    if (e == hipSuccess) e = mapped_alloc(&P.etab_host, &P.etab_host_dev, sizeof(void*) * 3 * kMaxTopK);
    if (e == hipSuccess) e = hipMalloc(&P.etab_dev, sizeof(void*) * 3 * kMaxTopK);
    if (e == hipSuccess) e = hipMalloc(&P.iota_dev, sizeof(int) * kMaxTopK);
    if (e == hipSuccess) e = hipMalloc(&P.shared_out, sizeof(float) * c.d);
    if (e == hipSuccess && g.max_tokens > 1) {
        P.max_waves = (c.E + wave_size(slots, c.E + 1) - 1) / wave_size(slots, c.E + 1) + 1;
        e = mapped_alloc(&P.idx_batch_host, &P.idx_batch_host_dev, sizeof(int) * (size_t)g.max_tokens * c.k);
        if (e == hipSuccess)
            e = mapped_alloc(&P.w_batch_host, &P.w_batch_host_dev, sizeof(float) * (size_t)g.max_tokens * c.k);
        if (e == hipSuccess)
            e = mapped_alloc(&P.wave_tabs, &P.wave_tabs_dev, sizeof(void*) * 3 * (size_t)(c.E + 1) * P.max_waves);
    }
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
// after the last kernel that read the slot: one copy of the whole expert when
// its three matrices lie back to back in host memory (the reference's expert
// block, uploaded with one copy, cuda_backend.cpp:416-418), else one per matrix.
static int copy_expert(const LayerState& L, int eid, int slot) {
    StreamPool& P = g.pool;
    const size_t proj = (size_t)g.cfg.I * g.cfg.d;
    uint16_t* dst = P.base + (size_t)slot * (P.slot_bytes / 2);
    const uint16_t* const* m = &L.host_experts[3 * (size_t)eid];
    hipError_t e = hipStreamWaitEvent(g.copy_stream, P.consumed[slot], 0);
    if (e == hipSuccess && m[1] == m[0] + proj && m[2] == m[1] + proj)
        e = hipMemcpyAsync(dst, m[0], 3 * proj * 2, hipMemcpyHostToDevice, g.copy_stream);
    else
        for (int q = 0; q < 3 && e == hipSuccess; ++q)
            e = hipMemcpyAsync(dst + q * proj, m[q], proj * 2, hipMemcpyHostToDevice, g.copy_stream);
    if (e == hipSuccess) e = hipEventRecord(P.copied[slot], g.copy_stream);
    if (e != hipSuccess) {
        P.policy.drop_slot(slot);  // the slot holds no copy of the expert: never serve it
        return fail_hip(e, "expert H2D");
    }
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
    e = routing_to_host(P.idx_host_dev, P.w_host_dev, c.k, s);
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
    for (int r = 0; r < c.k; ++r)
        if (P.idx_host[r] < 0 || P.idx_host[r] >= c.E)
            return fail(HFMOE_ERR_HIP, "router produced expert id %d", P.idx_host[r]);

    // The scheduler hears the routing first (history, heat, pins, guesses for
    // the next layer), then the layer looks its experts up.
    auto nx = g.layers.find(layer + 1);
    const bool has_next = nx != g.layers.end();
    const bool next_streamed = has_next && nx->second.location == HFMOE_EXPERTS_HOST_PINNED;
    const std::vector<int> guess = P.policy.route_done(layer, P.idx_host, P.w_host, c.k, has_next, next_streamed);

    int used[2 * kMaxTopK + kMaxTopK];
    const size_t proj = (size_t)c.I * c.d;
    for (int r = 0; r < c.k; ++r) {
        const int eid = P.idx_host[r];
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
    // call) are not victims.
    int nclaimed = c.k;
    for (int eid : guess) {
        if (eid < 0 || eid >= c.E || nclaimed >= (int)(sizeof used / sizeof used[0])) continue;
        const int slot = P.policy.stage(layer + 1, eid, used, nclaimed);
        if (slot < 0) continue;
        int rc2 = copy_expert(nx->second, eid, slot);
        if (rc2) return rc2;
        used[nclaimed++] = slot;
    }
    e = launch_copy_u64(reinterpret_cast<const uint64_t*>(P.etab_host_dev), reinterpret_cast<uint64_t*>(P.etab_dev),
                        3 * (size_t)c.k, s);
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

int streamed_forward_batch(int layer, LayerState& L, const float* x, int T, float* out, hipStream_t s,
                           const hfmoe_route_debug* dbg) {
    int rc = pool_init();
    if (rc) return rc;
    StreamPool& P = g.pool;
    const Cfg& c = g.cfg;
    if (!P.idx_batch_host || !P.w_batch_host || !P.wave_tabs)
        return fail(HFMOE_ERR_NOT_INITIALIZED, "multi-token staging buffers are not allocated");
    rc = grouped_route(L, x, T, s);
    if (rc) return rc;
    const int npairs = T * c.k;
    hipError_t e = routing_to_host(P.idx_batch_host_dev, P.w_batch_host_dev, (size_t)npairs, s);
    if (e == hipSuccess) e = hipEventSynchronize(P.routed);
    if (e != hipSuccess) return fail_hip(e, "routing readback");

    // The batch's distinct experts, resident ones first (their waves compute
    // while the others cross PCIe), then in order of first use.
    std::vector<char> seen(c.E, 0);
    std::vector<int> order, missing;
    for (int i = 0; i < npairs; ++i) {
        const int eid = P.idx_batch_host[i];
        if (eid < 0 || eid >= c.E) return fail(HFMOE_ERR_HIP, "router produced expert id %d", eid);
        if (seen[eid]) continue;
        seen[eid] = 1;
        (P.policy.find(expert_key(layer, eid)) >= 0 ? order : missing).push_back(eid);
    }
    order.insert(order.end(), missing.begin(), missing.end());
    const int U = (int)order.size();
    // The scheduler hears each token's routing in order, as the reference's
    // token loop reports it (onLayerRouterDone per token); the copy-ahead
    // follows the last token's guesses, queued after the batch's own copies.
    auto nx = g.layers.find(layer + 1);
    const bool has_next = nx != g.layers.end();
    const bool next_streamed = has_next && nx->second.location == HFMOE_EXPERTS_HOST_PINNED;
    std::vector<int> guess;
    for (int t = 0; t < T; ++t)
        guess = P.policy.route_done(layer, P.idx_batch_host + (size_t)t * c.k, P.w_batch_host + (size_t)t * c.k, c.k,
                                    has_next, next_streamed && t == T - 1);
    const int ws = wave_size(P.slots, U);
    const int nwaves = (U + ws - 1) / ws;
    if (nwaves > P.max_waves) return fail(HFMOE_ERR_HIP, "%d waves exceed the %d staged tables", nwaves, P.max_waves);
    const size_t ntab = 3 * (size_t)(c.E + 1);
    const size_t proj = (size_t)c.I * c.d;
    const bool dynamic_items = grouped_tile_rows(T) == kPrefillTileRows;
    std::vector<int> claimed;
    // At most kWavesAhead waves of copies queued: before a wave's copies go in,
    // the host waits for the copies of the wave that many places back.  With a
    // prefill's whole ~700 copies queued at once they ran progressively slower
    // (25 MB from 448 to ~630 us each) with gaps between them; two waves ahead
    // keep the copy engine fed at the pinned copy rate.
    constexpr int kWavesAhead = 2;
    std::vector<int> wave_last_slot(nwaves, -1);
    for (int wv = 0; wv < nwaves; ++wv) {
        if (wv >= kWavesAhead && wave_last_slot[wv - kWavesAhead] >= 0) {
            e = hipEventSynchronize(P.copied[wave_last_slot[wv - kWavesAhead]]);
            if (e != hipSuccess) return fail_hip(e, "wait for an earlier wave's copies");
        }
        const uint16_t** tab = P.wave_tabs + (size_t)wv * ntab;
        std::fill(tab, tab + ntab, nullptr);
        claimed.clear();
        for (int i = wv * ws; i < std::min(U, (wv + 1) * ws); ++i) {
            const int eid = order[i];
            bool copy = false;
            const int slot = P.policy.lookup(layer, eid, claimed.data(), (int)claimed.size(), &copy);
            if (slot < 0) return fail(HFMOE_ERR_HIP, "expert slot pool exhausted");
            if (copy) {
                rc = copy_expert(L, eid, slot);
                if (rc) return rc;
                wave_last_slot[wv] = slot;
            }
            claimed.push_back(slot);
            const uint16_t* base = P.base + (size_t)slot * (P.slot_bytes / 2);
            tab[3 * eid] = base;
            tab[3 * eid + 1] = base + proj;
            tab[3 * eid + 2] = base + 2 * proj;
            e = hipStreamWaitEvent(s, P.copied[slot], 0);
            if (e != hipSuccess) return fail_hip(e, "wait for expert H2D");
        }
        if (wv == 0 && c.n_shared > 0) {  // the shared expert (group E) is HBM-resident: first wave only
            tab[3 * c.E] = L.dev.sg;
            tab[3 * c.E + 1] = L.dev.su;
            tab[3 * c.E + 2] = L.dev.sd;
        }
        // The table goes up by a small kernel reading the mapped pinned copy: a
        // DMA copy here would queue behind the next wave's weight copies.
        e = launch_copy_u64(reinterpret_cast<const uint64_t*>(P.wave_tabs_dev + (size_t)wv * ntab),
                            reinterpret_cast<uint64_t*>(L.etab_dev), ntab, s);
        if (e == hipSuccess && wv > 0 && dynamic_items)  // the dispatch zeroed them for the first wave
            e = launch_clear_u32(g.gws.item_ctr, kItemCounters, s);
        if (e != hipSuccess) return fail_hip(e, "wave table upload");
        rc = grouped_experts(L.etab_dev, T, s);
        if (rc) return rc;
        for (int slot : claimed) {
            e = hipEventRecord(P.consumed[slot], s);
            if (e != hipSuccess) return fail_hip(e, "slot release");
        }
    }
    for (int eid : guess) {
        if (eid < 0 || eid >= c.E) continue;
        const int slot = P.policy.stage(layer + 1, eid, claimed.data(), (int)claimed.size());
        if (slot < 0) continue;
        rc = copy_expert(nx->second, eid, slot);
        if (rc) return rc;
        claimed.push_back(slot);
    }
    rc = grouped_combine(T, out, s);
    return rc ? rc : copy_debug(dbg, T, s);
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
    if (o->extra_depth < 0 || o->extra_depth > kMaxTopK)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "extra_depth=%d must be in 0..%d", o->extra_depth, kMaxTopK);
    StreamPolicyOptions& so = g.stream_opt;
    so.prefetch = o->prefetch_next_layer != 0;
    so.ema_predictor = o->ema_predictor != 0;
    so.ema_alpha = o->ema_alpha;
    so.overlap_floor = o->overlap_floor;
    so.overlap_alpha = o->overlap_alpha;
    so.extra_depth = o->extra_depth;
    so.prob_resident = o->prob_resident != 0;
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
    o->extra_depth = so.extra_depth;
    o->prob_resident = so.prob_resident;
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
    out->pinned = n.pinned > (uint64_t)INT32_MAX ? INT32_MAX : (int32_t)n.pinned;
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
