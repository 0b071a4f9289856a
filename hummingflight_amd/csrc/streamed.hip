// streamed.hip -- decode with routed experts resident in pinned host RAM.
//
// The on-device counterpart of the reference's scheduler + GPU staging window
// (Scheduler::getExpertPtr scheduler.cpp:646-741 feeding gpuExpertStage,
// cuda_backend.cpp:395-428, from moeLayer glm_forward.cpp:562-602): only the k
// experts the router selects cross PCIe.
//
// Per call (T = 1), on the caller's stream s and the library's copy stream:
//   s:    router -> D2H of the k selected ids (pinned) -> event `routed`
//   s:    shared expert gate/up + down into shared_out (overlaps the copies)
//   host: wait `routed`; for each selected expert look up the HBM slot pool
//         (LRU keyed by layer and expert): a hit reuses the slot, a miss
//         queues three hipMemcpyAsync (gate, up, down) on the copy stream
//         after the slot's previous reader finished, then records `copied`
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
    // else two layers' worth of selected experts; never fewer than k.
    int slots = 2 * c.k;
    if (g.vram_budget) slots = (int)(g.vram_budget / P.slot_bytes);
    if (slots < c.k) slots = c.k;
    hipError_t e = hipMalloc(&P.base, P.slot_bytes * (size_t)slots);
    if (e != hipSuccess)
        return fail(HFMOE_ERR_OUT_OF_MEMORY, "expert staging pool (%d x %zu bytes): %s", slots,
                    P.slot_bytes, hipGetErrorString(e));
    P.slots = slots;
    P.copied.assign(slots, nullptr);
    P.consumed.assign(slots, nullptr);
    P.key.assign(slots, ~0ull);
    P.last_use.assign(slots, 0);
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

    int used[kMaxTopK];
    const size_t proj = (size_t)c.I * c.d;
    for (int r = 0; r < c.k; ++r) {
        const int eid = P.idx_host[r];
        if (eid < 0 || eid >= c.E) return fail(HFMOE_ERR_HIP, "router produced expert id %d", eid);
        const uint64_t key = ((uint64_t)(uint32_t)layer << 32) | (uint32_t)eid;
        int slot = -1;
        for (int i = 0; i < P.slots; ++i)
            if (P.key[i] == key) slot = i;
        if (slot >= 0) {
            ++P.hits;
        } else {
            // LRU victim among slots this call has not claimed.
            uint64_t oldest = ~0ull;
            for (int i = 0; i < P.slots; ++i) {
                bool taken = false;
                for (int q = 0; q < r; ++q) taken |= (used[q] == i);
                if (taken) continue;
                if (P.key[i] == ~0ull) {
                    slot = i;
                    break;
                }
                if (P.last_use[i] < oldest) {
                    oldest = P.last_use[i];
                    slot = i;
                }
            }
            uint16_t* dst = P.base + (size_t)slot * (P.slot_bytes / 2);
            e = hipStreamWaitEvent(g.copy_stream, P.consumed[slot], 0);
            for (int q = 0; q < 3 && e == hipSuccess; ++q)
                e = hipMemcpyAsync(dst + q * proj, L.host_experts[3 * eid + q], proj * 2,
                                   hipMemcpyHostToDevice, g.copy_stream);
            if (e == hipSuccess) e = hipEventRecord(P.copied[slot], g.copy_stream);
            if (e != hipSuccess) return fail_hip(e, "expert H2D");
            P.key[slot] = key;
            ++P.misses;
            g.pcie_bytes += 3 * proj * 2;
        }
        P.last_use[slot] = ++P.clock;
        used[r] = slot;
        const uint16_t* base = P.base + (size_t)slot * (P.slot_bytes / 2);
        P.etab_host[3 * r] = base;
        P.etab_host[3 * r + 1] = base + proj;
        P.etab_host[3 * r + 2] = base + 2 * proj;
        e = hipStreamWaitEvent(s, P.copied[slot], 0);
        if (e != hipSuccess) return fail_hip(e, "wait for expert H2D");
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
