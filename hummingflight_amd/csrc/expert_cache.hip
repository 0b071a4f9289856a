// expert_cache.hip -- the per-expert GPU plugin surface of the reference
// (src/compute/cuda_backend.h:64-90, cuda_backend.cpp:196-554) on gfx950:
// an HBM-resident LRU of whole experts keyed by (layer, expert), fed through
// round-robin pinned staging slots with asynchronous H2D on a copy stream and
// per-expert completion events, and an expert FFN that waits on its expert's
// event, runs the decode GEMV kernels and copies the result back.
#include "hf_api_internal.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <thread>

namespace hf {
namespace {

struct DevExpert {
    uint16_t* w = nullptr;   // [gate | up | down], 6*hidden*inter bytes
    uint64_t key = ~0ull;
    uint64_t last_use = 0;
    bool pending = false;    // H2D queued, not yet waited on by an FFN
    int stage_slot = -1;
    hipEvent_t uploaded = nullptr;
};

struct ExpertCache {
    int capacity = 0;
    int depth = 2;
    int hidden = 0, inter = 0;
    bool allocated = false;
    std::vector<DevExpert> experts;
    std::vector<uint16_t*> stage_host;    // pinned staging slots
    std::vector<hipEvent_t> stage_done;   // copy of the slot finished
    std::vector<char> stage_busy;
    int next_stage = 0;
    float* x = nullptr;
    float* h = nullptr;
    float* out = nullptr;
    float* io_pin = nullptr;              // pinned coherent [2, hidden]: x, then out, of an FFN call
    float* io_pin_dev = nullptr;          // its device address (null: DMA copies instead)
    uint64_t clock = 0;
    std::unordered_map<uint64_t, int> where;

    static uint64_t key_of(int layer, int eid) {
        return ((uint64_t)(uint32_t)layer << 32) | (uint64_t)(uint32_t)eid;
    }
    size_t expert_bytes() const { return (size_t)hidden * inter * 6; }

    void release() {
        for (auto& e : experts) {
            if (e.w) hipFree(e.w);
            if (e.uploaded) hipEventDestroy(e.uploaded);
        }
        experts.clear();
        for (auto p : stage_host)
            if (p) hipHostFree(p);
        for (auto ev : stage_done)
            if (ev) hipEventDestroy(ev);
        stage_host.clear();
        stage_done.clear();
        stage_busy.clear();
        if (x) hipFree(x);
        if (h) hipFree(h);
        if (out) hipFree(out);
        if (io_pin) hipHostFree(io_pin);
        x = h = out = io_pin = io_pin_dev = nullptr;
        where.clear();
        allocated = false;
    }

    int alloc(int hd, int it) {
        hidden = hd;
        inter = it;
        experts.assign(capacity, DevExpert{});
        stage_host.assign(depth, nullptr);
        stage_done.assign(depth, nullptr);
        stage_busy.assign(depth, 0);
        next_stage = 0;
        const size_t one = expert_bytes();
        hipError_t e = hipSuccess;
        for (int s = 0; s < depth && e == hipSuccess; ++s) {
            e = hipHostMalloc(reinterpret_cast<void**>(&stage_host[s]), one, hipHostMallocDefault);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&stage_done[s], hipEventDisableTiming);
        }
        for (int i = 0; i < capacity && e == hipSuccess; ++i) {
            e = hipMalloc(&experts[i].w, one);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&experts[i].uploaded, hipEventDisableTiming);
        }
        if (e == hipSuccess) e = hipMalloc(&x, sizeof(float) * hd);
        if (e == hipSuccess) e = hipMalloc(&h, sizeof(float) * it);
        if (e == hipSuccess) e = hipMalloc(&out, sizeof(float) * hd);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void**>(&io_pin), 2 * sizeof(float) * hd,
                              hipHostMallocCoherent | hipHostMallocMapped);
        if (e == hipSuccess && hipHostGetDevicePointer(reinterpret_cast<void**>(&io_pin_dev), io_pin, 0) != hipSuccess) {
            (void)hipGetLastError();
            io_pin_dev = nullptr;
        }
        if (e != hipSuccess) {
            release();
            return fail(HFMOE_ERR_OUT_OF_MEMORY, "expert cache allocation failed: %s", hipGetErrorString(e));
        }
        allocated = true;
        return HFMOE_OK;
    }

    // Resident lookup, or LRU admission evicting the least recently used entry
    // (cuda_backend.cpp:322-363).
    int acquire(uint64_t k, bool& need_upload) {
        auto it = where.find(k);
        if (it != where.end()) {
            experts[it->second].last_use = ++clock;
            need_upload = false;
            return it->second;
        }
        int victim = 0;
        uint64_t oldest = std::numeric_limits<uint64_t>::max();
        for (int i = 0; i < capacity; ++i) {
            if (experts[i].key == ~0ull) {
                victim = i;
                break;
            }
            if (experts[i].last_use < oldest) {
                oldest = experts[i].last_use;
                victim = i;
            }
        }
        DevExpert& d = experts[victim];
        if (d.key != ~0ull) where.erase(d.key);
        d.key = k;
        d.last_use = ++clock;
        d.pending = false;
        where[k] = victim;
        need_upload = true;
        return victim;
    }

    // Unmap a slot whose upload could not be queued: its bytes are the evicted
    // expert's, so a later stage of the key must copy again and an FFN call
    // must report the expert as not resident.
    void forget(int slot) {
        DevExpert& d = experts[slot];
        if (d.key != ~0ull) where.erase(d.key);
        d.key = ~0ull;
        d.last_use = 0;
        d.pending = false;
    }

    // Round-robin staging slot; a slot whose copy is still queued is drained
    // first so its host bytes are never overwritten in flight
    // (cuda_backend.cpp:302-312).
    int claim_stage() {
        const int s = next_stage;
        next_stage = (next_stage + 1) % depth;
        if (stage_busy[s]) {
            hipError_t e = hipEventSynchronize(stage_done[s]);
            if (e != hipSuccess) return -1;
            stage_busy[s] = 0;
        }
        return s;
    }
};

ExpertCache* g_cache = nullptr;

}  // namespace
}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_expert_cache_config(int capacity, int staging_depth) {
    int rc = require_init();
    if (rc) return rc;
    if (capacity <= 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "capacity must be positive");
    hfmoe_expert_cache_shutdown();
    g_cache = new ExpertCache();
    g_cache->capacity = capacity;
    g_cache->depth = staging_depth < 1 ? 1 : staging_depth;
    return HFMOE_OK;
}

void hfmoe_expert_cache_shutdown(void) {
    if (!g_cache) return;
    if (g.inited) hipDeviceSynchronize();
    g_cache->release();
    delete g_cache;
    g_cache = nullptr;
}

int hfmoe_experts_enabled(void) { return (g.inited && g_cache) ? 1 : 0; }

// Copy into a pinned staging slot with several host threads: one thread's
// memcpy (~16 GB/s) is slower than the PCIe copy it feeds.
static void staging_memcpy(void* dst, const void* src, size_t bytes) {
    const unsigned hw = std::thread::hardware_concurrency();
    const size_t nt = std::min<size_t>(8, hw ? hw : 1);
    if (bytes < (size_t)(8 << 20) || nt < 2) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const size_t chunk = (bytes / nt + 4095) & ~(size_t)4095;
    std::vector<std::thread> pool;
    for (size_t i = 1; i < nt && i * chunk < bytes; ++i)
        pool.emplace_back([=] {
            const size_t off = i * chunk;
            std::memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off,
                        std::min(chunk, bytes - off));
        });
    std::memcpy(dst, src, std::min(chunk, bytes));
    for (auto& t : pool) t.join();
}

int hfmoe_expert_stage(int layer, int expert_id, const uint16_t* w, int hidden, int inter) {
    if (!hfmoe_experts_enabled())
        return fail(HFMOE_ERR_NOT_INITIALIZED, "expert cache not configured");
    if (!w || hidden <= 0 || inter <= 0 || hidden % 8 || inter % 8 || hidden > 8192 || inter > 4096)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "bad expert shape %dx%d", hidden, inter);
    ExpertCache& c = *g_cache;
    if (!c.allocated) {
        int rc = c.alloc(hidden, inter);
        if (rc) return rc;
    }
    if (c.hidden != hidden || c.inter != inter)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "expert shape %dx%d differs from the cache's %dx%d",
                    hidden, inter, c.hidden, c.inter);
    bool need = false;
    const int slot = c.acquire(ExpertCache::key_of(layer, expert_id), need);
    if (!need) return HFMOE_OK;
    const int st = c.claim_stage();
    if (st < 0) {
        c.forget(slot);
        return fail(HFMOE_ERR_HIP, "staging slot drain failed");
    }
    const size_t bytes = c.expert_bytes();
    staging_memcpy(c.stage_host[st], w, bytes);
    hipError_t e = hipMemcpyAsync(c.experts[slot].w, c.stage_host[st], bytes, hipMemcpyHostToDevice,
                                  g.copy_stream);
    if (e == hipSuccess) e = hipEventRecord(c.stage_done[st], g.copy_stream);
    if (e == hipSuccess) e = hipEventRecord(c.experts[slot].uploaded, g.copy_stream);
    if (e != hipSuccess) {
        // The copy may be queued with its events unrecorded: drain it before
        // the staging slot or the HBM slot is reused.
        (void)hipStreamSynchronize(g.copy_stream);
        c.forget(slot);
        return fail_hip(e, "expert upload");
    }
    c.stage_busy[st] = 1;
    c.experts[slot].pending = true;
    c.experts[slot].stage_slot = st;
    g.pcie_bytes += bytes;
    return HFMOE_OK;
}

int hfmoe_expert_ffn(int layer, int expert_id, const float* x, float* out, int hidden, int inter) {
    if (!hfmoe_experts_enabled())
        return fail(HFMOE_ERR_NOT_INITIALIZED, "expert cache not configured");
    ExpertCache& c = *g_cache;
    if (!c.allocated || c.hidden != hidden || c.inter != inter)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "expert shape mismatch or nothing staged");
    if (!x || !out) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null buffer");
    auto it = c.where.find(ExpertCache::key_of(layer, expert_id));
    if (it == c.where.end())
        return fail(HFMOE_ERR_NOT_REGISTERED, "expert (%d,%d) is not resident", layer, expert_id);
    DevExpert& d = c.experts[it->second];
    hipStream_t s = g.stream;
    hipError_t e = hipSuccess;
    if (d.pending) {
        e = hipStreamWaitEvent(s, d.uploaded, 0);
        if (e != hipSuccess) return fail_hip(e, "wait for expert upload");
        d.pending = false;
    }
    const size_t half = (size_t)hidden * inter;
    // x and out cross PCIe through the coherent pinned io buffer, read and
    // written by a small kernel on the compute stream (or by DMA copies where
    // the buffer has no device address).
    const size_t xb = sizeof(float) * hidden;
    memcpy(c.io_pin, x, xb);
    e = c.io_pin_dev ? launch_copy_f32(c.io_pin_dev, c.x, hidden, s)
                     : hipMemcpyAsync(c.x, c.io_pin, xb, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return fail_hip(e, "H2D x");
    g.pcie_bytes += xb;
    e = launch_expert_ffn(d.w, d.w + half, d.w + 2 * half, c.x, c.h, c.out, hidden, inter,
                          gu_blocks(), dn_blocks(), s);
    if (e != hipSuccess) return fail_hip(e, "expert ffn launch");
    e = c.io_pin_dev ? launch_copy_f32(c.out, c.io_pin_dev + hidden, hidden, s)
                     : hipMemcpyAsync(c.io_pin + hidden, c.out, xb, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail_hip(e, "D2H out");
    memcpy(out, c.io_pin + hidden, xb);
    g.pcie_bytes += xb;
    return HFMOE_OK;
}

// Device-vs-host parity of one staged expert, the analogue of
// cudaExpertSelfTest (cuda_backend.cpp:494-554): cases (hidden, inter) =
// (64, 32) and (6144, 2048), weights and x from std::mt19937(1) uniform in
// [-1, 1) (x scaled by 0.7), relative tolerance 1e-2.  The host loop below is
// this check's own yardstick only; it never produces a result for a caller.
int hfmoe_self_test(void) {
    int rc = require_init();
    if (rc) return rc;
    const int cases[2][2] = {{64, 32}, {6144, 2048}};
    ExpertCache* prev = g_cache;
    g_cache = nullptr;
    int result = HFMOE_OK;
    for (auto& cs : cases) {
        const int hd = cs[0], it = cs[1];
        const size_t half = (size_t)hd * it;
        std::vector<uint16_t> w(3 * half);
        std::mt19937 rng(1);
        std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
        for (auto& v : w) {
            const float f = dist(rng);
            uint32_t u;
            std::memcpy(&u, &f, 4);
            v = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
        }
        std::vector<float> x(hd), y(hd), ref(hd);
        for (auto& v : x) v = 0.7f * dist(rng);
        rc = hfmoe_expert_cache_config(2, 2);
        if (!rc) rc = hfmoe_expert_stage(1, 3, w.data(), hd, it);
        if (!rc) rc = hfmoe_expert_stage(1, 7, w.data(), hd, it);
        if (!rc) rc = hfmoe_expert_ffn(1, 3, x.data(), y.data(), hd, it);
        hfmoe_expert_cache_shutdown();
        if (rc) {
            result = rc;
            break;
        }
        auto bf = [](uint16_t b) {
            uint32_t u = (uint32_t)b << 16;
            float f;
            std::memcpy(&f, &u, 4);
            return f;
        };
        std::vector<float> gg(it), uu(it), m(it);
        for (int r = 0; r < it; ++r) {
            float a = 0.0f, b = 0.0f;
            for (int k = 0; k < hd; ++k) {
                a += bf(w[(size_t)r * hd + k]) * x[k];
                b += bf(w[half + (size_t)r * hd + k]) * x[k];
            }
            gg[r] = a;
            uu[r] = b;
            m[r] = (a / (1.0f + std::exp(-a))) * b;
        }
        for (int j = 0; j < hd; ++j) {
            float a = 0.0f;
            for (int r = 0; r < it; ++r) a += bf(w[2 * half + (size_t)j * it + r]) * m[r];
            ref[j] = a;
        }
        for (int j = 0; j < hd; ++j) {
            const bool bad = std::fabs(ref[j]) > 1e-8f
                                 ? std::fabs(y[j] - ref[j]) / std::fabs(ref[j]) > 1e-2f
                                 : std::fabs(y[j]) > 1e-6f;
            if (bad) {
                result = fail(HFMOE_ERR_HIP, "self-test %dx%d: element %d device %g host %g", hd, it,
                              j, (double)y[j], (double)ref[j]);
                break;
            }
        }
        if (result) break;
    }
    g_cache = prev;
    return result;
}

}  // extern "C"
