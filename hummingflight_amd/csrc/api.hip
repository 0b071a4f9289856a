// api.hip -- C-ABI entry points of libhfmoe.so (declared in include/hfmoe.h).
//
// Process-global state, one device, one caller thread (the reference's GPU
// backend is a process-global singleton too, cuda_backend.cpp:366).  Owns the
// per-layer device weight tables, the routing/activation workspace and the
// library stream, and turns every failure into a status code plus a message.
#include "hf_api_internal.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace hf {

State g;
LaunchTiming g_timing;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g.last_error = buf;
    return code;
}

int fail_hip(hipError_t e, const char* what) {
    return fail(HFMOE_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

hipStream_t pick_stream(void* s) { return s ? reinterpret_cast<hipStream_t>(s) : g.stream; }

// ---- profiling: the launches of a section record their dispatch timestamps
// into a pair of pooled events (launch() in hf_kernels.h) ----
static hipEvent_t pooled_event() {
    hipEvent_t e = nullptr;
    if (!g.event_pool.empty()) {
        e = g.event_pool.back();
        g.event_pool.pop_back();
    } else if (hipEventCreate(&e) != hipSuccess) {
        e = nullptr;
    }
    return e;
}

void prof_begin(Pending& p, const char* name, hipStream_t s) {
    (void)s;
    p.name = nullptr;
    if (!g.prof_on) return;
    hipEvent_t a = pooled_event();
    if (!a) return;
    hipEvent_t b = pooled_event();
    if (!b) {
        g.event_pool.push_back(a);
        return;
    }
    p.name = name;
    p.start = a;
    p.stop = b;
    g_timing.start = a;
    g_timing.stop = b;
}

void prof_end(Pending& p, hipStream_t s) {
    (void)s;
    if (!p.name) return;
    const bool launched = g_timing.start != p.start;
    g_timing = LaunchTiming{};
    if (!launched) {  // nothing was launched in the section
        g.event_pool.push_back(p.start);
        g.event_pool.push_back(p.stop);
    } else {
        g.pending.push_back(p);
    }
    p.name = nullptr;  // ended: a second prof_end is a no-op
}

void prof_drain() {
    for (auto& p : g.pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            auto& st = g.kstats[p.name];
            st.first += 1;
            st.second += ms;
            g.gpu_active_ns += (uint64_t)(ms * 1e6);
        }
        g.event_pool.push_back(p.start);
        g.event_pool.push_back(p.stop);
    }
    g.pending.clear();
}

static void free_workspace() {
    Workspace& w = g.ws;
    void* ptrs[] = {w.logits, w.scores, w.idx, w.wts, w.h, w.counter, w.x_io, w.out_io, w.tmp};
    for (void* p : ptrs)
        if (p) hipFree(p);
    if (w.io_pin) hipHostFree(w.io_pin);
    w = Workspace{};
}

static int alloc_workspace() {
    free_workspace();
    Workspace& w = g.ws;
    const Cfg& c = g.cfg;
    const int T = g.max_tokens;
    const int nslots = c.k + c.n_shared;
    struct A {
        void** p;
        size_t bytes;
    } list[] = {
        {(void**)&w.logits, sizeof(float) * (size_t)T * c.E},
        {(void**)&w.scores, sizeof(float2) * (size_t)T * c.E},
        {(void**)&w.idx, sizeof(int) * (size_t)T * c.k},
        {(void**)&w.wts, sizeof(float) * (size_t)T * c.k},
        {(void**)&w.h, sizeof(float) * (size_t)nslots * c.I},
        {(void**)&w.counter, 256},
        {(void**)&w.x_io, sizeof(float) * (size_t)c.d},
        {(void**)&w.out_io, sizeof(float) * (size_t)c.d},
        {(void**)&w.tmp, sizeof(float) * 2 * (size_t)T * c.d},
    };
    for (auto& a : list) {
        hipError_t e = hipMalloc(a.p, a.bytes);
        if (e != hipSuccess) {
            free_workspace();
            return fail(HFMOE_ERR_OUT_OF_MEMORY, "workspace allocation of %zu bytes failed: %s",
                        a.bytes, hipGetErrorString(e));
        }
    }
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&w.io_pin), 2 * sizeof(float) * (size_t)c.d,
                                 hipHostMallocCoherent | hipHostMallocMapped);
    if (e != hipSuccess) {
        free_workspace();
        return fail(HFMOE_ERR_OUT_OF_MEMORY, "pinned io buffer: %s", hipGetErrorString(e));
    }
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&w.io_pin_dev), w.io_pin, 0) != hipSuccess) {
        (void)hipGetLastError();
        w.io_pin_dev = nullptr;
    }
    e = hipMemset(w.counter, 0, 256);
    if (e != hipSuccess) return fail_hip(e, "hipMemset(counter)");
    return HFMOE_OK;
}

int require_init() {
    if (!g.inited) return fail(HFMOE_ERR_NOT_INITIALIZED, "hfmoe_init has not been called");
    return HFMOE_OK;
}

int require_cfg() {
    int rc = require_init();
    if (rc) return rc;
    if (!g.configured) return fail(HFMOE_ERR_NOT_INITIALIZED, "hfmoe_configure has not been called");
    return HFMOE_OK;
}

int check_align(int layer, const char* what, const void* p, size_t align) {
    if (reinterpret_cast<uintptr_t>(p) % align)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: %s weights at %p are not %zu-byte aligned", layer, what, p,
                    align);
    return HFMOE_OK;
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_init(int device) {
    if (g.inited) {
        if (device == g.device) return HFMOE_OK;
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "already initialised on device %d", g.device);
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(HFMOE_ERR_NO_DEVICE, "no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "device %d out of range (count %d)", device, count);
    if ((e = hipSetDevice(device)) != hipSuccess) return fail_hip(e, "hipSetDevice");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return fail_hip(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(HFMOE_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950",
                    device, prop.gcnArchName);
    // The allocation-free entry point's scratch address is optional: when it
    // cannot be taken the library still initialises, and only
    // hfmoe_moe_forward_noalloc reports HFMOE_ERR_NOT_INITIALIZED (with this
    // reason).
    noalloc_setup(device);
    g.device = device;
    g.num_cus = prop.multiProcessorCount;
    g.total_mem = prop.totalGlobalMem;
    snprintf(g.name, sizeof g.name, "%s", prop.name);
    if ((e = hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking)) != hipSuccess)
        return fail_hip(e, "hipStreamCreate");
    if ((e = hipStreamCreateWithFlags(&g.copy_stream, hipStreamNonBlocking)) != hipSuccess)
        return fail_hip(e, "hipStreamCreate(copy)");
    g.inited = true;
    return HFMOE_OK;
}

void hfmoe_shutdown(void) {
    if (!g.inited) return;
    hipDeviceSynchronize();
    hfmoe_expert_cache_shutdown();
    stream_pool_release();
    for (auto& kv : g.layers)
        if (kv.second.etab_dev) hipFree(kv.second.etab_dev);
    g.layers.clear();
    free_workspace();
    grouped_workspace_free();
    dense_workspace_free();
    lm_head_release();
    prof_drain();
    for (auto ev : g.event_pool) hipEventDestroy(ev);
    g.event_pool.clear();
    if (g.stream) hipStreamDestroy(g.stream);
    if (g.copy_stream) hipStreamDestroy(g.copy_stream);
    g.stream = g.copy_stream = nullptr;
    g.inited = false;
    g.configured = false;
}

int hfmoe_available(void) { return g.inited ? 1 : 0; }

int hfmoe_device_name(char* buf, size_t len) {
    if (!buf || len == 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null buffer");
    buf[0] = 0;
    int rc = require_init();
    if (rc) return rc;
    snprintf(buf, len, "%s", g.name);
    return HFMOE_OK;
}

size_t hfmoe_device_memory_mb(void) { return g.inited ? g.total_mem / (1024 * 1024) : 0; }

const char* hfmoe_last_error(void) { return g.last_error.c_str(); }

int hfmoe_configure(const hfmoe_config* cfg) {
    int rc = require_init();
    if (rc) return rc;
    if (!cfg) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null config");
    // A rejected configuration leaves the earlier one in force; once the old
    // workspace is released below, only a fully allocated new one counts.
    Cfg c{};
    c.d = cfg->hidden;
    c.I = cfg->moe_intermediate;
    c.E = cfg->n_routed_experts;
    c.k = cfg->num_experts_per_tok;
    c.n_group = cfg->n_group <= 0 ? 1 : cfg->n_group;
    c.topk_group = cfg->topk_group <= 0 ? 1 : cfg->topk_group;
    c.n_shared = cfg->n_shared_experts;
    c.norm = cfg->norm_topk_prob ? 1 : 0;
    c.scale = cfg->routed_scaling_factor;
    c.eps = cfg->rms_norm_eps;
    if (c.d <= 0 || c.d % 8 || c.d > 8192)
        return fail(HFMOE_ERR_UNSUPPORTED, "hidden=%d: must be a positive multiple of 8, <= 8192", c.d);
    if (c.I <= 0 || c.I % 8 || c.I > 4096)
        return fail(HFMOE_ERR_UNSUPPORTED, "moe_intermediate=%d: must be a positive multiple of 8, <= 4096", c.I);
    if (c.E <= 0 || c.E > kMaxExperts)
        return fail(HFMOE_ERR_UNSUPPORTED, "n_routed_experts=%d: must be in 1..%d", c.E, kMaxExperts);
    if (c.k <= 0 || c.k > kMaxTopK || c.k > c.E)
        return fail(HFMOE_ERR_UNSUPPORTED, "num_experts_per_tok=%d: must be in 1..min(8, E)", c.k);
    if (c.n_group > 64 || c.E % c.n_group)
        return fail(HFMOE_ERR_UNSUPPORTED, "n_group=%d must divide E=%d and be <= 64", c.n_group, c.E);
    if (c.n_group > 1 && c.topk_group * (c.E / c.n_group) < c.k)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "topk_group=%d keeps fewer than k=%d experts",
                    c.topk_group, c.k);
    if (c.n_shared < 0 || c.k + c.n_shared > kMaxSlots)
        return fail(HFMOE_ERR_UNSUPPORTED, "n_shared_experts=%d too large", c.n_shared);
    if ((size_t)(c.k + c.n_shared) * c.I * sizeof(float) > 160 * 1024)
        return fail(HFMOE_ERR_UNSUPPORTED, "(k + n_shared) * I FP32 activations exceed LDS");
    if (cfg->max_tokens < 0 || cfg->max_tokens > kMaxTokens)
        return fail(HFMOE_ERR_UNSUPPORTED, "max_tokens=%d: must be in 0..%d", cfg->max_tokens, kMaxTokens);
    g.configured = false;
    g.cfg = c;
    g.max_tokens = cfg->max_tokens > 0 ? cfg->max_tokens : 1;
    g.vram_budget = cfg->vram_budget_bytes;
    for (auto& kv : g.layers)
        if (kv.second.etab_dev) hipFree(kv.second.etab_dev);
    g.layers.clear();
    stream_pool_release();
    dense_workspace_free();
    lm_head_release();
    rc = alloc_workspace();
    if (rc) return rc;
    rc = grouped_workspace_alloc();
    if (rc) {
        free_workspace();
        return rc;
    }
    g.configured = true;
    return HFMOE_OK;
}

int hfmoe_register_layer(int layer, const hfmoe_layer_weights* w) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!w || !w->router_dev || !w->experts)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: router and expert table are required", layer);
    const Cfg& c = g.cfg;
    if (c.n_shared > 0 && (!w->shared_gate_dev || !w->shared_up_dev || !w->shared_down_dev))
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: shared expert weights missing", layer);
    if (w->experts_location != HFMOE_EXPERTS_DEVICE && w->experts_location != HFMOE_EXPERTS_HOST_PINNED)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: unknown experts_location %d", layer,
                    w->experts_location);
    for (int i = 0; i < 3 * c.E; ++i)
        if (!w->experts[i]) return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: expert pointer %d is NULL", layer, i);
    // Alignment the kernels' loads need: 16 bytes for every BF16 matrix read
    // from HBM (16-byte vector loads and LDS DMA), 4 for the F32 bias, 2 for the
    // norm weight.  Host-pinned experts are copied by the DMA engines into the
    // library's own slots, which carry no requirement.
    rc = check_align(layer, "router", w->router_dev, 16);
    if (!rc && c.n_shared > 0) rc = check_align(layer, "shared gate", w->shared_gate_dev, 16);
    if (!rc && c.n_shared > 0) rc = check_align(layer, "shared up", w->shared_up_dev, 16);
    if (!rc && c.n_shared > 0) rc = check_align(layer, "shared down", w->shared_down_dev, 16);
    if (!rc) rc = check_align(layer, "e_score_correction_bias", w->score_bias_dev, 4);
    if (!rc) rc = check_align(layer, "post_attention_norm", w->post_attention_norm_dev, 2);
    for (int i = 0; !rc && w->experts_location == HFMOE_EXPERTS_DEVICE && i < 3 * c.E; ++i)
        if (reinterpret_cast<uintptr_t>(w->experts[i]) & 15)
            rc = fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d: HBM expert %d %s weights at %p are not 16-byte aligned",
                      layer, i / 3, i % 3 == 0 ? "gate" : i % 3 == 1 ? "up" : "down", (const void*)w->experts[i]);
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it != g.layers.end() && it->second.etab_dev) hipFree(it->second.etab_dev);
    g.pool.policy.forget_layer(layer);  // cached HBM copies hold the old weights
    LayerState st;
    st.location = w->experts_location;
    st.host_experts.assign(w->experts, w->experts + 3 * c.E);
    st.norm_w = w->post_attention_norm_dev;
    // Device table of 3 * (E + 1) pointers: the routed experts' (gate, up,
    // down), then the shared expert's, which the multi-token path multiplies
    // as one more group (a single shared expert has a routed expert's shape).
    hipError_t e = hipMalloc(&st.etab_dev, sizeof(void*) * 3 * (size_t)(c.E + 1));
    if (e != hipSuccess) return fail_hip(e, "hipMalloc(expert table)");
    if (st.location == HFMOE_EXPERTS_DEVICE) {
        std::vector<const void*> tab(w->experts, w->experts + 3 * c.E);
        tab.push_back(w->shared_gate_dev);
        tab.push_back(w->shared_up_dev);
        tab.push_back(w->shared_down_dev);
        e = hipMemcpy(st.etab_dev, tab.data(), sizeof(void*) * tab.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            hipFree(st.etab_dev);
            return fail_hip(e, "hipMemcpy(expert table)");
        }
    }
    st.dev.router = w->router_dev;
    st.dev.bias = w->score_bias_dev;
    st.dev.sg = w->shared_gate_dev;
    st.dev.su = w->shared_up_dev;
    st.dev.sd = w->shared_down_dev;
    st.dev.etab = const_cast<const uint16_t* const*>(st.etab_dev);
    g.layers[layer] = st;
    return HFMOE_OK;
}

int hfmoe_moe_forward(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream) {
    return hfmoe_moe_forward_debug(layer, x_dev, T, out_dev, stream, nullptr);
}

int hfmoe_moe_forward_debug(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream,
                            const hfmoe_route_debug* dbg) {
    int rc = require_cfg();
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it == g.layers.end()) return fail(HFMOE_ERR_NOT_REGISTERED, "layer %d is not registered", layer);
    if (T < 0 || T > g.max_tokens)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "T=%d outside 0..max_tokens=%d", T, g.max_tokens);
    if (T == 0) return HFMOE_OK;
    if (!x_dev || !out_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null activation pointer");
    if ((reinterpret_cast<uintptr_t>(x_dev) | reinterpret_cast<uintptr_t>(out_dev)) & 15)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "activations must be 16-byte aligned");
    hipStream_t s = pick_stream(stream);
    LayerState& L = it->second;
    if (L.dense) return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d is a dense MLP layer", layer);
    if (L.location == HFMOE_EXPERTS_HOST_PINNED) {
        if (T == 1) return streamed_forward_t1(layer, L, x_dev, out_dev, s, dbg);
        if (g.gws.xh) return streamed_forward_batch(layer, L, x_dev, T, out_dev, s, dbg);
        // Shapes the grouped GEMM does not tile: token by token.
        for (int t = 0; t < T; ++t) {
            hfmoe_route_debug d1{};
            if (dbg) {
                d1.logits_dev = dbg->logits_dev ? dbg->logits_dev + (size_t)t * g.cfg.E : nullptr;
                d1.idx_dev = dbg->idx_dev ? dbg->idx_dev + (size_t)t * g.cfg.k : nullptr;
                d1.weight_dev = dbg->weight_dev ? dbg->weight_dev + (size_t)t * g.cfg.k : nullptr;
            }
            rc = streamed_forward_t1(layer, L, x_dev + (size_t)t * g.cfg.d, out_dev + (size_t)t * g.cfg.d, s,
                                     dbg ? &d1 : nullptr);
            if (rc) return rc;
        }
        return HFMOE_OK;
    }
    if (T == 1) return forward_t1(L, x_dev, out_dev, s, dbg);
    // Two tokens go through the decode kernels one at a time: 0.225 against
    // 0.25-0.26 ms per layer at full shape (the grouped path's seven launches
    // and dispatch cost more than a second read of the few experts the two
    // share); from three tokens on the grouped path is as fast or faster.  A
    // debug call takes the grouped path, whose dispatch it reports.
    if (!dbg && T <= env_int("HFMOE_TOKENWISE_MAX_T", 2)) {
        for (int t = 0; t < T; ++t) {
            rc = forward_t1(L, x_dev + (size_t)t * g.cfg.d, out_dev + (size_t)t * g.cfg.d, s, nullptr);
            if (rc) return rc;
        }
        return HFMOE_OK;
    }
    return forward_grouped(L, x_dev, T, out_dev, s, dbg);
}

int hfmoe_moe_forward_bf16(int layer, const uint16_t* x_dev, int32_t T, float* out_dev, void* stream) {
    int rc = require_cfg();
    if (rc) return rc;
    if (T < 0 || T > g.max_tokens)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "T=%d outside 0..max_tokens=%d", T, g.max_tokens);
    if (T == 0) return HFMOE_OK;
    if (!x_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null activation pointer");
    if (reinterpret_cast<uintptr_t>(x_dev) & 15) return fail(HFMOE_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
    if (!g.ws.tmp) return fail(HFMOE_ERR_NOT_INITIALIZED, "workspace is not allocated");
    // x widened to FP32 (exactly) in the workspace's [max_tokens, d] scratch
    // rows, then the FP32 forward on the same stream.
    hipError_t e = launch_bf16_to_f32(x_dev, g.ws.tmp, (size_t)T * g.cfg.d, pick_stream(stream));
    if (e != hipSuccess) return fail_hip(e, "x BF16 -> FP32");
    return hfmoe_moe_forward_debug(layer, g.ws.tmp, T, out_dev, stream, nullptr);
}

int hfmoe_moe_layer(int layer, const float* input_host, float* output_host) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!input_host || !output_host) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null buffer");
    // x and out cross PCIe through the coherent pinned io buffer, read and
    // written by a small kernel on the compute stream (no DMA-engine round
    // trip per 24 KB), or by DMA copies where the buffer has no device address.
    const size_t bytes = sizeof(float) * (size_t)g.cfg.d;
    if (!g.ws.io_pin || !g.ws.x_io || !g.ws.out_io)
        return fail(HFMOE_ERR_NOT_INITIALIZED, "host-contract buffers are not allocated");
    float* pin = g.ws.io_pin;
    float* pin_dev = g.ws.io_pin_dev;
    memcpy(pin, input_host, bytes);
    hipError_t e = pin_dev ? launch_copy_f32(pin_dev, g.ws.x_io, g.cfg.d, g.stream)
                           : hipMemcpyAsync(g.ws.x_io, pin, bytes, hipMemcpyHostToDevice, g.stream);
    if (e != hipSuccess) return fail_hip(e, "H2D input");
    g.pcie_bytes += bytes;
    rc = hfmoe_moe_forward(layer, g.ws.x_io, 1, g.ws.out_io, nullptr);
    if (rc) {
        hipStreamSynchronize(g.stream);  // the pinned buffer is reused by the next call
        return rc;
    }
    e = pin_dev ? launch_copy_f32(g.ws.out_io, pin_dev + g.cfg.d, g.cfg.d, g.stream)
                : hipMemcpyAsync(pin + g.cfg.d, g.ws.out_io, bytes, hipMemcpyDeviceToHost, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e != hipSuccess) return fail_hip(e, "D2H output");
    memcpy(output_host, pin + g.cfg.d, bytes);
    g.pcie_bytes += bytes;
    return HFMOE_OK;
}

int hfmoe_mlp_block(int layer, float* h_dev, int32_t T, void* stream) {
    int rc = require_cfg();
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it == g.layers.end()) return fail(HFMOE_ERR_NOT_REGISTERED, "layer %d is not registered", layer);
    if (T < 0 || T > g.max_tokens)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "T=%d outside 0..max_tokens=%d", T, g.max_tokens);
    if (T == 0) return HFMOE_OK;
    // The RMSNorm reads and the residual add writes h in 16-byte vectors.
    if (!h_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null hidden state pointer");
    if (reinterpret_cast<uintptr_t>(h_dev) & 15)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "hidden state must be 16-byte aligned");
    if (!g.ws.tmp) return fail(HFMOE_ERR_NOT_INITIALIZED, "workspace is not allocated");
    hipStream_t s = pick_stream(stream);
    float* xn = g.ws.tmp;
    float* mo = g.ws.tmp + (size_t)T * g.cfg.d;
    Pending p;
    prof_begin(p, "rmsnorm", s);
    hipError_t e = launch_rmsnorm(h_dev, it->second.norm_w, xn, T, g.cfg.d, g.cfg.eps, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "rmsnorm launch");
    rc = it->second.dense ? hfmoe_dense_mlp_forward(layer, xn, T, mo, s) : hfmoe_moe_forward(layer, xn, T, mo, s);
    if (rc) return rc;
    prof_begin(p, "residual_add", s);
    e = launch_add_inplace(h_dev, mo, (size_t)T * g.cfg.d, s);
    prof_end(p, s);
    if (e != hipSuccess) return fail_hip(e, "residual launch");
    return HFMOE_OK;
}

int hfmoe_malloc(void** ptr, size_t bytes) {
    int rc = require_init();
    if (rc) return rc;
    if (!ptr) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null out pointer");
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) return fail(HFMOE_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return HFMOE_OK;
}

int hfmoe_free(void* ptr) {
    if (!ptr) return HFMOE_OK;
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "hipFree");
}

int hfmoe_host_alloc(void** ptr, size_t bytes) {
    int rc = require_init();
    if (rc) return rc;
    if (!ptr) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null out pointer");
    hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
    if (e != hipSuccess) return fail(HFMOE_ERR_OUT_OF_MEMORY, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return HFMOE_OK;
}

int hfmoe_host_free(void* ptr) {
    if (!ptr) return HFMOE_OK;
    hipError_t e = hipHostFree(ptr);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "hipHostFree");
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    int rc = require_init();
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "hipMemcpy");
}

int hfmoe_memcpy_h2d(void* dst, const void* src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyHostToDevice); }
int hfmoe_memcpy_d2h(void* dst, const void* src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyDeviceToHost); }
int hfmoe_memcpy_d2d(void* dst, const void* src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyDeviceToDevice); }

int hfmoe_memset(void* ptr, int value, size_t bytes) {
    int rc = require_init();
    if (rc) return rc;
    hipError_t e = hipMemsetAsync(ptr, value, bytes, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "hipMemset");
}

int hfmoe_synchronize(void) {
    int rc = require_init();
    if (rc) return rc;
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "hipDeviceSynchronize");
}

int hfmoe_fill_normal_bf16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t tensor, uint64_t first,
                           float mean, float stdev) {
    int rc = require_init();
    if (rc) return rc;
    if (!dst && n) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null destination");
    hipError_t e = launch_fill_normal_bf16(dst, n, seed, tensor, first, mean, stdev, g.stream);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "fill_normal_bf16");
}

int hfmoe_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t tensor, uint64_t first,
                          float mean, float stdev) {
    int rc = require_init();
    if (rc) return rc;
    if (!dst && n) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null destination");
    hipError_t e = launch_fill_normal_f32(dst, n, seed, tensor, first, mean, stdev, g.stream);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "fill_normal_f32");
}

int hfmoe_profile_enable(int on) {
    int rc = require_init();
    if (rc) return rc;
    g.prof_on = on != 0;
    return HFMOE_OK;
}

int hfmoe_profile_read(hfmoe_kernel_stat* out, int max_entries, int* n_entries) {
    int rc = require_init();
    if (rc) return rc;
    prof_drain();
    int n = 0;
    for (auto& kv : g.kstats) {
        if (out && n < max_entries) {
            snprintf(out[n].name, sizeof out[n].name, "%s", kv.first.c_str());
            out[n].launches = kv.second.first;
            out[n].total_ms = kv.second.second;
        }
        ++n;
    }
    if (n_entries) *n_entries = n;
    return HFMOE_OK;
}

int hfmoe_profile_reset(void) {
    int rc = require_init();
    if (rc) return rc;
    prof_drain();
    g.kstats.clear();
    return HFMOE_OK;
}

int hfmoe_stats(uint64_t* pcie_bytes, uint64_t* gpu_active_ns) {
    if (pcie_bytes) *pcie_bytes = g.pcie_bytes;
    if (gpu_active_ns) *gpu_active_ns = g.gpu_active_ns;
    return HFMOE_OK;
}

}  // extern "C"
