// noalloc.hip -- the decode forward for callers that cannot allocate.
//
// hfmoe_moe_forward_noalloc runs the same T = 1 kernels as hfmoe_moe_forward
// (forward_t1_on, forward.hip), with their scratch -- router logits, score
// pairs, selected ids, routing weights and h -- in `scratch`, a file-scope
// device array of kScratchBytes that every GPU the library runs on holds until
// the process ends.  The call allocates nothing and creates no events.
//
// Host code never uses the array's name as an address: in host code it is a
// stand-in, not a device pointer.  hfmoe_init calls noalloc_setup(device) with
// that device current, which takes the device's own address of its copy with
// hipGetSymbolAddress once, and the entry point passes only that address to
// the kernels.  A failed setup does not fail hfmoe_init: only this entry
// point is then unavailable.
//
// Every call on one GPU shares that GPU's array and the last call's contents
// stay in it; each buffer is written in full by an earlier kernel of the same
// call before any kernel reads it, so nothing needs clearing.  Calls that
// overlap on one GPU (two streams, two threads) race on the array.
#include "hf_api_internal.h"

namespace hf {
namespace {

// Largest scratch of a configuration hfmoe_configure accepts: E <= 1024
// (logits 4 KB, score pairs 8 KB), k <= 8 (ids, weights) and
// (k + n_shared) * I * 4 <= 160 KB for h, each part 256-byte aligned.
constexpr size_t kScratchBytes = 192 * 1024;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

unsigned char* g_scratch_dev[kMaxDevices];  // per device: its copy's address
std::string g_setup_error;                   // why the last setup left no address

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Byte offsets of the five buffers for the configured layer shape; returns the
// total.
size_t layout(const Cfg& c, size_t off[5]) {
    const size_t sizes[5] = {sizeof(float) * (size_t)c.E, sizeof(float2) * (size_t)c.E, sizeof(int) * (size_t)c.k,
                             sizeof(float) * (size_t)c.k, sizeof(float) * (size_t)(c.k + c.n_shared) * c.I};
    size_t at = 0;
    for (int i = 0; i < 5; ++i) {
        off[i] = at;
        at += align256(sizes[i]);
    }
    return at;
}

}  // namespace

// Never fails hfmoe_init: on any error the device's address stays null, the
// reason is kept for the entry point's error message, and a sticky HIP error
// is cleared so that it does not surface in the next, unrelated call.
// HFMOE_NOALLOC_DISABLE=1 leaves the address unset on purpose (the entry
// point then reports HFMOE_ERR_NOT_INITIALIZED).
void noalloc_setup(int device) {
    char why[160];
    if (env_int("HFMOE_NOALLOC_DISABLE", 0)) {
        g_setup_error = "disabled by HFMOE_NOALLOC_DISABLE";
        return;
    }
    if (device < 0 || device >= kMaxDevices) {
        snprintf(why, sizeof why, "device %d: the scratch covers devices 0..%d", device, kMaxDevices - 1);
        g_setup_error = why;
        return;
    }
    if (g_scratch_dev[device]) return;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        snprintf(why, sizeof why, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_setup_error = why;
        return;
    }
    g_scratch_dev[device] = static_cast<unsigned char*>(p);
}

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_moe_forward_noalloc(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream) {
    int rc = require_cfg();
    if (rc) return rc;
    auto it = g.layers.find(layer);
    if (it == g.layers.end()) return fail(HFMOE_ERR_NOT_REGISTERED, "layer %d is not registered", layer);
    LayerState& L = it->second;
    if (L.dense) return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d is a dense MLP layer", layer);
    if (L.location != HFMOE_EXPERTS_DEVICE)
        return fail(HFMOE_ERR_UNSUPPORTED, "layer %d: the no-allocation forward needs HBM-resident experts", layer);
    if (T < 0 || T > 1)
        return fail(HFMOE_ERR_UNSUPPORTED, "T=%d: the no-allocation forward takes one token (T <= 1)", T);
    if (T == 0) return HFMOE_OK;
    if (!x_dev || !out_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null activation pointer");
    if ((reinterpret_cast<uintptr_t>(x_dev) | reinterpret_cast<uintptr_t>(out_dev)) & 15)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "activations must be 16-byte aligned");
    size_t off[5];
    const size_t need = layout(g.cfg, off);
    if (need > kScratchBytes)
        return fail(HFMOE_ERR_UNSUPPORTED, "layer shape needs %zu bytes of scratch, more than the %zu available", need,
                    kScratchBytes);
    unsigned char* base = (g.device >= 0 && g.device < kMaxDevices) ? g_scratch_dev[g.device] : nullptr;
    if (!base)
        return fail(HFMOE_ERR_NOT_INITIALIZED, "no-allocation scratch of device %d is not set up (%s)", g.device,
                    g_setup_error.empty() ? "unknown" : g_setup_error.c_str());
    const T1Buffers b{reinterpret_cast<float*>(base + off[0]), reinterpret_cast<float2*>(base + off[1]),
                      reinterpret_cast<int*>(base + off[2]), reinterpret_cast<float*>(base + off[3]),
                      reinterpret_cast<float*>(base + off[4])};
    return forward_t1_on(L, x_dev, out_dev, pick_stream(stream), b, false);
}

}  // extern "C"
