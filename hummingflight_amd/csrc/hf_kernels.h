// hf_kernels.h -- launchers of the MoE-block kernels (host side).
#pragma once

#include <hip/hip_ext.h>

#include "hf_common.h"

namespace hf {

// Timing hook: while set, launches record their dispatch timestamps into
// these events (hipExtLaunchKernelGGL): the first launch of a timed section
// records `start` (then cleared), every launch re-records `stop`, so a section
// of one kernel measures that kernel alone, with no extra packets queued, and
// a section of several spans the first one's start to the last one's end.
struct LaunchTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
extern LaunchTiming g_timing;

template <typename... Params>
inline hipError_t launch_exact(void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t shmem,
                               hipStream_t s, Params... args) {
    // The launch reports through the thread's last-error slot: clear what an
    // earlier call left there (a refused allocation, say) so it is not taken
    // for this launch's failure.
    (void)hipGetLastError();
    if (g_timing.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, g_timing.start, g_timing.stop, 0u, args...);
        g_timing.start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
    }
    return hipGetLastError();
}

// Launch with every argument converted to the kernel's exact parameter type
// (the extended launch packs arguments by their own types).
template <typename... Params, typename... Args>
inline hipError_t launch(void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t shmem,
                         hipStream_t s, Args... args) {
    static_assert(sizeof...(Params) == sizeof...(Args), "kernel argument count");
    return launch_exact<Params...>(kernel, grid, block, shmem, s, static_cast<Params>(args)...);
}

constexpr int kRouterTokTile = 8;   // tokens per pass of the multi-token router GEMV
// Largest max_tokens of a configuration: keeps every [rows, hidden] index of
// the multi-token path (rows = T * (k + n_shared) <= 131072) below 2^31.
constexpr int kMaxTokens = 8192;
constexpr int kMaxSlots = 16;       // routed + shared slices handled by the T=1 GEMVs
constexpr int kDownMaxRows = 64;    // output rows per block of the decode down projection

// router.hip
// Logits [E] of one token (x FP32 [d]) and score pairs (sigmoid, sigmoid + bias).
hipError_t launch_router_logits_t1(const float* x, const LayerDev& L, const Cfg& c, float* logits,
                                   float2* scores, hipStream_t s);
// Logits and score pairs [T, E] of T tokens.
hipError_t launch_router_logits(const float* x, int T, const LayerDev& L, const Cfg& c,
                                float* logits, float2* scores, hipStream_t s);
// (Group-limited) top-k + normalise + scale from score pairs, one wave per
// token: sel_idx/sel_w [T, k].
hipError_t launch_select(const float2* scores, int T, const Cfg& c, int* sel_idx, float* sel_w,
                         hipStream_t s);

// expert_gemv.hip -- decode (T = 1) expert SwiGLU.
// Slots 0..k-1 are the selected experts (sel_idx), slots k.. are the shared
// expert's n_shared slices of I rows.  h: FP32 [nslots, I].
// With `scores` (E <= 256) the kernel routes in place and writes sel_idx/sel_w;
// without, sel_idx holds the k routed ids on entry.
hipError_t launch_gateup_t1(const float* x, const LayerDev& L, const Cfg& c, const float2* scores,
                            int* sel_idx, float* sel_w, float* h, int nslots, int blocks,
                            hipStream_t s);
// out[j] = sum_s weight_s * (Wd_s[j,:] . h_s) (+ addend[j] when addend is not null);
// weight = sel_w for routed slots, 1 for shared slices.
hipError_t launch_down_t1(const float* h, const LayerDev& L, const Cfg& c, const int* sel_idx,
                          const float* sel_w, const float* addend, float* out, int nslots,
                          int blocks, hipStream_t s);

// Single-expert FFN on explicit device weights (the per-expert boundary of
// gpuExpertFFN, cuda_backend.h:79-85): out = Wd.(silu(Wg.x) * (Wu.x)).
hipError_t launch_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                             const float* x, float* h, float* out, int d, int I, int gu_blocks,
                             int dn_blocks, hipStream_t s);

// rng.hip -- seeded synthetic tensors (same bits as the generator the tests use).
hipError_t launch_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                   uint64_t first, float mean, float stdev, hipStream_t s);
hipError_t launch_fill_normal_f32(float* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                  uint64_t first, float mean, float stdev, hipStream_t s);

}  // namespace hf
