// hf_kernels.h -- launchers of the MoE-block kernels (host side).
#pragma once

#include "hf_common.h"

namespace hf {

constexpr int kMaxExperts = 1024;   // selection keeps ceil(E/64) scores per lane
constexpr int kRouterTokTile = 8;   // tokens per pass of the multi-token router GEMV
constexpr int kMaxSlots = 16;       // routed + shared slices handled by the T=1 GEMVs

// router.hip
hipError_t launch_router_t1(const float* x, const LayerDev& L, const Cfg& c, float* logits,
                            int* sel_idx, float* sel_w, unsigned int* counter, hipStream_t s);
hipError_t launch_router_tokens(const float* x, int T, const LayerDev& L, const Cfg& c,
                                float* logits, int* sel_idx, float* sel_w, hipStream_t s);

// expert_gemv.hip -- decode (T = 1) expert SwiGLU.
// Slots 0..k-1 are the selected experts (sel_idx), slots k.. are the shared
// expert's n_shared slices of I rows.  h: FP32 [nslots, I].
hipError_t launch_gateup_t1(const float* x, const LayerDev& L, const Cfg& c, const int* sel_idx,
                            float* h, int nslots, int blocks, hipStream_t s);
// out[j] = sum_s weight_s * (Wd_s[j,:] . h_s) (+ addend[j] when addend is not null);
// weight = sel_w for routed slots, 1 for shared slices.
hipError_t launch_down_t1(const float* h, const LayerDev& L, const Cfg& c, const int* sel_idx,
                          const float* sel_w, const float* addend, float* out, int nslots,
                          int blocks, hipStream_t s);

// Single-expert FFN on explicit device weights (the per-expert boundary of
// gpuExpertFFN, cuda_backend.h:79-85): out = Wd.(silu(Wg.x) * (Wu.x)).
hipError_t launch_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                             const float* x, float* h, float* out, int d, int I, int blocks,
                             hipStream_t s);

// rng.hip -- seeded synthetic tensors (same bits as the generator the tests use).
hipError_t launch_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                   uint64_t first, float mean, float stdev, hipStream_t s);
hipError_t launch_fill_normal_f32(float* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                  uint64_t first, float mean, float stdev, hipStream_t s);

}  // namespace hf
