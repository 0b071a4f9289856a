// hf_common.h -- shared device helpers for the MoE-block kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hf {

// Layer configuration as the kernels see it (ModelConfig MoE fields,
// src/model/config.h:49-58, plus the group-limited routing extension).
struct Cfg {
    int d;           // hidden
    int I;           // moe_intermediate (one routed expert)
    int E;           // routed experts
    int k;           // experts per token (<= 8)
    int n_group;     // 1 = flat selection
    int topk_group;
    int n_shared;    // shared expert = n_shared slices of I rows
    int norm;        // norm_topk_prob
    float scale;     // routed_scaling_factor
    float eps;       // rms_norm_eps
};

// Device view of one layer's weights.  etab holds 3*E device pointers
// (gate_e [I,d], up_e [I,d], down_e [d,I]) in HBM.
struct LayerDev {
    const uint16_t* router;   // [E, d]
    const float* bias;        // [E] or null
    const uint16_t* sg;       // [n_shared*I, d]
    const uint16_t* su;       // [n_shared*I, d]
    const uint16_t* sd;       // [d, n_shared*I]
    const uint16_t* const* etab;
};

constexpr int kMaxTopK = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// Round-to-nearest-even F32 -> BF16 bits (same rule as dtype_bf16.h:27-33).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// 8 BF16 (one 16-byte chunk) dotted with 8 FP32 values.
__device__ __forceinline__ float dot8(const u32x4 w, const float* x, float acc) {
    acc = fmaf(bf_lo(w.x), x[0], acc);
    acc = fmaf(bf_hi(w.x), x[1], acc);
    acc = fmaf(bf_lo(w.y), x[2], acc);
    acc = fmaf(bf_hi(w.y), x[3], acc);
    acc = fmaf(bf_lo(w.z), x[4], acc);
    acc = fmaf(bf_hi(w.z), x[5], acc);
    acc = fmaf(bf_lo(w.w), x[6], acc);
    acc = fmaf(bf_hi(w.w), x[7], acc);
    return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Wave-wide argmax over (value desc, index asc); every lane gets the winner.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(v, o, 64);
        const int i2 = __shfl_xor(i, o, 64);
        if (v2 > v || (v2 == v && i2 < i)) {
            v = v2;
            i = i2;
        }
    }
}

// Weight loads that stream through the cache hierarchy once.
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ u32x4 ld_plain(const u32x4* p) { return *p; }

}  // namespace hf
