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
constexpr int kMaxGroups = 64;
constexpr int kMaxExperts = 1024;

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

// ---- cross-lane steps on the DPP network (GFX9 encodings) ----
// quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_ror:4 = 0x124,
// row_ror:8 = 0x128, row_mirror = 0x140, row_half_mirror = 0x141.
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes; every lane gets the same value (fixed order: rows by
// DPP butterfly, then (row0 + row1) + (row2 + row3)).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kDppQuadXor1>(v);
    v += dpp_f<kDppQuadXor2>(v);
    v += dpp_f<kDppRowRor4>(v);
    v += dpp_f<kDppRowRor8>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
    const float v2 = dpp_f<CTRL>(v);
    const int i2 = dpp_i<CTRL>(i);
    if (ranks_before(v2, i2, v, i)) {
        v = v2;
        i = i2;
    }
}

// Wave-wide argmax over (value desc, index asc); every lane gets the winner.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    argmax_step<kDppQuadXor1>(v, i);
    argmax_step<kDppQuadXor2>(v, i);
    argmax_step<kDppRowRor4>(v, i);
    argmax_step<kDppRowRor8>(v, i);
    float bv = readlane_f(v, 0);
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float rv = readlane_f(v, r);
        const int ri = __builtin_amdgcn_readlane(i, r);
        if (ranks_before(rv, ri, bv, bi)) {
            bv = rv;
            bi = ri;
        }
    }
    v = bv;
    i = bi;
}

// Weight loads that stream through the cache hierarchy once.
// Through a global (not generic) pointer: a generic one compiles to a FLAT
// load, which counts in both vmcnt and lgkmcnt, so every wait for it becomes
// vmcnt(0) lgkmcnt(0) and no load can stay in flight across a wait.
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)p);
}

__device__ __forceinline__ u32x4 ld_plain(const u32x4* p) { return *p; }

}  // namespace hf
