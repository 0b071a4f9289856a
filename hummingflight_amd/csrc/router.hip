// router.hip -- MoE router for gfx950: BF16 gate GEMV and the per-token
// selection kernel (sigmoid, e_score_correction bias, (group-limited) top-k,
// normalisation, routed scaling; hf_select.h).
//
// Reference arithmetic: router GEMV glm_forward.cpp:519-520 (gemv_bf16_f32,
// cpu_kernels.cpp:43-94), then the selection of hf_select.h.
#include "hf_common.h"
#include "hf_kernels.h"
#include "hf_select.h"

namespace hf {

// Decode router GEMV (T = 1): block e computes logit e over 256 threads and
// its score pair (sigmoid, sigmoid + bias).  x is FP32, as the reference's
// moeLayer input (glm_forward.cpp:509).  Selection follows in a later kernel:
// a kernel boundary orders the scores for it, which costs less than a
// device-scope fence and counter in every block.
__global__ __launch_bounds__(256) void router_t1_kernel(const float* __restrict__ x, LayerDev L,
                                                        Cfg c, float* __restrict__ logits,
                                                        float2* __restrict__ scores) {
    __shared__ float red[4];
    const int e = blockIdx.x;
    const int t = threadIdx.x;
    const uint16_t* row = L.router + (size_t)e * c.d;
    // hidden <= 8192: at most 4 chunks of 8 per thread, all loads issued
    // before the first product.
    constexpr int kMaxCh = 8192 / 8 / 256;
    u32x4 w[kMaxCh];
    float4 xa[kMaxCh], xb[kMaxCh];
#pragma unroll
    for (int j = 0; j < kMaxCh; ++j) {
        const int ch = t + 256 * j;
        if (ch * 8 < c.d) {
            w[j] = ld_plain(reinterpret_cast<const u32x4*>(row) + ch);
            xa[j] = reinterpret_cast<const float4*>(x)[2 * ch];
            xb[j] = reinterpret_cast<const float4*>(x)[2 * ch + 1];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxCh; ++j) {
        if ((t + 256 * j) * 8 < c.d) {
            const float xv[8] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w, xb[j].x, xb[j].y, xb[j].z, xb[j].w};
            acc = dot8(w[j], xv, acc);
        }
    }
    acc = wave_sum(acc);
    if ((t & 63) == 0) red[t >> 6] = acc;
    __syncthreads();
    if (t == 0) {
        const float lg = (red[0] + red[1]) + (red[2] + red[3]);
        logits[e] = lg;
        scores[e] = score_pair(lg, L.bias, e);
    }
}

// Router logits for T tokens: block e reads router row e once and dots it with
// every token (x FP32 [T, d] from L2).  Output logits and score pairs [T, E].
__global__ __launch_bounds__(256) void router_logits_kernel(const float* __restrict__ x, int T,
                                                            LayerDev L, Cfg c,
                                                            float* __restrict__ logits,
                                                            float2* __restrict__ scores) {
    __shared__ float red[4][kRouterTokTile];
    const int e = blockIdx.x;
    const int t = threadIdx.x;
    const uint16_t* row = L.router + (size_t)e * c.d;
    const int nch = c.d / 8;
    for (int t0 = 0; t0 < T; t0 += kRouterTokTile) {
        const int nt = (T - t0) < kRouterTokTile ? (T - t0) : kRouterTokTile;
        float acc[kRouterTokTile];
#pragma unroll
        for (int j = 0; j < kRouterTokTile; ++j) acc[j] = 0.0f;
        for (int ch = t; ch < nch; ch += 256) {
            const u32x4 w = ld_plain(reinterpret_cast<const u32x4*>(row) + ch);
#pragma unroll
            for (int j = 0; j < kRouterTokTile; ++j) {
                if (j < nt) {
                    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)(t0 + j) * c.d);
                    const float4 xa = xr[2 * ch], xb = xr[2 * ch + 1];
                    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                    acc[j] = dot8(w, xv, acc[j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kRouterTokTile; ++j) {
            const float v = wave_sum(acc[j]);
            if ((t & 63) == 0) red[t >> 6][j] = v;
        }
        __syncthreads();
        if (t < nt) {
            const float lg = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
            logits[(size_t)(t0 + t) * c.E + e] = lg;
            scores[(size_t)(t0 + t) * c.E + e] = score_pair(lg, L.bias, e);
        }
        __syncthreads();
    }
}

// Selection for T tokens: one 256-thread block per token.
__global__ __launch_bounds__(kSelectThreads) void select_kernel(const float2* __restrict__ scores,
                                                                int T, Cfg c,
                                                                int* __restrict__ sel_idx,
                                                                float* __restrict__ sel_w) {
    __shared__ SelectSmem sm;
    const int tok = blockIdx.x;
    if (tok >= T) return;
    SelectRegs regs;
    select_fetch(scores + (size_t)tok * c.E, c.E, regs);
    const int kk = select_block(regs, c, sm);
    if ((int)threadIdx.x < kk) {
        sel_idx[(size_t)tok * c.k + threadIdx.x] = sm.sel[threadIdx.x];
        sel_w[(size_t)tok * c.k + threadIdx.x] = sm.w[threadIdx.x];
    }
}

hipError_t launch_router_logits_t1(const float* x, const LayerDev& L, const Cfg& c, float* logits,
                                   float2* scores, hipStream_t s) {
    return launch(router_t1_kernel, dim3(c.E), dim3(256), 0, s, x, L, c, logits, scores);
}

hipError_t launch_router_logits(const float* x, int T, const LayerDev& L, const Cfg& c,
                                float* logits, float2* scores, hipStream_t s) {
    return launch(router_logits_kernel, dim3(c.E), dim3(256), 0, s, x, T, L, c, logits, scores);
}

hipError_t launch_select(const float2* scores, int T, const Cfg& c, int* sel_idx, float* sel_w,
                         hipStream_t s) {
    return launch(select_kernel, dim3(T), dim3(kSelectThreads), 0, s, scores, T, c, sel_idx, sel_w);
}

}  // namespace hf
