// router.hip -- MoE router for gfx950: BF16 gate GEMV, sigmoid,
// e_score_correction bias, (group-limited) top-k, normalisation, scaling.
//
// Reference arithmetic: router GEMV glm_forward.cpp:519-520 (gemv_bf16_f32,
// cpu_kernels.cpp:43-94), sigmoid glm_forward.cpp:522-524, F32 bias
// glm_forward.cpp:534-539, topKScores moe_router.h:29-57.  Group-limited
// selection is the DeepSeek-V3 noaux_tc rule (the reference parses topk_group
// but never applies it, config.cpp:117).
#include "hf_common.h"
#include "hf_kernels.h"

// Exact IEEE steps: no multiply-add contraction in this file.
#pragma clang fp contract(off)

namespace hf {

// sigmoid with a correctly rounded exp: exp evaluated in double and rounded
// once to float, then 1/(1+e) in IEEE single precision, matching the
// reference's 1.0f/(1.0f+std::exp(-x)) operation by operation.
__device__ __forceinline__ float sigmoid_cr(float x) {
    const float e = (float)exp(-(double)x);
    return 1.0f / (1.0f + e);
}

// One wavefront selects k experts for one token from its E router logits.
// Values live in registers, contiguous per lane (expert = lane*PER + v).
// Ranking key: score+bias descending, lower expert index first on ties.
template <int PER>
__device__ void select_token(const float* __restrict__ logits, const float* __restrict__ bias,
                             const Cfg& c, int* __restrict__ idx_out, float* __restrict__ w_out) {
    const int lane = threadIdx.x & 63;
    float val[PER], sc[PER];
#pragma unroll
    for (int v = 0; v < PER; ++v) {
        const int e = lane * PER + v;
        val[v] = -INFINITY;
        sc[v] = 0.0f;
        if (e < c.E) {
            sc[v] = sigmoid_cr(logits[e]);
            val[v] = bias ? sc[v] + bias[e] : sc[v];
        }
    }

    if (c.n_group > 1) {
        const int gs = c.E / c.n_group;
        float gscore = -INFINITY;  // lane g holds group g's score
        for (int g = 0; g < c.n_group; ++g) {
            float m1 = -INFINITY;
            int i1 = 0x7fffffff;
#pragma unroll
            for (int v = 0; v < PER; ++v) {
                const int e = lane * PER + v;
                if (e < c.E && e / gs == g && (val[v] > m1 || (val[v] == m1 && e < i1))) {
                    m1 = val[v];
                    i1 = e;
                }
            }
            wave_argmax(m1, i1);
            float m2 = -INFINITY;
            int i2 = 0x7fffffff;
#pragma unroll
            for (int v = 0; v < PER; ++v) {
                const int e = lane * PER + v;
                if (e < c.E && e / gs == g && e != i1 && (val[v] > m2 || (val[v] == m2 && e < i2))) {
                    m2 = val[v];
                    i2 = e;
                }
            }
            wave_argmax(m2, i2);
            const float score = (gs >= 2) ? m1 + m2 : m1;
            if (lane == g) gscore = score;
        }
        uint64_t kept = 0;
        float gv = (lane < c.n_group) ? gscore : -INFINITY;
        const int tg = c.topk_group < c.n_group ? c.topk_group : c.n_group;
        for (int r = 0; r < tg; ++r) {
            float bv = gv;
            int bi = (lane < c.n_group) ? lane : 0x7fffffff;
            wave_argmax(bv, bi);
            kept |= 1ull << bi;
            if (lane == bi) gv = -INFINITY;
        }
#pragma unroll
        for (int v = 0; v < PER; ++v) {
            const int e = lane * PER + v;
            if (e < c.E && !((kept >> (e / gs)) & 1ull)) val[v] = -INFINITY;
        }
    }

    int kk = c.k < kMaxTopK ? c.k : kMaxTopK;
    if (kk > c.E) kk = c.E;
    int sel[kMaxTopK];
    float w[kMaxTopK];
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r) {
        w[r] = 0.0f;
        sel[r] = 0;
        if (r >= kk) continue;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int v = 0; v < PER; ++v) {
            const int e = lane * PER + v;
            if (val[v] > bv || (val[v] == bv && e < bi)) {
                bv = val[v];
                bi = e;
            }
        }
        wave_argmax(bv, bi);
        float own = 0.0f;
#pragma unroll
        for (int v = 0; v < PER; ++v) {
            if (lane * PER + v == bi) {
                own = sc[v];
                val[v] = -INFINITY;
            }
        }
        // No finite candidate left (NaN logits): emit expert 0 with weight 0 so
        // every index handed to the expert kernels stays inside the table.
        const bool valid = bi < c.E;
        // moe_router.h:49-52: the winner's unbiased score, summed in rank order.
        w[r] = valid ? __shfl(own, bi / PER, 64) : 0.0f;
        if (!valid) bi = 0;
        sel[r] = bi;
        sum = sum + w[r];
    }
    if (lane == 0) {
        // moe_router.h:53-56: normalise, then scale.
#pragma unroll
        for (int r = 0; r < kMaxTopK; ++r) {
            if (r >= kk) continue;
            float wr = w[r];
            if (c.norm && sum > 0.0f) wr = wr / sum;
            wr = wr * c.scale;
            idx_out[r] = sel[r];
            w_out[r] = wr;
        }
    }
}

// Selection dispatch on E (values per lane = ceil(E/64)).
__device__ void select_any(const float* logits, const float* bias, const Cfg& c, int* idx_out,
                           float* w_out) {
    if (c.E <= 64)
        select_token<1>(logits, bias, c, idx_out, w_out);
    else if (c.E <= 128)
        select_token<2>(logits, bias, c, idx_out, w_out);
    else if (c.E <= 256)
        select_token<4>(logits, bias, c, idx_out, w_out);
    else if (c.E <= 512)
        select_token<8>(logits, bias, c, idx_out, w_out);
    else
        select_token<16>(logits, bias, c, idx_out, w_out);
}

// Decode router (T = 1): block e computes logit e over 256 threads, the last
// block to finish (agent-scope counter) runs the selection.  x is FP32, as the
// reference's moeLayer input (glm_forward.cpp:509).
__global__ __launch_bounds__(256) void router_t1_kernel(const float* __restrict__ x, LayerDev L,
                                                        Cfg c, float* __restrict__ logits,
                                                        int* __restrict__ sel_idx,
                                                        float* __restrict__ sel_w,
                                                        unsigned int* __restrict__ counter) {
    __shared__ float red[4];
    __shared__ int am_last;
    const int e = blockIdx.x;
    const int t = threadIdx.x;
    const uint16_t* row = L.router + (size_t)e * c.d;
    float acc = 0.0f;
    for (int ch = t; ch * 8 < c.d; ch += 256) {
        const u32x4 w = ld_plain(reinterpret_cast<const u32x4*>(row) + ch);
        const float4 xa = reinterpret_cast<const float4*>(x)[2 * ch];
        const float4 xb = reinterpret_cast<const float4*>(x)[2 * ch + 1];
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        acc = dot8(w, xv, acc);
    }
    acc = wave_sum(acc);
    if ((t & 63) == 0) red[t >> 6] = acc;
    __syncthreads();
    if (t == 0) {
        logits[e] = (red[0] + red[1]) + (red[2] + red[3]);
        __threadfence();
        const unsigned int prev = atomicAdd(counter, 1u);
        am_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!am_last) return;
    __threadfence();
    if (t < 64) {
        select_any(logits, L.bias, c, sel_idx, sel_w);
        if (t == 0) *counter = 0u;
    }
}

// Router logits for T tokens: block e reads router row e once and dots it with
// every token (x FP32 [T, d] from L2).  Output logits [T, E].
__global__ __launch_bounds__(256) void router_logits_kernel(const float* __restrict__ x, int T,
                                                            LayerDev L, Cfg c,
                                                            float* __restrict__ logits) {
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
        if (t < nt) logits[(size_t)(t0 + t) * c.E + e] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
        __syncthreads();
    }
}

// Selection for T tokens: one wave per token.
__global__ __launch_bounds__(64) void select_kernel(const float* __restrict__ logits, int T,
                                                    LayerDev L, Cfg c, int* __restrict__ sel_idx,
                                                    float* __restrict__ sel_w) {
    const int tok = blockIdx.x;
    if (tok >= T) return;
    select_any(logits + (size_t)tok * c.E, L.bias, c, sel_idx + (size_t)tok * c.k,
               sel_w + (size_t)tok * c.k);
}

hipError_t launch_router_t1(const float* x, const LayerDev& L, const Cfg& c, float* logits,
                            int* sel_idx, float* sel_w, unsigned int* counter, hipStream_t s) {
    hipLaunchKernelGGL(router_t1_kernel, dim3(c.E), dim3(256), 0, s, x, L, c, logits, sel_idx,
                       sel_w, counter);
    return hipGetLastError();
}

hipError_t launch_router_tokens(const float* x, int T, const LayerDev& L, const Cfg& c,
                                float* logits, int* sel_idx, float* sel_w, hipStream_t s) {
    hipLaunchKernelGGL(router_logits_kernel, dim3(c.E), dim3(256), 0, s, x, T, L, c, logits);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(select_kernel, dim3(T), dim3(64), 0, s, logits, T, L, c, sel_idx, sel_w);
    return hipGetLastError();
}

}  // namespace hf
