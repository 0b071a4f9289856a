// hf_select.h -- noaux_tc expert selection for one token by one 256-thread block.
//
// Reference arithmetic: sigmoid glm_forward.cpp:522-524 (moe_router.h:19-21),
// F32 correction bias glm_forward.cpp:534-539, topKScores moe_router.h:29-57
// (rank on score + bias, weights = unbiased scores of the winners summed in
// rank order, divided by that sum when normalising, then scaled).  Group-limited
// selection is the DeepSeek-V3 noaux_tc rule (the reference parses topk_group
// but never applies it, config.cpp:117): group score = largest + second largest
// biased score of the group, keep the best topk_group groups, then top-k among
// their experts.  Ties: lower expert (or group) index first.
//
// Rank by counting on 64-bit keys: high word = the ranking value's bits mapped
// to an order-preserving unsigned integer, low word = ~expert, so "ranks
// before" is one unsigned compare and every key is distinct.  Stage A ranks
// each expert inside its chunk (its group, or 32 experts); only a chunk's top
// 8 can reach the global top 8, so stage D ranks those few candidates against
// each other.  All ranks are counted in parallel from LDS: no chain of
// wave-wide reductions.
//
// Every floating-point step is a single IEEE operation written out in this
// file with contraction off, and the sigmoid is glibc's expf algorithm
// (hf_expf.h), so given the same logits the selection and the weights are the
// reference's bit for bit.
#pragma once

#include "hf_common.h"
#include "hf_expf.h"

namespace hf {

constexpr int kSelectThreads = 256;
constexpr int kSelectPerThread = kMaxExperts / kSelectThreads;
constexpr int kSelectChunk = 32;    // preferred chunk size for stage A
constexpr int kSelectMaxChunks = 64;

// Score pair of one expert, written by the router kernels next to its logit:
// s = sigmoid(logit) (glm_forward.cpp:522-524) and key = s + bias
// (moe_router.h:38-41), the value experts are ranked on.
__device__ __forceinline__ float2 score_pair(float logit, const float* bias, int e) {
#pragma clang fp contract(off)
    const float s = router_sigmoid(logit);
    return make_float2(s, bias ? s + bias[e] : s);
}

// Order-preserving map of a float to uint32 (-0 folded onto +0, NaN below -inf).
__device__ __forceinline__ uint32_t ordered_bits(float v) {
    if (v != v) return 0u;
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float ordered_value(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

__device__ __forceinline__ uint64_t select_key(float v, int e) {
    return ((uint64_t)ordered_bits(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

__device__ __forceinline__ int key_expert(uint64_t k) {
    return (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
}

// Number of keys[j], j in [j0, j0 + n), greater than ke.  keys lives in LDS;
// lanes reading the same chunk share each read (broadcast).
__device__ __forceinline__ int count_greater(const uint64_t* keys, int j0, int n, uint64_t ke) {
    int cnt = 0;
    int j = j0;
    if ((j0 & 1) == 0) {
        for (; j + 8 <= j0 + n; j += 8) {
            const ulonglong2 a = *reinterpret_cast<const ulonglong2*>(keys + j);
            const ulonglong2 b = *reinterpret_cast<const ulonglong2*>(keys + j + 2);
            const ulonglong2 c = *reinterpret_cast<const ulonglong2*>(keys + j + 4);
            const ulonglong2 d = *reinterpret_cast<const ulonglong2*>(keys + j + 6);
            cnt += (a.x > ke) + (a.y > ke) + (b.x > ke) + (b.y > ke) + (c.x > ke) + (c.y > ke) +
                   (d.x > ke) + (d.y > ke);
        }
    }
    for (; j < j0 + n; ++j) cnt += keys[j] > ke;
    return cnt;
}

// LDS of one block-level selection.
struct SelectSmem {
    uint64_t key[kMaxExperts] __attribute__((aligned(16)));
    uint64_t top[kSelectMaxChunks][kMaxTopK];  // per chunk: keys by chunk rank
    float sc[kMaxExperts];                     // unbiased scores
    float gscore[kMaxGroups];
    int kept[kSelectMaxChunks];                // per chunk: its group is kept
    int sel[kMaxTopK];
    float w[kMaxTopK];
};

// This thread's score pairs (experts t, t + 256, ...), loaded ahead of other
// memory traffic so that later waits on them do not queue behind it.
struct SelectRegs {
    float2 p[kSelectPerThread];
};

__device__ __forceinline__ void select_fetch(const float2* __restrict__ scores, int E,
                                             SelectRegs& r) {
#pragma unroll
    for (int v = 0; v < kSelectPerThread; ++v) {
        const int e = (int)threadIdx.x + v * kSelectThreads;
        r.p[v] = e < E ? scores[e] : make_float2(0.0f, 0.0f);
    }
}

// Chunk size for E experts in groups of gs: the group itself when it has at
// most 32 experts, else 32 when that tiles the group, else the whole group.
__device__ __forceinline__ int select_chunk(int gs) {
    return gs <= kSelectChunk ? gs : (gs % kSelectChunk == 0 ? kSelectChunk : gs);
}

// Select k experts for one token from its score pairs [E] (fetched by
// select_fetch).  Must be called by all 256 threads of the block (it
// synchronises the block).  On return sm.sel[r] / sm.w[r] (r < k) hold the ids
// in rank order and the final weights; the return value is k.
__device__ __forceinline__ int select_block(const SelectRegs& regs, const Cfg& c, SelectSmem& sm) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    int kk = c.k < kMaxTopK ? c.k : kMaxTopK;
    if (kk > c.E) kk = c.E;
    const int ng = c.n_group > 1 ? c.n_group : 1;
    const int gs = c.E / ng;
    const int cs = select_chunk(gs);
    const int nchunks = c.E / cs;
    const int per_chunk = cs < kMaxTopK ? cs : kMaxTopK;
    uint64_t mykey[kSelectPerThread];
#pragma unroll
    for (int v = 0; v < kSelectPerThread; ++v) {
        const int e = t + v * kSelectThreads;
        mykey[v] = 0;
        if (e < c.E) {
            sm.sc[e] = regs.p[v].x;
            mykey[v] = select_key(regs.p[v].y, e);
            sm.key[e] = mykey[v];
        }
    }
    if (t < kMaxTopK) {
        sm.sel[t] = 0;
        sm.w[t] = 0.0f;
    }
    if (t < nchunks) sm.kept[t] = 1;
    __syncthreads();

    // Stage A: rank inside the chunk; the chunk's top entries in rank order.
#pragma unroll
    for (int v = 0; v < kSelectPerThread; ++v) {
        const int e = t + v * kSelectThreads;
        if (e < c.E) {
            const int ch = e / cs;
            const int rk = count_greater(sm.key, ch * cs, cs, mykey[v]);
            if (rk < kMaxTopK) sm.top[ch][rk] = mykey[v];
        }
    }
    __syncthreads();

    if (ng > 1) {
        // Stage B: group score = largest + second largest key value of the group.
        const int cpg = gs / cs;  // chunks per group
        if (t < ng) {
            uint64_t b1 = 0, b2 = 0;
            for (int ch = t * cpg; ch < (t + 1) * cpg; ++ch) {
                for (int r = 0; r < 2 && r < per_chunk; ++r) {
                    const uint64_t k = sm.top[ch][r];
                    if (k > b1) {
                        b2 = b1;
                        b1 = k;
                    } else if (k > b2) {
                        b2 = k;
                    }
                }
            }
            const float v1 = ordered_value((uint32_t)(b1 >> 32));
            sm.gscore[t] = gs >= 2 ? v1 + ordered_value((uint32_t)(b2 >> 32)) : v1;
        }
        __syncthreads();
        // Stage C: keep the topk_group best groups (ties: lower group index).
        if (t < ng) {
            const float gv = sm.gscore[t];
            int rk = 0;
            for (int g = 0; g < ng; ++g) {
                const float o = sm.gscore[g];
                rk += (o > gv || (o == gv && g < t)) ? 1 : 0;
            }
            const int keep = rk < c.topk_group;
            for (int ch = t * cpg; ch < (t + 1) * cpg; ++ch) sm.kept[ch] = keep;
        }
        __syncthreads();
    }

    // Stage D: rank each kept chunk's top entries against all of them.
    for (int cand = t; cand < nchunks * kMaxTopK; cand += kSelectThreads) {
        const int ch = cand / kMaxTopK, r = cand % kMaxTopK;
        if (r >= per_chunk || !sm.kept[ch]) continue;
        const uint64_t k = sm.top[ch][r];
        int rk = 0;
        for (int o = 0; o < nchunks; ++o) {
            if (!sm.kept[o]) continue;
#pragma unroll
            for (int q = 0; q < kMaxTopK; ++q) rk += (q < per_chunk && sm.top[o][q] > k) ? 1 : 0;
        }
        if (rk < kk) {
            const int e = key_expert(k);
            sm.sel[rk] = e;
            sm.w[rk] = sm.sc[e];
        }
    }
    __syncthreads();
    if (t == 0) {
        // moe_router.h:49-56: rank-order sum of the unbiased scores, normalise, scale.
        float sum = 0.0f;
        for (int r = 0; r < kk; ++r) sum = sum + sm.w[r];
        for (int r = 0; r < kk; ++r) {
            float wr = sm.w[r];
            if (c.norm && sum > 0.0f) wr = wr / sum;
            sm.w[r] = wr * c.scale;
        }
    }
    __syncthreads();
    return kk;
}

}  // namespace hf
