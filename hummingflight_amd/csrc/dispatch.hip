// dispatch.hip -- token-to-expert dispatch as a stable counting sort (gfx950).
//
// The reference has no batched MoE (it loops token by token, glm_forward.cpp:755,
// and expert by expert, :581); this is the multi-token path's dispatch: pairs
// p = t*k + r sorted by (expert, p), with per-expert counts and offsets, the
// same order the CPU oracle's orc_dispatch produces (its stable counting sort).
//
// One workgroup of 1024 threads:
//   1. histogram of experts (LDS atomics: order cannot matter for counts);
//   2. block-wide exclusive scans of the counts and of the per-expert M-tile
//      counts ceil(count_e / tile_rows) -> offsets[E+1] and the M-tile list of
//      the grouped GEMM, in expert order, then the tiles of the shared group;
//   3. stable scatter, 1024 pairs per pass in pair order: a pair's slot is
//      cursor[e] + (same-expert pairs in earlier wavefronts of the pass) +
//      (same-expert pairs in earlier lanes of its wavefront).  The in-wave
//      match mask comes from one ballot per key bit, so the result is fully
//      deterministic with no atomics on positions.
#include "hf_api_internal.h"
#include "hf_grouped.h"

namespace hf {

constexpr int kDispatchThreads = 1024;
constexpr int kDispatchWaves = kDispatchThreads / 64;

// Inclusive scan of v over the 1024 threads of the block (wsum: [16] LDS).
__device__ __forceinline__ int block_scan(int v, int* wsum) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(v, off);
        if (lane >= off) v += y;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    __syncthreads();
    return v + before;
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int* __restrict__ idx, int npairs, int k, int E, int key_bits, int tile_rows, int shared_rows,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ perm,
    int* __restrict__ row_token, int* __restrict__ tile_expert, int* __restrict__ tile_row0,
    int* __restrict__ ntiles_out) {
    extern __shared__ int smem[];
    int* cnt = smem;                        // [E]
    int* cursor = cnt + E;                  // [E]
    int* whist = cursor + E;                // [waves][E]
    __shared__ int wsum[kDispatchWaves];
    __shared__ int totals[2];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;

    for (int e = t; e < E; e += kDispatchThreads) cnt[e] = 0;
    __syncthreads();
    for (int p = t; p < npairs; p += kDispatchThreads) {
        const int e = min(max(idx[p], 0), E - 1);
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Scans over experts in chunks of 1024 (E <= 1024 in practice: one chunk).
    int run_rows = 0, run_tiles = 0;
    for (int e0 = 0; e0 < E; e0 += kDispatchThreads) {
        const int e = e0 + t;
        const int c = e < E ? cnt[e] : 0;
        const int nt = (c + tile_rows - 1) / tile_rows;
        const int c_inc = block_scan(c, wsum);
        const int t_inc = block_scan(nt, wsum);
        if (e < E) {
            const int r0 = run_rows + c_inc - c;
            const int tl0 = run_tiles + t_inc - nt;
            offsets[e] = r0;
            cursor[e] = r0;
            counts[e] = c;
            for (int j = 0; j < nt; ++j) {
                tile_expert[tl0 + j] = e;
                tile_row0[tl0 + j] = r0 + j * tile_rows;
            }
        }
        if (t == kDispatchThreads - 1) {
            totals[0] = c_inc;
            totals[1] = t_inc;
        }
        __syncthreads();
        run_rows += totals[0];
        run_tiles += totals[1];
        __syncthreads();
    }
    // The shared group: rows npairs + i <- token i.
    const int shared_tiles = (shared_rows + tile_rows - 1) / tile_rows;
    for (int j = t; j < shared_tiles; j += kDispatchThreads) {
        tile_expert[run_tiles + j] = E;
        tile_row0[run_tiles + j] = npairs + j * tile_rows;
    }
    for (int i = t; i < shared_rows; i += kDispatchThreads) {
        perm[npairs + i] = npairs + i;
        row_token[npairs + i] = i;
    }
    if (t == 0) {
        offsets[E] = run_rows;
        offsets[E + 1] = run_rows + shared_rows;
        *ntiles_out = run_tiles + shared_tiles;
    }
    __syncthreads();

    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < npairs; base += kDispatchThreads) {
        for (int i = t; i < kDispatchWaves * E; i += kDispatchThreads) whist[i] = 0;
        __syncthreads();
        const int p = base + t;
        const bool valid = p < npairs;
        const int e = valid ? min(max(idx[p], 0), E - 1) : 0;
        uint64_t same = __ballot(valid);
        for (int b = 0; b < key_bits; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t vote = __ballot(bit);
            same &= bit ? vote : ~vote;
        }
        const int rank_in_wave = __popcll(same & lt_mask);
        if (valid && rank_in_wave == 0) whist[wave * E + e] = __popcll(same);
        __syncthreads();
        if (valid) {
            int before = 0;
            for (int w = 0; w < wave; ++w) before += whist[w * E + e];
            const int slot = cursor[e] + before + rank_in_wave;
            perm[slot] = p;
            row_token[slot] = p / k;
        }
        __syncthreads();
        for (int ee = t; ee < E; ee += kDispatchThreads) {
            int add = 0;
            for (int w = 0; w < kDispatchWaves; ++w) add += whist[w * E + ee];
            cursor[ee] += add;
        }
        __syncthreads();
    }
}

hipError_t launch_dispatch(const int* idx, int T, int k, int E, int tile_rows, int shared_rows,
                           int* counts, int* offsets, int* perm, int* row_token, int* tile_expert,
                           int* tile_row0, int* ntiles, hipStream_t s) {
    int bits = 1;
    while ((1 << bits) < E) ++bits;
    const size_t lds = sizeof(int) * (size_t)E * (2 + kDispatchWaves);
    static size_t lds_raised = 0;
    if (lds > 48 * 1024 && lds > lds_raised) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(dispatch_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        lds_raised = lds;
    }
    return launch(dispatch_kernel, dim3(1), dim3(kDispatchThreads), (uint32_t)lds, s, idx, T * k, k,
                  E, bits, tile_rows, shared_rows, counts, offsets, perm, row_token, tile_expert,
                  tile_row0, ntiles);
}

}  // namespace hf
