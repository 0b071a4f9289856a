// dispatch.hip -- token-to-expert dispatch as a stable counting sort (gfx950).
//
// The reference has no batched MoE (it loops token by token, glm_forward.cpp:755,
// and expert by expert, :581); this is the multi-token path's dispatch: pairs
// p = t*k + r sorted by (expert, p), with per-expert counts and offsets, the
// same order the CPU oracle's orc_dispatch produces (its stable counting sort).
//
// Small batches, one workgroup of 1024 threads (large batches split steps 1
// and 3 over pair chunks, see dispatch_count_kernel):
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
// From this many passes of 1024 pairs on, the counting and the scatter run
// in up to kDispatchMaxChunks workgroups (three launches instead of one).
constexpr int kDispatchSplitPasses = 8;

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

// Offsets, counts and the M-tile lists (tl[0], and tl[1] when its rows are
// set) from the per-expert counts cnt[E] (LDS); cursor[e] = offsets[e].  Then
// the shared group: rows npairs + i <- token i.
__device__ void dispatch_plan(const int* cnt, int* cursor, int npairs, int E, const TileList* tl, int shared_rows,
                              int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ perm,
                              int* __restrict__ row_token, unsigned* __restrict__ item_ctr, int* wsum, int* totals) {
    const int t = threadIdx.x;
    if (item_ctr && t < kItemCounters) item_ctr[t] = 0u;  // the grouped GEMMs' work counters
    const int nl = tl[1].rows > 0 ? 2 : 1;
    // Scans over experts in chunks of 1024 (E <= 1024 in practice: one chunk).
    int run_rows = 0, run_tiles[2] = {0, 0};
    for (int e0 = 0; e0 < E; e0 += kDispatchThreads) {
        const int e = e0 + t;
        const int c = e < E ? cnt[e] : 0;
        const int c_inc = block_scan(c, wsum);
        const int r0 = run_rows + c_inc - c;
        if (e < E) {
            offsets[e] = r0;
            cursor[e] = r0;
            counts[e] = c;
        }
        if (t == kDispatchThreads - 1) totals[0] = c_inc;
#pragma unroll
        for (int l = 0; l < 2; ++l) {
            if (l >= nl) break;
            const int rows = tl[l].rows;
            const int nt = (c + rows - 1) / rows;
            const int t_inc = block_scan(nt, wsum);
            const int tl0 = run_tiles[l] + t_inc - nt;
            for (int j = 0; j < nt; ++j) {
                tl[l].expert[tl0 + j] = e;
                tl[l].row0[tl0 + j] = r0 + j * rows;
            }
            if (t == kDispatchThreads - 1) totals[1 + l] = t_inc;
        }
        __syncthreads();
        run_rows += totals[0];
#pragma unroll
        for (int l = 0; l < 2; ++l)
            if (l < nl) run_tiles[l] += totals[1 + l];
        __syncthreads();
    }
#pragma unroll
    for (int l = 0; l < 2; ++l) {
        if (l >= nl) break;
        const int rows = tl[l].rows;
        const int shared_tiles = (shared_rows + rows - 1) / rows;
        for (int j = t; j < shared_tiles; j += kDispatchThreads) {
            tl[l].expert[run_tiles[l] + j] = E;
            tl[l].row0[run_tiles[l] + j] = npairs + j * rows;
        }
        if (t == 0) *tl[l].count = run_tiles[l] + shared_tiles;
    }
    for (int i = t; i < shared_rows; i += kDispatchThreads) {
        perm[npairs + i] = npairs + i;
        row_token[npairs + i] = i;
    }
    if (t == 0) {
        offsets[E] = run_rows;
        offsets[E + 1] = run_rows + shared_rows;
    }
    __syncthreads();
}

// Stable scatter of pairs [begin, end), 1024 per pass in pair order: a pair's
// slot is cursor[e] + (same-expert pairs in earlier wavefronts of the pass) +
// (same-expert pairs in earlier lanes of its wavefront); cursor (LDS) advances.
__device__ void dispatch_scatter(const int* __restrict__ idx, int begin, int end, int k, int E, int key_bits,
                                 int* cursor, int* whist, int* __restrict__ perm, int* __restrict__ row_token) {
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = begin; base < end; base += kDispatchThreads) {
        for (int i = t; i < kDispatchWaves * E; i += kDispatchThreads) whist[i] = 0;
        __syncthreads();
        const int p = base + t;
        const bool valid = p < end;
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

// Histogram of experts over pairs [begin, end) into cnt[E] (LDS atomics:
// order cannot matter for counts).
__device__ void dispatch_count(const int* __restrict__ idx, int begin, int end, int E, int* cnt) {
    for (int e = threadIdx.x; e < E; e += kDispatchThreads) cnt[e] = 0;
    __syncthreads();
    for (int p = begin + (int)threadIdx.x; p < end; p += kDispatchThreads) atomicAdd(&cnt[min(max(idx[p], 0), E - 1)], 1);
    __syncthreads();
}

// Small batches: everything in one workgroup.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int* __restrict__ idx, int npairs, int k, int E, int key_bits, TileList tl0, TileList tl1,
    int shared_rows, int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ perm,
    int* __restrict__ row_token, unsigned* __restrict__ item_ctr) {
    extern __shared__ int smem[];
    int* cnt = smem;              // [E]
    int* cursor = cnt + E;        // [E]
    int* whist = cursor + E;      // [waves][E]
    __shared__ int wsum[kDispatchWaves];
    __shared__ int totals[3];
    const TileList tl[2] = {tl0, tl1};
    dispatch_count(idx, 0, npairs, E, cnt);
    dispatch_plan(cnt, cursor, npairs, E, tl, shared_rows, counts, offsets, perm, row_token, item_ctr, wsum, totals);
    dispatch_scatter(idx, 0, npairs, k, E, key_bits, cursor, whist, perm, row_token);
}

// Large batches, step 1 of 3: workgroup b counts the experts of pair chunk b
// (pairs [b * chunk, (b + 1) * chunk)) into chunk_hist[b][E].
__global__ __launch_bounds__(kDispatchThreads) void dispatch_count_kernel(const int* __restrict__ idx, int npairs,
                                                                          int E, int chunk,
                                                                          int* __restrict__ chunk_hist) {
    extern __shared__ int smem[];
    const int b = blockIdx.x;
    dispatch_count(idx, b * chunk, min(npairs, (b + 1) * chunk), E, smem);
    for (int e = threadIdx.x; e < E; e += kDispatchThreads) chunk_hist[(size_t)b * E + e] = smem[e];
}

// Step 2: one workgroup sums the chunk counts, plans offsets and tiles, and
// turns chunk_hist[b][e] into the first slot of chunk b's expert-e pairs.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_plan_kernel(
    int nchunks, int npairs, int E, TileList tl0, TileList tl1, int shared_rows, int* __restrict__ chunk_hist,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ perm, int* __restrict__ row_token,
    unsigned* __restrict__ item_ctr) {
    extern __shared__ int smem[];
    int* cnt = smem;        // [E]
    int* cursor = cnt + E;  // [E]
    __shared__ int wsum[kDispatchWaves];
    __shared__ int totals[3];
    const TileList tl[2] = {tl0, tl1};
    for (int e = threadIdx.x; e < E; e += kDispatchThreads) {
        int c = 0;
#pragma unroll 8
        for (int b = 0; b < nchunks; ++b) c += chunk_hist[(size_t)b * E + e];
        cnt[e] = c;
    }
    __syncthreads();
    dispatch_plan(cnt, cursor, npairs, E, tl, shared_rows, counts, offsets, perm, row_token, item_ctr, wsum, totals);
    for (int e = threadIdx.x; e < E; e += kDispatchThreads) {
        int run = cursor[e];
#pragma unroll 8
        for (int b = 0; b < nchunks; ++b) {
            const int c = chunk_hist[(size_t)b * E + e];
            chunk_hist[(size_t)b * E + e] = run;
            run += c;
        }
    }
}

// Step 3: workgroup b scatters chunk b from its first slots.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_scatter_kernel(
    const int* __restrict__ idx, int npairs, int k, int E, int key_bits, int chunk,
    const int* __restrict__ chunk_base, int* __restrict__ perm, int* __restrict__ row_token) {
    extern __shared__ int smem[];
    int* cursor = smem;        // [E]
    int* whist = cursor + E;   // [waves][E]
    const int b = blockIdx.x;
    for (int e = threadIdx.x; e < E; e += kDispatchThreads) cursor[e] = chunk_base[(size_t)b * E + e];
    __syncthreads();
    dispatch_scatter(idx, b * chunk, min(npairs, (b + 1) * chunk), k, E, key_bits, cursor, whist, perm, row_token);
}

static hipError_t raise_lds(const void* fn, size_t lds, size_t& raised) {
    if (lds <= 48 * 1024 || lds <= raised) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) raised = lds;
    return e;
}

hipError_t launch_dispatch(const int* idx, int T, int k, int E, const TileList& tl0, const TileList& tl1,
                           int shared_rows, int* counts, int* offsets, int* perm, int* row_token, int* chunk_hist,
                           unsigned* item_ctr, hipStream_t s) {
    if (tl0.rows <= 0 || tl1.rows < 0) return hipErrorInvalidValue;
    int bits = 1;
    while ((1 << bits) < E) ++bits;
    const int npairs = T * k;
    const size_t lds = sizeof(int) * (size_t)E * (2 + kDispatchWaves);
    const int passes = (npairs + kDispatchThreads - 1) / kDispatchThreads;
    if (passes < kDispatchSplitPasses || !chunk_hist) {
        static size_t raised = 0;
        hipError_t e = raise_lds(reinterpret_cast<const void*>(dispatch_kernel), lds, raised);
        if (e != hipSuccess) return e;
        return launch(dispatch_kernel, dim3(1), dim3(kDispatchThreads), (uint32_t)lds, s, idx, npairs, k, E, bits,
                      tl0, tl1, shared_rows, counts, offsets, perm, row_token, item_ctr);
    }
    // One chunk of whole passes per workgroup, at most kDispatchMaxChunks chunks.
    const int per = (passes + kDispatchMaxChunks - 1) / kDispatchMaxChunks;
    const int chunk = per * kDispatchThreads;
    const int nchunks = (npairs + chunk - 1) / chunk;
    static size_t raised_count = 0, raised_plan = 0, raised_scatter = 0;
    const size_t lds_count = sizeof(int) * (size_t)E, lds_plan = 2 * sizeof(int) * (size_t)E,
                 lds_scatter = sizeof(int) * (size_t)E * (1 + kDispatchWaves);
    hipError_t e = raise_lds(reinterpret_cast<const void*>(dispatch_count_kernel), lds_count, raised_count);
    if (e == hipSuccess) e = raise_lds(reinterpret_cast<const void*>(dispatch_plan_kernel), lds_plan, raised_plan);
    if (e == hipSuccess)
        e = raise_lds(reinterpret_cast<const void*>(dispatch_scatter_kernel), lds_scatter, raised_scatter);
    if (e == hipSuccess)
        e = launch(dispatch_count_kernel, dim3(nchunks), dim3(kDispatchThreads), (uint32_t)lds_count, s, idx, npairs, E,
                   chunk, chunk_hist);
    if (e == hipSuccess)
        e = launch(dispatch_plan_kernel, dim3(1), dim3(kDispatchThreads), (uint32_t)lds_plan, s, nchunks, npairs, E,
                   tl0, tl1, shared_rows, chunk_hist, counts, offsets, perm, row_token, item_ctr);
    if (e == hipSuccess)
        e = launch(dispatch_scatter_kernel, dim3(nchunks), dim3(kDispatchThreads), (uint32_t)lds_scatter, s, idx,
                   npairs, k, E, bits, chunk, static_cast<const int*>(chunk_hist), perm, row_token);
    return e;
}

}  // namespace hf
