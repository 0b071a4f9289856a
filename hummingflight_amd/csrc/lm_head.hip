// lm_head.hip -- final RMSNorm, LM-head logits and greedy argmax
// (GLMForward::lmHeadAndSample, glm_forward.cpp:663-731).
//
// logits[v] = lm_head[v, :] . RMSNorm(h) over the whole vocabulary (154880 x
// 6144 BF16 = 1.9 GB at GLM-5.2: a bandwidth-bound GEMV), then the first
// index of the largest logit (the reference's serial scan keeps the first
// maximum; its OpenMP merge of per-thread winners is the same unless two
// threads hold exactly equal maxima).
//
// T = 1: a persistent GEMV.  Each block stages the normalised hidden state in
//   LDS; each wavefront streams whole vocabulary rows, two at a time, 16-byte
//   non-temporal loads (lane l: elements 512j + 8l .. +7; the weights are read
//   once and kept out of the caches' way); lane 0 writes the logit and
//   keeps the wavefront's running winner, the block merges its four, and one
//   small launch merges the blocks' winners (lowest row on equal values).
// T > 1: the grouped GEMM (one group, fixed B = lm_head) writes the logits,
//   then one block per token finds its argmax.
#include "hf_api_internal.h"
#include "hf_grouped.h"

#include <climits>

namespace hf {

struct ArgMax {
    float v;
    int i;
};

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

constexpr int kLmBlock = 256;

template <int KCH, int RF>
__global__ __launch_bounds__(kLmBlock) void lm_gemv_kernel(const uint16_t* __restrict__ W,
                                                           const float* __restrict__ x, int V, int K,
                                                           float* __restrict__ logits,
                                                           ArgMax* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) float xs[KCH * 512];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = gridDim.x * (kLmBlock / 64);
    const int gw = blockIdx.x * (kLmBlock / 64) + wave;
    for (int i = threadIdx.x; i < KCH * 512; i += kLmBlock) xs[i] = i < K ? x[i] : 0.0f;
    __syncthreads();
    float best = -INFINITY;
    int best_i = INT_MAX;
    for (int r0 = gw * RF; r0 < V; r0 += nwaves * RF) {
        u32x4 w[RF][KCH];
#pragma unroll
        for (int u = 0; u < RF; ++u) {
            const int r = min(r0 + u, V - 1);
            const uint16_t* row = W + (size_t)r * K;
#pragma unroll
            for (int j = 0; j < KCH; ++j) {
                const int k0 = j * 512 + lane * 8;
                w[u][j] = k0 < K ? ld_stream(reinterpret_cast<const u32x4*>(row + k0)) : (u32x4){0, 0, 0, 0};
            }
        }
        float acc[RF];
#pragma unroll
        for (int u = 0; u < RF; ++u) acc[u] = 0.0f;
        // Re-read x from LDS for every row pair: an opaque offset keeps the
        // compiler from hoisting the reads (and 96 registers) out of the loop.
        int xo = lane * 8;
        asm volatile("" : "+v"(xo));
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const float4 xa = *reinterpret_cast<const float4*>(xs + j * 512 + xo);
            const float4 xb = *reinterpret_cast<const float4*>(xs + j * 512 + xo + 4);
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int u = 0; u < RF; ++u) {
                const u32x4 v = w[u][j];
                const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc[u] = fmaf(__uint_as_float(ws[q] << 16), xv[2 * q], acc[u]);
                    acc[u] = fmaf(__uint_as_float(ws[q] & 0xFFFF0000u), xv[2 * q + 1], acc[u]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < RF; ++u) {
            const float dot = wave_sum(acc[u]);
            const int r = r0 + u;
            if (r < V) {
                if (lane == 0) logits[r] = dot;
                if (better(dot, r, best, best_i)) {
                    best = dot;
                    best_i = r;
                }
            }
        }
    }
    if (!part) return;  // plain matvec: no winner wanted
    __shared__ ArgMax wbest[kLmBlock / 64];
    if (lane == 0) wbest[wave] = {best, best_i};
    __syncthreads();
    if (threadIdx.x == 0) {
        ArgMax b = wbest[0];
        for (int i = 1; i < kLmBlock / 64; ++i)
            if (better(wbest[i].v, wbest[i].i, b.v, b.i)) b = wbest[i];
        part[blockIdx.x] = b;
    }
}

// Winner of n partial winners (one block).
__global__ __launch_bounds__(256) void argmax_merge_kernel(const ArgMax* __restrict__ part, int n,
                                                           int* __restrict__ out) {
    __shared__ ArgMax s[256];
    ArgMax b{-INFINITY, INT_MAX};
    for (int i = threadIdx.x; i < n; i += 256)
        if (better(part[i].v, part[i].i, b.v, b.i)) b = part[i];
    s[threadIdx.x] = b;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w && better(s[threadIdx.x + w].v, s[threadIdx.x + w].i, s[threadIdx.x].v,
                                          s[threadIdx.x].i))
            s[threadIdx.x] = s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = s[0].i == INT_MAX ? 0 : s[0].i;
}

// One block per row of a [T, V] matrix: first index of the row's maximum.
__global__ __launch_bounds__(256) void row_argmax_kernel(const float* __restrict__ logits, int V,
                                                         int* __restrict__ out) {
    __shared__ ArgMax s[256];
    const float* row = logits + (size_t)blockIdx.x * V;
    ArgMax b{-INFINITY, INT_MAX};
    for (int i = threadIdx.x; i < V; i += 256)
        if (better(row[i], i, b.v, b.i)) b = {row[i], i};
    s[threadIdx.x] = b;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w && better(s[threadIdx.x + w].v, s[threadIdx.x + w].i, s[threadIdx.x].v,
                                          s[threadIdx.x].i))
            s[threadIdx.x] = s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = s[0].i == INT_MAX ? 0 : s[0].i;
}

template <int KCH>
static hipError_t lm_gemv_inst(const uint16_t* W, const float* x, int V, int K, float* logits, ArgMax* part,
                               int grid, hipStream_t s) {
    constexpr int RF = KCH <= 12 ? 2 : 1;
    return launch(lm_gemv_kernel<KCH, RF>, dim3(grid), dim3(kLmBlock), 0, s, W, x, V, K, logits, part);
}

hipError_t launch_row_argmax(const float* x, int T, int n, int* out, hipStream_t s) {
    return launch(row_argmax_kernel, dim3(T), dim3(256), 0, s, x, n, out);
}

static hipError_t launch_lm_gemv(const uint16_t* W, const float* x, int V, int K, float* logits, ArgMax* part,
                                 int grid, hipStream_t s) {
    const int kch = (K + 511) / 512;
    if (kch <= 4) return lm_gemv_inst<4>(W, x, V, K, logits, part, grid, s);
    if (kch <= 8) return lm_gemv_inst<8>(W, x, V, K, logits, part, grid, s);
    if (kch <= 12) return lm_gemv_inst<12>(W, x, V, K, logits, part, grid, s);
    if (kch <= 16) return lm_gemv_inst<16>(W, x, V, K, logits, part, grid, s);
    return hipErrorInvalidValue;
}

// Two 4-wave blocks per CU (two rows of loads in flight per wavefront take
// ~176 registers at hidden 6144; more rows or blocks measured no faster).
// y[M] = W[M, K] . x[K] (K a multiple of 8, at most 8192), no argmax.
hipError_t launch_matvec_bf16(const uint16_t* W, const float* x, int M, int K, float* y, hipStream_t s) {
    return launch_lm_gemv(W, x, M, K, y, nullptr, g.num_cus * 2, s);
}

static int lm_grid() { return env_int("HFMOE_LM_BLOCKS", g.num_cus * 2); }
// Workgroups of a T = 1 call: HFMOE_LM_BLOCKS as read now, within the
// per-workgroup winners allocated at registration.
static int lm_call_grid() { return std::max(1, std::min(lm_grid(), g.lm.part_n)); }

void lm_head_release() {
    if (g.lm.part) hipFree(g.lm.part);
    g.lm = LmHead{};
}

#define HF_CHECK_LAUNCH(expr, what)                      \
    do {                                                 \
        hipError_t e_ = (expr);                          \
        prof_end(p, s);                                  \
        if (e_ != hipSuccess) return fail_hip(e_, what); \
    } while (0)

static int lm_head_forward(const float* h, int T, float* logits, int* token, hipStream_t s) {
    const Cfg& c = g.cfg;
    const LmHead& L = g.lm;
    float* xn = g.ws.tmp;  // [T, d]
    Pending p;
    prof_begin(p, "lm_norm", s);
    HF_CHECK_LAUNCH(launch_rmsnorm(h, L.norm, xn, T, c.d, c.eps, s), "final norm");
    const bool gemm = T > 1 && g.gws.xh && c.d % kGemmTileK == 0;
    if (!gemm) {
        const int grid = lm_call_grid();
        for (int t = 0; t < T; ++t) {
            prof_begin(p, "lm_head_gemv", s);
            HF_CHECK_LAUNCH(launch_lm_gemv(L.w, xn + (size_t)t * c.d, L.vocab, c.d, logits + (size_t)t * L.vocab,
                                           static_cast<ArgMax*>(L.part), grid, s),
                            "lm head gemv");
            if (token) {
                prof_begin(p, "lm_argmax", s);
                HF_CHECK_LAUNCH(launch(argmax_merge_kernel, dim3(1), dim3(256), 0, s,
                                       static_cast<const ArgMax*>(L.part), grid, token + t),
                                "argmax");
            }
        }
        return HFMOE_OK;
    }
    GroupedWorkspace& gw = g.gws;
    prof_begin(p, "split_x", s);
    HF_CHECK_LAUNCH(launch_split_bf16(xn, gw.xh, gw.xl, (size_t)T * c.d, gw.lo_flag, s), "split x");
    // Past one 128-row M tile, the 256-row tiles (HFMOE_LM_MIN_TOKENS): a
    // second 128-row M tile streams the whole table again (GLM vocab:
    // T = 129-191 1.53-1.56 ms against 0.89-1.03 on one 256-row tile; up to
    // 128 tokens the two are even, 0.77-0.88 ms).
    const int TR = T >= env_int("HFMOE_LM_MIN_TOKENS", kGemmTileRows + 1) ? kDenseTileRows : kGemmTileRows;
    GemmArgs a{};
    a.K = c.d;
    a.N = L.vocab;
    a.tile_rows = TR;
    a.tile_cols = gemm_tile_cols(TR, EPI_PARTIAL);
    a.n_tiles = gemm_n_tiles(EPI_PARTIAL, L.vocab, a.tile_cols);
    a.m_tiles = (T + TR - 1) / TR;
    a.rows_total = T;
    a.a_hi = gw.xh;
    a.a_lo = gw.xl;
    a.a_lo_flag = gw.lo_flag;
    a.b_fixed0 = L.w;
    a.b_ld = c.d;
    a.out_f32 = logits;
    a.ksplit = 1;
    prof_begin(p, "lm_head_gemm", s);
    HF_CHECK_LAUNCH(launch_grouped_gemm(EPI_PARTIAL, a, gemm_blocks(TR), s), "lm head gemm");
    if (token) {
        prof_begin(p, "lm_argmax", s);
        HF_CHECK_LAUNCH(launch(row_argmax_kernel, dim3(T), dim3(256), 0, s, static_cast<const float*>(logits),
                               L.vocab, token),
                        "argmax");
    }
    return HFMOE_OK;
}

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_register_lm_head(const uint16_t* lm_head_dev, const uint16_t* final_norm_dev, int32_t vocab) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!lm_head_dev || vocab <= 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "lm head weights and vocab > 0 required");
    if ((reinterpret_cast<uintptr_t>(lm_head_dev) & 15) || g.cfg.d % 8)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "lm head must be 16-byte aligned with hidden a multiple of 8");
    if (g.cfg.d > 8192) return fail(HFMOE_ERR_UNSUPPORTED, "hidden %d > 8192", g.cfg.d);
    lm_head_release();
    const int part_n = std::max(1, lm_grid());
    hipError_t e = hipMalloc(&g.lm.part, sizeof(ArgMax) * (size_t)part_n);
    if (e != hipSuccess) return fail_hip(e, "lm head workspace");
    g.lm.part_n = part_n;
    g.lm.w = lm_head_dev;
    g.lm.norm = final_norm_dev;
    g.lm.vocab = vocab;
    return HFMOE_OK;
}

int hfmoe_lm_head(const float* h_dev, int32_t T, float* logits_dev, int32_t* token_dev, void* stream) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!g.lm.w) return fail(HFMOE_ERR_NOT_REGISTERED, "no lm head registered");
    if (T < 0 || T > g.max_tokens)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "T=%d outside 0..max_tokens=%d", T, g.max_tokens);
    if (T == 0) return HFMOE_OK;
    if (!h_dev || !logits_dev) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null hidden state or logits pointer");
    if ((reinterpret_cast<uintptr_t>(h_dev) | reinterpret_cast<uintptr_t>(logits_dev)) & 15)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "buffers must be 16-byte aligned");
    return lm_head_forward(h_dev, T, logits_dev, token_dev, pick_stream(stream));
}

}  // extern "C"
