// grouped_gemm.hip -- BF16 MFMA grouped GEMM for multi-token MoE (gfx950).
//
// C[m, n] = sum_k A[m, k] * B[n, k] (both operands K-contiguous, the
// reference's row-major [out, in] weight layout, weight_index.h:28-36), FP32
// accumulation with v_mfma_f32_16x16x32_bf16.  Rows are grouped by expert
// (dispatch.hip's M-tile list); each group multiplies by its own B.
//
// Exactness: an FP32 operand is carried as hi + lo BF16 pairs (hi = RNE(v),
// lo = RNE(v - hi)) and both halves go through the MFMA, so products keep
// about 16 significand bits instead of 8.  The activations x skip the lo half
// when it is zero everywhere (BF16-valued inputs, checked on the device); the
// SwiGLU intermediate h always uses both halves (BF16 h alone misses the
// 1e-2/2e-3 tolerance at d = 6144).
//
// Tile 128 x 128 x 32, 256 threads as 2 x 2 wavefronts of 64 x 64 (4 x 4
// MFMA tiles of 16 x 16), LDS double-buffered, persistent workgroups walking a
// contiguous range of (m-tile, n-tile) items per XCD so that neighbouring
// tiles of one expert share that XCD's L2.
//
// Epilogues:
//   PARTIAL  split-K partial sums (router logits; reduced in fixed order later)
//   SWIGLU   B rows = 64 gate rows then the 64 matching up rows; writes
//            h = silu(g) * u as BF16 hi/lo (glm_forward.cpp:444-446)
//   SCATTER  y for one (token, rank) pair per row, stored at its pair slot
//   COMBINE  shared-expert down projection + the weighted merge: out[t] =
//            (sum_r w[t,r] * y[t,r]) + shared[t] in rank order
//            (glm_forward.cpp:639-640,658-660)
#include "hf_api_internal.h"
#include "hf_grouped.h"
#include "hf_select.h"

namespace hf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int GBM = kGemmTileRows, GBN = 128, GBK = 32, GLD = GBK + 8;

struct GemmSmem {
    uint16_t a_hi[2][GBM][GLD];
    uint16_t a_lo[2][GBM][GLD];
    uint16_t b[2][GBN][GLD];
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ u32x4 lds_frag(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

template <int EPI>
__global__ __launch_bounds__(256, 2) void grouped_gemm_kernel(GemmArgs a) {
    __shared__ GemmSmem sm;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    constexpr int cols_per_tile = EPI == EPI_SWIGLU ? GBN / 2 : GBN;

    const int m_tiles = a.ntiles_dev ? *a.ntiles_dev : a.m_tiles;
    const int total = m_tiles * a.n_tiles * a.ksplit;
    // Contiguous range of items per XCD (blocks are dealt to XCDs round-robin).
    const int nxcd = gridDim.x >= 8 ? 8 : 1;
    const int xcd = blockIdx.x % nxcd;
    const int per_xcd_blocks = (int)gridDim.x / nxcd + (xcd < (int)gridDim.x % nxcd ? 1 : 0);
    const int local = blockIdx.x / nxcd;
    const int chunk = (total + nxcd - 1) / nxcd;
    const int item_begin = xcd * chunk;
    const int item_end = min(total, item_begin + chunk);
    const bool use_lo = a.a_lo && (a.a_lo_flag ? (*a.a_lo_flag != 0u) : true);
    const int Kc = a.K / a.ksplit;
    const int nk = Kc / GBK;

    // Loader mapping: thread t fills 16 bytes of rows (t >> 2) and (t >> 2) + 64.
    const int lrow = t >> 2;
    const int lc = (t & 3) * 8;

    for (int item = item_begin + local; item < item_end; item += per_xcd_blocks) {
        const int ks = item % a.ksplit;
        const int rest = item / a.ksplit;
        const int nt = rest % a.n_tiles;
        const int mt = rest / a.n_tiles;
        const int g = a.tile_group ? a.tile_group[mt] : 0;
        const int row0 = a.tile_row0 ? a.tile_row0[mt] : mt * GBM;
        const int row_end = a.group_end ? a.group_end[g] : a.rows_total;
        const int rows = min(GBM, row_end - row0);
        const int n0 = nt * cols_per_tile;
        const uint16_t* b0;
        const uint16_t* b1 = nullptr;
        if (a.b_tab) {
            b0 = a.b_tab[3 * g + a.b_which];
            if (EPI == EPI_SWIGLU) b1 = a.b_tab[3 * g + a.b_which + 1];
        } else {
            b0 = a.b_fixed0;
            b1 = a.b_fixed1;
        }
        const int kbase = ks * Kc;

        // Global source rows of this thread's two A rows and two B rows.
        const uint16_t* ah[2];
        const uint16_t* al[2];
        const uint16_t* bp[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int r = lrow + 64 * h2;
            ah[h2] = nullptr;
            al[h2] = nullptr;
            if (r < rows) {
                const int gr = row0 + r;
                const int src = a.a_rowmap ? a.a_rowmap[gr] : gr;
                ah[h2] = a.a_hi + (size_t)src * a.K + kbase + lc;
                if (use_lo) al[h2] = a.a_lo + (size_t)src * a.K + kbase + lc;
            }
            bp[h2] = nullptr;
            if (EPI == EPI_SWIGLU) {
                const int n = n0 + (r & 63);
                if (n < a.N) bp[h2] = (r < 64 ? b0 : b1) + (size_t)n * a.b_ld + kbase + lc;
            } else {
                const int n = n0 + r;
                if (n < a.N) bp[h2] = b0 + (size_t)n * a.b_ld + kbase + lc;
            }
        }

        u32x4 ra[2], rl[2], rb[2];
        auto gload = [&](int kt) {
            const int ko = kt * GBK;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const u32x4 zero = {0u, 0u, 0u, 0u};
                ra[h2] = ah[h2] ? *reinterpret_cast<const u32x4*>(ah[h2] + ko) : zero;
                rl[h2] = al[h2] ? *reinterpret_cast<const u32x4*>(al[h2] + ko) : zero;
                rb[h2] = bp[h2] ? ld_stream(reinterpret_cast<const u32x4*>(bp[h2] + ko)) : zero;
            }
        };
        auto lstore = [&](int buf) {
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int r = lrow + 64 * h2;
                *reinterpret_cast<u32x4*>(&sm.a_hi[buf][r][lc]) = ra[h2];
                if (use_lo) *reinterpret_cast<u32x4*>(&sm.a_lo[buf][r][lc]) = rl[h2];
                *reinterpret_cast<u32x4*>(&sm.b[buf][r][lc]) = rb[h2];
            }
        };

        f32x4_t acc[4][4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};

        // B-tile row bases of this wavefront's four 16-column subtiles.
        int nb[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            nb[ni] = EPI == EPI_SWIGLU ? (ni < 2 ? wn * 32 + 16 * ni : 64 + wn * 32 + 16 * (ni - 2))
                                       : wn * 64 + 16 * ni;
        const int fr = lane & 15;
        const int fk = (lane >> 4) * 8;

        gload(0);
        lstore(0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int buf = kt & 1;
            if (kt + 1 < nk) gload(kt + 1);
            bf16x8_t af[4], bfr[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) af[mi] = as_bf16x8(lds_frag(&sm.a_hi[buf][wm * 64 + 16 * mi + fr][fk]));
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bfr[ni] = as_bf16x8(lds_frag(&sm.b[buf][nb[ni] + fr][fk]));
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
            if (use_lo) {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) af[mi] = as_bf16x8(lds_frag(&sm.a_lo[buf][wm * 64 + 16 * mi + fr][fk]));
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
            }
            if (kt + 1 < nk) lstore(buf ^ 1);
            __syncthreads();
        }

        // Epilogue: lane holds D[4*(lane>>4) + q][lane & 15] of each 16 x 16 tile.
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int rl_ = wm * 64 + 16 * mi + 4 * (lane >> 4) + q;
                if (rl_ >= rows) continue;
                const int gr = row0 + rl_;
                if (EPI == EPI_SWIGLU) {
#pragma unroll
                    for (int ni = 0; ni < 2; ++ni) {
                        const int col = n0 + wn * 32 + 16 * ni + fr;
                        if (col >= a.N) continue;
                        const float gv = acc[mi][ni][q];
                        const float uv = acc[mi][ni + 2][q];
                        const float hv = gv / (1.0f + expf(-gv)) * uv;
                        const uint16_t hb = f32_to_bf16(hv);
                        const float hr = hv - __uint_as_float((uint32_t)hb << 16);
                        a.h_hi[(size_t)gr * a.N + col] = hb;
                        a.h_lo[(size_t)gr * a.N + col] = f32_to_bf16(hr);
                    }
                } else {
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        const int col = n0 + wn * 64 + 16 * ni + fr;
                        if (col >= a.N) continue;
                        const float v = acc[mi][ni][q];
                        if (EPI == EPI_PARTIAL) {
                            a.out_f32[((size_t)ks * a.rows_total + gr) * a.N + col] = v;
                        } else if (EPI == EPI_SCATTER) {
                            a.out_f32[(size_t)a.scatter_rows[gr] * a.N + col] = v;
                        } else {
                            float moe = 0.0f;
                            for (int r = 0; r < a.comb_k; ++r)
                                moe += a.comb_w[(size_t)gr * a.comb_k + r] *
                                       a.comb_y[((size_t)gr * a.comb_k + r) * a.N + col];
                            a.out_f32[(size_t)gr * a.N + col] = moe + v;
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
}

// x FP32 [n] -> BF16 hi/lo; *flag |= 1 when any lo is nonzero.
__global__ void split_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ hi,
                                  uint16_t* __restrict__ lo, size_t n, unsigned* __restrict__ flag) {
    bool nz = false;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        const uint16_t h = f32_to_bf16(v);
        const uint16_t l = f32_to_bf16(v - __uint_as_float((uint32_t)h << 16));
        hi[i] = h;
        lo[i] = l;
        nz |= (l & 0x7FFF) != 0;
    }
    if (__ballot(nz) != 0ull && (threadIdx.x & 63) == 0) atomicOr(flag, 1u);
}

__global__ void clear_u32_kernel(unsigned* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Router logits from split-K partials (summed in split order) and score pairs.
__global__ void router_reduce_kernel(const float* __restrict__ part, int ksplit, int T, int E,
                                     const float* __restrict__ bias, float* __restrict__ logits,
                                     float2* __restrict__ scores) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * E) return;
    float s = 0.0f;
    for (int q = 0; q < ksplit; ++q) s += part[(size_t)q * T * E + i];
    logits[i] = s;
    scores[i] = score_pair(s, bias, i % E);
}

hipError_t launch_grouped_gemm(int epi, const GemmArgs& a, int blocks, hipStream_t s) {
    switch (epi) {
        case EPI_PARTIAL: return launch(grouped_gemm_kernel<EPI_PARTIAL>, dim3(blocks), dim3(256), 0, s, a);
        case EPI_SWIGLU: return launch(grouped_gemm_kernel<EPI_SWIGLU>, dim3(blocks), dim3(256), 0, s, a);
        case EPI_SCATTER: return launch(grouped_gemm_kernel<EPI_SCATTER>, dim3(blocks), dim3(256), 0, s, a);
        case EPI_COMBINE: return launch(grouped_gemm_kernel<EPI_COMBINE>, dim3(blocks), dim3(256), 0, s, a);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, size_t n, unsigned* flag,
                             hipStream_t s) {
    hipError_t e = launch(clear_u32_kernel, dim3(1), dim3(64), 0, s, flag, 1);
    if (e != hipSuccess) return e;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    return launch(split_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, hi, lo, n, flag);
}

hipError_t launch_router_reduce(const float* part, int ksplit, int T, int E, const float* bias,
                                float* logits, float2* scores, hipStream_t s) {
    const int n = T * E;
    return launch(router_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, s, part, ksplit, T, E,
                  bias, logits, scores);
}

}  // namespace hf
