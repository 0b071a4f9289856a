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
// The MoE GEMMs stream expert weights (B) far more than they compute: at
// T = 4096 each expert sees ~128 rows, 128 FLOP per weight byte, below the
// MI355X ridge (~312), and at T = 64 a few rows.  So the kernels are built to
// keep B streaming and to spend MFMA cycles only on rows that exist.  Three
// tile shapes:
//   * 128 (M) x 128 (N) x 64 (K), 4 wavefronts (batched decode, router):
//     wavefront w owns tile rows [32w, 32w + 32) across all 128 columns and
//     skips the MFMAs of 16-row blocks past the group's last row, so a 3-row
//     expert costs one 16-row block of work, not 128.  B goes from global
//     memory into an LDS ring by DMA (global_load_lds_dwordx4), A fragments
//     straight into registers (L2-resident activations, row-gathered through
//     a_rowmap), both 2-4 K stages ahead of the one multiplied;
//   * 192 (M) x 256 or 384 (N) x 64 (K), 8 wavefronts (prefill GEMMs whose
//     sizes do not fit the wide tiles, dense layers, LM head): both operands
//     by DMA into LDS, wavefronts split 2 (row-block parity) x 4 (column
//     groups) -- gemm_item_split below;
//   * 192 or 160 (M) x 512 (N) x 64 (K), 8 wavefronts of 64 weight rows each
//     over all rows (prefill gate/up, 160-row tiles when x has a lo half;
//     prefill down projection, 160-row tiles): weights through private
//     per-wavefront LDS rings -- gemm_item_wide below.
// Persistent workgroups walk per-XCD item lists, n fastest, so an M tile's
// activations are reused within that XCD's L2 (item_range).
//
// Epilogues:
//   PARTIAL  split-K partial sums (router logits; reduced in fixed order
//            later), or plain FP32 rows with ksplit = 1 (dense down)
//   SWIGLU   B rows = gate rows then as many matching up rows; writes
//            h = silu(g) * u as BF16 hi/lo (glm_forward.cpp:444-446)
//   SCATTER  y for one (token, rank) pair per row, stored at row scatter_rows[r]
#include "hf_api_internal.h"
#include "hf_grouped.h"
#include "hf_select.h"
#include "item_deal.h"
#include "split_pipeline.h"

#include <type_traits>

namespace hf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int GBN = 128, GBK = kGemmTileK;

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16-byte load through a global-address-space pointer.  Pointers read from
// memory (the expert table) are generic; a generic load is a FLAT instruction,
// which also counts against the LDS counter and is not ordered with other
// vector loads, so every LDS wait would drain the weight prefetch.
__device__ __forceinline__ u32x4 ld_global(const uint16_t* p) {
    return *(const __attribute__((address_space(1))) u32x4*)(p);
}

// B stages in LDS: 128 rows x 64 k of BF16, 128-byte rows whose 16-byte
// chunks are XOR-swizzled by (row & 7), which keeps both the DMA writes
// (lane-contiguous) and the fragment reads (16 rows x 16 bytes per quarter
// wave) free of bank conflicts.
constexpr int kDmaPolicy = 2;  // cache-policy bits of the weight DMA: non-temporal
typedef uint16_t BStage[GBN * GBK];
// Prefetch distance (K stages) of A and B: deeper when only the hi half of A
// is multiplied (half the MFMA work per stage, same bytes); the ring holds
// distance + 1 stages.
constexpr int kDepthHi = 4, kDepthLo = 2;
constexpr size_t kRingBytes = sizeof(BStage) * (kDepthHi + 1);

// Weight DMA with the non-temporal hint: each weight tile is read by at most
// the few M tiles of one expert, close together in time, while the activation
// rows are re-read by every N tile of their M tile and must stay in L2.
// (POLICY 0: the activations' DMA, which should stay in L2.)
template <int POLICY = kDmaPolicy>
__device__ __forceinline__ void dma16(const uint16_t* g, uint16_t* l) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                     (__attribute__((address_space(3))) void*)l, 16, 0, POLICY);
}

// The same DMA through a raw buffer resource (buffer_load_dwordx4 ... lds):
// lane l's 16 bytes at base + voff + soff (bytes) land at l + 16 l bytes.
// Unlike the FLAT-encoded global_load_lds, which the compiler must assume
// may still be writing LDS when an LDS read's wait is placed (it then waits
// for every LDS read with lgkmcnt(0)), a buffer DMA leaves the compiler free
// to wait for just the read it needs, so LDS reads can run ahead of the
// multiplies that use them.
// c ? x : y on values: a conditional on two named resources can compile to a
// select of their addresses, which keeps them in scratch memory.
template <class T>
__device__ __forceinline__ T pick(bool c, T x, T y) {
    return c ? x : y;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
    // stride 0, 4 GiB of records, 32-bit data format (untyped loads)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
// A wavefront-uniform pointer moved into scalar registers.  A pointer read
// from memory the kernel also writes (the expert table) comes back from a
// vector load; a buffer resource built from it would sit in vector registers
// and every buffer instruction on it would run as a loop over its distinct
// values (readfirstlane, compare, exec mask) -- once, but at a dozen
// instructions per DMA.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}
template <int POLICY = kDmaPolicy>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint16_t* l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)l, 16, voff, soff, 0, POLICY);
}

// f(integral_constant<int, i>) for i = N, N - 1, ..., 1.
template <int N, class F>
__device__ __forceinline__ void static_for_desc(F&& f) {
    if constexpr (N > 0) {
        f(std::integral_constant<int, N>{});
        static_for_desc<N - 1>(f);
    }
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without the release fence of __syncthreads(), which would
// drain every outstanding load (the weight DMA of later stages included);
// the asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Barrier that also makes this wavefront's LDS writes visible (lgkmcnt(0)
// first), still without waiting for global loads or stores.
__device__ __forceinline__ void lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The items (m-tile, n-tile, k-split) a persistent workgroup walks.  The
// hardware deals workgroups to the 8 XCDs round-robin, so blockIdx.x % 8 is
// the XCD, and each XCD takes a contiguous range of items (an M tile's N
// tiles, which share its activation rows, run side by side in one L2).
// DEAL_M (prefill tiles, at least one M tile per XCD): whole M tiles are
// dealt to the XCDs round-robin instead, which keeps the first property and
// spreads runs of heavy tiles -- the shared expert's full 192-row tiles sit
// together at the end of the list, with half as much again the MFMA work of a
// routed expert's ~128 rows -- over all XCDs rather than the last one.
struct ItemRange {
    int begin, end, stride;  // local item indices begin, begin + stride, ... < end
    int xcd, nxcd, per_m;    // per_m = n_tiles * ksplit items per M tile
    bool by_mtile;
    // by_ntile: this XCD's block of N tiles [n0, n0 + n_local) x M tiles
    // [m0, m0 + m_cnt), M tiles fastest
    bool by_ntile;
    int n0, n_local, m0, m_cnt, ksplit;
    // Dynamic by_mtile dealing (item_deal.h), the shared expert's last
    // sh_m M tiles dealt by blocks of N tiles (GemmArgs::shared_mtiles;
    // 0: none).
    int m_tiles, sh_m;
    __device__ __forceinline__ XcdDeal deal() const { return XcdDeal{m_tiles, per_m, nxcd, sh_m}; }
    __device__ __forceinline__ int item(int li) const {
        if (by_ntile) {
            const int per_n = m_cnt * ksplit;
            const int nt = n0 + li / per_n;
            const int rem = li % per_n;
            return ((m0 + rem / ksplit) * (per_m / ksplit) + nt) * ksplit + rem % ksplit;
        }
        return by_mtile ? (xcd + nxcd * (li / per_m)) * per_m + li % per_m : li;
    }
};

template <bool DEAL_M>
__device__ __forceinline__ ItemRange item_range(const GemmArgs& a, int m_tiles) {
    ItemRange r;
    r.nxcd = gridDim.x >= 8 ? 8 : 1;
    r.xcd = blockIdx.x % r.nxcd;
    r.stride = (int)gridDim.x / r.nxcd + (r.xcd < (int)gridDim.x % r.nxcd ? 1 : 0);
    r.per_m = a.n_tiles * a.ksplit;
    r.ksplit = a.ksplit;
    // a.by_ntile N groups x (nxcd / a.by_ntile) M groups, one block per XCD;
    // every group the same size, else whole N-tile ranges (one M group)
    int gn = a.by_ntile;
    if (gn > 0 && (r.nxcd % gn || a.n_tiles % gn || m_tiles % (r.nxcd / gn))) gn = r.nxcd;
    r.by_ntile = gn > 0 && !a.tile_group && r.nxcd > 1 && a.n_tiles % gn == 0;
    if (r.by_ntile) {
        const int gm = r.nxcd / gn;
        r.n_local = a.n_tiles / gn;
        r.n0 = (r.xcd % gn) * r.n_local;
        r.m_cnt = m_tiles / gm;
        r.m0 = (r.xcd / gn) * r.m_cnt;
    }
    r.by_mtile = !r.by_ntile && DEAL_M && m_tiles >= r.nxcd;
    r.m_tiles = m_tiles;
    const bool sh = r.by_mtile && a.item_ctr && a.ksplit == 1 && a.shared_mtiles > 0 && a.shared_mtiles <= m_tiles;
    r.sh_m = sh ? a.shared_mtiles : 0;
    const int local = blockIdx.x / r.nxcd;
    if (r.by_ntile) {
        r.begin = local;
        r.end = r.n_local * r.m_cnt * a.ksplit;
    } else if (r.by_mtile) {
        const int m_local = (m_tiles - r.xcd + r.nxcd - 1) / r.nxcd;
        r.begin = local;
        r.end = m_local * r.per_m;
    } else {
        const int total = m_tiles * r.per_m;
        const int chunk = (total + r.nxcd - 1) / r.nxcd;
        r.begin = r.xcd * chunk + local;
        r.end = min(total, r.xcd * chunk + chunk);
    }
    return r;
}

// Stores one lane's share of a finished tile row gr: acc[cb][q] is output
// column col0 + 16*cb + q (q = 0..3).  SWIGLU: blocks [0, NCB/2) are gate and
// [NCB/2, NCB) the matching up columns; writes h = silu(g) * u
// (glm_forward.cpp:444-446) as BF16 hi / lo halves, 8 bytes per array.
// PARTIAL / SCATTER: 16-byte FP32 stores (row stride N is a multiple
// of 4 whenever N is a multiple of 64; a ragged router width falls back to
// single floats) to output row orow_idx (SCATTER: the token-order row of gr;
// PARTIAL: gr).  NT: non-temporal stores.
// h = silu(g) * u with the hardware exp2 and reciprocal (a few ulp of FP32):
// far below the rounding of h to a BF16 hi + lo pair.  The one formula of the
// GEMM epilogue and of the split-K SwiGLU kernel.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

template <int EPI, int NCB, bool NT = false>
__device__ __forceinline__ void store_tile_row(const GemmArgs& a, const f32x4_t (&acc)[NCB], int gr, int col0,
                                               int ks, int orow_idx) {
    if (EPI == EPI_SWIGLU) {
        float hv[NCB / 2][4];
#pragma unroll
        for (int cb = 0; cb < NCB / 2; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q) hv[cb][q] = silu_mul(acc[cb][q], acc[cb + NCB / 2][q]);
        {  // BF16 hi + lo halves
            uint16_t* hrow = a.h_hi + (size_t)gr * a.N;
            uint16_t* lrow = a.h_lo + (size_t)gr * a.N;
#pragma unroll
            for (int cb = 0; cb < NCB / 2; ++cb) {
                const int col = col0 + 16 * cb;
                if (col >= a.N) continue;
                uint32_t hw[2], lw[2];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t v0 = f32_to_bf16(hv[cb][q]);
                    const uint32_t v1 = f32_to_bf16(hv[cb][q] - __uint_as_float(v0 << 16));
                    if (q & 1) {
                        hw[q >> 1] |= v0 << 16;
                        lw[q >> 1] |= v1 << 16;
                    } else {
                        hw[q >> 1] = v0;
                        lw[q >> 1] = v1;
                    }
                }
                *reinterpret_cast<uint2*>(hrow + col) = make_uint2(hw[0], hw[1]);
                *reinterpret_cast<uint2*>(lrow + col) = make_uint2(lw[0], lw[1]);
            }
        }
    } else {
        float* orow = EPI == EPI_PARTIAL ? a.out_f32 + ((size_t)ks * a.rows_total + orow_idx) * a.N
                                         : a.out_f32 + (size_t)orow_idx * a.N;
        const bool vec = (a.N & 3) == 0;
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            const int col = col0 + 16 * cb;
            if (vec && col + 3 < a.N) {
                if constexpr (NT)
                    __builtin_nontemporal_store(acc[cb], reinterpret_cast<f32x4_t*>(orow + col));
                else
                    *reinterpret_cast<f32x4_t*>(orow + col) = acc[cb];
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (col + q < a.N) orow[col + q] = acc[cb][q];
            }
        }
    }
}

// One (m-tile, n-tile, k-split) item.  USE_LO: multiply the A lo half too.
//
// Pipeline per K stage s (64 k), prefetch distance D: every wave waits until
// its A registers and its DMA of B for stage s have landed, the workgroup
// meets at a barrier, then each wave issues A of stage s+D (registers) and
// its quarter of B stage s+D (DMA into the ring slot stage s-1 used), and
// multiplies stage s.  A and B of one stage are issued together, so waiting
// for stage s (in-order load counter) never waits for a later stage.
// NRB: this wavefront's 16-row blocks that hold rows (0, 1 or 2), fixed per
// instantiation so that a wavefront loads A fragments only for rows that
// exist (the activation requests otherwise take up to a third of the CU's
// queue of outstanding requests at batched-decode sizes) while every load
// count stays a compile-time constant for the counter waits.
template <int EPI, bool USE_LO, int WAVES, int NRB>
__device__ __forceinline__ void gemm_item(const GemmArgs& a, int item, BStage* ring, int t, int wave) {
    constexpr int GBM = 32 * WAVES;     // tile rows: 32 per wavefront
    constexpr int BJ = 16 / WAVES;      // 1 KB weight DMAs per wave per stage
    constexpr int cols_per_tile = EPI == EPI_SWIGLU ? GBN / 2 : GBN;
    constexpr int NA = NRB * (USE_LO ? 4 : 2);  // A loads per wave per stage
    constexpr int D = USE_LO ? kDepthLo : kDepthHi;
    constexpr int RING = D + 1;
    const int lane = t & 63;
    const int fr = lane & 15;  // fragment row (A) / column (B, D)
    const int fq = lane >> 4;  // fragment k quarter
    const int Kc = a.K / a.ksplit;
    const int nk = Kc / GBK;

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
    constexpr int nrb = NRB;

    // A fragment sources: lane row fr of row blocks 0 and 1, clamped to the
    // tile's last row (rows past it are loaded but never multiplied or stored).
    // (the lo half sits at a fixed offset from the hi half: one pointer per row block)
    const uint16_t* ap[2];
    const ptrdiff_t lo_off = USE_LO ? a.a_lo - a.a_hi : 0;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int lr = min(32 * wave + 16 * rb + fr, rows - 1);
        const int gr = row0 + lr;
        const size_t src = (size_t)(a.a_rowmap ? a.a_rowmap[gr] : gr);
        ap[rb] = a.a_hi + src * a.K + kbase + fq * 8;
    }
    // B DMA sources: wave w fills ring slots (BJ*w + j) * 64 + lane, j < BJ,
    // each 16 bytes: slot i holds chunk (i & 7) ^ (row & 7) of tile row i >> 3.
    // Rows past N are clamped to row N-1 (their columns are never stored).  A
    // wavefront's slot rows lie in one half (gate or up), so one base pointer
    // plus 32-bit element offsets addresses them.
    const uint16_t* bbase = (EPI == EPI_SWIGLU && wave >= WAVES / 2) ? b1 : b0;
    uint32_t boff[BJ];
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
        const int i = (wave * BJ + j) * 64 + lane;
        const int r = i >> 3;
        const int c = (i & 7) ^ (r & 7);
        int n = EPI == EPI_SWIGLU ? n0 + (r & 63) : n0 + r;
        n = min(n, a.N - 1);
        boff[j] = (uint32_t)((size_t)n * a.b_ld + kbase + c * 8);
    }

    f32x4_t acc[2][8];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[rb][cb] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};

    // Loads are unconditional (stage indices clamped to the last stage) so the
    // number of loads in flight, which the counter waits rely on, is fixed.
    auto issue_b = [&](int s) {
        uint16_t* dst = ring[s % RING] + wave * BJ * 512;
        s = min(s, nk - 1);
#pragma unroll
        for (int j = 0; j < BJ; ++j) dma16(bbase + boff[j] + s * GBK, dst + j * 512);
    };
    typedef u32x4 AFrag[2][2][2];  // [hi/lo][row block][k half]
    auto load_a = [&](AFrag& f, int s) {
        s = min(s, nk - 1);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                f[0][rb][kh] = ld_global(ap[rb] + s * GBK + kh * 32);
                if (USE_LO) f[1][rb][kh] = ld_global(ap[rb] + lo_off + s * GBK + kh * 32);
            }
    };
    // Four groups of four column blocks (k half kh = g >> 1, column half
    // ch = g & 1); the B fragments of group g+1 are read from LDS while the
    // MFMAs of group g run.
    constexpr int NB = 2;  // B fragment sets
    auto compute = [&](const uint16_t* bt, const AFrag& f) {
        if (nrb == 0) return;
        bf16x8_t bf[NB][4];
        auto read_group = [&](int g, bf16x8_t(&dst)[4]) {
            const int kh = g >> 1, ch = g & 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = 16 * (4 * ch + j) + fr;
                const int c = (kh * 4 + fq) ^ (r & 7);
                dst[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(bt + r * GBK + c * 8));
            }
        };
        if (NB == 2) read_group(0, bf[0]);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (NB == 1)
                read_group(g, bf[0]);
            else if (g + 1 < 4)
                read_group(g + 1, bf[(g + 1) % NB]);
            const int kh = g >> 1, ch = g & 1;
            const bf16x8_t(&b)[4] = bf[g % NB];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                if (rb == 1 && nrb < 2) break;
                const bf16x8_t af = as_bf16x8(f[0][rb][kh]);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[rb][4 * ch + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], af, acc[rb][4 * ch + j], 0, 0, 0);
                if (USE_LO) {
                    const bf16x8_t alf = as_bf16x8(f[1][rb][kh]);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[rb][4 * ch + j] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], alf, acc[rb][4 * ch + j], 0, 0, 0);
                }
            }
        }
    };
    // Steady-state steps wait for stage s with stages s+1 .. s+D-1 still in
    // flight.  Tail steps (after the loop) drain instead: the compiler drops
    // the A loads whose registers are never read again, so the count of
    // loads issued after stage s is no longer fixed there.
    auto step = [&](int s, const AFrag& cur, AFrag& ahead, auto tail) {
        if constexpr (decltype(tail)::value)
            wait_vmcnt<0>();
        else
            wait_vmcnt<(D - 1) * (NA + BJ)>();
        lds_barrier();
        load_a(ahead, s + D);
        issue_b(s + D);
        compute(ring[s % RING], cur);
    };

    AFrag A[RING];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load_a(A[j], j);
        issue_b(j);
    }
    // Whole rotations only inside the loop: a back edge that always follows
    // the same steps lets the compiler's own counter waits stay exact.
    int s = 0;
    for (; s + RING <= nk; s += RING) {
#pragma unroll
        for (int u = 0; u < RING; ++u) step(s + u, A[u], A[(u + D) % RING], std::false_type{});
    }
#pragma unroll
    for (int u = 0; u < RING - 1; ++u)
        if (s + u < nk) step(s + u, A[u], A[(u + D) % RING], std::true_type{});

    // Epilogue.  The MFMAs take the weight fragment as their A operand, so a
    // lane holds output columns 16*cb + 4*fq + q (q = 0..3, consecutive) of
    // tile row 32*wave + 16*rb + fr: each store writes 4 adjacent columns.
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        if (rb >= nrb) break;
        const int rl = 32 * wave + 16 * rb + fr;
        if (rl < rows)
            store_tile_row<EPI, 8>(a, acc[rb], row0 + rl, n0 + 4 * fq, ks,
                                   EPI == EPI_SCATTER ? a.scatter_rows[row0 + rl] : row0 + rl);
    }
}

// How the A operand's lo half is handled: kLoNone (A is BF16), kLoByFlag
// (x: multiplied only when the device flag says some lo half is nonzero),
// kLoAlways (h: always; the kernel is compiled for that path alone, which
// also leaves it more registers).
enum { kLoNone = 0, kLoByFlag = 1, kLoAlways = 2 };

// A group whose weight-table entry is null takes no part in this launch: its
// tiles are skipped (streamed experts are multiplied a wave of groups at a
// time, the other groups' entries left null).
__device__ __forceinline__ bool group_absent(const GemmArgs& a, int g) {
    return a.b_tab && a.b_tab[3 * g + a.b_which] == nullptr;
}

// WAVES = 4: 128-row tiles, two workgroups per CU.
template <int EPI, int LOM, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void grouped_gemm_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) BStage ring[];  // kRingBytes
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: scalar branches

    const int m_tiles = a.ntiles_dev ? *a.ntiles_dev : a.m_tiles;
    const ItemRange r = item_range<false>(a, m_tiles);
    const bool use_lo = LOM == kLoAlways || (LOM == kLoByFlag && *a.a_lo_flag != 0u);

    for (int li = r.begin; li < r.end; li += r.stride) {
        const int item = r.item(li);
        // Row blocks of this wavefront in the item's tile (wave-uniform).
        const int mt = item / a.ksplit / a.n_tiles;
        const int g = a.tile_group ? a.tile_group[mt] : 0;
        if (group_absent(a, g)) continue;  // workgroup-uniform: no barrier is skipped by some waves only
        const int row0 = a.tile_row0 ? a.tile_row0[mt] : mt * 32 * WAVES;
        const int row_end = a.group_end ? a.group_end[g] : a.rows_total;
        const int wrows = min(max(min(32 * WAVES, row_end - row0) - 32 * wave, 0), 32);
        const int nrb = (wrows + 15) >> 4;
        auto run = [&](auto lo_c) {
            constexpr bool LO = decltype(lo_c)::value;
            if (nrb == 2)
                gemm_item<EPI, LO, WAVES, 2>(a, item, ring, t, wave);
            else if (nrb == 1)
                gemm_item<EPI, LO, WAVES, 1>(a, item, ring, t, wave);
            else
                gemm_item<EPI, LO, WAVES, 0>(a, item, ring, t, wave);
        };
        if constexpr (LOM == kLoAlways)
            run(std::true_type{});
        else if (LOM == kLoByFlag && use_lo)
            run(std::integral_constant<bool, LOM == kLoByFlag>{});
        else
            run(std::false_type{});
        __syncthreads();  // all DMA landed and all ring reads done before the next item
    }
}

// ---------------------------------------------------------------------------
// Split tiles for prefill: ROWS (M) x 64*CB (N) x 64 (K), eight wavefronts,
// one workgroup per CU.  Both operands go by DMA into LDS rings in whole
// 128-byte lines: activations (A, up to ROWS rows of the group, L2-resident)
// and weights (B, 64*CB weight rows streamed from HBM with the non-temporal
// hint).  Wavefront w takes column group w & 3 (16*CB output columns; SWIGLU:
// 8*CB h columns from as many gate and up rows) and the row blocks of parity
// w >> 2, so each wavefront reads a quarter of B and half of A from LDS, and a
// group of n row blocks gives every wavefront ceil(n / 2) or floor(n / 2) of
// them: the MFMA work stays even across the SIMDs for any row count.
//
// ROWS = 192 for the MoE GEMMs: a routed expert's ~128 rows at T = 4096 fit
// one tile with room to spare (an expert with more takes several M tiles and
// re-reads its weights).  ROWS = 256 for one-group GEMMs (dense layers, LM
// head), whose weights are re-read once per M tile.
//
// At T = 4096 the weight stream alone (this kernel's DMA pattern, no
// multiplies) and the multiplies alone (no DMA) each take about 70 % of the
// kernel's time: what is lost is their overlap, with one workgroup of eight
// wavefronts per CU meeting at a barrier every stage.  Tiles are as wide as
// registers and LDS allow (fewer items, fewer activation re-reads): the down
// projection's 384 columns (CB = 6, 144 registers of accumulators per lane),
// and gate/up's 256 weight rows (CB = 4) so that its weights run two stages
// ahead in the LDS; one stage ahead costs it more than wider tiles bring.
//
// The lo half of A runs as its own sub-step against the same B stage, so an
// A stage is always one half (ROWS x 64 BF16).  Depths, ring sizes and wait
// counts: split_pipeline.h.
template <int EPI, int ROWS>
constexpr int split_cb() { return split_cb(EPI == EPI_SWIGLU, ROWS); }
static_assert(split_lds_max(192, 4) <= 160 * 1024 && split_lds_max(192, 6) <= 160 * 1024 &&
                  split_lds_max(256, 4) <= 160 * 1024,
              "LDS");

// on_setup() runs once the item's own loads (tile table, row map) are out,
// before its first DMA.
template <int EPI, int ROWS, int HALVES, class Setup>
__device__ __forceinline__ void gemm_item_split(const GemmArgs& a, int item, uint16_t* lds, int t, int wave,
                                                Setup&& on_setup) {
    constexpr int CB = split_cb<EPI, ROWS>();
    constexpr int RBW = ROWS / 32;                 // row blocks per wavefront
    constexpr int AST = ROWS * GBK;                // elements per A stage
    constexpr int NAD = ROWS / 64, NBD = CB;       // 1 KB DMAs per wave per stage: activations, weights
    constexpr int DA = split_da(ROWS, CB, HALVES), DB = split_db(ROWS, CB, HALVES);
    constexpr int RA = DA + 1, RB = DB + 1;
    constexpr int cols_per_tile = EPI == EPI_SWIGLU ? 32 * CB : 64 * CB;
    uint16_t* aring = lds;
    uint16_t* bring = lds + RA * AST;
    const int lane = t & 63;
    const int fr = lane & 15;
    const int fq = lane >> 4;
    const int cg = wave & 3;
    const int par = wave >> 2;
    const int Kc = a.K / a.ksplit;
    const int nk = Kc / GBK;
    const int nj = nk * HALVES;

    // The item comes through LDS on the dynamic path: make it (and all that
    // derives from it: tile, rows, the row-block guards) provably uniform, so
    // that its loads are scalar and its guards scalar branches rather than
    // exec-mask juggling on every multiply of the K loop.
    item = __builtin_amdgcn_readfirstlane(item);
    const int ks = item % a.ksplit;
    const int rest = item / a.ksplit;
    const int nt = rest % a.n_tiles;
    const int mt = rest / a.n_tiles;
    const int g = a.tile_group ? a.tile_group[mt] : 0;
    const int row0 = a.tile_row0 ? a.tile_row0[mt] : mt * ROWS;
    const int row_end = a.group_end ? a.group_end[g] : a.rows_total;
    const int rows = min(ROWS, row_end - row0);
    const int nrb = (rows + 15) >> 4;
    const int nmine = (nrb - par + 1) >> 1;  // row blocks 2j + par, j < nmine
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

    // DMA slot i (16 bytes) of a stage holds chunk (i & 7) ^ (r & 7) of stage
    // row r = i >> 3.  Activation DMA j of a wavefront fills the 8-row block
    // 8 j + wave (the blocks spread over the wavefronts); rows past the tile's
    // end re-read its last row, and with SKIP_A the blocks past its last
    // 16-row block, which nothing multiplies, are not loaded at all: an
    // activation DMA takes a slot of the memory pipeline's queue even when it
    // hits in L1, and near-uniform prefill fills a 192-row tile to ~128 rows.
    // Weight rows: SWIGLU rows [0, 32 CB) are gate rows n0.., the next
    // 32 CB the matching up rows; a wavefront's 8 CB slot rows lie in one half.
    constexpr bool SKIP_A = split_a_may_skip(HALVES, DA, DB, NAD, NBD);
    const int nab = 2 * nrb;
    uint32_t aoff[NAD], boff[NBD];
#pragma unroll
    for (int j = 0; j < NAD; ++j) {
        const int i = (j * 8 + wave) * 64 + lane;
        const int r = i >> 3;
        const int c = (i & 7) ^ (r & 7);
        const int gr = row0 + min(r, rows - 1);
        const size_t src = (size_t)(a.a_rowmap ? a.a_rowmap[gr] : gr);
        aoff[j] = (uint32_t)(2 * (src * a.K + kbase + c * 8));
    }
    // A PARTIAL tile past b_split lies wholly in the second matrix: its
    // output columns n are rows n - b_split of b_fixed1.
    const bool second = EPI == EPI_PARTIAL && a.b_split > 0 && n0 >= a.b_split;
    const int nsub = second ? a.b_split : 0;
#pragma unroll
    for (int j = 0; j < NBD; ++j) {
        const int i = (wave * NBD + j) * 64 + lane;
        const int r = i >> 3;
        const int c = (i & 7) ^ (r & 7);
        int n = EPI == EPI_SWIGLU ? n0 + r % (32 * CB) : n0 + r;
        n = min(n, a.N - 1) - nsub;
        boff[j] = (uint32_t)(2 * ((size_t)n * a.b_ld + kbase + c * 8));
    }
    // Byte offsets within 4 GiB of each operand's base (every activation and
    // weight buffer of a layer is far smaller).
    const __amdgpu_buffer_rsrc_t rb =
        raw_rsrc(uniform_ptr(((EPI == EPI_SWIGLU && wave >= 4) || second) ? b1 : b0));
    const __amdgpu_buffer_rsrc_t ra0 = raw_rsrc(a.a_hi);
    const __amdgpu_buffer_rsrc_t ra1 = raw_rsrc(HALVES == 2 ? a.a_lo : a.a_hi);

    f32x4_t acc[RBW][CB];
#pragma unroll
    for (int j = 0; j < RBW; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[j][cb] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};

    // Sub-step / stage indices outside [0, nj) / [0, nk) (prologue and tail)
    // load nothing.  The prologue's are issued before every real load, so no
    // wait count includes them; the waits that could count a missing tail
    // load wait for everything instead (substep).
    auto issue_a = [&](int j, int nab_s) {  // A half of sub-step j
        if (j < 0 || j >= nj) return;
        uint16_t* dst = aring + (j % RA) * AST;
        const __amdgpu_buffer_rsrc_t ra = j % HALVES ? ra1 : ra0;
        const uint32_t soff = (uint32_t)(j / HALVES) * (2 * GBK);
#pragma unroll
        for (int i = 0; i < NAD; ++i)
            if (!SKIP_A || i * 8 + wave < nab_s) dma16<0>(ra, aoff[i], soff, dst + (i * 8 + wave) * 512);
    };
    auto issue_b = [&](int s) {  // B of K stage s
        if (s < 0 || s >= nk) return;
        uint16_t* dst = bring + (s % RB) * (64 * CB * GBK) + wave * NBD * 512;
#pragma unroll
        for (int i = 0; i < NBD; ++i) dma16(rb, boff[i], (uint32_t)s * (2 * GBK), dst + i * 512);
    };
    // B stage row of this wavefront's column block cb.  The weights are the
    // MFMA's first operand, so lane (fr, fq) ends with output columns
    // 4 fq .. 4 fq + 3 of the block for row fr of the row block.
    auto brow = [&](int cb) {
        return EPI == EPI_SWIGLU ? (cb < CB / 2 ? 8 * CB * cg + 16 * cb : 32 * CB + 8 * CB * cg + 16 * (cb - CB / 2)) + fr
                                 : 16 * CB * cg + 16 * cb + fr;
    };
    // LDS fragments: weights of column block cb, activations of row block j,
    // K half kh of the stage.
    auto wfrag = [&](const uint16_t* bt, int cb, int kh) {
        const int r = brow(cb);
        const int c = (kh * 4 + fq) ^ (r & 7);
        return *reinterpret_cast<const u32x4*>(bt + r * GBK + c * 8);
    };
    auto afrag = [&](const uint16_t* at, int j, int kh) {
        const int r = 16 * (2 * j + par) + fr;
        const int c = (kh * 4 + fq) ^ (r & 7);
        return *reinterpret_cast<const u32x4*>(at + r * GBK + c * 8);
    };
    // One stage's multiplies as a chain of steps (kh, j), j < nmine, each
    // reading the next step's activation fragment before its own multiplies
    // so that the LDS latency hides under them.  Every step's fragment has a
    // variable of its own (av[kh][j], all indices compile-time), so no copy
    // has to wait for a read in flight.  Per accumulator the order of the
    // multiplies is kh = 0 then 1, as ever.
    // One stage's multiplies for a wavefront with NM row blocks, as straight
    // code: a guard per row block inside the K loop becomes a branch per
    // block, and the counter waits at the branches' joins fall back to
    // lgkmcnt(0), which serialises every fragment read with its multiplies.
    // With two halves of A the weight fragments of a K stage are read once,
    // in the hi sub-step, and kept in registers (wk) for the lo sub-step: the
    // stage's ring slot is not refilled before the next stage's barrier, and
    // the lo sub-step reads only its activations.
    u32x4 wk[2][CB];
    auto compute_n = [&](const uint16_t* at, const uint16_t* bt, auto nm_c, auto half_c) {
        constexpr int NM = decltype(nm_c)::value;
        constexpr bool READ_W = HALVES == 1 || decltype(half_c)::value == 0;
        u32x4 av[2][NM];
        if constexpr (READ_W) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) wk[0][cb] = wfrag(bt, cb, 0);
        }
        av[0][0] = afrag(at, 0, 0);
        // kh = 1's weights now too, registers permitting (not for 384 columns
        // or 256 rows with one half, where they are read after kh = 0)
        constexpr bool W1_EARLY = RBW * CB <= 24 || HALVES == 2;
        if constexpr (READ_W && W1_EARLY) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) wk[1][cb] = wfrag(bt, cb, 1);
        }
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            if constexpr (READ_W && !W1_EARLY) {
                if (kh == 1) {
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) wk[1][cb] = wfrag(bt, cb, 1);
                }
            }
#pragma unroll
            for (int j = 0; j < NM; ++j) {
                if (j + 1 < NM)
                    av[kh][j + 1] = afrag(at, j + 1, kh);
                else if (kh == 0)
                    av[1][0] = afrag(at, 0, 1);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[j][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wk[kh][cb]), as_bf16x8(av[kh][j]),
                                                                         acc[j][cb], 0, 0, 0);
            }
        }
    };
    // The same with the row-block count known only at run time (a guard per
    // row block): for tiles whose accumulators leave no registers for a K
    // loop per row-block count (384 columns, or 256 rows).
    auto compute_rt = [&](const uint16_t* at, const uint16_t* bt, int nm, auto half_c) {
        constexpr bool READ_W = HALVES == 1 || decltype(half_c)::value == 0;
        u32x4 (&w)[2][CB] = wk;
        u32x4 av[2][RBW];
        if constexpr (READ_W) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) w[0][cb] = wfrag(bt, cb, 0);
        }
        av[0][0] = afrag(at, 0, 0);
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            if (READ_W && kh == 1) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) w[1][cb] = wfrag(bt, cb, 1);
            }
#pragma unroll
            for (int j = 0; j < RBW; ++j) {
                if (j < nm) {  // a guard, not a break: acc must stay in registers
                    if (j + 1 < nm) {
                        if (j + 1 < RBW) av[kh][j + 1] = afrag(at, j + 1, kh);
                    } else if (kh == 0) {
                        av[1][0] = afrag(at, 0, 1);
                    }
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
                        acc[j][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            as_bf16x8(w[kh][cb]), as_bf16x8(av[kh][j]), acc[j][cb], 0, 0, 0);
                }
            }
        }
    };
    // One K loop per row-block count where registers allow it (192-row
    // gate/up tiles: 96 accumulator registers; any tile whose weight
    // fragments serve two halves, as they need no second set of registers),
    // else one K loop with guards.
    constexpr bool PER_NM = RBW * CB <= 24;
    auto substep = [&](int s, auto half_c, auto nm_c) {
        constexpr int half = decltype(half_c)::value;
        const int j = s * HALVES + half;
        // The loads issued before this sub-step go up to A(j - 1 + DA) and
        // B(floor((j - 1) / H) + DB): while all exist the steady count holds.
        const int jp = j - 1;
        const int sp = (jp >= 0 ? jp : jp - (HALVES - 1)) / HALVES;  // floor
        if (jp + DA < nj && sp + DB < nk)
            wait_vmcnt<split_after(HALVES, DA, DB, half, NAD, NBD)>();
        else
            wait_vmcnt<0>();
        lds_barrier();
        // Fresh scalar copies of the item's bounds in every sub-step: the
        // compiler would otherwise hoist each guard's comparison out of the K
        // loop as a lane mask and rebuild a branch from it at every guard.
        int nm = nmine, nab_s = nab;
        asm volatile("" : "+s"(nm), "+s"(nab_s));
        issue_a(j + DA, nab_s);
        if (half == 0) issue_b(s + DB);
        const uint16_t* at = aring + (j % RA) * AST;
        const uint16_t* bt = bring + (s % RB) * (64 * CB * GBK);
        if constexpr (!PER_NM)
            compute_rt(at, bt, nm, half_c);
        else if constexpr (decltype(nm_c)::value > 0)
            compute_n(at, bt, nm_c, half_c);
    };
    // SCATTER: the token-order output rows of the epilogue, read now (192-row
    // tiles; the 256-row tiles have no registers to spare) so that their
    // latency hides under the item.
    constexpr bool EARLY_ROWS = EPI == EPI_SCATTER && ROWS == kPrefillTileRows && HALVES == 1;
    [[maybe_unused]] int orow[EARLY_ROWS ? RBW : 1];
    if constexpr (EARLY_ROWS) {
#pragma unroll
        for (int j = 0; j < RBW; ++j) {
            const int rl = 16 * (2 * j + par) + fr;
            orow[j] = j < nmine && rl < rows ? a.scatter_rows[row0 + rl] : 0;
        }
    }
    on_setup();
    // Prologue: the sub-steps before 0 of the steady pattern (ops with an
    // index below 0 load nothing), so the counts split_after assumes hold
    // from sub-step 0 on.
    constexpr int Q = DA > HALVES * DB ? DA : HALVES * DB;
#pragma unroll
    for (int q = -Q; q < 0; ++q) {
        issue_a(q + DA, nab);
        if ((q % HALVES) == 0) issue_b(q / HALVES + DB);
    }
    // The K loop, compiled once per row-block count of the wavefront (0 ..
    // RBW) and chosen once per item, so each stage's multiplies are straight
    // code with exact counter waits.
    auto kloop = [&](auto nm_c) {
        for (int s = 0; s < nk; ++s) {
            substep(s, std::integral_constant<int, 0>{}, nm_c);
            if constexpr (HALVES == 2) substep(s, std::integral_constant<int, 1>{}, nm_c);
        }
    };
    if constexpr (PER_NM) {
        static_for_desc<RBW + 1>([&](auto n1_c) {
            if (nmine == decltype(n1_c)::value - 1) kloop(std::integral_constant<int, decltype(n1_c)::value - 1>{});
        });
    } else {
        kloop(std::integral_constant<int, -1>{});
    }

    // Every load of the item has landed (the last sub-steps wait for all).
    // Epilogue: the output rows (SCATTER: y, read once by the combine) go out
    // with non-temporal stores.
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
        const int rl = 16 * (2 * j + par) + fr;
        const int col0 = EPI == EPI_SWIGLU ? n0 + 8 * CB * cg + 4 * fq : n0 + 16 * CB * cg + 4 * fq;
        if (j < nmine && rl < rows) {
            int dst = row0 + rl;
            if constexpr (EARLY_ROWS)
                dst = orow[j];
            else if (EPI == EPI_SCATTER)
                dst = a.scatter_rows[row0 + rl];
            store_tile_row<EPI, CB, EPI == EPI_SCATTER>(a, acc[j], row0 + rl, col0, ks, dst);
        }
    }
}

// Dynamic items of the prefill kernel: each XCD's workgroups take the XCD's
// items (item_deal.h: its block of the shared expert's items, then its own M
// tiles) in order from a counter (zeroed by the dispatch), then help the
// other XCDs with theirs, so the kernel ends when the last item does, not
// when the workgroup dealt the most items does.  Thread 0 takes the next item
// while the current one runs (its atomic goes out with the item's first
// loads), so no workgroup waits on the counter between items.  Every grab
// advances a counter and each counter stops yielding at its XCD's item count:
// the loop ends.
template <class Run>
__device__ __forceinline__ void dynamic_items(const GemmArgs& a, const ItemRange& r, Run&& run) {
    const int t = threadIdx.x;
    __shared__ int next_item;
    int probe = 0;  // thread 0: counters found spent, in probing order from this XCD's
    auto grab = [&]() { return (int)atomicAdd(a.item_ctr + (r.xcd + probe) % r.nxcd, 1u); };
    // Thread 0: the item of grab li, probing the next counters once one is spent; -1 when all are.
    auto settle = [&](int li) {
        for (;;) {
            const int x = (r.xcd + probe) % r.nxcd;
            if (li < xcd_items(r.deal(), x)) return xcd_item(r.deal(), x, li);
            if (++probe >= r.nxcd) return -1;
            li = grab();
        }
    };
    auto publish = [&](int v) {  // thread 0's value to the workgroup
        if (t == 0) next_item = v;
        lds_sync();
        v = next_item;
        lds_sync();
        return v;
    };
    int item = publish(t == 0 ? settle(grab()) : 0);
    while (item >= 0) {
        int li = 0;
        run(item, [&] {
            if (t == 0 && probe < r.nxcd) li = grab();
        });
        item = publish(t == 0 ? (probe < r.nxcd ? settle(li) : -1) : 0);
    }
}

template <int EPI, int LOM, int ROWS>
__global__ __launch_bounds__(512, 1) void grouped_gemm_split_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t slds[];  // split_lds_max(ROWS, CB) bytes
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int m_tiles = a.ntiles_dev ? *a.ntiles_dev : a.m_tiles;
    const ItemRange r = item_range<true>(a, m_tiles);
    const bool use_lo = LOM == kLoAlways || (LOM == kLoByFlag && *a.a_lo_flag != 0u);
    // One item, then a barrier: every wavefront is done with the LDS rings
    // before the next item's loads land in them.  (The item's own loads have
    // all landed; its stores need not have.)
    auto run = [&](int item, auto&& on_setup) {
        if (group_absent(a, a.tile_group ? a.tile_group[item / a.ksplit / a.n_tiles] : 0)) {
            on_setup();
            return;
        }
        if (LOM != kLoNone && use_lo)
            gemm_item_split<EPI, ROWS, 2>(a, item, slds, t, wave, on_setup);
        else
            gemm_item_split<EPI, ROWS, 1>(a, item, slds, t, wave, on_setup);
        lds_barrier();
    };
    // 256-row tiles fill the whole 160 KB of LDS, leaving none for the
    // dynamic loop's shared item slot: they always take static items.
    if (ROWS != kPrefillTileRows || !a.item_ctr || !r.by_mtile) {
        for (int li = r.begin; li < r.end; li += r.stride) run(r.item(li), [] {});
        return;
    }
    if constexpr (ROWS == kPrefillTileRows) dynamic_items(a, r, run);
}

// ---------------------------------------------------------------------------
// Wide prefill tiles: gate/up 192 (M) x 512 (N: 256 gate + 256 up weight
// rows) x 64 (K), or 160 x 512 x 64 when x has a lo half; the down projection
// 160 x 512 x 64 (h: always two halves).  Eight wavefronts, one workgroup per
// CU.
//
// What bounds the prefill GEMMs is the CU's stream of line requests to L2:
// the weights once, plus the activation rows once per N tile.  Per weight
// byte the activations add rows x halves / N; 512 weight rows per tile instead
// of 256 cut that from 0.56 to 0.28 (gate/up, BF16-valued x) and from 1.12
// to 0.56 (FP32 x: hi and lo halves), and instead of the down projection's
// 384 from 0.75 to about 0.5.  Registers and LDS set the layout:
//   * wavefront w owns weight rows [64 w, 64 w + 64) of the tile (32 gate
//     rows then the 32 matching up rows) and all rows of the M tile: up to
//     12 x 4 accumulator blocks, 192 of its 256 registers, and no weight
//     fragment is read by two wavefronts;
//   * so each wavefront streams its own weights, in 128-byte lines, through a
//     private LDS ring of three half-stages (32 rows x 64 k, 4 KB), reading
//     a stage's weight fragments into registers before multiplying with them
//     (with two halves of A, all 32 registers of them once per stage, kept
//     for the second half: room that the 160-row tiles' 160 accumulator
//     registers leave, and the reason for those tiles); the slots read are
//     refilled with the next half-stages as soon as their reads have landed,
//     so 1.5 stages of weights stay in flight per wavefront with no barrier
//     among wavefronts for them;
//   * the activations (shared by all eight wavefronts) go by DMA into a
//     two-slot ring of sub-steps (up to 192 rows x 64 k; a K stage has one
//     sub-step per half of A), with one barrier per sub-step.
// 2 x 24 KB of activations + 8 x 3 x 4 KB of weights = 144 KB of LDS.
// With one half of A the 192-row tiles measure faster (fewer shared-expert
// tiles); the 160-row ones still hold a near-uniform prefill's ~128-row
// experts in one tile.  The cost of this layout is LDS reads: every
// wavefront reads all rows' activation fragments (with the weight fragments
// kept for the second half, about 5 bytes per weight byte, as on the 384-row
// split tiles).
constexpr int kWideWaves = 8;
constexpr int kWideWaveRows = kWideTileCols / kWideWaves;  // weight rows per wavefront
constexpr int kWideHalfRows = kWideWaveRows / 2;           // weight rows per half-stage
constexpr int kWideWRing = 3;                              // half-stages per wavefront ring
constexpr size_t kWideLds = 2 * (2 * (size_t)kPrefillTileRows * GBK +
                                 (size_t)kWideWaves * kWideWRing * kWideHalfRows * GBK);
static_assert(kWideLds + 64 <= 160 * 1024, "wide LDS");

// Sub-step j = H * s + half multiplies A half `half` of K stage s.  The
// first sub-step of a stage reads the wavefront's weight fragments of stage s
// (half-stages 2s, 2s + 1) from its ring; with two halves it reads them all
// at once and keeps them in registers for the second.  Issue order: sub-step
// j issues A(j + 1) over its first k half (after its barrier) and weight
// half-stages over its second k half, into the ring slots stage s came from
// (whose reads have all landed by then): 2s + 3 and 2s + 4 with one half,
// else 2s + 3 from the first sub-step and 2s + 4 from the second.  Loads
// complete in issue order, so a sub-step may leave exactly the last weight
// half-stage issued before it outstanding (split_pipeline.h: wide_after).
// EPI_SWIGLU: the gate/up GEMM (x, one or two halves); EPI_SCATTER: the down
// projection (h, two halves), each wavefront's 64 weight rows 64 consecutive
// output columns (half-stage h: rows 32 h + [0, 32) of them).
template <int EPI, int HALVES, class Setup>
__device__ __forceinline__ void gemm_item_wide(const GemmArgs& a, int item, uint16_t* lds, int t, int wave,
                                               Setup&& on_setup) {
    static_assert(EPI == EPI_SWIGLU || (EPI == EPI_SCATTER && HALVES == 2), "wide tiles");
    constexpr bool SW = EPI == EPI_SWIGLU;
    constexpr int ROWS = HALVES == 1 ? kPrefillTileRows : kWideTileRows;
    constexpr int AST = ROWS * GBK;                 // elements per A sub-step slot
    constexpr int NAD = (ROWS / 8 + kWideWaves - 1) / kWideWaves;  // A DMAs (8 rows x 128 bytes) per wavefront
    constexpr int NWH = kWideHalfRows / 8;          // weight DMAs per half-stage
    constexpr int NWS = wide_w_per_substep(HALVES);  // weight half-stages issued per sub-step
    static_assert(NAD == 3 && NWH == 4, "the counts tests/split_pipeline checks the waits with");
    constexpr int WHS = kWideHalfRows * GBK;        // elements per weight half-stage slot
    constexpr int CB = kWideWaveRows / 16;          // column blocks per wavefront
    uint16_t* aring = lds;
    uint16_t* wring = lds + 2 * AST + wave * (kWideWRing * WHS);
    const int lane = t & 63;
    const int fr = lane & 15;
    const int fq = lane >> 4;
    const int nk = a.K / GBK;
    const int nj = nk * HALVES;

    item = __builtin_amdgcn_readfirstlane(item);
    const int nt = item % a.n_tiles;
    const int mt = item / a.n_tiles;
    // (the tile table is read with vector loads: the kernel writes memory too)
    const int g = __builtin_amdgcn_readfirstlane(a.tile_group ? a.tile_group[mt] : 0);
    const int row0 = __builtin_amdgcn_readfirstlane(a.tile_row0 ? a.tile_row0[mt] : mt * ROWS);
    const int row_end = __builtin_amdgcn_readfirstlane(a.group_end ? a.group_end[g] : a.rows_total);
    const int rows = min(ROWS, row_end - row0);
    const int nrb = (rows + 15) >> 4;
    const int n0 = nt * (SW ? kWideTileCols / 2 : kWideTileCols);  // first output column of the tile
    const uint16_t* b0 = a.b_tab ? a.b_tab[3 * g + a.b_which] : a.b_fixed0;  // gate (down) rows
    const uint16_t* b1 = !SW ? b0 : a.b_tab ? a.b_tab[3 * g + a.b_which + 1] : a.b_fixed1;  // up rows

    // DMA lane l of an 8-row block loads chunk (l & 7) ^ (l >> 3) of block row
    // l >> 3, so 16-byte chunk c of slot row r sits at position c ^ (r & 7):
    // conflict-free for the lane-contiguous DMA writes and for the fragment
    // reads (16 rows x 16 bytes per quarter wavefront).
    const int dr = lane >> 3;
    const int dc = (lane & 7) ^ dr;
    // A: 8-row block 8 i + wave of the tile (rows past the item's last re-read
    // it; blocks past its last 16-row block are not loaded at all).
    uint32_t aoff[NAD];
#pragma unroll
    for (int i = 0; i < NAD; ++i) {
        const int r = 8 * (kWideWaves * i + wave) + dr;
        const int gr = row0 + min(r, rows - 1);
        const size_t src = (size_t)(a.a_rowmap ? a.a_rowmap[gr] : gr);
        aoff[i] = (uint32_t)(2 * (src * a.K + dc * 8));
    }
    // Weights: half-stage h of this wavefront is gate rows (h = 0) or the
    // matching up rows (h = 1) n0 + 32 w + [0, 32), or down rows
    // n0 + 64 w + 32 h + [0, 32); DMA i covers 8 of them.
    const int wrow = n0 + (SW ? kWideHalfRows : kWideWaveRows) * wave + dr;
    const uint32_t woff = (uint32_t)(2 * ((size_t)wrow * a.b_ld + dc * 8));
    const __amdgpu_buffer_rsrc_t rw0 = raw_rsrc(uniform_ptr(b0));
    const __amdgpu_buffer_rsrc_t rw1 = raw_rsrc(uniform_ptr(b1));
    const __amdgpu_buffer_rsrc_t ra0 = raw_rsrc(a.a_hi);
    const __amdgpu_buffer_rsrc_t ra1 = raw_rsrc(HALVES == 2 ? a.a_lo : a.a_hi);
    const uint32_t wrow_bytes = (uint32_t)a.b_ld * 2;

    // DMA i of A sub-step j (nothing past the last sub-step or the item's rows).
    auto issue_a1 = [&](int j, int i, int nab) {
        const int blk = kWideWaves * i + wave;
        if (j >= nj || blk >= nab) return;
        dma16<0>(pick((j % HALVES) != 0, ra1, ra0), aoff[i], (uint32_t)(j / HALVES) * (2 * GBK), aring + (j & 1) * AST + blk * 512);
    };
    auto issue_a = [&](int j, int nab) {
#pragma unroll
        for (int i = 0; i < NAD; ++i) issue_a1(j, i, nab);
    };
    // DMA i of weight half-stage q = 2 s + h (nothing past the last).
    auto issue_w1 = [&](int q, int i) {
        if (q >= 2 * nk) return;
        const int s = q >> 1, h = q & 1;
        dma16(pick(h != 0, rw1, rw0), woff,
              (uint32_t)s * (2 * GBK) + (uint32_t)(8 * i + (SW ? 0 : kWideHalfRows * h)) * wrow_bytes,
              wring + (q % kWideWRing) * WHS + i * 512);
    };
    auto issue_w = [&](int q) {
#pragma unroll
        for (int i = 0; i < NWH; ++i) issue_w1(q, i);
    };
    // Fragments: slot row r, 16-byte chunk c at position c ^ (r & 7).
    auto frag = [&](const uint16_t* slot, int r, int c) {
        return *reinterpret_cast<const u32x4*>(slot + r * GBK + ((c ^ (r & 7)) * 8));
    };

    on_setup();
    const int nab0 = 2 * nrb;
    issue_a(0, nab0);
    issue_w(0);
    issue_w(1);
    issue_w(2);

    // The K loop, compiled per row-block count of the item (all eight
    // wavefronts share it), so every sub-step's multiplies are straight code.
    auto kloop = [&](auto nm_c) __attribute__((always_inline)) {
        constexpr int NM = decltype(nm_c)::value;
        f32x4_t acc[NM > 0 ? NM : 1][CB];
#pragma unroll
        for (int j = 0; j < NM; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) acc[j][cb] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
        u32x4 wk[2][CB];  // the stage's weight fragments [k half][column block]
        // One sub-step's multiplies: per k half, the CB weight fragments of
        // that half, each activation fragment (read one step ahead) against
        // them.  The weight fragments come from the wavefront's ring: with one
        // half of A, the second k half's reads go out one by one as the first
        // half's last multiplies free their registers; with two, a stage's
        // first sub-step reads all of them up front and the second reuses
        // them.  The DMAs go out one at a time between row blocks rather than
        // in a burst (a DMA waits at issue while the CU's queue of line
        // requests is full, holding up the multiplies behind it): A(j + 1)
        // over the first k half; the weight half-stages from wq on over the
        // second, once every read of the ring slots they overwrite has landed.
        auto compute = [&](const uint16_t* at, int s, bool first, int jn, int nab, int wq)
                           __attribute__((always_inline)) {
            const uint16_t* w0 = wring + ((2 * s) % kWideWRing) * WHS;
            const uint16_t* w1 = wring + ((2 * s + 1) % kWideWRing) * WHS;
            auto wfrag = [&](int cb, int kh) {
                return frag(cb < CB / 2 ? w0 : w1, 16 * (cb % (CB / 2)) + fr, kh * 4 + fq);
            };
            auto dma = [&](auto&& f) {
                asm volatile("" ::: "memory");
                f();
                asm volatile("" ::: "memory");
            };
            // After row block r of k half kh (r == -1: before any).
            auto dmas_after = [&](int kh, int r) {
                constexpr int NMX = NM > 0 ? NM : 1;
                constexpr int NW = NWS * NWH;
                if (kh == 0) {  // A(jn): DMA r + 1 after row block r, the rest after the last
#pragma unroll
                    for (int i = 0; i < NAD; ++i)
                        if (i == r + 1 || (r == NMX - 1 && i > r + 1)) dma([&] { issue_a1(jn, i, nab); });
                } else {  // NW weight DMAs spread over the row blocks
                    if (r == -1) {
                        asm volatile("" ::: "memory");
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slots' reads are done
                    }
#pragma unroll
                    for (int k = 0; k < NW; ++k)
                        if (k * NMX / NW == r + 1 || (r == NMX - 1 && k * NMX / NW > r))
                            dma([&] { issue_w1(wq + k / NWH, k % NWH); });
                }
            };
            if constexpr (NM > 0) {
                if constexpr (HALVES == 1) {
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) wk[0][cb] = wfrag(cb, 0);
                } else if (first) {
#pragma unroll
                    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                        for (int cb = 0; cb < CB; ++cb) wk[kh][cb] = wfrag(cb, kh);
                }
                u32x4 av[2][NM];
                av[0][0] = frag(at, fr, fq);
#pragma unroll
                for (int kh = 0; kh < 2; ++kh) {
                    dmas_after(kh, -1);
#pragma unroll
                    for (int j = 0; j < NM; ++j) {
                        if (j + 1 < NM)
                            av[kh][j + 1] = frag(at, 16 * (j + 1) + fr, kh * 4 + fq);
                        else if (kh == 0)
                            av[1][0] = frag(at, fr, 4 + fq);
#pragma unroll
                        for (int cb = 0; cb < CB; ++cb) {
                            acc[j][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                as_bf16x8(wk[kh][cb]), as_bf16x8(av[kh][j]), acc[j][cb], 0, 0, 0);
                            if (HALVES == 1 && kh == 0 && j == NM - 1) wk[1][cb] = wfrag(cb, 1);
                        }
                        dmas_after(kh, j);
                        // Keep the reads one step ahead: hoisted further, they
                        // would hold registers the accumulators need.
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            } else {
                issue_a(jn, nab);
#pragma unroll
                for (int k = 0; k < NWS; ++k) issue_w(wq + k);
            }
        };
        for (int j = 0; j < nj; ++j) {
            // Sub-step j: A(j); the first of a stage also weight half-stages
            // 2s, 2s+1.
            const int s = j / HALVES;
            const bool first = HALVES == 1 || (j & 1) == 0;
            // (two ways, as here: a three-way branch around the waits made the
            // compiler schedule the two-half K loop ~35 % slower)
            if (wide_steady(s, nk))
                wait_vmcnt<wide_after(NWH)>();
            else
                wait_vmcnt<0>();
            lds_barrier();
            int nab = nab0;
            asm volatile("" : "+s"(nab));
            compute(aring + (j & 1) * AST, s, first, j + 1, nab, 2 * s + 3 + (first ? 0 : 1));
        }
        // Every load of the item has landed (the last stage waits for all).
        // SWIGLU: h columns n0 + 32 w + 16 cb + 4 fq + q from gate block cb
        // and up block cb + 2; SCATTER: y columns n0 + 64 w + 16 cb + 4 fq + q.
        const int col0 = n0 + (SW ? kWideHalfRows : kWideWaveRows) * wave + 4 * fq;
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            const int rl = 16 * j + fr;
            if (rl < rows)
                store_tile_row<EPI, CB>(a, acc[j], row0 + rl, col0, 0, SW ? row0 + rl : a.scatter_rows[row0 + rl]);
        }
    };
    // Row-block counts in buckets (8 .. 12 or 10 exact, the near-uniform
    // prefill's range; smaller ones rounded up to even): the extra blocks multiply rows
    // that were not loaded and are never stored.
    const int nb = nrb >= 8 ? nrb : (nrb + 1) & ~1;
    static_for_desc<ROWS / 16>([&](auto n_c) {
        constexpr int NM = decltype(n_c)::value;
        if constexpr (NM >= 8 || NM % 2 == 0) {
            if (nb == NM) kloop(std::integral_constant<int, NM>{});
        }
    });
}

// EPI_SWIGLU: x (BF16 hi, and lo when the device flag says x is not
// BF16-valued) times the gate and up weights, h = silu(g) * u out as BF16
// hi / lo; with the lo half the items are those of the 160-row M tiles
// (GemmArgs::lo_tiles), else of the 192-row ones.  EPI_SCATTER: h (hi and lo)
// times the down weights on the launch's own 160-row tiles, y rows scattered.
template <int EPI>
__global__ __launch_bounds__(64 * kWideWaves, 1) void grouped_gemm_wide_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t wlds[];  // kWideLds bytes
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    // One item, then a barrier: every wavefront is done with the activation
    // ring before the next item's loads land in it.
    auto items = [&](const GemmArgs& b, auto halves_c) __attribute__((always_inline)) {
        constexpr int HALVES = decltype(halves_c)::value;
        const int m_tiles = b.ntiles_dev ? *b.ntiles_dev : b.m_tiles;
        const ItemRange r = item_range<true>(b, m_tiles);
        auto run = [&](int item, auto&& on_setup) __attribute__((always_inline)) {
            if (group_absent(b, b.tile_group ? b.tile_group[item / b.n_tiles] : 0)) {
                on_setup();
                return;
            }
            gemm_item_wide<EPI, HALVES>(b, item, wlds, t, wave, on_setup);
            lds_barrier();
        };
        if (!b.item_ctr || !r.by_mtile) {
            for (int li = r.begin; li < r.end; li += r.stride) run(r.item(li), [] {});
            return;
        }
        dynamic_items(b, r, run);
    };
    if constexpr (EPI == EPI_SCATTER) {
        items(a, std::integral_constant<int, 2>{});
    } else if (*a.a_lo_flag != 0u) {
        GemmArgs b = a;
        b.tile_rows = kWideTileRows;
        b.tile_group = a.lo_tiles.group;
        b.tile_row0 = a.lo_tiles.row0;
        b.ntiles_dev = a.lo_tiles.count;
        b.shared_mtiles = a.lo_tiles.shared_mtiles;
        items(b, std::integral_constant<int, 2>{});
    } else {
        items(a, std::integral_constant<int, 1>{});
    }
}

// out[t] = (sum_r w[t, r] * y[t*k + r]) + y[shared_row0 + t] (when shared_row0 >= 0):
// the weighted merge in rank order, then the shared expert (glm_forward.cpp:639-640, 658-660).
__global__ void combine_kernel(const float* __restrict__ wts, const float* __restrict__ y, int T, int k,
                               int d, int shared_row0, float* __restrict__ out) {
    const size_t i4 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int d4 = d >> 2;
    if (i4 >= (size_t)T * d4) return;
    const int t = (int)(i4 / d4), n4 = (int)(i4 % d4);
    // y is read once: non-temporal loads.
    const f32x4_t* y4 = reinterpret_cast<const f32x4_t*>(y);
    float4 m = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r = 0; r < k; ++r) {
        const float w = wts[(size_t)t * k + r];
        const f32x4_t v = __builtin_nontemporal_load(y4 + ((size_t)t * k + r) * d4 + n4);
        m.x += w * v.x;
        m.y += w * v.y;
        m.z += w * v.z;
        m.w += w * v.w;
    }
    if (shared_row0 >= 0) {
        const f32x4_t v = __builtin_nontemporal_load(y4 + ((size_t)shared_row0 + t) * d4 + n4);
        m.x += v.x;
        m.y += v.y;
        m.z += v.z;
        m.w += v.w;
    }
    reinterpret_cast<float4*>(out)[i4] = m;
}

// x FP32 [n] -> BF16 hi/lo; *flag = 1 when any lo is nonzero.  Eight values
// per thread and step (two 16-byte loads, one 16-byte store per half) when x
// is 16-byte aligned, then single values for the rest.  x is read once:
// non-temporal loads; hi/lo are read again by the GEMMs that follow.
__global__ void split_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ hi,
                                  uint16_t* __restrict__ lo, size_t n, unsigned* __restrict__ flag) {
    bool nz = false;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(hi) |
                       reinterpret_cast<uintptr_t>(lo)) & 15) == 0;
    const size_t n8 = vec ? n / 8 : 0;
    for (size_t i = tid; i < n8; i += stride) {
        const f32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(x) + 2 * i);
        const f32x4_t b = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(x) + 2 * i + 1);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t h0 = f32_to_bf16(v[2 * q]), h1 = f32_to_bf16(v[2 * q + 1]);
            const uint32_t l0 = f32_to_bf16(v[2 * q] - __uint_as_float(h0 << 16));
            const uint32_t l1 = f32_to_bf16(v[2 * q + 1] - __uint_as_float(h1 << 16));
            hw[q] = h0 | (h1 << 16);
            lw[q] = l0 | (l1 << 16);
            nz |= ((l0 | l1) & 0x7FFFu) != 0;
        }
        reinterpret_cast<u32x4*>(hi)[i] = (u32x4){hw[0], hw[1], hw[2], hw[3]};
        reinterpret_cast<u32x4*>(lo)[i] = (u32x4){lw[0], lw[1], lw[2], lw[3]};
    }
    for (size_t i = n8 * 8 + tid; i < n; i += stride) {
        const float v = x[i];
        const uint16_t h = f32_to_bf16(v);
        const uint16_t l = f32_to_bf16(v - __uint_as_float((uint32_t)h << 16));
        hi[i] = h;
        lo[i] = l;
        nz |= (l & 0x7FFF) != 0;
    }
    // A plain store: the flag only goes from 0 (cleared by an earlier kernel)
    // to 1 and is read by later kernels; with FP32 activations every
    // wavefront sets it, and as many device-scope atomics on one address
    // serialise at the memory (x split of 4096 x 6144: 199 -> 37 us).
    if (__ballot(nz) != 0ull && (threadIdx.x & 63) == 0) *flag = 1u;
}

// out[i] = ((part[0][i] + part[1][i]) + part[2][i]) + ...: the K splits of a
// PARTIAL GEMM ([ks][n] FP32) summed in split order, four values per thread
// (n a multiple of 4, both arrays 16-byte aligned).
__global__ void sum_splits_kernel(const float* __restrict__ part, int ks, size_t n4, float* __restrict__ out) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(part) + i);
        for (int k = 1; k < ks; ++k) v += __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(part) + k * n4 + i);
        reinterpret_cast<f32x4_t*>(out)[i] = v;
    }
}

hipError_t launch_sum_splits(const float* part, int ks, size_t n, float* out, hipStream_t s) {
    if (ks < 1 || n % 4 || ((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(out)) & 15))
        return hipErrorInvalidValue;
    const size_t n4 = n / 4;
    size_t blocks = (n4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    return launch(sum_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, ks, n4, out);
}

// Four consecutive h columns of one token per thread: g and u summed over the
// splits in split order (as sum_splits_kernel sums), then the epilogue's
// silu_mul and hi / lo split.
__global__ void swiglu_splits_kernel(const float* __restrict__ part, int ks, int T, int I,
                                     uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo) {
    const int i4 = I >> 2;
    const size_t n4 = (size_t)T * i4;
    const size_t split4 = (size_t)T * (I >> 1);  // f32x4 elements per split: [T][2 I]
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(part);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const size_t t = i / i4, c4 = i % i4;
        const size_t gi = t * 2 * i4 + c4;  // gate columns 4 c4.., up columns I + 4 c4..
        f32x4_t gv = __builtin_nontemporal_load(p4 + gi);
        f32x4_t uv = __builtin_nontemporal_load(p4 + gi + i4);
        for (int k = 1; k < ks; ++k) {
            gv += __builtin_nontemporal_load(p4 + k * split4 + gi);
            uv += __builtin_nontemporal_load(p4 + k * split4 + gi + i4);
        }
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float h = silu_mul(gv[q], uv[q]);
            const uint32_t v0 = f32_to_bf16(h);
            const uint32_t v1 = f32_to_bf16(h - __uint_as_float(v0 << 16));
            if (q & 1) {
                hw[q >> 1] |= v0 << 16;
                lw[q >> 1] |= v1 << 16;
            } else {
                hw[q >> 1] = v0;
                lw[q >> 1] = v1;
            }
        }
        reinterpret_cast<uint2*>(h_hi)[i] = make_uint2(hw[0], hw[1]);
        reinterpret_cast<uint2*>(h_lo)[i] = make_uint2(lw[0], lw[1]);
    }
}

hipError_t launch_swiglu_splits(const float* part, int ks, int T, int I, uint16_t* h_hi, uint16_t* h_lo,
                                hipStream_t s) {
    if (ks < 1 || T < 0 || I <= 0 || I % 4 ||
        ((reinterpret_cast<uintptr_t>(part) & 15) | (reinterpret_cast<uintptr_t>(h_hi) & 7) |
         (reinterpret_cast<uintptr_t>(h_lo) & 7)))
        return hipErrorInvalidValue;
    const size_t n4 = (size_t)T * (I / 4);
    size_t blocks = (n4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    return launch(swiglu_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, ks, T, I, h_hi, h_lo);
}

__global__ void clear_u32_kernel(unsigned* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

hipError_t launch_clear_u32(unsigned* p, int n, hipStream_t s) {
    return launch(clear_u32_kernel, dim3((n + 63) / 64), dim3(64), 0, s, p, n);
}

// Router logits from split-K partials (summed in split order) and score pairs.
__global__ void router_reduce_kernel(const float* __restrict__ part, int ksplit, int T, int E,
                                     const float* __restrict__ bias, float* __restrict__ logits,
                                     float2* __restrict__ scores) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * E) return;
    const size_t st = (size_t)T * E;
    // Eight partials loaded at a time, summed in split order.
    float s = 0.0f;
    int q = 0;
    for (; q + 8 <= ksplit; q += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(part + (q + u) * st + i);
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; q < ksplit; ++q) s += part[q * st + i];
    logits[i] = s;
    scores[i] = score_pair(s, bias, i % E);
}

template <int EPI, int LOM, int WAVES>
static hipError_t launch_gemm(const GemmArgs& a, int blocks, hipStream_t s) {
    static bool raised = false;  // the ring exceeds the default 64 KB of dynamic LDS
    if (!raised) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(grouped_gemm_kernel<EPI, LOM, WAVES>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRingBytes);
        if (e != hipSuccess) return e;
        raised = true;
    }
    return launch(grouped_gemm_kernel<EPI, LOM, WAVES>, dim3(blocks), dim3(64 * WAVES), (uint32_t)kRingBytes, s, a);
}

template <int EPI, int LOM, int ROWS>
static hipError_t launch_gemm_split(const GemmArgs& a, int blocks, hipStream_t s) {
    constexpr size_t lds = split_lds_max(ROWS, split_cb<EPI, ROWS>());
    static bool raised = false;
    if (!raised) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(grouped_gemm_split_kernel<EPI, LOM, ROWS>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        raised = true;
    }
    return launch(grouped_gemm_split_kernel<EPI, LOM, ROWS>, dim3(blocks), dim3(512), (uint32_t)lds, s, a);
}

template <int EPI>
static hipError_t launch_gemm_wide(const GemmArgs& a, int blocks, hipStream_t s) {
    static bool raised = false;
    if (!raised) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(grouped_gemm_wide_kernel<EPI>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWideLds);
        if (e != hipSuccess) return e;
        raised = true;
    }
    return launch(grouped_gemm_wide_kernel<EPI>, dim3(blocks), dim3(64 * kWideWaves), (uint32_t)kWideLds, s, a);
}

template <int EPI, int LOM>
static hipError_t launch_shape(const GemmArgs& a, int blocks, hipStream_t s) {
    if (a.tile_cols == kWideTileCols) {
        // The MoE gate/up GEMM (on x, whose lo half goes by the device flag,
        // with the 160-row tile list for it) on 192-row tiles, and the MoE
        // down projection (h, both halves) on 160-row tiles: whole wide tiles
        // (their weight DMAs are not clamped at N), one K split.
        if constexpr (EPI == EPI_SWIGLU && LOM == kLoByFlag) {
            if (a.tile_rows == kPrefillTileRows && a.N % (kWideTileCols / 2) == 0 && a.ksplit == 1 &&
                a.a_lo_flag && a.lo_tiles.count)
                return launch_gemm_wide<EPI_SWIGLU>(a, blocks, s);
        }
        if constexpr (EPI == EPI_SCATTER && LOM == kLoAlways) {
            if (a.tile_rows == kWideTileRows && a.N % kWideTileCols == 0 && a.ksplit == 1 && a.scatter_rows)
                return launch_gemm_wide<EPI_SCATTER>(a, blocks, s);
        }
        return hipErrorInvalidValue;
    }
    if (a.tile_rows == 192 && a.tile_cols == 64 * split_cb<EPI, 192>()) return launch_gemm_split<EPI, LOM, 192>(a, blocks, s);
    if (a.tile_rows == 256 && a.tile_cols == 64 * split_cb<EPI, 256>()) return launch_gemm_split<EPI, LOM, 256>(a, blocks, s);
    if (a.tile_rows == kGemmTileRows && a.tile_cols == GBN) return launch_gemm<EPI, LOM, 4>(a, blocks, s);
    return hipErrorInvalidValue;
}

template <int EPI>
static hipError_t launch_epi(const GemmArgs& a, int blocks, hipStream_t s) {
    if (!a.a_lo) return launch_shape<EPI, kLoNone>(a, blocks, s);
    if (a.a_lo_flag) {
        // the flag is x's (gate/up, router, dense layers); the down
        // projection's h always carries both halves
        if constexpr (EPI != EPI_SCATTER) return launch_shape<EPI, kLoByFlag>(a, blocks, s);
        return hipErrorInvalidValue;
    }
    return launch_shape<EPI, kLoAlways>(a, blocks, s);
}

hipError_t launch_grouped_gemm(int epi, const GemmArgs& a, int blocks, hipStream_t s) {
    // The prefill kernel addresses each operand through a buffer resource
    // with 32-bit byte offsets: every weight matrix and activation array of a
    // launch must lie within 4 GiB of its base (at most a few hundred MB at
    // the supported shapes).
    const size_t lim = (size_t)1 << 32;
    if (a.tile_rows != kGemmTileRows &&
        ((size_t)a.N * (size_t)a.b_ld * 2 >= lim || (size_t)a.rows_total * (size_t)a.K * 2 >= lim))
        return hipErrorInvalidValue;
    // A second fixed matrix along N: split-kernel PARTIAL tiles that stay on
    // one side of the boundary.
    if (a.b_split && (epi != EPI_PARTIAL || a.b_tab || !a.b_fixed1 || a.b_split < 0 || a.b_split >= a.N ||
                      (a.tile_rows != kPrefillTileRows && a.tile_rows != kDenseTileRows) ||
                      a.b_split % a.tile_cols))
        return hipErrorInvalidValue;
    switch (epi) {
        case EPI_PARTIAL: return launch_epi<EPI_PARTIAL>(a, blocks, s);
        case EPI_SWIGLU: return launch_epi<EPI_SWIGLU>(a, blocks, s);
        case EPI_SCATTER: return launch_epi<EPI_SCATTER>(a, blocks, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_combine(const float* wts, const float* y, int T, int k, int d, int shared_row0,
                          float* out, hipStream_t s) {
    const size_t n4 = (size_t)T * (d / 4);
    return launch(combine_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, wts, y, T, k, d,
                  shared_row0, out);
}

hipError_t launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, size_t n, unsigned* flag,
                             hipStream_t s) {
    // flag[0]: x has a nonzero lo half (set below).
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
