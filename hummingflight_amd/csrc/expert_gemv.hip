// expert_gemv.hip -- decode (T = 1) expert SwiGLU as bandwidth-bound BF16 GEMVs.
//
// Reference arithmetic: expertFFNRaw glm_forward.cpp:434-449 (g = Wg.x,
// u = Wu.x, h = g/(1+exp(-g))*u, y = Wd.h), sharedExpertFFNRaw :459-479 and the
// weighted merge :555-556,639-640,658-660 (out = sum_r w_r*y_r + y_shared).
//
// Two launches over all selected experts at once:
//   gate/up: one wavefront per (slot, row i): streams row i of gate and up
//            (2*d BF16, 16-byte coalesced loads) against x staged in LDS as
//            FP32, writes h[slot][i] = silu(g)*u in FP32.  Shared-expert rows
//            come first; with in-kernel routing each block ranks the experts
//            (hf_select.h) once its wavefronts' first (shared) rows have
//            landed, while the other blocks' rows keep HBM busy.
//   down:    one block per set of output rows (groups of U consecutive rows,
//            interleaved across blocks so each batch of the chip reads one
//            contiguous stretch of every slot's down matrix), one wavefront
//            per slot streaming those rows with h_slot in VGPRs; the per-slot
//            products meet in LDS and are summed in a fixed order.
// No atomics: every output element has one fixed summation order, so results
// repeat bit for bit from run to run.
#include "hf_common.h"
#include "hf_kernels.h"
#include "hf_select.h"

namespace hf {

struct SlotW {
    const uint16_t* g;
    const uint16_t* u;
    const uint16_t* dn;
    int ld;  // row stride of the down matrix (I for routed, n_shared*I for shared)
};

// Slot s: s < k is routed expert e, else shared slice s - k.
__device__ __forceinline__ SlotW slot_weights(const LayerDev& L, const Cfg& c, int s, int e) {
    SlotW r;
    if (s < c.k) {
        e = min(max(e, 0), c.E - 1);  // ids come from the router; stay in the table
        r.g = L.etab[3 * e];
        r.u = L.etab[3 * e + 1];
        r.dn = L.etab[3 * e + 2];
        r.ld = c.I;
    } else {
        const int sh = s - c.k;
        const size_t off = (size_t)sh * c.I * c.d;
        r.g = L.sg + off;
        r.u = L.su + off;
        r.dn = L.sd + (size_t)sh * c.I;
        r.ld = c.n_shared * c.I;
    }
    return r;
}

// Up to 8 expert ids packed 16 bits apiece into two wave-uniform words, so a
// runtime slot index never indexes a register array.
struct PackedIds {
    uint64_t lo = 0, hi = 0;
    __device__ __forceinline__ void set(int r, int e) {
        const uint64_t v = (uint64_t)(e & 0xFFFF);
        if (r < 4) lo |= v << (16 * r);
        else hi |= v << (16 * (r - 4));
    }
    __device__ __forceinline__ int get(int r) const {
        return (int)(((r < 4 ? lo >> (16 * r) : hi >> (16 * (r - 4)))) & 0xFFFF);
    }
};

// Work item q -> (slot, row): shared slices first, then routed slots.
__device__ __forceinline__ void gateup_item(const Cfg& c, int shared_items, int q, int& s, int& i) {
    if (q < shared_items) {
        s = c.k + q / c.I;
        i = q - (s - c.k) * c.I;
    } else {
        const int rq = q - shared_items;
        s = rq / c.I;
        i = rq - s * c.I;
    }
}

// KCH = 16-byte chunks per lane per row (d <= 512*KCH; tail chunks masked).
// ROUTE: the block ranks the experts itself from the router's score pairs and
// block 0 publishes ids/weights to sel_io/selw_out; otherwise sel_io holds the
// k routed ids.  Block size is 256 threads.
template <int KCH, bool ROUTE>
__global__ __launch_bounds__(256) void gateup_t1_kernel(const float* __restrict__ x, LayerDev L,
                                                        Cfg c, const float2* __restrict__ scores,
                                                        int* __restrict__ sel_io,
                                                        float* __restrict__ selw_out,
                                                        float* __restrict__ h, int nslots) {
    const int lane = threadIdx.x & 63;
    const int gw = (int)((blockIdx.x * 256u + threadIdx.x) >> 6);
    const int nw = (int)gridDim.x * 4;
    const int nch = c.d >> 3;

    // x in LDS, chunk ch = x[8ch .. 8ch+8) split into halves xa[ch], xb[ch] so
    // that a wavefront's 16-byte LDS reads are consecutive (no bank conflicts).
    __shared__ float4 xa[64 * KCH], xb[64 * KCH];
    for (int ch = threadIdx.x; ch < 64 * KCH; ch += 256) {
        if (ch < nch) {
            xa[ch] = reinterpret_cast<const float4*>(x)[2 * ch];
            xb[ch] = reinterpret_cast<const float4*>(x)[2 * ch + 1];
        } else {
            xa[ch] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            xb[ch] = xa[ch];
        }
    }

    const int shared_items = (nslots - c.k) * c.I;
    const int total = nslots * c.I;
    PackedIds ids;
    u32x4 gv[KCH], uv[KCH];
    auto issue = [&](int q) {
        int s, i;
        gateup_item(c, shared_items, q, s, i);
        const SlotW sw = slot_weights(L, c, s, s < c.k ? ids.get(s) : 0);
        const u32x4* g4 = reinterpret_cast<const u32x4*>(sw.g + (size_t)i * c.d);
        const u32x4* u4 = reinterpret_cast<const u32x4*>(sw.u + (size_t)i * c.d);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const int ch = lane + 64 * j;
            if (ch < nch) {
                gv[j] = ld_stream(g4 + ch);
                uv[j] = ld_stream(u4 + ch);
            }
        }
    };

    int q = gw;
    bool preloaded = false;
    if (ROUTE) {
        __shared__ SelectSmem sm;
        // Scores first, then the first (shared) row's weights (routing-free).
        // The selection's block barriers wait for those weight loads as well;
        // a version that let the ranking run ahead of them (x and scores by LDS
        // DMA, LDS-only barriers) measured the same: the shared rows keep HBM
        // saturated meanwhile.
        SelectRegs regs;
        select_fetch(scores, c.E, regs);
        if (q < total && q < shared_items) {
            issue(q);
            preloaded = true;
        }
        const int kk = select_block(regs, c, sm);
        for (int r = 0; r < kk; ++r) ids.set(r, sm.sel[r]);
        if (blockIdx.x == 0 && (int)threadIdx.x < kk) {
            sel_io[threadIdx.x] = sm.sel[threadIdx.x];
            selw_out[threadIdx.x] = sm.w[threadIdx.x];
        }
    } else {
        for (int r = 0; r < c.k; ++r) ids.set(r, sel_io[r]);
        __syncthreads();
    }

    for (; q < total; q += nw) {
        int s, i;
        gateup_item(c, shared_items, q, s, i);
        if (!preloaded) issue(q);
        preloaded = false;
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const int ch = lane + 64 * j;
            if (ch < nch) {
                const float4 a = xa[ch], b = xb[ch];
                const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                ga = dot8(gv[j], xv, ga);
                ua = dot8(uv[j], xv, ua);
            }
        }
        ga = wave_sum(ga);
        ua = wave_sum(ua);
        if (lane == 0) h[(size_t)s * c.I + i] = ga / (1.0f + expf(-ga)) * ua;
    }
}

// ICH = 16-byte chunks per lane per down row (I <= 512*ICH).
// Rows go out in batches of U consecutive rows: batch j of block b (of G) is
// rows j*G*U + b*U .. + U - 1, so each batch of the chip covers G*U
// consecutive rows (`rows`, a multiple of U, per block).  Block b has nslots
// wavefronts; wavefront s keeps h_s in VGPRs and streams those rows of slot
// s's down matrix, one batch at a time (U*ICH 16-byte loads per lane in
// flight, U*I*2 contiguous bytes), writing w_s * (row . h_s) to LDS.  Each output row is then summed
// over the slots in a fixed order -- routed slots in rank order, then the
// shared slices, then `addend` -- the association of glm_forward.cpp:639-640,
// 658-660 (moeOut += w*y; out = moeOut + sharedOut).
// (one row per batch from 8 chunks on: two rows' weights beside h would take
// more than the 128 registers a 1024-thread block leaves a lane, and spill)
constexpr int down_batch_rows(int ich) { return ich >= 8 ? 1 : 16 / ich; }

template <int ICH>
__global__ __launch_bounds__(1024) void down_t1_kernel(const float* __restrict__ h, LayerDev L,
                                                       Cfg c, const int* __restrict__ sel,
                                                       const float* __restrict__ selw,
                                                       const float* __restrict__ addend,
                                                       float* __restrict__ out, int nslots,
                                                       int rows) {
    constexpr int U = down_batch_rows(ICH);
    __shared__ float part[kMaxSlots][kDownMaxRows];
    const int s = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int G = (int)gridDim.x;
    const int b = (int)blockIdx.x;
    const int nch = c.I >> 3;
    const bool routed = s < c.k;
    const SlotW sw = slot_weights(L, c, s, routed ? sel[s] : 0);

    // The first batch's weight loads go out before h and the slot weight,
    // which they do not depend on.
    u32x4 wv[U][ICH];
    auto load_batch = [&](int i0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = (i0 / U) * G * U + b * U + u;
            if (i0 + u < rows && row < c.d) {
                const u32x4* r4 = reinterpret_cast<const u32x4*>(sw.dn + (size_t)row * sw.ld);
#pragma unroll
                for (int jj = 0; jj < ICH; ++jj) {
                    const int ch = lane + 64 * jj;
                    if (ch < nch) wv[u][jj] = ld_stream(r4 + ch);
                }
            }
        }
    };
    load_batch(0);
    const float ws = routed && selw ? selw[s] : 1.0f;

    float hv[ICH][8];
#pragma unroll
    for (int jj = 0; jj < ICH; ++jj) {
        const int ch = lane + 64 * jj;
        if (ch < nch) {
            const float4* hp = reinterpret_cast<const float4*>(h + (size_t)s * c.I) + 2 * ch;
            const float4 a = hp[0], bb = hp[1];
            hv[jj][0] = a.x; hv[jj][1] = a.y; hv[jj][2] = a.z; hv[jj][3] = a.w;
            hv[jj][4] = bb.x; hv[jj][5] = bb.y; hv[jj][6] = bb.z; hv[jj][7] = bb.w;
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) hv[jj][q] = 0.0f;
        }
    }

    for (int i0 = 0; i0 < rows; i0 += U) {
        if (i0 > 0) load_batch(i0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = (i0 / U) * G * U + b * U + u;
            if (i0 + u < rows && row < c.d) {
                float dot = 0.0f;
#pragma unroll
                for (int jj = 0; jj < ICH; ++jj) {
                    const int ch = lane + 64 * jj;
                    if (ch < nch) dot = dot8(wv[u][jj], hv[jj], dot);
                }
                dot = wave_sum(dot);
                if (lane == 0) part[s][i0 + u] = ws * dot;
            }
        }
    }
    __syncthreads();
    const int nrouted = c.k < nslots ? c.k : nslots;
    for (int t = threadIdx.x; t < rows; t += blockDim.x) {
        const int row = (t / U) * G * U + b * U + t % U;
        if (row >= c.d) continue;
        float moe = 0.0f;
        for (int q = 0; q < nrouted; ++q) moe += part[q][t];
        if (nslots > nrouted) {
            float shared = 0.0f;
            for (int q = nrouted; q < nslots; ++q) shared += part[q][t];
            moe += shared;
        }
        if (addend) moe += addend[row];
        out[row] = moe;
    }
}

template <int KCH>
static hipError_t gateup_inst(const float* x, const LayerDev& L, const Cfg& c,
                              const float2* scores, int* sel, float* selw, float* h, int nslots,
                              int blocks, hipStream_t s) {
    if (scores)
        return launch(gateup_t1_kernel<KCH, true>, dim3(blocks), dim3(256), 0, s, x, L, c, scores,
                      sel, selw, h, nslots);
    return launch(gateup_t1_kernel<KCH, false>, dim3(blocks), dim3(256), 0, s, x, L, c, scores, sel,
                  selw, h, nslots);
}

hipError_t launch_gateup_t1(const float* x, const LayerDev& L, const Cfg& c, const float2* scores,
                            int* sel_idx, float* sel_w, float* h, int nslots, int blocks,
                            hipStream_t s) {
    if (nslots < 1 || blocks < 1) return hipErrorInvalidValue;
    const int kch = (c.d + 511) / 512;
    if (kch <= 1) return gateup_inst<1>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    if (kch <= 2) return gateup_inst<2>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    if (kch <= 4) return gateup_inst<4>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    if (kch <= 8) return gateup_inst<8>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    if (kch <= 12) return gateup_inst<12>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    if (kch <= 16) return gateup_inst<16>(x, L, c, scores, sel_idx, sel_w, h, nslots, blocks, s);
    return hipErrorInvalidValue;
}

template <int ICH>
static hipError_t down_inst(const float* h, const LayerDev& L, const Cfg& c, const int* sel,
                            const float* selw, const float* addend, float* out, int nslots,
                            int blocks, hipStream_t s) {
    // rows per block: a multiple of the batch (the row mapping covers
    // [0, grid * rows) exactly then), at most kDownMaxRows.
    constexpr int U = down_batch_rows(ICH);
    static_assert(kDownMaxRows % U == 0, "batch");
    int grid = blocks < c.d ? blocks : c.d;
    int rows = (c.d + grid - 1) / grid;
    rows = (rows + U - 1) / U * U;
    if (rows > kDownMaxRows) rows = kDownMaxRows;
    grid = (c.d + rows - 1) / rows;
    return launch(down_t1_kernel<ICH>, dim3(grid), dim3(64 * nslots), 0, s, h, L, c, sel, selw,
                  addend, out, nslots, rows);
}

hipError_t launch_down_t1(const float* h, const LayerDev& L, const Cfg& c, const int* sel_idx,
                          const float* sel_w, const float* addend, float* out, int nslots,
                          int blocks, hipStream_t s) {
    if (nslots < 1 || nslots > kMaxSlots || blocks < 1) return hipErrorInvalidValue;
    const int ich = (c.I + 511) / 512;
    if (ich <= 1) return down_inst<1>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 2) return down_inst<2>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 4) return down_inst<4>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 8) return down_inst<8>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    return hipErrorInvalidValue;
}

hipError_t launch_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                             const float* x, float* h, float* out, int d, int I, int gu_blocks,
                             int dn_blocks, hipStream_t s) {
    LayerDev L{};
    L.sg = Wg;
    L.su = Wu;
    L.sd = Wd;
    Cfg c{};
    c.d = d;
    c.I = I;
    c.k = 0;
    c.n_shared = 1;
    hipError_t err = launch_gateup_t1(x, L, c, nullptr, nullptr, nullptr, h, 1, gu_blocks, s);
    if (err != hipSuccess) return err;
    return launch_down_t1(h, L, c, nullptr, nullptr, nullptr, out, 1, dn_blocks, s);
}

}  // namespace hf
