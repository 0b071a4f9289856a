// expert_gemv.hip -- decode (T = 1) expert SwiGLU as bandwidth-bound BF16 GEMVs.
//
// Reference arithmetic: expertFFNRaw glm_forward.cpp:434-449 (g = Wg.x,
// u = Wu.x, h = g/(1+exp(-g))*u, y = Wd.h), sharedExpertFFNRaw :459-479 and the
// weighted merge :555-556,639-640,658-660 (out = sum_r w_r*y_r + y_shared).
//
// Two launches over all selected experts at once:
//   gate/up: one wavefront per (slot, row i): streams row i of gate and up
//            (2*d BF16, 16-byte coalesced loads), x held in VGPRs as FP32,
//            writes h[slot][i] = silu(g)*u in FP32;
//   down:    h of every slot staged in LDS; one wavefront per output row j
//            streams row j of every slot's down matrix and accumulates
//            w_slot * (row . h_slot) in lane registers, then one reduction.
// No atomics: each output element is produced by one wavefront, so results
// repeat bit for bit from run to run.
#include "hf_common.h"
#include "hf_kernels.h"

namespace hf {

struct SlotW {
    const uint16_t* g;
    const uint16_t* u;
    const uint16_t* dn;
    int ld;      // row stride of the down matrix (I for routed, n_shared*I for shared)
    float w;
};

__device__ __forceinline__ SlotW slot_weights(const LayerDev& L, const Cfg& c,
                                              const int* __restrict__ sel,
                                              const float* __restrict__ selw, int s) {
    SlotW r;
    if (s < c.k) {
        const int e = min(max(sel[s], 0), c.E - 1);  // ids come from the router; stay in the table
        r.g = L.etab[3 * e];
        r.u = L.etab[3 * e + 1];
        r.dn = L.etab[3 * e + 2];
        r.ld = c.I;
        r.w = selw ? selw[s] : 1.0f;
    } else {
        const int sh = s - c.k;
        const size_t off = (size_t)sh * c.I * c.d;
        r.g = L.sg + off;
        r.u = L.su + off;
        r.dn = L.sd + (size_t)sh * c.I;
        r.ld = c.n_shared * c.I;
        r.w = 1.0f;
    }
    return r;
}

// KCH = 16-byte chunks per lane per row (d <= 512*KCH; tail chunks masked).
template <int KCH>
__global__ __launch_bounds__(256) void gateup_t1_kernel(const float* __restrict__ x, LayerDev L,
                                                        Cfg c, const int* __restrict__ sel,
                                                        float* __restrict__ h, int nslots) {
    const int lane = threadIdx.x & 63;
    const int gw = (int)((blockIdx.x * 256u + threadIdx.x) >> 6);
    const int nw = (int)gridDim.x * 4;
    const int nch = c.d >> 3;

    float xr[KCH][8];
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
        const int ch = lane + 64 * j;
        if (ch < nch) {
            const float4 a = reinterpret_cast<const float4*>(x)[2 * ch];
            const float4 b = reinterpret_cast<const float4*>(x)[2 * ch + 1];
            xr[j][0] = a.x; xr[j][1] = a.y; xr[j][2] = a.z; xr[j][3] = a.w;
            xr[j][4] = b.x; xr[j][5] = b.y; xr[j][6] = b.z; xr[j][7] = b.w;
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) xr[j][q] = 0.0f;
        }
    }

    const int total = nslots * c.I;
    for (int q = gw; q < total; q += nw) {
        const int s = q / c.I;
        const int i = q - s * c.I;
        const SlotW sw = slot_weights(L, c, sel, nullptr, s);
        const u32x4* g4 = reinterpret_cast<const u32x4*>(sw.g + (size_t)i * c.d);
        const u32x4* u4 = reinterpret_cast<const u32x4*>(sw.u + (size_t)i * c.d);
        u32x4 gv[KCH], uv[KCH];
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const int ch = lane + 64 * j;
            if (ch < nch) {
                gv[j] = ld_stream(g4 + ch);
                uv[j] = ld_stream(u4 + ch);
            }
        }
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const int ch = lane + 64 * j;
            if (ch < nch) {
                ga = dot8(gv[j], xr[j], ga);
                ua = dot8(uv[j], xr[j], ua);
            }
        }
        ga = wave_sum(ga);
        ua = wave_sum(ua);
        if (lane == 0) h[q] = ga / (1.0f + expf(-ga)) * ua;
    }
}

// ICH = 16-byte chunks per lane per down row (I <= 512*ICH).  Dynamic LDS holds
// h for all slots (nslots*I floats).  Slots are streamed three at a time so
// 3*ICH loads per lane are in flight before the first FMA.
template <int ICH>
__global__ __launch_bounds__(512) void down_t1_kernel(const float* __restrict__ h, LayerDev L,
                                                      Cfg c, const int* __restrict__ sel,
                                                      const float* __restrict__ selw,
                                                      const float* __restrict__ addend,
                                                      float* __restrict__ out, int nslots) {
    extern __shared__ float4 hs4[];
    const float* hs = reinterpret_cast<const float*>(hs4);
    const int n4 = (nslots * c.I) >> 2;
    for (int t = threadIdx.x; t < n4; t += 512) hs4[t] = reinterpret_cast<const float4*>(h)[t];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int gw = (int)((blockIdx.x * 512u + threadIdx.x) >> 6);
    const int nw = (int)gridDim.x * 8;
    const int nch = c.I >> 3;
    constexpr int SG = 3;

    for (int j = gw; j < c.d; j += nw) {
        float acc = 0.0f;
        for (int s0 = 0; s0 < nslots; s0 += SG) {
            u32x4 wv[SG][ICH];
            float wt[SG];
#pragma unroll
            for (int ss = 0; ss < SG; ++ss) {
                const int s = s0 + ss;
                wt[ss] = 0.0f;
                if (s < nslots) {
                    const SlotW sw = slot_weights(L, c, sel, selw, s);
                    wt[ss] = sw.w;
                    const u32x4* r4 = reinterpret_cast<const u32x4*>(sw.dn + (size_t)j * sw.ld);
#pragma unroll
                    for (int jj = 0; jj < ICH; ++jj) {
                        const int ch = lane + 64 * jj;
                        if (ch < nch) wv[ss][jj] = ld_stream(r4 + ch);
                    }
                }
            }
#pragma unroll
            for (int ss = 0; ss < SG; ++ss) {
                const int s = s0 + ss;
                if (s < nslots) {
                    float part = 0.0f;
#pragma unroll
                    for (int jj = 0; jj < ICH; ++jj) {
                        const int ch = lane + 64 * jj;
                        if (ch < nch) {
                            const float4* hp = reinterpret_cast<const float4*>(hs + (size_t)s * c.I) + 2 * ch;
                            const float4 a = hp[0], b = hp[1];
                            const float hv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                            part = dot8(wv[ss][jj], hv, part);
                        }
                    }
                    acc = fmaf(wt[ss], part, acc);
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) out[j] = addend ? acc + addend[j] : acc;
    }
}

template <int KCH>
static hipError_t gateup_inst(const float* x, const LayerDev& L, const Cfg& c, const int* sel,
                              float* h, int nslots, int blocks, hipStream_t s) {
    hipLaunchKernelGGL(gateup_t1_kernel<KCH>, dim3(blocks), dim3(256), 0, s, x, L, c, sel, h,
                       nslots);
    return hipGetLastError();
}

hipError_t launch_gateup_t1(const float* x, const LayerDev& L, const Cfg& c, const int* sel_idx,
                            float* h, int nslots, int blocks, hipStream_t s) {
    const int kch = (c.d + 511) / 512;
    if (kch <= 1) return gateup_inst<1>(x, L, c, sel_idx, h, nslots, blocks, s);
    if (kch <= 2) return gateup_inst<2>(x, L, c, sel_idx, h, nslots, blocks, s);
    if (kch <= 4) return gateup_inst<4>(x, L, c, sel_idx, h, nslots, blocks, s);
    if (kch <= 8) return gateup_inst<8>(x, L, c, sel_idx, h, nslots, blocks, s);
    if (kch <= 12) return gateup_inst<12>(x, L, c, sel_idx, h, nslots, blocks, s);
    if (kch <= 16) return gateup_inst<16>(x, L, c, sel_idx, h, nslots, blocks, s);
    return hipErrorInvalidValue;
}

template <int ICH>
static hipError_t down_inst(const float* h, const LayerDev& L, const Cfg& c, const int* sel,
                            const float* selw, const float* addend, float* out, int nslots,
                            int blocks, hipStream_t s) {
    const size_t lds = sizeof(float) * (size_t)nslots * c.I;
    static int lds_limit = 0;  // per instantiation: raise the dynamic LDS cap once
    if ((int)lds > lds_limit) {
        hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(down_t1_kernel<ICH>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             160 * 1024);
        if (err != hipSuccess) return err;
        lds_limit = 160 * 1024;
    }
    hipLaunchKernelGGL(down_t1_kernel<ICH>, dim3(blocks), dim3(512), lds, s, h, L, c, sel, selw,
                       addend, out, nslots);
    return hipGetLastError();
}

hipError_t launch_down_t1(const float* h, const LayerDev& L, const Cfg& c, const int* sel_idx,
                          const float* sel_w, const float* addend, float* out, int nslots,
                          int blocks, hipStream_t s) {
    const int ich = (c.I + 511) / 512;
    if (ich <= 1) return down_inst<1>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 2) return down_inst<2>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 4) return down_inst<4>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    if (ich <= 8) return down_inst<8>(h, L, c, sel_idx, sel_w, addend, out, nslots, blocks, s);
    return hipErrorInvalidValue;
}

hipError_t launch_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                             const float* x, float* h, float* out, int d, int I, int blocks,
                             hipStream_t s) {
    LayerDev L{};
    L.sg = Wg;
    L.su = Wu;
    L.sd = Wd;
    Cfg c{};
    c.d = d;
    c.I = I;
    c.k = 0;
    c.n_shared = 1;
    hipError_t err = launch_gateup_t1(x, L, c, nullptr, h, 1, blocks, s);
    if (err != hipSuccess) return err;
    return launch_down_t1(h, L, c, nullptr, nullptr, nullptr, out, 1, blocks, s);
}

}  // namespace hf
