/*
 * oracle.h -- CPU restatement of HummingFlight's MoE-block forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP path
 * (hummingflight_amd/csrc) is compared against.  Only tests/, the smoke() entry
 * and the cpu_baseline leg of bench.py may load it; the product never links,
 * loads or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Floating-point order follows the reference's Linux/GCC build exactly: scalar
 * serial accumulation, separate multiply and add (this file is compiled with
 * -ffp-contract=off and no -march, as CMakeLists.txt:62-77 builds the
 * reference), glibc expf for std::exp(float).
 *
 * Functions that go beyond the reference (group-limited selection, dispatch,
 * the seeded generator) say so and how each is pinned.
 */
#ifndef HF_ORACLE_H
#define HF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- BF16 (src/compute/dtype_bf16.h:19-33) ---- */
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_bf16_from_f32(float f);

/* ---- GEMV y = alpha*A.x + beta*y, A BF16 [M,K] row-major ----
 * Scalar serial order of the reference's non-MSVC branch
 * (src/compute/cpu_kernels.cpp:82-92). */
void orc_gemv_bf16_f32(const uint16_t* A, const float* x, float* y,
                       int M, int K, float alpha, float beta);

/* Same contract, restating the MSVC AVX2 branch (cpu_kernels.cpp:47-81):
 * 8 lanes, one FMA accumulator, 16 elements per iteration, hadd reduction,
 * scalar tail.  Built only when the compiler targets AVX2+FMA; returns -1
 * (and leaves y untouched) otherwise. */
int orc_gemv_bf16_f32_avx2(const uint16_t* A, const float* x, float* y,
                           int M, int K, float alpha, float beta);

/* ---- sigmoid (src/compute/moe_router.h:19-21, glm_forward.cpp:522-524) ---- */
float orc_sigmoid(float x);
void orc_sigmoid_n(const float* x, float* y, int64_t n);

/* ---- flat noaux_tc top-k (src/compute/moe_router.h:29-57) ----
 * Ranks experts on scores[i]+bias[i] (bias may be NULL), keeps k (<= 8) in
 * descending order.  Exact ties: lower expert index first (the reference's
 * std::partial_sort leaves tie order unspecified).  Weights are the unbiased
 * scores of the winners, divided by their rank-order sum when norm != 0 and the
 * sum is > 0, then multiplied by scale.  Returns k. */
int orc_topk_flat(const float* scores, int E, const float* bias, int k,
                  float scale, int norm, int* idx, float* w);

/* ---- group-limited noaux_tc top-k (beyond the reference, which parses
 * topk_group but never uses it, src/model/config.cpp:117) ----
 * E experts in n_group equal contiguous groups.  Group score = sum of the two
 * largest biased scores in the group (largest + second largest, one float add;
 * a group of one expert scores that expert alone).  Keep the topk_group
 * best groups (ties: lower group index first), then take the k best biased
 * scores among experts of kept groups exactly as orc_topk_flat does.
 * With n_group == 1 this is orc_topk_flat.  Pinned by brute-force enumeration
 * on tiny E and by the n_group == 1 reduction. */
int orc_topk_grouped(const float* scores, int E, const float* bias, int k,
                     int n_group, int topk_group, float scale, int norm,
                     int* idx, float* w);

/* ---- dispatch: stable counting sort of (token, rank) pairs by expert
 * (beyond the reference, which loops token by token,
 * glm_forward.cpp:755, and expert by expert, :581) ----
 * idx: int [T*k] expert per pair, pair p = t*k + r.
 * counts[E], offsets[E+1] (exclusive scan), perm[T*k]: pair ids ordered by
 * (expert, pair id).  Pinned by brute force (sort of (expert, p)). */
void orc_dispatch(const int* idx, int T, int k, int E,
                  int* counts, int* offsets, int* perm);

/* ---- expert SwiGLU (glm_forward.cpp:434-449, shared :459-479) ----
 * g = Wg.x, u = Wu.x (Wg, Wu BF16 [inter, hidden]); h_i = g_i/(1+exp(-g_i))*u_i;
 * y = Wd.h (Wd BF16 [hidden, inter]).  scratch: 3*inter floats. */
void orc_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                    const float* x, float* y, int hidden, int inter,
                    float* scratch);

/* ---- plugin helpers (cuda_backend.h:36-48; the reference's CPU forms,
 * cuda_backend.cpp:27-57 and :564-594) ---- */
/* x <- exp(x - max) * (1 / sum), serial order, libm expf. */
void orc_softmax(float* x, int n);
/* First index of the largest element (strictly greater replaces). */
int orc_argmax(const float* x, int n);

/* ---- RMSNorm (glm_forward.cpp:185-197) in place; w BF16 [n] or NULL ---- */
void orc_rmsnorm(const uint16_t* w, float* x, int n, float eps);

/* ---- one MoE layer for one token (GLMForward::moeLayer,
 * glm_forward.cpp:509-661, direct-weight path :630-635) ---- */
typedef struct orc_moe_cfg {
    int hidden;        /* ModelConfig::hiddenSize */
    int inter;         /* moeIntermediateSize */
    int n_experts;     /* numLocalExperts */
    int top_k;         /* numExpertsPerTok (<= 8) */
    int n_group;       /* 1 = the reference's flat selection */
    int topk_group;
    int n_shared;      /* nSharedExperts; shared inter = n_shared*inter */
    int norm_topk_prob;
    float routed_scaling_factor;
} orc_moe_cfg;

typedef struct orc_moe_weights {
    const uint16_t* router;             /* BF16 [E, hidden] */
    const float* bias;                  /* F32 [E] or NULL */
    const uint16_t* shared_gate;        /* BF16 [n_shared*inter, hidden] or NULL */
    const uint16_t* shared_up;
    const uint16_t* shared_down;        /* BF16 [hidden, n_shared*inter] */
    const uint16_t* const* expert_gate; /* [E] -> BF16 [inter, hidden]; entries of */
    const uint16_t* const* expert_up;   /* unselected experts may be NULL          */
    const uint16_t* const* expert_down; /* [E] -> BF16 [hidden, inter] */
} orc_moe_weights;

/* x f32[hidden] -> out f32[hidden].  Optional outputs (NULL to skip):
 * logits f32[E] (router GEMV before sigmoid), idx int[k], w f32[k].
 * Returns 0, or -1 when a selected expert has no weights. */
int orc_moe_layer(const orc_moe_cfg* cfg, const orc_moe_weights* W,
                  const float* x, float* out,
                  float* logits, int* idx, float* w);

/* Selection only, from given router logits f32[E] (pre-sigmoid): sigmoid,
 * bias, top-k (flat or grouped per cfg).  Returns k. */
int orc_route_from_logits(const orc_moe_cfg* cfg, const float* logits,
                          const float* bias, int* idx, float* w);

/* MoE layer body given a fixed selection (idx/w for one token): routed experts
 * in rank order, weighted FP32 sum, plus the shared expert. */
int orc_moe_combine(const orc_moe_cfg* cfg, const orc_moe_weights* W,
                    const float* x, const int* idx, const float* w, int k,
                    float* out);

/* The CPU baseline: `iters` moeLayer calls for one token, seconds in total
 * (-1 when a selected expert has no weights).  avx2 = 0 runs the reference's
 * Linux GEMV (scalar, serial, cpu_kernels.cpp:82-92), 1 its MSVC AVX2+FMA GEMV
 * restated (:47-81).  copy_scratch (NULL, or >= 3*inter*hidden*2 bytes)
 * receives each selected expert's [gate|up|down] by one memcpy before its
 * FFN, as Scheduler::getExpertPtr copies a resident expert into its scratch
 * (scheduler.cpp:646-660).  Threads: the OpenMP setting of the caller. */
double orc_moe_layer_bench(const orc_moe_cfg* cfg, const orc_moe_weights* W, const float* x, float* out,
                           int avx2, void* copy_scratch, int iters);

/* ---- seeded counter-based generator (beyond the reference) ----
 * Element i of tensor `tensor` under `seed`: three SplitMix64 outputs give
 * twelve 16-bit uniforms; z = (sum - 393210) / 65536 (exact, mean 0, var ~1,
 * Irwin-Hall(12) approximation of N(0,1)); value = z*std (rounded) + mean
 * (rounded); BF16 variants round that float to nearest-even.  Integer-only up
 * to two IEEE float operations, so CPU and GPU produce identical bits. */
float orc_rng_normal_f32(uint64_t seed, uint64_t tensor, uint64_t i,
                         float mean, float std);
void orc_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed,
                          uint64_t tensor, uint64_t first, float mean, float std);
void orc_fill_normal_f32(float* out, uint64_t n, uint64_t seed,
                         uint64_t tensor, uint64_t first, float mean, float std);

#ifdef __cplusplus
}
#endif
#endif
