/*
 * oracle.c -- CPU restatement of HummingFlight's MoE-block forward.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against, never part of it.
 * Built by oracle/Makefile with gcc -O2 -ffp-contract=off (no -march): scalar,
 * serial FP32 accumulation with separate multiply and add, which is what the
 * reference's CMake build produces on Linux/GCC (CMakeLists.txt:62-77 adds no
 * -mavx2/-mfma; cpu_kernels.cpp:82-92 is the branch that compiles).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* dtype_bf16.h:19-24 -- zero-extend into the high half. */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* dtype_bf16.h:27-33 -- round to nearest even by adding 0x7FFF + lsb
 * (no NaN special case, as in the reference). */
uint16_t orc_bf16_from_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + bias) >> 16);
}

/* cpu_kernels.cpp:82-92 -- one row per iteration, serial K loop. */
void orc_gemv_bf16_f32(const uint16_t* A, const float* x, float* y,
                       int M, int K, float alpha, float beta) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const uint16_t* row = A + (int64_t)i * K;
        float dot = 0.0f;
        for (int j = 0; j < K; ++j) dot += orc_bf16_to_f32(row[j]) * x[j];
        y[i] = alpha * dot + beta * y[i];
    }
}

/* moe_router.h:19-21 and glm_forward.cpp:522-524: 1/(1+exp(-x)) with the C
 * library's single-precision exp (std::exp(float) is expf). */
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* orc_sigmoid over an array (the GPU tests compare millions of inputs). */
void orc_sigmoid_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_sigmoid(x[i]);
}

/* Strict "a ranks before b": larger value first, then lower index. */
static int ranks_before(float va, int ia, float vb, int ib) {
    if (va > vb) return 1;
    if (va < vb) return 0;
    return ia < ib;
}

/* Select the k best (value, index) pairs of cand[0..n) into out (descending),
 * by repeated scans; n is at most a few hundred. */
static int select_best(const float* val, const int* cand, int n, int k, int* out) {
    if (k > n) k = n;
    char* used = (char*)calloc((size_t)(n > 0 ? n : 1), 1);
    for (int r = 0; r < k; ++r) {
        int best = -1;
        for (int c = 0; c < n; ++c) {
            if (used[c]) continue;
            if (best < 0 || ranks_before(val[cand[c]], cand[c], val[cand[best]], cand[best]))
                best = c;
        }
        used[best] = 1;
        out[r] = cand[best];
    }
    free(used);
    return k;
}

/* moe_router.h:38-56 -- weights from the winners' unbiased scores, summed in
 * rank order, optionally normalised, then scaled. */
static void finish_weights(const float* scores, const int* idx, int k,
                           float scale, int norm, float* w) {
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) {
        w[i] = scores[idx[i]];
        sum += w[i];
    }
    if (norm && sum > 0.0f)
        for (int i = 0; i < k; ++i) w[i] /= sum;
    for (int i = 0; i < k; ++i) w[i] *= scale;
}

/* moe_router.h:29-57. */
int orc_topk_flat(const float* scores, int E, const float* bias, int k,
                  float scale, int norm, int* idx, float* w) {
    if (E <= 0 || k <= 0) return 0;
    if (k > 8) k = 8;
    float* ranked = (float*)malloc(sizeof(float) * (size_t)E);
    int* cand = (int*)malloc(sizeof(int) * (size_t)E);
    for (int i = 0; i < E; ++i) {
        ranked[i] = scores[i] + (bias ? bias[i] : 0.0f);
        cand[i] = i;
    }
    k = select_best(ranked, cand, E, k, idx);
    finish_weights(scores, idx, k, scale, norm, w);
    free(ranked);
    free(cand);
    return k;
}

/* Group-limited selection (DeepSeek-V3 noaux_tc convention; beyond the
 * reference, see oracle.h). */
int orc_topk_grouped(const float* scores, int E, const float* bias, int k,
                     int n_group, int topk_group, float scale, int norm,
                     int* idx, float* w) {
    if (E <= 0 || k <= 0) return 0;
    if (n_group <= 1) return orc_topk_flat(scores, E, bias, k, scale, norm, idx, w);
    if (E % n_group != 0 || topk_group <= 0) return -1;
    if (k > 8) k = 8;
    const int gs = E / n_group;
    if (topk_group > n_group) topk_group = n_group;
    float* ranked = (float*)malloc(sizeof(float) * (size_t)E);
    for (int i = 0; i < E; ++i) ranked[i] = scores[i] + (bias ? bias[i] : 0.0f);

    float* gscore = (float*)malloc(sizeof(float) * (size_t)n_group);
    int* gid = (int*)malloc(sizeof(int) * (size_t)n_group);
    for (int g = 0; g < n_group; ++g) {
        int cand2[2];
        int* members = (int*)malloc(sizeof(int) * (size_t)gs);
        for (int j = 0; j < gs; ++j) members[j] = g * gs + j;
        int n2 = select_best(ranked, members, gs, 2, cand2);
        gscore[g] = (n2 == 2) ? ranked[cand2[0]] + ranked[cand2[1]] : ranked[cand2[0]];
        gid[g] = g;
        free(members);
    }
    int* keep = (int*)malloc(sizeof(int) * (size_t)n_group);
    int nk = select_best(gscore, gid, n_group, topk_group, keep);

    int* cand = (int*)malloc(sizeof(int) * (size_t)E);
    int nc = 0;
    for (int g = 0; g < n_group; ++g) {        /* ascending expert order */
        int kept = 0;
        for (int q = 0; q < nk; ++q) kept |= (keep[q] == g);
        if (!kept) continue;
        for (int j = 0; j < gs; ++j) cand[nc++] = g * gs + j;
    }
    k = select_best(ranked, cand, nc, k, idx);
    finish_weights(scores, idx, k, scale, norm, w);
    free(ranked); free(gscore); free(gid); free(keep); free(cand);
    return k;
}

void orc_dispatch(const int* idx, int T, int k, int E,
                  int* counts, int* offsets, int* perm) {
    const int N = T * k;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int p = 0; p < N; ++p) counts[idx[p]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int* cursor = (int*)malloc(sizeof(int) * (size_t)(E > 0 ? E : 1));
    for (int e = 0; e < E; ++e) cursor[e] = offsets[e];
    for (int p = 0; p < N; ++p) perm[cursor[idx[p]]++] = p;
    free(cursor);
}

/* glm_forward.cpp:434-449 (expertFFNRaw); the SiLU loop is serial there. */
void orc_expert_ffn(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                    const float* x, float* y, int hidden, int inter,
                    float* scratch) {
    float* g = scratch;
    float* u = scratch + inter;
    float* m = scratch + 2 * inter;
    for (int i = 0; i < 3 * inter; ++i) scratch[i] = 0.0f;
    orc_gemv_bf16_f32(Wg, x, g, inter, hidden, 1.0f, 0.0f);
    orc_gemv_bf16_f32(Wu, x, u, inter, hidden, 1.0f, 0.0f);
    for (int i = 0; i < inter; ++i) m[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
    orc_gemv_bf16_f32(Wd, m, y, hidden, inter, 1.0f, 0.0f);
}

/* cuda_backend.cpp:39-49 (and the CUDA-less gpuSoftmax, :577-588). */
void orc_softmax(float* x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; ++i) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

/* cuda_backend.cpp:51-57. */
int orc_argmax(const float* x, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}

/* glm_forward.cpp:185-197. */
void orc_rmsnorm(const uint16_t* w, float* x, int n, float eps) {
    float sq = 0.0f;
    for (int i = 0; i < n; ++i) sq += x[i] * x[i];
    float rms = 1.0f / sqrtf(sq / (float)n + eps);
    if (w) {
        for (int i = 0; i < n; ++i) x[i] = x[i] * rms * orc_bf16_to_f32(w[i]);
    } else {
        for (int i = 0; i < n; ++i) x[i] = x[i] * rms;
    }
}

int orc_route_from_logits(const orc_moe_cfg* cfg, const float* logits,
                          const float* bias, int* idx, float* w) {
    const int E = cfg->n_experts;
    float* s = (float*)malloc(sizeof(float) * (size_t)E);
    for (int i = 0; i < E; ++i) s[i] = 1.0f / (1.0f + expf(-logits[i]));
    int k = orc_topk_grouped(s, E, bias, cfg->top_k, cfg->n_group, cfg->topk_group,
                             cfg->routed_scaling_factor, cfg->norm_topk_prob, idx, w);
    free(s);
    return k;
}

/* glm_forward.cpp:555-556, 581-660: routed experts in rank order into a
 * zeroed FP32 accumulator, then output = moeOut + sharedOut. */
int orc_moe_combine(const orc_moe_cfg* cfg, const orc_moe_weights* W,
                    const float* x, const int* idx, const float* w, int k,
                    float* out) {
    const int H = cfg->hidden, I = cfg->inter;
    const int Is = cfg->n_shared * I;
    const int Imax = Is > I ? Is : I;
    float* moe = (float*)calloc((size_t)H, sizeof(float));
    float* eo = (float*)calloc((size_t)H, sizeof(float));
    float* so = (float*)calloc((size_t)H, sizeof(float));
    float* scratch = (float*)calloc((size_t)(3 * Imax), sizeof(float));
    int rc = 0;
    for (int r = 0; r < k; ++r) {
        const int e = idx[r];
        if (!W->expert_gate[e] || !W->expert_up[e] || !W->expert_down[e]) { rc = -1; break; }
        for (int j = 0; j < H; ++j) eo[j] = 0.0f;
        orc_expert_ffn(W->expert_gate[e], W->expert_up[e], W->expert_down[e], x, eo, H, I, scratch);
        const float wr = w[r];
        for (int j = 0; j < H; ++j) moe[j] += wr * eo[j];
    }
    if (rc == 0) {
        /* sharedExpertFFN (glm_forward.cpp:481-493): absent weights give zeros. */
        if (Is > 0 && W->shared_gate && W->shared_up && W->shared_down)
            orc_expert_ffn(W->shared_gate, W->shared_up, W->shared_down, x, so, H, Is, scratch);
        for (int j = 0; j < H; ++j) out[j] = moe[j] + so[j];
    }
    free(moe); free(eo); free(so); free(scratch);
    return rc;
}

/* ---- CPU-baseline form: the reference's two GEMV builds, optional
 * scheduler copy, timed over `iters` calls ---- */
typedef void (*orc_gemv_fn)(const uint16_t*, const float*, float*, int, int, float, float);

static void gemv_avx2_void(const uint16_t* A, const float* x, float* y, int M, int K, float alpha, float beta) {
    (void)orc_gemv_bf16_f32_avx2(A, x, y, M, K, alpha, beta);
}

/* orc_expert_ffn with the GEMV build as a parameter. */
static void expert_ffn_g(orc_gemv_fn gemv, const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd,
                         const float* x, float* y, int hidden, int inter, float* scratch) {
    float* g = scratch;
    float* u = scratch + inter;
    float* m = scratch + 2 * inter;
    gemv(Wg, x, g, inter, hidden, 1.0f, 0.0f);
    gemv(Wu, x, u, inter, hidden, 1.0f, 0.0f);
    for (int i = 0; i < inter; ++i) m[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
    gemv(Wd, m, y, hidden, inter, 1.0f, 0.0f);
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

double orc_moe_layer_bench(const orc_moe_cfg* cfg, const orc_moe_weights* W, const float* x, float* out,
                           int avx2, void* copy_scratch, int iters) {
    const int E = cfg->n_experts, H = cfg->hidden, I = cfg->inter;
    const int Is = cfg->n_shared * I;
    const int Imax = Is > I ? Is : I;
    const size_t proj = (size_t)I * H;
    orc_gemv_fn gemv = avx2 ? gemv_avx2_void : orc_gemv_bf16_f32;
    float* lg = (float*)calloc((size_t)E, sizeof(float));
    float* moe = (float*)calloc((size_t)H, sizeof(float));
    float* eo = (float*)calloc((size_t)H, sizeof(float));
    float* so = (float*)calloc((size_t)H, sizeof(float));
    float* scratch = (float*)calloc((size_t)(3 * Imax), sizeof(float));
    uint16_t* cp = (uint16_t*)copy_scratch;
    double t0 = now_s(), t = -1.0;
    for (int it = 0; it < iters; ++it) {
        int sel[8];
        float sw[8];
        gemv(W->router, x, lg, E, H, 1.0f, 0.0f);
        const int k = orc_route_from_logits(cfg, lg, W->bias, sel, sw);
        for (int j = 0; j < H; ++j) moe[j] = 0.0f;
        for (int r = 0; r < k; ++r) {
            const int e = sel[r];
            const uint16_t *g = W->expert_gate[e], *u = W->expert_up[e], *d = W->expert_down[e];
            if (!g || !u || !d) goto done;
            if (cp) { /* getExpertPtr: the resident expert copied into exScratch_ */
                memcpy(cp, g, proj * 2);
                memcpy(cp + proj, u, proj * 2);
                memcpy(cp + 2 * proj, d, proj * 2);
                g = cp;
                u = cp + proj;
                d = cp + 2 * proj;
            }
            expert_ffn_g(gemv, g, u, d, x, eo, H, I, scratch);
            for (int j = 0; j < H; ++j) moe[j] += sw[r] * eo[j];
        }
        for (int j = 0; j < H; ++j) so[j] = 0.0f;
        if (Is > 0 && W->shared_gate && W->shared_up && W->shared_down)
            expert_ffn_g(gemv, W->shared_gate, W->shared_up, W->shared_down, x, so, H, Is, scratch);
        for (int j = 0; j < H; ++j) out[j] = moe[j] + so[j];
    }
    t = now_s() - t0;
done:
    free(lg); free(moe); free(eo); free(so); free(scratch);
    return t;
}

/* glm_forward.cpp:509-661 for one token. */
int orc_moe_layer(const orc_moe_cfg* cfg, const orc_moe_weights* W,
                  const float* x, float* out,
                  float* logits, int* idx, float* w) {
    const int E = cfg->n_experts, H = cfg->hidden;
    float* lg = (float*)calloc((size_t)E, sizeof(float));
    orc_gemv_bf16_f32(W->router, x, lg, E, H, 1.0f, 0.0f);
    if (logits) memcpy(logits, lg, sizeof(float) * (size_t)E);
    int sel[8];
    float sw[8];
    int k = orc_route_from_logits(cfg, lg, W->bias, sel, sw);
    free(lg);
    if (k < 0) return -1;
    if (idx) memcpy(idx, sel, sizeof(int) * (size_t)k);
    if (w) memcpy(w, sw, sizeof(float) * (size_t)k);
    return orc_moe_combine(cfg, W, x, sel, sw, k, out);
}

/* ---- seeded counter-based generator ---- */
static uint64_t sm64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint32_t sum16x4(uint64_t v) {
    return (uint32_t)(v & 0xFFFF) + (uint32_t)((v >> 16) & 0xFFFF) +
           (uint32_t)((v >> 32) & 0xFFFF) + (uint32_t)(v >> 48);
}

static float rng_z(uint64_t key, uint64_t i) {
    const uint64_t c = key + 3ull * i;
    const uint32_t s = sum16x4(sm64(c)) + sum16x4(sm64(c + 1)) + sum16x4(sm64(c + 2));
    return (float)((int32_t)s - 393210) * (1.0f / 65536.0f);
}

static uint64_t rng_key(uint64_t seed, uint64_t tensor) { return sm64(seed ^ sm64(tensor)); }

float orc_rng_normal_f32(uint64_t seed, uint64_t tensor, uint64_t i,
                         float mean, float std) {
    float v = rng_z(rng_key(seed, tensor), i) * std;
    return v + mean;
}

void orc_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed,
                          uint64_t tensor, uint64_t first, float mean, float std) {
    const uint64_t key = rng_key(seed, tensor);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (int64_t)n; ++j) {
        float v = rng_z(key, first + (uint64_t)j) * std;
        v = v + mean;
        out[j] = orc_bf16_from_f32(v);
    }
}

void orc_fill_normal_f32(float* out, uint64_t n, uint64_t seed,
                         uint64_t tensor, uint64_t first, float mean, float std) {
    const uint64_t key = rng_key(seed, tensor);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (int64_t)n; ++j) {
        float v = rng_z(key, first + (uint64_t)j) * std;
        out[j] = v + mean;
    }
}
