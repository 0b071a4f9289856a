// ref_harness.cpp -- C entry points over the reference's own compiled sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile (target `ref`) compiles this file
// together with the reference's translation units where they lie under the
// reference checkout into oracle/_ref/libhfref.so.  It is used to pin the C
// restatement in oracle.c (tests/golden/gen_golden.py) and as the "reference"
// CPU baseline.  Nothing here restates reference arithmetic: every compute
// call goes into the reference's code.
//
// GLMForward::moeLayer and GLMForward::rmsNorm are private
// (src/model/glm_forward.h:93,84); they are reached through the standard
// explicit-instantiation access rule (a pointer to member named in an explicit
// template instantiation is not access-checked), with no change to any
// reference header.
#include "compute/cpu_kernels.h"
#include "compute/cuda_backend.h"
#include "compute/dtype_bf16.h"
#include "compute/moe_router.h"
#include "model/glm_forward.h"
#include "model/weight_index.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace {

template <typename Tag, typename Tag::type M>
struct Expose {
    friend typename Tag::type get(Tag) { return M; }
};

struct MoeLayerTag {
    using type = void (glm::GLMForward::*)(int, const float*, float*);
    friend type get(MoeLayerTag);
};
template struct Expose<MoeLayerTag, &glm::GLMForward::moeLayer>;

struct RmsNormTag {
    using type = void (glm::GLMForward::*)(const glm::TensorLocation&, float*, int);
    friend type get(RmsNormTag);
};
template struct Expose<RmsNormTag, &glm::GLMForward::rmsNorm>;

struct DenseMlpTag {
    using type = void (glm::GLMForward::*)(const glm::LayerWeights&, const float*, float*);
    friend type get(DenseMlpTag);
};
template struct Expose<DenseMlpTag, &glm::GLMForward::denseMlp>;

struct LmHeadTag {
    using type = int (glm::GLMForward::*)(const float*, std::vector<float>*);
    friend type get(LmHeadTag);
};
template struct Expose<LmHeadTag, &glm::GLMForward::lmHeadAndSample>;

struct FinalNormTag {
    using type = std::vector<float> glm::GLMForward::*;
    friend type get(FinalNormTag);
};
template struct Expose<FinalNormTag, &glm::GLMForward::finalNorm_>;

bool writeAt(int fd, const void* src, size_t bytes, uint64_t off) {
    const char* p = static_cast<const char*>(src);
    while (bytes > 0) {
        ssize_t n = pwrite(fd, p, bytes, off_t(off));
        if (n <= 0) return false;
        p += n;
        bytes -= size_t(n);
        off += uint64_t(n);
    }
    return true;
}

glm::TensorLocation loc(const std::string& path, uint64_t off, uint64_t bytes,
                        std::vector<int> shape, const char* dtype) {
    glm::TensorLocation t;
    t.shardPath = path;
    t.byteOffset = off;
    t.byteSize = bytes;
    t.shape = std::move(shape);
    t.dtype = dtype;
    return t;
}

}  // namespace

extern "C" {

// Mirrors orc_moe_cfg / orc_moe_weights in oracle.h.
struct ref_moe_cfg {
    int hidden, inter, n_experts, top_k, n_group, topk_group, n_shared, norm_topk_prob;
    float routed_scaling_factor;
};
struct ref_moe_weights {
    const uint16_t* router;
    const float* bias;
    const uint16_t* shared_gate;
    const uint16_t* shared_up;
    const uint16_t* shared_down;
    const uint16_t* const* expert_gate;
    const uint16_t* const* expert_up;
    const uint16_t* const* expert_down;
};

// src/compute/cpu_kernels.cpp:43-94 as compiled for this host.
void ref_gemv_bf16_f32(const uint16_t* A, const float* x, float* y, int M, int K,
                       float alpha, float beta) {
    glm::gemv_bf16_f32(reinterpret_cast<const glm::BFloat16*>(A), x, y, M, K, alpha, beta);
}

// src/compute/moe_router.h:19-21.
float ref_sigmoid(float x) { return glm::sigmoid_f32(x); }

// src/compute/dtype_bf16.h:19-33.
uint16_t ref_bf16_from_f32(float f) { return glm::BFloat16::fromF32(f).bits_; }
float ref_bf16_to_f32(uint16_t b) { return glm::BFloat16(b).toF32(); }

// src/compute/moe_router.h:29-57.  Returns k.
int ref_topk_scores(const float* scores, int E, const float* bias, int k, float scale,
                    int norm, int* idx, float* w) {
    glm::TopKResult r = glm::topKScores(scores, E, bias, k, scale, norm != 0);
    for (int i = 0; i < r.k; ++i) {
        idx[i] = r.indices[i];
        w[i] = r.weights[i];
    }
    return r.k;
}

// GLMForward::moeLayer (src/model/glm_forward.cpp:509-661) on a one-layer
// WeightIndex whose tensors live in a scratch file at `path` (created, mapped
// by the reference's own getShardView, then removed).  Experts whose pointers
// are NULL are left as holes of zeros.  The layer runs `iters` times on the
// same input (iters >= 1); *sec_per_call, when not NULL, receives the mean
// steady_clock time of those calls (moeLayer only: no file or index setup).
// Returns 0 on success.
int ref_moe_layer_timed(const char* path, const ref_moe_cfg* c, const ref_moe_weights* W,
                        const float* x, float* out, int iters, double* sec_per_call) {
    const uint64_t H = uint64_t(c->hidden), I = uint64_t(c->inter), E = uint64_t(c->n_experts);
    const uint64_t Is = uint64_t(c->n_shared) * I;
    const uint64_t routerB = E * H * 2, biasB = W->bias ? E * 4 : 0, shB = Is * H * 2;
    const uint64_t projB = I * H * 2;
    uint64_t off = 0;
    const uint64_t routerOff = off; off += routerB;
    const uint64_t biasOff = off; off += (biasB + 255) & ~uint64_t(255);
    const uint64_t sgOff = off; off += shB;
    const uint64_t suOff = off; off += shB;
    const uint64_t sdOff = off; off += shB;
    const uint64_t expOff = off; off += E * 3 * projB;

    int fd = ::open(path, O_CREAT | O_TRUNC | O_RDWR, 0600);
    if (fd < 0) return -1;
    bool ok = ftruncate(fd, off_t(off)) == 0;
    ok = ok && writeAt(fd, W->router, routerB, routerOff);
    if (W->bias) ok = ok && writeAt(fd, W->bias, biasB, biasOff);
    if (Is > 0) {
        ok = ok && writeAt(fd, W->shared_gate, shB, sgOff) && writeAt(fd, W->shared_up, shB, suOff) &&
             writeAt(fd, W->shared_down, shB, sdOff);
    }
    for (uint64_t e = 0; e < E && ok; ++e) {
        const uint64_t b = expOff + e * 3 * projB;
        if (W->expert_gate[e]) ok = writeAt(fd, W->expert_gate[e], projB, b);
        if (ok && W->expert_up[e]) ok = writeAt(fd, W->expert_up[e], projB, b + projB);
        if (ok && W->expert_down[e]) ok = writeAt(fd, W->expert_down[e], projB, b + 2 * projB);
    }
    ::close(fd);
    if (!ok) {
        ::unlink(path);
        return -2;
    }

    int rc = 0;
    {
        glm::WeightIndex idx;
        auto& cfg = idx.config;
        cfg.hiddenSize = c->hidden;
        cfg.moeIntermediateSize = c->inter;
        cfg.numLocalExperts = c->n_experts;
        cfg.numExpertsPerTok = c->top_k;
        cfg.nSharedExperts = c->n_shared;
        cfg.routedScalingFactor = c->routed_scaling_factor;
        cfg.normTopkProb = c->norm_topk_prob != 0;
        cfg.topkGroup = c->topk_group;
        idx.layers.resize(1);
        auto& lw = idx.layers[0];
        const std::string p(path);
        lw.isMoe = true;
        lw.mlpGate = loc(p, routerOff, routerB, {int(E), int(H)}, "BF16");
        if (W->bias) lw.gateBias = loc(p, biasOff, biasB, {int(E)}, "F32");
        if (Is > 0) {
            lw.sharedGateProj = loc(p, sgOff, shB, {int(Is), int(H)}, "BF16");
            lw.sharedUpProj = loc(p, suOff, shB, {int(Is), int(H)}, "BF16");
            lw.sharedDownProj = loc(p, sdOff, shB, {int(H), int(Is)}, "BF16");
        }
        idx.routedExperts.resize(1);
        idx.routedExperts[0].resize(size_t(E));
        for (uint64_t e = 0; e < E; ++e) {
            const uint64_t b = expOff + e * 3 * projB;
            auto& ew = idx.routedExperts[0][size_t(e)];
            ew.gateProj = loc(p, b, projB, {int(I), int(H)}, "BF16");
            ew.upProj = loc(p, b + projB, projB, {int(I), int(H)}, "BF16");
            ew.downProj = loc(p, b + 2 * projB, projB, {int(H), int(I)}, "BF16");
        }
        if (!idx.getShardView(p)) {
            rc = -3;
        } else {
            glm::GLMForward fwd(idx);
            std::vector<float> o(size_t(H), 0.0f);
            if (iters < 1) iters = 1;
            const auto t0 = std::chrono::steady_clock::now();
            for (int it = 0; it < iters; ++it) (fwd.*get(MoeLayerTag()))(0, x, o.data());
            const auto t1 = std::chrono::steady_clock::now();
            if (sec_per_call) *sec_per_call = std::chrono::duration<double>(t1 - t0).count() / iters;
            std::memcpy(out, o.data(), sizeof(float) * size_t(H));
        }
    }
    ::unlink(path);
    return rc;
}

int ref_moe_layer(const char* path, const ref_moe_cfg* c, const ref_moe_weights* W,
                  const float* x, float* out) {
    return ref_moe_layer_timed(path, c, W, x, out, 1, nullptr);
}

// GLMForward::rmsNorm (src/model/glm_forward.cpp:185-197), weight via a
// scratch file as above.  w may be NULL (byteSize 0: the reference returns
// without touching x).
int ref_rmsnorm(const char* path, const uint16_t* w, float* x, int n, float eps) {
    glm::WeightIndex idx;
    idx.config.rmsNormEps = eps;
    glm::TensorLocation t;
    if (w) {
        int fd = ::open(path, O_CREAT | O_TRUNC | O_RDWR, 0600);
        if (fd < 0) return -1;
        bool ok = writeAt(fd, w, size_t(n) * 2, 0);
        ::close(fd);
        if (!ok) {
            ::unlink(path);
            return -2;
        }
        t = loc(path, 0, uint64_t(n) * 2, {n}, "BF16");
    }
    {
        glm::GLMForward fwd(idx);
        (fwd.*get(RmsNormTag()))(t, x, n);
    }
    if (w) ::unlink(path);
    return 0;
}

// GLMForward::denseMlp (src/model/glm_forward.cpp:410-432): gate, up and down
// [inter, hidden] / [inter, hidden] / [hidden, inter] via a scratch file.
int ref_dense_mlp(const char* path, const uint16_t* gate, const uint16_t* up, const uint16_t* down,
                  int hidden, int inter, const float* x, float* out) {
    const uint64_t B = uint64_t(hidden) * uint64_t(inter) * 2;
    int fd = ::open(path, O_CREAT | O_TRUNC | O_RDWR, 0600);
    if (fd < 0) return -1;
    bool ok = writeAt(fd, gate, B, 0) && writeAt(fd, up, B, B) && writeAt(fd, down, B, 2 * B);
    ::close(fd);
    if (!ok) {
        ::unlink(path);
        return -2;
    }
    int rc = 0;
    {
        glm::WeightIndex idx;
        idx.config.hiddenSize = hidden;
        idx.config.intermediateSize = inter;
        glm::LayerWeights lw;
        const std::string p(path);
        lw.mlpGate = loc(p, 0, B, {inter, hidden}, "BF16");
        lw.mlpUp = loc(p, B, B, {inter, hidden}, "BF16");
        lw.mlpDown = loc(p, 2 * B, B, {hidden, inter}, "BF16");
        if (!idx.getShardView(p)) {
            rc = -3;
        } else {
            glm::GLMForward fwd(idx);
            (fwd.*get(DenseMlpTag()))(lw, x, out);
        }
    }
    ::unlink(path);
    return rc;
}

// GLMForward::lmHeadAndSample (src/model/glm_forward.cpp:663-731): final
// RMSNorm with the norm weight (finalNorm_, filled as init() does from
// model.norm.weight, :135-148), logits over the vocabulary, greedy argmax.
// lm_head [vocab, hidden] via a scratch file; norm NULL means all ones.
int ref_lm_head(const char* path, const uint16_t* lm_head, const uint16_t* norm, int hidden, int vocab,
                float eps, const float* h, float* logits, int* best) {
    const uint64_t B = uint64_t(hidden) * uint64_t(vocab) * 2;
    int fd = ::open(path, O_CREAT | O_TRUNC | O_RDWR, 0600);
    if (fd < 0) return -1;
    bool ok = writeAt(fd, lm_head, B, 0);
    ::close(fd);
    if (!ok) {
        ::unlink(path);
        return -2;
    }
    int rc = 0;
    {
        glm::WeightIndex idx;
        idx.config.hiddenSize = hidden;
        idx.config.vocabSize = vocab;
        idx.config.rmsNormEps = eps;
        const std::string p(path);
        idx.lmHead = loc(p, 0, B, {vocab, hidden}, "BF16");
        if (!idx.getShardView(p)) {
            rc = -3;
        } else {
            glm::GLMForward fwd(idx);
            std::vector<float>& fn = fwd.*get(FinalNormTag());
            fn.assign(size_t(hidden), 1.0f);
            if (norm)
                for (int i = 0; i < hidden; ++i) fn[size_t(i)] = glm::BFloat16(norm[i]).toF32();
            std::vector<float> lg;
            *best = (fwd.*get(LmHeadTag()))(h, &lg);
            std::memcpy(logits, lg.data(), sizeof(float) * size_t(vocab));
        }
    }
    ::unlink(path);
    return rc;
}

// The plugin helpers of src/compute/cuda_backend.h:36-48 as the reference
// builds them without CUDA (cuda_backend.cpp:564-594): embedding row lookup,
// row-major BF16 matvec, in-place softmax, argmax.
void ref_embedding_lookup(const uint16_t* emb, int token, float* out, int hidden) {
    glm::gpuEmbeddingLookup(reinterpret_cast<const glm::BFloat16*>(emb), token, out, hidden);
}
void ref_matvec_bf16(const uint16_t* W, const float* x, float* y, int M, int K) {
    glm::gpuMatvecBf16(reinterpret_cast<const glm::BFloat16*>(W), x, y, M, K);
}
void ref_softmax(float* x, int n) { glm::gpuSoftmax(x, n); }
int ref_argmax(const float* x, int n) { return glm::gpuArgmax(x, n); }

}  // extern "C"
