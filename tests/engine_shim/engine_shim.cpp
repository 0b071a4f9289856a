// engine_shim.cpp -- the engine side of the drop-in, built the way the C++
// engine would build it: include/hfmoe.h, link libhfmoe.so, no other runtime.
//
// A miniature engine with one MoE layer: start-up as --gpu-experts does
// (main.cpp:571-580: a requested but unavailable device is a hard start-up
// error, exit code 2), the layer's tensors in HBM from the library's seeded
// generator (standing in for the WeightIndex handles, weight_index.h:28-67),
// and moeLayer(layer, input, output) with the host float[hidden] contract of
// GLMForward::moeLayer (glm_forward.h:93), restarting on the CPU path when the
// device call fails (glm_forward.cpp:594-602) -- here the restart only reports.
//
//   engine_shim <seed> <tokens>   prints one line per token: the 32-bit
//                                  patterns of output[0..hidden) in hex
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "hfmoe.h"

namespace {

// Tensor ids of the seeded synthetic layer: (layer << 40) | (role << 32) | expert.
enum Role { kRouter = 0, kBias = 1, kSharedGate = 2, kSharedUp = 3, kSharedDown = 4,
            kGate = 5, kUp = 6, kDown = 7, kX = 8 };
uint64_t tensor_id(uint64_t layer, uint64_t role, uint64_t expert) {
    return (layer << 40) | (role << 32) | expert;
}

struct Layer {
    int hidden = 2048, inter = 1024, experts = 64, top_k = 8;
    std::vector<void*> owned;
    void* dev(size_t bytes) {
        void* p = nullptr;
        if (hfmoe_malloc(&p, bytes) != HFMOE_OK) return nullptr;
        owned.push_back(p);
        return p;
    }
    ~Layer() {
        for (void* p : owned) hfmoe_free(p);
    }
};

bool fill_bf16(void* p, size_t n, uint64_t seed, uint64_t tensor, float mean, float std) {
    return p && hfmoe_fill_normal_bf16(static_cast<uint16_t*>(p), n, seed, tensor, 0, mean, std) == HFMOE_OK;
}

// The engine's per-layer call: GPU first, CPU restart on any failure.
bool moe_layer(int layer, const float* input, float* output) {
    if (hfmoe_moe_layer(layer, input, output) == HFMOE_OK) return true;
    std::fprintf(stderr, "MoE layer %d on GPU failed (%s): CPU restart\n", layer, hfmoe_last_error());
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    const uint64_t seed = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
    const int tokens = argc > 2 ? std::atoi(argv[2]) : 1;
    if (hfmoe_init(0) != HFMOE_OK) {
        std::fprintf(stderr, "--gpu-experts: no usable device: %s\n", hfmoe_last_error());
        return 2;
    }
    Layer L;
    const size_t d = L.hidden, I = L.inter, E = L.experts;
    hfmoe_config c{};
    c.hidden = L.hidden;
    c.moe_intermediate = L.inter;
    c.n_routed_experts = L.experts;
    c.num_experts_per_tok = L.top_k;
    c.n_group = 8;
    c.topk_group = 4;
    c.n_shared_experts = 1;
    c.norm_topk_prob = 1;
    c.routed_scaling_factor = 2.5f;
    c.rms_norm_eps = 1e-5f;
    c.max_tokens = 1;
    if (hfmoe_configure(&c) != HFMOE_OK) {
        std::fprintf(stderr, "configure: %s\n", hfmoe_last_error());
        return 1;
    }
    void* router = L.dev(E * d * 2);
    void* bias = L.dev(E * 4);
    void* sg = L.dev(I * d * 2);
    void* su = L.dev(I * d * 2);
    void* sd = L.dev(d * I * 2);
    void* ex = L.dev(E * 3 * I * d * 2);
    bool ok = fill_bf16(router, E * d, seed, tensor_id(0, kRouter, 0), 0.0f, 0.02f) &&
              hfmoe_fill_normal_f32(static_cast<float*>(bias), E, seed, tensor_id(0, kBias, 0), 0, 0.0f,
                                    0.01f) == HFMOE_OK &&
              fill_bf16(sg, I * d, seed, tensor_id(0, kSharedGate, 0), 0.0f, 0.02f) &&
              fill_bf16(su, I * d, seed, tensor_id(0, kSharedUp, 0), 0.0f, 0.02f) &&
              fill_bf16(sd, d * I, seed, tensor_id(0, kSharedDown, 0), 0.0f, 0.02f);
    std::vector<const uint16_t*> table(3 * E);
    for (size_t e = 0; ok && e < E; ++e) {
        uint16_t* base = static_cast<uint16_t*>(ex) + e * 3 * I * d;
        for (int q = 0; q < 3; ++q) {
            table[3 * e + q] = base + q * I * d;
            ok = ok && fill_bf16(base + q * I * d, I * d, seed, tensor_id(0, kGate + q, e), 0.0f, 0.02f);
        }
    }
    if (!ok) {
        std::fprintf(stderr, "weights: %s\n", hfmoe_last_error());
        return 1;
    }
    hfmoe_layer_weights w{};
    w.router_dev = static_cast<const uint16_t*>(router);
    w.score_bias_dev = static_cast<const float*>(bias);
    w.shared_gate_dev = static_cast<const uint16_t*>(sg);
    w.shared_up_dev = static_cast<const uint16_t*>(su);
    w.shared_down_dev = static_cast<const uint16_t*>(sd);
    w.experts = table.data();
    w.experts_location = HFMOE_EXPERTS_DEVICE;
    if (hfmoe_register_layer(0, &w) != HFMOE_OK) {
        std::fprintf(stderr, "register: %s\n", hfmoe_last_error());
        return 1;
    }
    // Activations: BF16-valued N(0, 1) held as float, token t of the seeded x tensor.
    void* xb = L.dev(static_cast<size_t>(tokens) * d * 2);
    if (!fill_bf16(xb, static_cast<size_t>(tokens) * d, seed, tensor_id(0, kX, 0), 0.0f, 1.0f)) return 1;
    std::vector<uint16_t> bits(static_cast<size_t>(tokens) * d);
    if (hfmoe_memcpy_d2h(bits.data(), xb, bits.size() * 2) != HFMOE_OK) return 1;
    std::vector<float> in(d), out(d);
    for (int t = 0; t < tokens; ++t) {
        for (size_t j = 0; j < d; ++j) {
            const uint32_t u = static_cast<uint32_t>(bits[t * d + j]) << 16;
            std::memcpy(&in[j], &u, 4);
        }
        if (!moe_layer(0, in.data(), out.data())) return 3;
        for (size_t j = 0; j < d; ++j) {
            uint32_t u;
            std::memcpy(&u, &out[j], 4);
            std::printf(j ? " %08x" : "%08x", u);
        }
        std::printf("\n");
    }
    hfmoe_shutdown();
    return 0;
}
