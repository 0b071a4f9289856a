// rng.hip -- seeded, counter-based synthetic tensors generated in HBM.
//
// Element i of tensor `tensor` under `seed`: key = SplitMix64(seed ^
// SplitMix64(tensor)); three SplitMix64 outputs of key + 3i, +1, +2 give twelve
// 16-bit uniforms; z = (sum - 393210) / 65536 (integer arithmetic, then an exact
// conversion and power-of-two scaling: mean 0, variance ~1, an Irwin-Hall(12)
// approximation of N(0,1)); value = (z*std) + mean with two IEEE roundings and
// no contraction.  Any host that evaluates the same integer steps gets the same
// bits, so the CPU oracle can regenerate any expert independently of the GPU.
#include "hf_common.h"
#include "hf_kernels.h"

// Exact IEEE steps: no multiply-add contraction in this file.
#pragma clang fp contract(off)

namespace hf {

__device__ __forceinline__ uint64_t sm64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint32_t sum16x4(uint64_t v) {
    return (uint32_t)(v & 0xFFFF) + (uint32_t)((v >> 16) & 0xFFFF) +
           (uint32_t)((v >> 32) & 0xFFFF) + (uint32_t)(v >> 48);
}

__device__ __forceinline__ float rng_value(uint64_t key, uint64_t i, float mean, float stdev) {
    const uint64_t c = key + 3ull * i;
    const uint32_t s = sum16x4(sm64(c)) + sum16x4(sm64(c + 1)) + sum16x4(sm64(c + 2));
    // Plain operators: this file is compiled with contraction off, so these are
    // two separately rounded IEEE operations (z is exact).
    const float z = (float)((int32_t)s - 393210) * (1.0f / 65536.0f);
    const float scaled = z * stdev;
    return scaled + mean;
}

static uint64_t host_sm64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_bf16_kernel(uint16_t* __restrict__ out, uint64_t n, uint64_t key,
                                 uint64_t first, float mean, float stdev) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride)
        out[j] = f32_to_bf16(rng_value(key, first + j, mean, stdev));
}

__global__ void fill_f32_kernel(float* __restrict__ out, uint64_t n, uint64_t key, uint64_t first,
                                float mean, float stdev) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride)
        out[j] = rng_value(key, first + j, mean, stdev);
}

static unsigned fill_blocks(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

hipError_t launch_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                   uint64_t first, float mean, float stdev, hipStream_t s) {
    const uint64_t key = host_sm64(seed ^ host_sm64(tensor));
    return launch(fill_bf16_kernel, dim3(fill_blocks(n)), dim3(256), 0, s, out, n, key,
                       first, mean, stdev);
}

hipError_t launch_fill_normal_f32(float* out, uint64_t n, uint64_t seed, uint64_t tensor,
                                  uint64_t first, float mean, float stdev, hipStream_t s) {
    const uint64_t key = host_sm64(seed ^ host_sm64(tensor));
    return launch(fill_f32_kernel, dim3(fill_blocks(n)), dim3(256), 0, s, out, n, key, first,
                       mean, stdev);
}

}  // namespace hf
