// misc.hip -- RMSNorm and residual add around the MoE block
// (glm_forward.cpp:185-197 and :785-796).
#include "hf_api_internal.h"

namespace hf {

// One block of 1024 threads per token: r = 1/sqrt(sum(x^2)/n + eps);
// out = x*r*w (w BF16 or 1).  Each thread loads its (at most two) float4
// chunks once and keeps them in registers for the second pass, so a token
// costs one round trip to memory, not two.
constexpr int kNormThreads = 1024;
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ h,
                                                               const uint16_t* __restrict__ w,
                                                               float* __restrict__ out, int d, float eps) {
    __shared__ float red[kNormThreads / 64];
    const float* x = h + (size_t)blockIdx.x * d;
    float* y = out + (size_t)blockIdx.x * d;
    const bool vec = (d & 3) == 0;
    float4 v[2];
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = 4 * (threadIdx.x + j * kNormThreads);
        v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (vec && i < d) v[j] = *reinterpret_cast<const float4*>(x + i);
        sq = fmaf(v[j].x, v[j].x, sq);
        sq = fmaf(v[j].y, v[j].y, sq);
        sq = fmaf(v[j].z, v[j].z, sq);
        sq = fmaf(v[j].w, v[j].w, sq);
    }
    if (!vec)
        for (int i = threadIdx.x; i < d; i += kNormThreads) sq = fmaf(x[i], x[i], sq);
    sq = wave_sum(sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
    const float r = 1.0f / sqrtf(tot / (float)d + eps);
    auto wt = [&](int i) { return w ? __uint_as_float((uint32_t)w[i] << 16) : 1.0f; };
    if (vec) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = 4 * (threadIdx.x + j * kNormThreads);
            if (i < d)
                *reinterpret_cast<float4*>(y + i) =
                    make_float4(v[j].x * r * wt(i), v[j].y * r * wt(i + 1), v[j].z * r * wt(i + 2), v[j].w * r * wt(i + 3));
        }
    } else {
        for (int i = threadIdx.x; i < d; i += kNormThreads) y[i] = x[i] * r * wt(i);
    }
}

__global__ void add_inplace_kernel(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] += src[i];
}

// n floats from src to dst, either of which may be mapped host memory: a
// small transfer done by the compute queue, without a DMA-engine round trip.
__global__ void copy_f32_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

hipError_t launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 64) blocks = 64;
    return launch(copy_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
}

// BF16 bits -> FP32 (exact: a BF16 value is the top half of its FP32), eight
// values per thread and step (a 16-byte load, two 16-byte stores) when both
// buffers are 16-byte aligned, then single values for the rest.
__global__ void bf16_to_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst, size_t n) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    const size_t n8 = vec ? n / 8 : 0;
    for (size_t i = tid; i < n8; i += stride) {
        const uint4 v = reinterpret_cast<const uint4*>(src)[i];
        float4* o = reinterpret_cast<float4*>(dst) + 2 * i;
        o[0] = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                           __uint_as_float(v.y & 0xFFFF0000u));
        o[1] = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u), __uint_as_float(v.w << 16),
                           __uint_as_float(v.w & 0xFFFF0000u));
    }
    for (size_t i = n8 * 8 + tid; i < n; i += stride) dst[i] = __uint_as_float((uint32_t)src[i] << 16);
}

hipError_t launch_bf16_to_f32(const uint16_t* src, float* dst, size_t n, hipStream_t s) {
    size_t blocks = (n / 8 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    return launch(bf16_to_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
}

__global__ void copy_u32_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

hipError_t launch_copy_u32(const uint32_t* src, uint32_t* dst, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 64) blocks = 64;
    return launch(copy_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
}

__global__ void copy_u64_kernel(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

hipError_t launch_copy_u64(const uint64_t* src, uint64_t* dst, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 64) blocks = 64;
    return launch(copy_u64_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
}

hipError_t launch_rmsnorm(const float* h, const uint16_t* w, float* out, int T, int d, float eps,
                          hipStream_t s) {
    if (d > 8 * kNormThreads) return hipErrorInvalidValue;
    return launch(rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, s, h, w, out, d, eps);
}

hipError_t launch_add_inplace(float* dst, const float* src, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    return launch(add_inplace_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, src, n);
}

}  // namespace hf
