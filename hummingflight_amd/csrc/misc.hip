// misc.hip -- RMSNorm and residual add around the MoE block
// (glm_forward.cpp:185-197 and :785-796).
#include "hf_api_internal.h"

namespace hf {

// One block per token: r = 1/sqrt(sum(x^2)/n + eps); out = x*r*w (w BF16 or 1).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ h,
                                                      const uint16_t* __restrict__ w,
                                                      float* __restrict__ out, int d, float eps) {
    __shared__ float red[4];
    const float* x = h + (size_t)blockIdx.x * d;
    float* y = out + (size_t)blockIdx.x * d;
    float sq = 0.0f;
    for (int i = threadIdx.x; i < d; i += 256) sq = fmaf(x[i], x[i], sq);
    sq = wave_sum(sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = 1.0f / sqrtf(tot / (float)d + eps);
    for (int i = threadIdx.x; i < d; i += 256) {
        const float v = x[i] * r;
        y[i] = w ? v * __uint_as_float((uint32_t)w[i] << 16) : v;
    }
}

__global__ void add_inplace_kernel(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] += src[i];
}

hipError_t launch_rmsnorm(const float* h, const uint16_t* w, float* out, int T, int d, float eps,
                          hipStream_t s) {
    return launch(rmsnorm_kernel, dim3(T), dim3(256), 0, s, h, w, out, d, eps);
}

hipError_t launch_add_inplace(float* dst, const float* src, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    return launch(add_inplace_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, src, n);
}

}  // namespace hf
