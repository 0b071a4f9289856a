// helpers.hip -- the GPU plugin's small dense helpers (cuda_backend.h:36-48):
// embedding row lookup, row-major BF16 matvec, softmax and argmax.
//
// The host-pointer entry points keep the reference's contract (host buffers
// in and out, synchronous; gpuEmbeddingLookup / gpuMatvecBf16 / gpuSoftmax /
// gpuArgmax, cuda_backend.cpp:104-164) and differ only in copying what the
// call needs (the reference uploads the first token_id + 1 embedding rows).
// The device-pointer forms replace the reference's CUDA helpers
// (glm_cuda::embeddingGather / matvec / softmax / argmax, cuda_kernels.h:8-11),
// with T-row generalisations of the embedding, softmax and argmax, and a
// stream argument.
//
// Arithmetic of the reference's CPU forms (cuda_backend.cpp:27-57): the
// embedding widens BF16 to FP32 exactly; softmax is exp(x - max) scaled by one
// reciprocal of the sum; argmax keeps the first largest element.
#include "hf_api_internal.h"
#include "hf_expf.h"

#include <climits>

namespace hf {

// out[t, i] = emb[ids[t], i] as FP32; rows of ids outside [0, vocab) are
// zeros.  ids == nullptr: the single row `id0` (already checked by the host).
__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t* __restrict__ emb, int vocab, int hidden,
                                                        const int* __restrict__ ids, int id0,
                                                        float* __restrict__ out) {
    const int t = blockIdx.y;
    const int id = ids ? ids[t] : id0;
    const bool ok = id >= 0 && id < vocab;
    const uint16_t* row = emb + (size_t)(ok ? id : 0) * hidden;
    float* o = out + (size_t)t * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        o[i] = ok ? __uint_as_float((uint32_t)row[i] << 16) : 0.0f;
}

// y[i] = sigmoid_f32(x[i]) (moe_router.h:19-21), the router's scoring function.
__global__ __launch_bounds__(256) void router_sigmoid_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = router_sigmoid(x[i]);
}

constexpr int kSoftmaxThreads = 1024;

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kSoftmaxThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

// One block per row, in place: x = exp(x - max(x)) * (1 / sum).
__global__ __launch_bounds__(kSoftmaxThreads) void softmax_rows_kernel(float* __restrict__ x, int n) {
    __shared__ float red[kSoftmaxThreads / 64];
    float* row = x + (size_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) mx = fmaxf(mx, row[i]);
    mx = block_reduce(mx, red, true);
    float sum = 0.0f;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) {
        const float e = expf(row[i] - mx);
        row[i] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    const float inv = 1.0f / sum;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) row[i] *= inv;
}

// y[r] = sum_k W[r, k] * x[k] for any K: one wavefront per row.
__global__ __launch_bounds__(256) void matvec_any_kernel(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                                         int M, int K, float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= M) return;
    const uint16_t* row = W + (size_t)r * K;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc = fmaf(__uint_as_float((uint32_t)row[k] << 16), x[k], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

static hipError_t launch_embedding(const uint16_t* emb, int vocab, int hidden, const int* ids, int id0, int T,
                                   float* out, hipStream_t s) {
    return launch(embedding_kernel, dim3(std::min((hidden + 255) / 256, 16), T), dim3(256), 0, s, emb, vocab,
                  hidden, ids, id0, out);
}

// The LDS-staged GEMV when its shape rules hold (K a multiple of 8 up to
// 8192, 16-byte aligned rows), else one wavefront per row.
static hipError_t launch_matvec(const uint16_t* W, const float* x, int M, int K, float* y, hipStream_t s) {
    if (K % 8 == 0 && K <= 8192 && (reinterpret_cast<uintptr_t>(W) & 15) == 0)
        return launch_matvec_bf16(W, x, M, K, y, s);
    return launch(matvec_any_kernel, dim3((M + 3) / 4), dim3(256), 0, s, W, x, M, K, y);
}

// Device scratch for the host-contract helpers, freed on return.
struct Scratch {
    void* p = nullptr;
    ~Scratch() {
        if (p) hipFree(p);
    }
};

}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_embedding(const uint16_t* emb_dev, int32_t vocab, int32_t hidden, const int32_t* ids_dev, int32_t T,
                    float* out_dev, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!emb_dev || !ids_dev || !out_dev || vocab <= 0 || hidden <= 0 || T < 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "embedding: null buffer or non-positive size");
    if (T == 0) return HFMOE_OK;
    hipError_t e = launch_embedding(emb_dev, vocab, hidden, static_cast<const int*>(ids_dev), 0, T, out_dev,
                                    pick_stream(stream));
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "embedding launch");
}

int hfmoe_embedding_gather(const uint16_t* emb_dev, int token_id, float* out_dev, int hidden, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!emb_dev || !out_dev || hidden <= 0 || token_id < 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "embedding gather: null buffer, hidden <= 0 or token < 0");
    hipError_t e = launch_embedding(emb_dev, INT_MAX, hidden, nullptr, token_id, 1, out_dev, pick_stream(stream));
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "embedding gather launch");
}

int hfmoe_matvec_bf16_dev(const uint16_t* w_dev, const float* x_dev, float* y_dev, int M, int K, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!w_dev || !x_dev || !y_dev || M <= 0 || K <= 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "matvec: null buffer or non-positive size");
    hipError_t e = launch_matvec(w_dev, x_dev, M, K, y_dev, pick_stream(stream));
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "matvec launch");
}

int hfmoe_softmax_rows(float* x_dev, int32_t T, int32_t n, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x_dev || n <= 0 || T < 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "softmax: null buffer or n <= 0");
    if (T == 0) return HFMOE_OK;
    hipError_t e = launch(softmax_rows_kernel, dim3(T), dim3(kSoftmaxThreads), 0, pick_stream(stream), x_dev, n);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "softmax launch");
}

int hfmoe_router_sigmoid(const float* x_dev, float* y_dev, int64_t n, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (n < 0 || (n > 0 && (!x_dev || !y_dev)))
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "router sigmoid: null buffer or n < 0");
    if (n == 0) return HFMOE_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    hipError_t e = launch(router_sigmoid_kernel, dim3((unsigned)blocks), dim3(256), 0, pick_stream(stream), x_dev,
                          y_dev, n);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "router sigmoid launch");
}

int hfmoe_argmax_rows(const float* x_dev, int32_t T, int32_t n, int32_t* best_dev, void* stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x_dev || !best_dev || n <= 0 || T < 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "argmax: null buffer or n <= 0");
    if (T == 0) return HFMOE_OK;
    hipError_t e = launch_row_argmax(x_dev, T, n, reinterpret_cast<int*>(best_dev), pick_stream(stream));
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "argmax launch");
}

int hfmoe_embedding_lookup(const uint16_t* emb_host, int token_id, float* out_host, int hidden) {
    int rc = require_init();
    if (rc) return rc;
    if (!emb_host || !out_host || hidden <= 0 || token_id < 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "embedding lookup: null buffer, hidden <= 0 or token < 0");
    Scratch row, out;
    hipError_t e = hipMalloc(&row.p, 2 * (size_t)hidden);
    if (e == hipSuccess) e = hipMalloc(&out.p, 4 * (size_t)hidden);
    if (e == hipSuccess) e = hipMemcpy(row.p, emb_host + (size_t)token_id * hidden, 2 * (size_t)hidden, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_embedding(static_cast<const uint16_t*>(row.p), 1, hidden, nullptr, 0, 1, static_cast<float*>(out.p),
                             g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(out_host, out.p, 4 * (size_t)hidden, hipMemcpyDeviceToHost);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "embedding lookup");
}

int hfmoe_matvec_bf16(const uint16_t* w_host, const float* x_host, float* y_host, int M, int K) {
    int rc = require_init();
    if (rc) return rc;
    if (!w_host || !x_host || !y_host || M <= 0 || K <= 0)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "matvec: null buffer or non-positive size");
    Scratch w, x, y;
    hipError_t e = hipMalloc(&w.p, 2 * (size_t)M * K);
    if (e == hipSuccess) e = hipMalloc(&x.p, 4 * (size_t)K);
    if (e == hipSuccess) e = hipMalloc(&y.p, 4 * (size_t)M);
    if (e == hipSuccess) e = hipMemcpy(w.p, w_host, 2 * (size_t)M * K, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(x.p, x_host, 4 * (size_t)K, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_matvec(static_cast<const uint16_t*>(w.p), static_cast<const float*>(x.p), M, K,
                          static_cast<float*>(y.p), g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(y_host, y.p, 4 * (size_t)M, hipMemcpyDeviceToHost);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "matvec");
}

int hfmoe_softmax(float* x_host, int n) {
    int rc = require_init();
    if (rc) return rc;
    if (!x_host || n <= 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "softmax: null buffer or n <= 0");
    Scratch x;
    hipError_t e = hipMalloc(&x.p, 4 * (size_t)n);
    if (e == hipSuccess) e = hipMemcpy(x.p, x_host, 4 * (size_t)n, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch(softmax_rows_kernel, dim3(1), dim3(kSoftmaxThreads), 0, g.stream, static_cast<float*>(x.p), n);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(x_host, x.p, 4 * (size_t)n, hipMemcpyDeviceToHost);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "softmax");
}

int hfmoe_argmax(const float* x_host, int n, int32_t* best) {
    int rc = require_init();
    if (rc) return rc;
    if (!x_host || !best || n <= 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "argmax: null buffer or n <= 0");
    Scratch x, o;
    hipError_t e = hipMalloc(&x.p, 4 * (size_t)n);
    if (e == hipSuccess) e = hipMalloc(&o.p, sizeof(int));
    if (e == hipSuccess) e = hipMemcpy(x.p, x_host, 4 * (size_t)n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_row_argmax(static_cast<const float*>(x.p), 1, n, static_cast<int*>(o.p), g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e == hipSuccess) e = hipMemcpy(best, o.p, sizeof(int), hipMemcpyDeviceToHost);
    return e == hipSuccess ? HFMOE_OK : fail_hip(e, "argmax");
}

}  // extern "C"
