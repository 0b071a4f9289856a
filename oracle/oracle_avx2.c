/*
 * oracle_avx2.c -- restatement of the reference's MSVC AVX2+FMA GEMV branch
 * (src/compute/cpu_kernels.cpp:47-81).  TEST INFRASTRUCTURE ONLY.
 *
 * Built with -mavx2 -mfma (oracle/Makefile).  Per row: 8-lane FP32 vector
 * accumulator fed by two FMAs per 16 elements while j + 8 < K8, one FMA per 8
 * after that, horizontal sum as (hi + lo) then two hadds, scalar tail without
 * contraction, then y = alpha*dot + beta*y.  Used as the "ref-avx2" CPU
 * baseline variant; the Linux reference build never reaches this code.
 */
#include "oracle.h"

#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>

static inline __m256 bf16x8(const uint16_t* p) {
    __m128i b = _mm_loadu_si128((const __m128i*)p);
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(b), 16));
}

int orc_gemv_bf16_f32_avx2(const uint16_t* A, const float* x, float* y,
                           int M, int K, float alpha, float beta) {
    const int K8 = K & ~7;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const uint16_t* row = A + (int64_t)i * K;
        __m256 sum = _mm256_setzero_ps();
        int j = 0;
        for (; j + 8 < K8; j += 16) {
            sum = _mm256_fmadd_ps(bf16x8(row + j), _mm256_loadu_ps(x + j), sum);
            sum = _mm256_fmadd_ps(bf16x8(row + j + 8), _mm256_loadu_ps(x + j + 8), sum);
        }
        for (; j < K8; j += 8)
            sum = _mm256_fmadd_ps(bf16x8(row + j), _mm256_loadu_ps(x + j), sum);
        __m128 s = _mm_add_ps(_mm256_extractf128_ps(sum, 1), _mm256_castps256_ps128(sum));
        s = _mm_hadd_ps(s, s);
        s = _mm_hadd_ps(s, s);
        float dot = _mm_cvtss_f32(s);
        for (; j < K; ++j) dot += orc_bf16_to_f32(row[j]) * x[j];
        y[i] = alpha * dot + beta * y[i];
    }
    return 0;
}
#else
int orc_gemv_bf16_f32_avx2(const uint16_t* A, const float* x, float* y,
                           int M, int K, float alpha, float beta) {
    (void)A; (void)x; (void)y; (void)M; (void)K; (void)alpha; (void)beta;
    return -1;
}
#endif
