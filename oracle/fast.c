/* CPU baseline for the decode hot path: int4 MatMulNBits on the host cores.
 *
 * TEST INFRASTRUCTURE ONLY. bench.py times this as the CPU baseline of the GEMV and
 * of the decoder's decode steps; tests/test_oracle.py pins it against the fp64
 * restatement orc_mnb_matmul. The shipped libraries never load it.
 *
 * The oracle proper (oracle.c) accumulates in fp64 with no vectorisation, which
 * makes a poor stand-in for what a CPU runs. This is the same product written
 * the way a CPU kernel would: fp32 accumulation, AVX2/FMA, one weight row per
 * OpenMP iteration (each block unpacked once for up to 8 activation rows), the
 * zero point folded per block,
 *   y[n] = sum_b s[n,b] * (sum_{k in b} a_k q_{n,k} - z_{n,b} * sum_{k in b} a_k),
 * which is quant.rs:570-601's dequantise-then-matmul regrouped by block (the
 * codes, zero points and block indexing are those of orc_mnb_matmul).
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* The 32 codes of one chunk (16 bytes, low nibble = even k) as floats: even
 * positions in q[0], q[1], odd positions in q[2], q[3]. */
__attribute__((target("avx2,fma"))) static inline void unpack_chunk(const uint8_t* w,
                                                                    __m256 q[4]) {
    const __m128i bytes = _mm_loadu_si128((const __m128i*)w);
    const __m128i mask = _mm_set1_epi8(0x0f);
    const __m128i lo = _mm_and_si128(bytes, mask);
    const __m128i hi = _mm_and_si128(_mm_srli_epi16(bytes, 4), mask);
    q[0] = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo));
    q[1] = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(lo, 8)));
    q[2] = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi));
    q[3] = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(hi, 8)));
}

/* acc += the chunk's codes times its activations split into even (ae) and odd (ao)
 * positions. */
__attribute__((target("avx2,fma"))) static inline __m256 chunk_fma(const __m256 q[4],
                                                                   const float* ae,
                                                                   const float* ao, __m256 acc) {
    acc = _mm256_fmadd_ps(q[0], _mm256_loadu_ps(ae), acc);
    acc = _mm256_fmadd_ps(q[1], _mm256_loadu_ps(ae + 8), acc);
    acc = _mm256_fmadd_ps(q[2], _mm256_loadu_ps(ao), acc);
    acc = _mm256_fmadd_ps(q[3], _mm256_loadu_ps(ao + 8), acc);
    return acc;
}

__attribute__((target("avx2,fma"))) static inline float hsum(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* Rows [n0, n1) of Y for CPB chunks of 32 codes per block (block = 32 CPB). */
#define DEFINE_GEMV_ROWS(CPB)                                                                  \
    __attribute__((target("avx2,fma,f16c"))) static void gemv_rows_##CPB(                      \
        const float* ae, const float* ao, const float* bsum, int64_t M, const uint8_t* B,      \
        const void* scales, int scale_f16, const uint8_t* zp, int64_t N, int64_t K,            \
        float* y) {                                                                            \
        const int64_t nb = K / (32 * CPB), row_bytes = K / 2, zp_cols = (nb + 1) / 2;          \
        const int64_t C = K / 32;                                                              \
        enum { kMT = 8 };                                                                      \
        _Pragma("omp for schedule(static)") for (int64_t n = 0; n < N; ++n) {                 \
            const uint8_t* row = B + n * row_bytes;                                            \
            for (int64_t m0 = 0; m0 < M; m0 += kMT) {                                          \
                const int64_t mt = M - m0 < kMT ? M - m0 : kMT;                                \
                __m256 tot[kMT];                                                               \
                float zterm[kMT];                                                              \
                for (int64_t i = 0; i < mt; ++i) {                                             \
                    tot[i] = _mm256_setzero_ps();                                              \
                    zterm[i] = 0.f;                                                            \
                }                                                                              \
                for (int64_t b = 0; b < nb; ++b) {                                             \
                    const float s = scale_f16                                                  \
                                        ? _cvtsh_ss(((const uint16_t*)scales)[n * nb + b])     \
                                        : ((const float*)scales)[n * nb + b];                  \
                    int z = 8;                                                                 \
                    if (zp) {                                                                  \
                        const uint8_t zb = zp[n * zp_cols + b / 2];                            \
                        z = (b & 1) ? zb >> 4 : zb & 15;                                       \
                    }                                                                          \
                    __m256 q[CPB][4];                                                          \
                    for (int j = 0; j < CPB; ++j) unpack_chunk(row + 16 * (b * CPB + j), q[j]); \
                    const __m256 sv = _mm256_set1_ps(s);                                       \
                    for (int64_t i = 0; i < mt; ++i) {                                         \
                        const int64_t m = m0 + i;                                              \
                        __m256 acc = _mm256_setzero_ps();                                      \
                        for (int j = 0; j < CPB; ++j) {                                        \
                            const int64_t c = b * CPB + j;                                     \
                            acc = chunk_fma(q[j], ae + (m * C + c) * 16, ao + (m * C + c) * 16, \
                                            acc);                                              \
                        }                                                                      \
                        tot[i] = _mm256_fmadd_ps(sv, acc, tot[i]);                             \
                        zterm[i] += s * (float)z * bsum[m * nb + b];                           \
                    }                                                                          \
                }                                                                              \
                for (int64_t i = 0; i < mt; ++i) y[(m0 + i) * N + n] = hsum(tot[i]) - zterm[i]; \
            }                                                                                  \
        }                                                                                      \
    }
DEFINE_GEMV_ROWS(1)
DEFINE_GEMV_ROWS(2)
DEFINE_GEMV_ROWS(3)
DEFINE_GEMV_ROWS(4)

/* Y[M, N] = A[M, K] x W^T for 4-bit W [N, K/32, 16] (ORT's MatMulNBits layout),
 * block sizes 32, 64, 96 or 128, K a multiple of the block. scales fp32 or
 * fp16 bits (scale_f16 = 1), zp packed nibbles or NULL (8). Returns -1 when the
 * form or the CPU (no AVX2/FMA) is outside what this path covers. */
int orc_mnb_matmul_fast(const float* A, int64_t M, const uint8_t* B, const void* scales,
                        int scale_f16, const uint8_t* zp, int64_t N, int64_t K, int block,
                        float* Y, int nthreads) {
    if (block < 32 || block > 128 || block % 32 || K % block || M < 1) return -1;
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
    const int64_t C = K / 32, nb = K / block;
    float* ae = (float*)malloc(sizeof(float) * (size_t)(16 * C * M));
    float* ao = (float*)malloc(sizeof(float) * (size_t)(16 * C * M));
    float* bsum = (float*)malloc(sizeof(float) * (size_t)(nb * M));
    if (!ae || !ao || !bsum) {
        free(ae);
        free(ao);
        free(bsum);
        return -1;
    }
    for (int64_t m = 0; m < M; ++m) {
        const float* a = A + m * K;
        for (int64_t c = 0; c < C; ++c)
            for (int i = 0; i < 16; ++i) {
                ae[(m * C + c) * 16 + i] = a[32 * c + 2 * i];
                ao[(m * C + c) * 16 + i] = a[32 * c + 2 * i + 1];
            }
        for (int64_t b = 0; b < nb; ++b) {
            float s = 0.f;
            for (int64_t k = b * block; k < (b + 1) * block; ++k) s += a[k];
            bsum[m * nb + b] = s;
        }
    }
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel
    {
        switch (block / 32) {
            case 1: gemv_rows_1(ae, ao, bsum, M, B, scales, scale_f16, zp, N, K, Y); break;
            case 2: gemv_rows_2(ae, ao, bsum, M, B, scales, scale_f16, zp, N, K, Y); break;
            case 3: gemv_rows_3(ae, ao, bsum, M, B, scales, scale_f16, zp, N, K, Y); break;
            default: gemv_rows_4(ae, ao, bsum, M, B, scales, scale_f16, zp, N, K, Y); break;
        }
    }
    free(ae);
    free(ao);
    free(bsum);
    return 0;
}
