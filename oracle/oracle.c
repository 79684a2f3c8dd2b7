/*
 * oracle.c -- CPU restatement of hshatti/Invision's dense linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libinvision_hip.so and the timed
 * CPU baseline.  The product never links or calls anything in this file.
 *
 * Written from the reference's Pascal and x86-64 assembly; each function cites
 * the file:line it follows (paths relative to the reference repository root).
 * Compile: see oracle/Makefile (gcc -O2 -fopenmp; AVX2 path selected at run
 * time, with a scalar path of identical association order).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#include <immintrin.h>

/* ======================================================================== */
/* RNG -- src/quicknn_sample.pas:212-276                                     */
/* ======================================================================== */

/* Initial state before any rng_seed call: quicknn_sample.pas:212-217. */
static uint64_t g_state[4] = {
    0x853c49e6748fea9bULL, 0xda3e39cb94b95bdbULL,
    0x647c4677a2884327ULL, 0xc6e7918d2e2969f5ULL};

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* xoshiro256ss: quicknn_sample.pas:226-237 (Vigna's xoshiro256**). */
uint64_t orc_xoshiro256ss(void) {
    const uint64_t result = rotl64(g_state[1] * 5u, 7) * 9u;
    const uint64_t t = g_state[1] << 17;
    g_state[2] ^= g_state[0];
    g_state[3] ^= g_state[1];
    g_state[1] ^= g_state[2];
    g_state[0] ^= g_state[3];
    g_state[2] ^= t;
    g_state[3] = rotl64(g_state[3], 45);
    return result;
}

/* rng_seed: quicknn_sample.pas:239-251 -- SplitMix64, four outputs. */
void orc_rng_seed(uint64_t seed) {
    for (int i = 0; i < 4; ++i) {
        seed += 0x9e3779b97f4a7c15ULL;
        uint64_t z = seed;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        g_state[i] = z ^ (z >> 31);
    }
}

void orc_rng_set_state(const uint64_t s[4]) { memcpy(g_state, s, sizeof g_state); }
void orc_rng_get_state(uint64_t s[4]) { memcpy(s, g_state, sizeof g_state); }

/* rand: quicknn_sample.pas:256-259.  The 53-bit integer times 2^-53 is exact in
 * double; the Pascal result type is single, so it is rounded to nearest. */
float orc_rand(void) {
    return (float)((double)(orc_xoshiro256ss() >> 11) * (1.0 / 9007199254740992.0));
}

/* random_normal: quicknn_sample.pas:261-270.  u1, u2 are singles (QNNFloat =
 * single, quicknn_common.pas:108); the transcendental part is evaluated in
 * double here and rounded to single on return. */
float orc_random_normal(void) {
    float u1 = orc_rand();
    float u2 = orc_rand();
    while (u1 == 0.0f) u1 = orc_rand();
    return (float)(sqrt(-2.0 * log((double)u1)) * cos(2.0 * 3.14159265358979323846 * (double)u2));
}

/* randn: quicknn_sample.pas:272-276. */
void orc_randn(float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_random_normal();
}

static inline uint16_t bf16_rne_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_randn_scaled(float *dst, int64_t n, float sigma, int round_bf16) {
    for (int64_t i = 0; i < n; ++i) {
        float v = sigma * orc_random_normal();
        dst[i] = round_bf16 ? bf16_bits_to_f32(bf16_rne_bits(v)) : v;
    }
}

/* ======================================================================== */
/* bf16 -- src/quicknn_common.pas:1991-2027                                  */
/* ======================================================================== */

/* BF16ToSingle: quicknn_common.pas:1991-2008 (exact widening, u32 = u16 << 16). */
void orc_bf16_to_f32(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = bf16_bits_to_f32(src[i]);
}

/* SingleToBF16: quicknn_common.pas:2010-2027 (truncation, u16 = u32 >> 16). */
void orc_f32_to_bf16_trunc(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &src[i], 4);
        dst[i] = (uint16_t)(u >> 16);
    }
}

/* The rounding the HIP path applies to fp32 activations: round to nearest,
 * ties to even, NaN kept quiet.  Not a reference function (the reference never
 * rounds activations); stated so that parity compares like with like. */
void orc_f32_to_bf16_rne(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = bf16_rne_bits(src[i]);
}

/* ======================================================================== */
/* GEMM -- src/quicknncpu.pas:1176-1496 and src/ops_avx2.inc                 */
/* ======================================================================== */

enum { ROW_MAJOR = 101, NO_TRANS = 111, TRANS = 112 };
enum { TILE_M = 8, TILE_N = 8, TILE_K = 8 }; /* quicknncpu.pas:1176-1180 */

static int g_has_avx2 = -1;
int orc_has_avx2(void) {
    if (g_has_avx2 < 0) {
        __builtin_cpu_init();
        g_has_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return g_has_avx2;
}
int orc_max_threads(void) { return omp_get_max_threads(); }

/* qscale: quicknncpu.pas:1067-1080 -> sScaleInplace_avx2.  X *= alpha; note
 * that beta = 0 multiplies (0 * NaN stays NaN), unlike BLAS. */
static void qscale(int64_t n, float alpha, float *x) {
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] * alpha;
}

/* qaxpy: quicknncpu.pas:1082-1093 -> saxpy_avx2 (ops_avx2.inc:839-907): y = fma(a, x, y). */
static void qaxpy(int64_t n, float a, const float *x, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = fmaf(a, x[i], y[i]);
}

/* Lane reduction shared by sdot_avx2 and sDot_x4_avx2 (ops_avx2.inc:827-832,
 * 1466-1483): lo+hi halves, then haddps twice -> (v0+v1)+(v2+v3). */
static inline float reduce8(const float l[8]) {
    float v0 = l[0] + l[4], v1 = l[1] + l[5], v2 = l[2] + l[6], v3 = l[3] + l[7];
    return (v0 + v1) + (v2 + v3);
}

/* sdot_avx2: ops_avx2.inc:757-837, scalar emulation.  Four 8-lane FMA
 * accumulators over 32-element chunks, combined (a0+a1)+(a2+a3); then 8-element
 * chunks into a0; then the masked K%8 tail into a0; then reduce8. */
static float sdot_emul(int64_t n, const float *a, const float *b) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    int64_t k = 0;
    int64_t n32 = n >> 5;
    for (int64_t it = 0; it < n32; ++it, k += 32)
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 8; ++l) acc[c][l] = fmaf(a[k + 8 * c + l], b[k + 8 * c + l], acc[c][l]);
    float s[8];
    if (n32) {
        for (int l = 0; l < 8; ++l) s[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    } else {
        memset(s, 0, sizeof s);
    }
    int64_t n8 = (n & 31) >> 3;
    for (int64_t it = 0; it < n8; ++it, k += 8)
        for (int l = 0; l < 8; ++l) s[l] = fmaf(a[k + l], b[k + l], s[l]);
    int64_t r = n & 7;
    for (int l = 0; l < r; ++l) s[l] = fmaf(a[k + l], b[k + l], s[l]);
    return reduce8(s);
}

/* sDot_x4_avx2: ops_avx2.inc:1407-1508, scalar emulation of the *intended*
 * arithmetic: four 8-lane accumulators (lane l sums k = l mod 8) for the four
 * B rows, reduce8 each, then C[j] = fma(dot_j, alpha, C[j]).  The assembly's
 * K%8 tail overwrites the accumulators with the masked loads (ops_avx2.inc:
 * 1442-1464); this restatement adds the tail product instead, which is what
 * the closed form requires.  All workload K are multiples of 8. */
static void sdot_x4_emul(const float *A, const float *B, float *C, int64_t K, int64_t ldb, float alpha) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    int64_t k = 0;
    for (int64_t it = 0; it < (K >> 3); ++it, k += 8)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) acc[j][l] = fmaf(A[k + l], B[j * ldb + k + l], acc[j][l]);
    for (int64_t l = 0; l < (K & 7); ++l)
        for (int j = 0; j < 4; ++j) acc[j][l] = fmaf(A[k + l], B[j * ldb + k + l], acc[j][l]);
    for (int j = 0; j < 4; ++j) C[j] = fmaf(reduce8(acc[j]), alpha, C[j]);
}

__attribute__((target("avx2,fma"))) static inline float reduce8_avx(__m256 v) {
    __m128 r = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    r = _mm_hadd_ps(r, r);
    r = _mm_hadd_ps(r, r);
    return _mm_cvtss_f32(r);
}

__attribute__((target("avx2,fma"))) static inline __m256i tail_mask(int64_t r) {
    const __m256i idx = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
    return _mm256_cmpgt_epi32(_mm256_set1_epi32((int)r), idx);
}

__attribute__((target("avx2,fma"))) static float sdot_avx(int64_t n, const float *a, const float *b) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    int64_t k = 0;
    for (int64_t it = 0; it < (n >> 5); ++it, k += 32) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + k), _mm256_loadu_ps(b + k), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + k + 8), _mm256_loadu_ps(b + k + 8), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + k + 16), _mm256_loadu_ps(b + k + 16), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + k + 24), _mm256_loadu_ps(b + k + 24), a3);
    }
    __m256 s = (n >> 5) ? _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)) : _mm256_setzero_ps();
    for (int64_t it = 0; it < ((n & 31) >> 3); ++it, k += 8)
        s = _mm256_fmadd_ps(_mm256_loadu_ps(a + k), _mm256_loadu_ps(b + k), s);
    if (n & 7) {
        __m256i m = tail_mask(n & 7);
        s = _mm256_fmadd_ps(_mm256_maskload_ps(a + k, m), _mm256_maskload_ps(b + k, m), s);
    }
    return reduce8_avx(s);
}

__attribute__((target("avx2,fma"))) static void sdot_x4_avx(const float *A, const float *B, float *C, int64_t K,
                                                             int64_t ldb, float alpha) {
    __m256 c0 = _mm256_setzero_ps(), c1 = c0, c2 = c0, c3 = c0;
    int64_t k = 0;
    for (int64_t it = 0; it < (K >> 3); ++it, k += 8) {
        __m256 a = _mm256_loadu_ps(A + k);
        c0 = _mm256_fmadd_ps(a, _mm256_loadu_ps(B + k), c0);
        c1 = _mm256_fmadd_ps(a, _mm256_loadu_ps(B + ldb + k), c1);
        c2 = _mm256_fmadd_ps(a, _mm256_loadu_ps(B + 2 * ldb + k), c2);
        c3 = _mm256_fmadd_ps(a, _mm256_loadu_ps(B + 3 * ldb + k), c3);
    }
    if (K & 7) {
        __m256i m = tail_mask(K & 7);
        __m256 a = _mm256_maskload_ps(A + k, m);
        c0 = _mm256_fmadd_ps(a, _mm256_maskload_ps(B + k, m), c0);
        c1 = _mm256_fmadd_ps(a, _mm256_maskload_ps(B + ldb + k, m), c1);
        c2 = _mm256_fmadd_ps(a, _mm256_maskload_ps(B + 2 * ldb + k, m), c2);
        c3 = _mm256_fmadd_ps(a, _mm256_maskload_ps(B + 3 * ldb + k, m), c3);
    }
    C[0] = fmaf(reduce8_avx(c0), alpha, C[0]);
    C[1] = fmaf(reduce8_avx(c1), alpha, C[1]);
    C[2] = fmaf(reduce8_avx(c2), alpha, C[2]);
    C[3] = fmaf(reduce8_avx(c3), alpha, C[3]);
}

/* One 8-row tile of gemm_nt: quicknncpu.pas:1250-1323. */
static void gemm_nt_tile(int64_t tm_start, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                         int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc,
                         int use_avx) {
    int64_t tm_finish = tm_start + TILE_M;
    if (tm_finish > M) tm_finish = M;
    for (int64_t tm = tm_start; tm < tm_finish; ++tm) qscale(N, beta, C + tm * ldc);
    for (int64_t tn_start = 0; tn_start < N; tn_start += TILE_N) {
        int64_t tn_finish = tn_start + TILE_N;
        if (tn_finish > N) tn_finish = N;
        for (int64_t tm = tm_start; tm < tm_finish; ++tm) {
            float *CC = C + tm * ldc;
            int64_t tn = tn_start;
            for (; tn + 4 <= tn_finish; tn += 4) {
                if (use_avx)
                    sdot_x4_avx(A + tm * lda, B + tn * ldb, CC + tn, K, ldb, alpha);
                else
                    sdot_x4_emul(A + tm * lda, B + tn * ldb, CC + tn, K, ldb, alpha);
            }
            for (; tn < tn_finish; ++tn) {
                /* a_part := ALPHA*qdot(...); CC[tn] := CC[tn] + a_part (two roundings) */
                float d = use_avx ? sdot_avx(K, A + tm * lda, B + tn * ldb) : sdot_emul(K, A + tm * lda, B + tn * ldb);
                float a_part = alpha * d;
                CC[tn] = CC[tn] + a_part;
            }
        }
    }
}

/* gemm_nn tile: quicknncpu.pas:1182-1239. */
static void gemm_nn_tile(int64_t tm_start, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                         int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    int64_t tm_finish = tm_start + TILE_M;
    if (tm_finish > M) tm_finish = M;
    for (int64_t tm = tm_start; tm < tm_finish; ++tm) qscale(N, beta, C + tm * ldc);
    for (int64_t tk_start = 0; tk_start < K; tk_start += TILE_K) {
        int64_t tk_finish = tk_start + TILE_K;
        if (tk_finish > K) tk_finish = K;
        for (int64_t tm = tm_start; tm < tm_finish; ++tm)
            for (int64_t tk = tk_start; tk < tk_finish; ++tk)
                qaxpy(N, alpha * A[tm * lda + tk], B + tk * ldb, C + tm * ldc);
    }
}

/* gemm_tn tile: quicknncpu.pas:1338-1395. */
static void gemm_tn_tile(int64_t tm_start, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                         int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    int64_t tm_finish = tm_start + TILE_M;
    if (tm_finish > M) tm_finish = M;
    for (int64_t tm = tm_start; tm < tm_finish; ++tm) qscale(N, beta, C + tm * ldc);
    for (int64_t tk_start = 0; tk_start < K; tk_start += TILE_K) {
        int64_t tk_finish = tk_start + TILE_K;
        if (tk_finish > K) tk_finish = K;
        for (int64_t tk = tk_start; tk < tk_finish; ++tk) {
            const float *AA = A + tk * lda;
            for (int64_t tm = tm_start; tm < tm_finish; ++tm)
                qaxpy(N, alpha * AA[tm], B + tk * ldb, C + tm * ldc);
        }
    }
}

/* qgemm: quicknncpu.pas:1398-1496.  Row tiles of 8 are distributed over
 * threads, as mp.&For does (quicknncpu.pas:1328-1329). */
int orc_qgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
              const float *A, int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc,
              int nthreads) {
    if (order != ROW_MAJOR || (transA == TRANS && transB == TRANS)) return -1;
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    const int use_avx = orc_has_avx2();
    const int64_t ntiles = (M + TILE_M - 1) / TILE_M;
    if (transA == NO_TRANS && transB == NO_TRANS) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t t = 0; t < ntiles; ++t)
            gemm_nn_tile(t * TILE_M, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    } else if (transA == NO_TRANS && transB == TRANS) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t t = 0; t < ntiles; ++t)
            gemm_nt_tile(t * TILE_M, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, use_avx);
    } else if (transA == TRANS && transB == NO_TRANS) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t t = 0; t < ntiles; ++t)
            gemm_tn_tile(t * TILE_M, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    } else {
        return -1;
    }
    return 0;
}

int orc_gemm_nt_scalar(int64_t M, int64_t N, int64_t K, float alpha, const float *A, int64_t lda,
                       const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    for (int64_t t = 0; t < M; t += TILE_M) gemm_nt_tile(t, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, 0);
    return 0;
}

/* fp64 gold for the closed form C = A . B^T. */
void orc_gemm_nt_f64(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda, const float *B, int64_t ldb,
                     double *C, int64_t ldc, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int64_t m = 0; m < M; ++m) {
        const float *a = A + m * lda;
        for (int64_t n = 0; n < N; ++n) {
            const float *b = B + n * ldb;
            double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            int64_t k = 0;
            for (; k + 4 <= K; k += 4) {
                s0 += (double)a[k] * b[k];
                s1 += (double)a[k + 1] * b[k + 1];
                s2 += (double)a[k + 2] * b[k + 2];
                s3 += (double)a[k + 3] * b[k + 3];
            }
            for (; k < K; ++k) s0 += (double)a[k] * b[k];
            C[m * ldc + n] = (s0 + s1) + (s2 + s3);
        }
    }
}

/* ======================================================================== */
/* Epilogue ops                                                              */
/* ======================================================================== */

float orc_silu_exact(float x) { return (float)((double)x / (1.0 + exp(-(double)x))); }

float orc_gelu_erf(float x) { return (float)(0.5 * (double)x * (1.0 + erf((double)x * 0.70710678118654752440))); }

/* fast_exp: quicknncpu.pas:305-330 (the non-AVX2 SiLU path). */
float orc_fast_exp(float x) {
    if (x < -87.33f) return 0.0f;
    if (x > 88.72f) return 1e38f;
    float n = floorf(x * 1.4426950408889634f + 0.5f);
    float r = x - n * 0.6931471805599453f;
    float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.16666667f + r * (0.04166667f + r * 0.00833333f))));
    int32_t bits;
    memcpy(&bits, &p, 4);
    bits += (int32_t)n << 23;
    memcpy(&p, &bits, 4);
    return p;
}

/* sSiLU_avx2: ops_avx2.inc:267-376 with constants ops_avx2.inc:22-35.
 * t = clamp(-x, MIN_EXP, MAX_EXP) * log2(e); n = floor(t); f = t - n;
 * p = (C0*f + C1)*f + C2 (two FMAs); exp(-x) ~= bits(p) + (n << 23);
 * sigma = 1/(1 + exp(-x)) -- vrcpps replaced by an exact division, because
 * the rcp bits are implementation defined (relative error <= 1.5 * 2^-12).
 * out_sigmoid <- sigma; dst <- sigma * x (* up if given). */
void orc_silu_qnn(int64_t n, const float *src, const float *up, float *out_sigmoid, float *dst) {
    const float L2E = 1.4426950408889634f, C2 = 1.00172476f, C1 = 0.657636276f, C0 = 0.3371894346f;
    const float MAX_EXP = 8.87e+001f, MIN_EXP = -8.73e+001f;
    for (int64_t i = 0; i < n; ++i) {
        float t = 0.0f - src[i];
        if (t >= MAX_EXP) t = MAX_EXP;
        if (t <= MIN_EXP) t = MIN_EXP;
        t = L2E * t;
        float fl = floorf(t);
        float f = t - fl;
        int32_t e = (int32_t)fl << 23;
        float p = fmaf(fmaf(C0, f, C1), f, C2);
        int32_t pb;
        memcpy(&pb, &p, 4);
        pb += e;
        float ex;
        memcpy(&ex, &pb, 4);
        float sig = 1.0f / (ex + 1.0f);
        if (out_sigmoid) out_sigmoid[i] = sig;
        if (dst) {
            float v = sig * src[i];
            if (up) v = v * up[i];
            dst[i] = v;
        }
    }
}

void orc_add_bias_rows(float *Y, const float *bias, int64_t M, int64_t N) {
    /* QNNLinear bias loop: quicknncpu.pas:1816-1819 -> QNNAddInplace :704-709. */
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) Y[i * N + j] = Y[i * N + j] + bias[j];
}

void orc_apply_epilogue(float *Y, int64_t n, int epilogue) {
    switch (epilogue) {
    case 1:
        for (int64_t i = 0; i < n; ++i) Y[i] = orc_silu_exact(Y[i]);
        break;
    case 2:
        for (int64_t i = 0; i < n; ++i) Y[i] = orc_gelu_erf(Y[i]);
        break;
    case 3:
        orc_silu_qnn(n, Y, NULL, NULL, Y);
        break;
    default:
        break;
    }
}

/* QNNGatedAdd: quicknncpu.pas:853-859, one QNNAccMul (:1752-1758) per row:
 * dst[i][j] = dst[i][j] + gate[j] * proj[i][j], product rounded to fp32 first. */
void orc_gated_add(float *dst, const float *gate, const float *proj, int64_t seq, int64_t hidden) {
    for (int64_t i = 0; i < seq; ++i)
        for (int64_t j = 0; j < hidden; ++j) {
            const float t = gate[j] * proj[i * hidden + j];
            dst[i * hidden + j] = dst[i * hidden + j] + t;
        }
}

/* QNNLinear / QNNLinearNoBias_BF16 / QNNLINEAR_BF16_OR_F32:
 * quicknncpu.pas:1807-1847, 3062-3071.  The bf16 weight is widened into a
 * workspace (:1842-1844), then cblas_gemm(RowMajor, NoTrans, Trans, M, N, K,
 * 1, X, K, W, K, 0, Y, N) (:1824-1827), then the per-row bias (:1816-1819),
 * then the epilogue op the caller applies next (QNNSilu etc.). */
int orc_linear_bf16w(const float *X, const uint16_t *W, const float *bias, float *Y, int64_t M, int64_t K,
                     int64_t N, int epilogue, int nthreads) {
    float *Wf = (float *)malloc((size_t)(N * K) * sizeof(float));
    if (!Wf) return -1;
    orc_bf16_to_f32(W, Wf, N * K);
    memset(Y, 0, (size_t)(M * N) * sizeof(float));
    int rc = orc_qgemm(ROW_MAJOR, NO_TRANS, TRANS, M, N, K, 1.0f, X, K, Wf, K, 0.0f, Y, N, nthreads);
    free(Wf);
    if (rc) return rc;
    if (bias) orc_add_bias_rows(Y, bias, M, N);
    orc_apply_epilogue(Y, M * N, epilogue);
    return 0;
}

/* ---- attention ---------------------------------------------------------------
 * The reference's transformer layout: Q [seq_q x heads*d], K and V
 * [seq_k x kv_heads*d], O [seq_q x heads*d], row-major; head h reads kv head
 * h / (heads / kv_heads) (quicknn_qwen3.pas:735-762).  With causal set, key j is
 * visible to query i iff j <= i + (seq_k - seq_q) (QNNMatTriangularFill before
 * the softmax, quicknn_qwen3.pas:752-754, for seq_q = seq_k). */

/* Closed form in fp64: O = softmax(scale * Q.K^T) . V per head and query -- the
 * mathematics of the per-head cblas_gemm / QNNSoftmaxRows / cblas_gemm loops
 * (quicknn_transformers.pas:1150-1311, 2228-2271; quicknn_qwen3.pas:727-769) and
 * of QNNFlashAttention (quicknncpu.pas:2763). */
int orc_attention_f64(const float *Q, const float *K, const float *V, double *O, int64_t heads, int64_t kv_heads,
                      int64_t seq_q, int64_t seq_k, int64_t d, double scale, int causal, const int32_t *key_mask,
                      int nthreads) {
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads) return -1;
    const int64_t hq = heads * d, hk = kv_heads * d, grp = heads / kv_heads, off = seq_k - seq_q;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    int bad = 0;
#pragma omp parallel
    {
        double *w = (double *)malloc((size_t)(seq_k > 0 ? seq_k : 1) * sizeof(double));
        if (!w) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for collapse(2) schedule(static)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t i = 0; i < seq_q; ++i) {
                if (!w) continue;
                const float *q = Q + i * hq + h * d;
                const int64_t g = h / grp;
                const int64_t last = causal ? (i + off < seq_k - 1 ? i + off : seq_k - 1) : seq_k - 1;
                double mx = -INFINITY;
                for (int64_t j = 0; j <= last; ++j) {
                    if (key_mask && !key_mask[j]) continue;
                    const float *k = K + j * hk + g * d;
                    double dot = 0.0;
                    for (int64_t e = 0; e < d; ++e) dot += (double)q[e] * (double)k[e];
                    w[j] = dot * scale;
                    if (w[j] > mx) mx = w[j];
                }
                double sum = 0.0;
                for (int64_t j = 0; j <= last; ++j) {
                    if (key_mask && !key_mask[j]) continue;
                    w[j] = exp(w[j] - mx);
                    sum += w[j];
                }
                double *o = O + i * hq + h * d;
                for (int64_t e = 0; e < d; ++e) o[e] = 0.0;
                for (int64_t j = 0; j <= last && sum > 0.0; ++j) {
                    if (key_mask && !key_mask[j]) continue;
                    const float *v = V + j * hk + g * d;
                    const double pj = w[j] / sum;
                    for (int64_t e = 0; e < d; ++e) o[e] += pj * (double)v[e];
                }
            }
        free(w);
    }
    return bad ? -2 : 0;
}

/* sSoftmax_avx2 (ops_avx2.inc:552-760) restated: t = x - max clamped to
 * [MIN_EXP, MAX_EXP] = [-87.3, 88.7] (:33-34, 600-603); n = floor(t log2 e + 0.5);
 * r = fma(n, -ln 2, t); p = Horner of 1 + r(1 + r(0.5 + r(0.16666667 +
 * r(0.04166667 + r 0.00833333)))) with fused multiply-adds; 2^n added to the
 * exponent bits; eight running lane sums, then the horizontal sum; every value
 * times 1/sum.  The reference takes 1/sum with rcpss (an approximation whose
 * bits are implementation-defined); this restatement divides exactly. */
void orc_softmax_qnn(float *x, int64_t n) {
    if (n <= 0) return;
    float mx = x[0];
    for (int64_t i = 1; i < n; ++i)
        if (x[i] > mx) mx = x[i];
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = 0; i < n; ++i) {
        float t = x[i] - mx;
        if (t >= 88.7f) t = 88.7f;
        if (t <= -87.3f) t = -87.3f;
        const float nn = floorf(t * 1.4426950408889634f + 0.5f);
        const float r = fmaf(nn, -0.6931471805599453f, t);
        float p = fmaf(r, 0.00833333f, 0.04166667f);
        p = fmaf(p, r, 0.16666667f);
        p = fmaf(p, r, 0.5f);
        p = fmaf(p, r, 1.0f);
        p = fmaf(p, r, 1.0f);
        int32_t bits;
        memcpy(&bits, &p, 4);
        bits += (int32_t)nn << 23;
        memcpy(&p, &bits, 4);
        x[i] = p;
        lane[i & 7] += p;
    }
    const float sum = ((lane[0] + lane[1]) + (lane[2] + lane[3])) + ((lane[4] + lane[5]) + (lane[6] + lane[7]));
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}

/* The reference's BLAS-bound attention as it runs (quicknn_transformers.pas:
 * 1163-1189; quicknn_qwen3.pas:741-768): scores = scale * Q_h . K_g^T summed in
 * fp32 (cblas_gemm with alpha = scale), -inf where causal or the key mask hides
 * the key (QNNMatTriangularFill, quicknncpu.pas:3017-3028), QNNSoftmaxRows
 * (orc_softmax_qnn), O_h = P . V_g summed in fp32. */
int orc_attention_qnn(const float *Q, const float *K, const float *V, float *O, int64_t heads, int64_t kv_heads,
                      int64_t seq_q, int64_t seq_k, int64_t d, float scale, int causal, const int32_t *key_mask,
                      int nthreads) {
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads) return -1;
    const int64_t hq = heads * d, hk = kv_heads * d, grp = heads / kv_heads, off = seq_k - seq_q;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    int bad = 0;
#pragma omp parallel
    {
        float *w = (float *)malloc((size_t)(seq_k > 0 ? seq_k : 1) * sizeof(float));
        if (!w) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for collapse(2) schedule(static)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t i = 0; i < seq_q; ++i) {
                if (!w) continue;
                const float *q = Q + i * hq + h * d;
                const int64_t g = h / grp;
                for (int64_t j = 0; j < seq_k; ++j) {
                    const float *k = K + j * hk + g * d;
                    float dot = 0.0f;
                    for (int64_t e = 0; e < d; ++e) dot += q[e] * k[e];
                    w[j] = ((causal && j > i + off) || (key_mask && !key_mask[j])) ? -INFINITY : scale * dot;
                }
                orc_softmax_qnn(w, seq_k);
                float *o = O + i * hq + h * d;
                for (int64_t e = 0; e < d; ++e) o[e] = 0.0f;
                for (int64_t j = 0; j < seq_k; ++j) {
                    const float *v = V + j * hk + g * d;
                    for (int64_t e = 0; e < d; ++e) o[e] += w[j] * v[e];
                }
            }
        free(w);
    }
    return bad ? -2 : 0;
}

/* ---- normalisations before the projections ---------------------------------
 * EPSILON = 1e-6 (quicknn_common.pas:51).  QNNAdaLN's eps argument is not used
 * by its body (quicknncpu.pas:3053): the constant always applies. */

/* QNNAdaLN (quicknncpu.pas:3042-3060): per row, mean = QNNSum / N (:679-685),
 * population variance = sum((x - mean)^2) / N (:687-695), stdInv = 1/sqrt(var +
 * EPSILON), out = (1 + scale[j]) * ((x - mean) * stdInv) + shift[j]. */
void orc_adaln(float *dst, const float *src, const float *shift, const float *scale, int64_t seq, int64_t hidden) {
    for (int64_t i = 0; i < seq; ++i) {
        const float *x = src + i * hidden;
        float *y = dst + i * hidden;
        float sum = 0.0f;
        for (int64_t j = 0; j < hidden; ++j) sum += x[j];
        const float mean = sum / (float)hidden;
        float sq = 0.0f;
        for (int64_t j = 0; j < hidden; ++j) sq += (x[j] - mean) * (x[j] - mean);
        const float var = sq / (float)hidden;
        const float inv = 1.0f / sqrtf(var + 1e-6f);
        for (int64_t j = 0; j < hidden; ++j) {
            const float norm = (x[j] - mean) * inv;
            y[j] = (1.0f + scale[j]) * norm + shift[j];
        }
    }
}

/* QNNRMSNormRows / QNNRMSNorm (quicknncpu.pas:2159-2198): invRMS = 1/sqrt(
 * QNNSumSqr / N + EPSILON); dst = src * weights * invRMS (src * invRMS without
 * weights). */
void orc_rmsnorm_rows(float *dst, const float *src, const float *weight, int64_t rows, int64_t dim) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = src + r * dim;
        float *y = dst + r * dim;
        float sq = 0.0f;
        for (int64_t j = 0; j < dim; ++j) sq += x[j] * x[j];
        const float inv = 1.0f / sqrtf(sq / (float)dim + 1e-6f);
        for (int64_t j = 0; j < dim; ++j) y[j] = weight ? x[j] * weight[j] * inv : x[j] * inv;
    }
}

/* QNNApplyRoPE2D (quicknncpu.pas:2968-2992): per token s and head h, for each
 * pair (d, d+1): x0 cos - x1 sin, x1 cos + x0 sin with cos/sin[s*hd + d]. */
void orc_rope_interleaved(float *x, const float *cos_t, const float *sin_t, int64_t seq, int64_t heads, int64_t d) {
    for (int64_t s = 0; s < seq; ++s)
        for (int64_t h = 0; h < heads; ++h) {
            float *v = x + (s * heads + h) * d;
            for (int64_t e = 0; e + 1 < d; e += 2) {
                const float c = cos_t[s * d + e], sn = sin_t[s * d + e];
                const float x0 = v[e], x1 = v[e + 1];
                v[e] = x0 * c - x1 * sn;
                v[e + 1] = x1 * c + x0 * sn;
            }
        }
}

/* QNNApplyRoPE3 -> QNNApplyRoPE2 (quicknncpu.pas:2892-2917): per token s and
 * head h, for i < d/2: x[i] cos[i] - x[i+d/2] sin[i], x[i] sin[i] + x[i+d/2] cos[i]
 * with cos/sin[s*d/2 + i]. */
void orc_rope_half(float *x, const float *cos_t, const float *sin_t, int64_t seq, int64_t heads, int64_t d) {
    const int64_t half = d / 2;
    for (int64_t s = 0; s < seq; ++s)
        for (int64_t h = 0; h < heads; ++h) {
            float *v = x + (s * heads + h) * d;
            for (int64_t i = 0; i < half; ++i) {
                const float c = cos_t[s * half + i], sn = sin_t[s * half + i];
                const float x0 = v[i], x1 = v[i + half];
                v[i] = x0 * c - x1 * sn;
                v[i + half] = x0 * sn + x1 * c;
            }
        }
}

/* QNNConv2d's direct form (quicknncpu.pas:2020-2039) in double; the output
 * channels run over threads. */
void orc_conv2d_f64(const float *src, const float *w, const float *bias, double *dst, int64_t in_ch,
                    int64_t out_ch, int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t stride,
                    int64_t pad, int64_t batch) {
    const int64_t outH = (H + 2 * pad - kH) / stride + 1, outW = (W + 2 * pad - kW) / stride + 1;
    for (int64_t b = 0; b < batch; ++b) {
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t oc = 0; oc < out_ch; ++oc)
            for (int64_t oh = 0; oh < outH; ++oh)
                for (int64_t ow = 0; ow < outW; ++ow) {
                    double sum = bias ? (double)bias[oc] : 0.0;
                    for (int64_t ic = 0; ic < in_ch; ++ic)
                        for (int64_t kr = 0; kr < kH; ++kr)
                            for (int64_t kc = 0; kc < kW; ++kc) {
                                const int64_t ih = oh * stride - pad + kr, iw = ow * stride - pad + kc;
                                if (ih >= 0 && ih < H && iw >= 0 && iw < W)
                                    sum += (double)src[((b * in_ch + ic) * H + ih) * W + iw] *
                                           (double)w[oc * in_ch * kH * kW + (ic * kH + kr) * kW + kc];
                            }
                    dst[((b * out_ch + oc) * outH + oh) * outW + ow] = sum;
                }
    }
}
