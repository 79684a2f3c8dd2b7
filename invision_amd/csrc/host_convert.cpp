// host_convert.cpp -- fp32 -> bf16 rounding of host rows (declared in
// host_convert.hpp).  An AVX2 body picked at run time, a portable one
// otherwise; both give the bits of the device's bf16_rne.
#include "host_convert.hpp"

#include <immintrin.h>
#include <string.h>

namespace inv {
namespace {

inline uint16_t rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void row_generic(uint16_t *d, const float *s, int64_t cols, int64_t cols_pad) {
    for (int64_t c = 0; c < cols; ++c) d[c] = rne(s[c]);
    for (int64_t c = cols; c < cols_pad; ++c) d[c] = 0;
}

// Eight fp32 bit patterns -> their bf16 bits in the low halves of the lanes.
__attribute__((target("avx2"))) inline __m256i rne8(__m256i u) {
    const __m256i one = _mm256_set1_epi32(1), half = _mm256_set1_epi32(0x7fff);
    const __m256i abs_mask = _mm256_set1_epi32(0x7fffffff), inf = _mm256_set1_epi32(0x7f800000);
    const __m256i quiet = _mm256_set1_epi32(0x40);
    const __m256i hi = _mm256_srli_epi32(u, 16);
    const __m256i rounded = _mm256_srli_epi32(_mm256_add_epi32(u, _mm256_add_epi32(half, _mm256_and_si256(hi, one))), 16);
    // |u| and inf are both below 2^31, so the signed compare is the unsigned one
    const __m256i nan = _mm256_cmpgt_epi32(_mm256_and_si256(u, abs_mask), inf);
    return _mm256_blendv_epi8(rounded, _mm256_or_si256(hi, quiet), nan);
}

__attribute__((target("avx2"))) void row_avx2(uint16_t *d, const float *s, int64_t cols, int64_t cols_pad) {
    int64_t c = 0;
    for (; c + 16 <= cols; c += 16) {
        const __m256i a = rne8(_mm256_loadu_si256((const __m256i *)(s + c)));
        const __m256i b = rne8(_mm256_loadu_si256((const __m256i *)(s + c + 8)));
        // packus keeps each 128-bit half in place: a0-3 b0-3 | a4-7 b4-7
        const __m256i p = _mm256_permute4x64_epi64(_mm256_packus_epi32(a, b), 0xd8);
        _mm256_storeu_si256((__m256i *)(d + c), p);
    }
    for (; c < cols; ++c) d[c] = rne(s[c]);
    for (; c < cols_pad; ++c) d[c] = 0;
}

bool have_avx2() {
#ifdef INV_HOST_CONVERT_GENERIC  // the portable body only (a test build)
    return false;
#else
    static const bool yes = (__builtin_cpu_init(), __builtin_cpu_supports("avx2") != 0);
    return yes;
#endif
}

}  // namespace

void host_f32_to_bf16_rows(uint16_t *dst, int64_t ldd, const float *src, int64_t lds, int64_t rows, int64_t cols,
                           int64_t cols_pad) {
    const bool avx2 = have_avx2();
    for (int64_t r = 0; r < rows; ++r) {
        if (avx2)
            row_avx2(dst + r * ldd, src + r * lds, cols, cols_pad);
        else
            row_generic(dst + r * ldd, src + r * lds, cols, cols_pad);
    }
}

}  // namespace inv
