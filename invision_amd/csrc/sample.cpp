// sample.cpp -- the reference's random sampler, for synthetic inputs of the
// reference's distributions (host code; no GPU).
//
// The stream follows src/quicknn_sample.pas:212-276: a 256-bit xoshiro256**
// state seeded by four SplitMix64 outputs (rng_seed, :239-251), uniform
// singles from the top 53 bits of each output (rand, :256-259) and one
// Box-Muller normal per two uniforms, cosine branch (random_normal,
// :261-270).  The state is per calling thread, so concurrent callers draw
// independent streams; a caller that wants the reference's draw order seeds
// once and draws its tensors in order.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/inv_hip.h"

namespace {

struct Xoshiro {
    // rng state before any seeding (src/quicknn_sample.pas:212-217)
    uint64_t s[4] = {0x853c49e6748fea9bULL, 0xda3e39cb94b95bdbULL, 0x647c4677a2884327ULL, 0xc6e7918d2e2969f5ULL};

    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

    void seed(uint64_t v) {
        for (uint64_t &w : s) {
            v += 0x9e3779b97f4a7c15ULL;
            uint64_t z = v;
            z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
            z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
            w = z ^ (z >> 31);
        }
    }
    uint64_t next() {
        const uint64_t out = rotl(s[1] * 5u, 7) * 9u;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return out;
    }
    // 53 random bits times 2^-53 (exact in double), rounded to single: the
    // Pascal result type of rand.
    float uniform() { return (float)((double)(next() >> 11) * 0x1p-53); }
    // Box-Muller on single-precision uniforms, the transcendental part in
    // double, rounded to single on return; u1 = 0 is redrawn.
    float normal() {
        float u1 = uniform();
        const float u2 = uniform();
        while (u1 == 0.0f) u1 = uniform();
        return (float)(sqrt(-2.0 * log((double)u1)) * cos(6.283185307179586476925 * (double)u2));
    }
};

thread_local Xoshiro t_rng;

uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

}  // namespace

// Records the message for inv_hip_last_error (defined in inv_hip.hip).
extern "C" int inv_hip_internal_fail(int code, const char *msg);

extern "C" {

int inv_hip_sample_seed(uint64_t seed) {
    t_rng.seed(seed);
    return INV_OK;
}

int inv_hip_sample_randn(float *dst, int64_t n, float sigma, int round_bf16) {
    if (n < 0 || (n > 0 && !dst)) return inv_hip_internal_fail(INV_ERR_ARG, "sample_randn: negative n or null dst");
    for (int64_t i = 0; i < n; ++i) {
        float v = sigma * t_rng.normal();
        if (round_bf16) {
            const uint32_t u = (uint32_t)bf16_rne(v) << 16;
            memcpy(&v, &u, 4);
        }
        dst[i] = v;
    }
    return INV_OK;
}

}  // extern "C"
