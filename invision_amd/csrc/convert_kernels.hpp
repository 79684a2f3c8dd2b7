// convert_kernels.hpp -- layout/precision staging for the GEMM operands.
//
// The GEMM consumes bf16 rows with K contiguous, K padded to a multiple of 8
// and rows 16-byte aligned.  These kernels produce that layout:
//  * fp32 rows -> bf16 rows (round to nearest even), the activation path of
//    inv_hip_linear (the reference keeps activations fp32, so this rounding is
//    the one precision step the HIP path adds);
//  * fp32 [R x C] -> bf16 [C x R] (transposed), for the CBLAS slot's
//    Trans-A / NoTrans-B operands;
//  * bf16 rows -> bf16 rows (re-pitch / pad) and bf16 transpose, for the bf16
//    slot and unaligned bf16 activations;
//  * an fp32 image -> its bf16 convolution patch matrix (im2col), for
//    inv_hip_conv2d.
// All are HBM-bound: 6 bytes (fp32 -> bf16) or 4 bytes (bf16) per element.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace inv {

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Split of an fp32 value into two bf16: hi = RNE(v), lo = RNE(v - hi), so that
// hi + lo carries 16 significant bits; a product (Ah + Al)(Bh + Bl) then
// differs from AB by the dropped Al*Bl term (relative 2^-16 or less).
__device__ __forceinline__ void bf16_split(float v, uint16_t &hi, uint16_t &lo) {
    hi = bf16_rne(v);
    const float h = __uint_as_float((uint32_t)hi << 16);
    lo = ((hi & 0x7f80u) == 0x7f80u) ? (uint16_t)0 : bf16_rne(v - h);
}

__device__ __forceinline__ uint4 pack8(const uint16_t (&h)[8]) {
    uint4 o;
    o.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    o.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
    o.z = (uint32_t)h[4] | ((uint32_t)h[5] << 16);
    o.w = (uint32_t)h[6] | ((uint32_t)h[7] << 16);
    return o;
}

// An image element as fp32: an fp32 image as it is, a bf16 image (an fp32
// image the host already rounded) widened exactly.
__device__ __forceinline__ float image_value(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float image_value(const uint16_t *p, int64_t i) {
    return __uint_as_float((uint32_t)p[i] << 16);
}

// Row-wise fp32 -> bf16 with nseg segments per output row: segment s of row r
// starts at dst + r*ldd + s*cols_pad and holds lo parts if bit s of lo_mask is
// set, hi parts otherwise (nseg = 1, lo_mask = 0: plain RNE rounding).
// Columns cols..cols_pad-1 of each segment are zero.  One thread per 8 columns;
// cols_pad % 8 == 0, ldd % 8 == 0, dst 16-byte aligned.
__global__ void __launch_bounds__(256) cvt_rows_f32_bf16(const float *__restrict__ src, int64_t lds,
                                                         uint16_t *__restrict__ dst, int64_t ldd, int64_t rows,
                                                         int64_t cols, int64_t cols_pad, int vec_src, int nseg,
                                                         int lo_mask) {
    const int64_t per_row = cols_pad >> 3;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row;
    const int64_t c0 = (idx - r * per_row) << 3;
    const float *s = src + r * lds + c0;
    float v[8];
    if (vec_src && c0 + 8 <= cols) {
        float4 a = *(const float4 *)s;
        float4 b = *(const float4 *)(s + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (c0 + e < cols) ? s[e] : 0.0f;
    }
    uint16_t *d = dst + r * ldd + c0;
    uint16_t hi[8];
    if (lo_mask == 0) {  // the plain rounding: no lo parts to form
#pragma unroll
        for (int e = 0; e < 8; ++e) hi[e] = bf16_rne(v[e]);
        const uint4 ohi = pack8(hi);
        for (int sg = 0; sg < nseg; ++sg) *(uint4 *)(d + sg * cols_pad) = ohi;
        return;
    }
    uint16_t lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bf16_split(v[e], hi[e], lo[e]);
    const uint4 ohi = pack8(hi);
    const uint4 olo = pack8(lo);
    for (int sg = 0; sg < nseg; ++sg) *(uint4 *)(d + sg * cols_pad) = ((lo_mask >> sg) & 1) ? olo : ohi;
}

// Normalisations that precede the reference's projections, applied while the
// fp32 activation is rounded into the GEMM's bf16 operand (the same one read of
// X and one bf16 write the plain conversion costs):
//  NORM_ADALN: (1 + a[c]) * ((x - mean) * rstd) + b[c], rstd = 1 / sqrt(var + eps),
//              mean and population variance over the row (QNNAdaLN,
//              src/quicknncpu.pas:3042-3060; QNNMean :679-685, QNNVariance :687-695);
//  NORM_RMS:   x * rstd * a[c] (a may be null), rstd = 1 / sqrt(sum(x^2) / cols + eps)
//              (QNNRMSNorm, src/quicknncpu.pas:2159-2185).
// One workgroup of 256 threads per row; the row is read from L2 once per pass.
// Columns cols..cols_pad-1 are zero; cols_pad % 8 == 0, ldd % 8 == 0, dst 16-byte aligned.
enum { NORM_ADALN = 1, NORM_RMS = 2 };

// Sum over the 256 threads of a workgroup (4 waves of 64); every thread gets it.
__device__ __forceinline__ float block_sum256(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();  // red is free (a previous call's readers are done)
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

template <int NORM>
__global__ void __launch_bounds__(256) norm_rows_f32_bf16(const float *__restrict__ src, int64_t lds,
                                                          const float *__restrict__ a, const float *__restrict__ b,
                                                          float eps, uint16_t *__restrict__ dst, int64_t ldd,
                                                          int64_t cols, int64_t cols_pad) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *x = src + r * lds;
    float mean = 0.0f, rstd;
    if constexpr (NORM == NORM_ADALN) {
        float s = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += 256) s += x[c];
        mean = block_sum256(s, red) / (float)cols;
        float q = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += 256) {
            const float d = x[c] - mean;
            q += d * d;
        }
        rstd = 1.0f / sqrtf(block_sum256(q, red) / (float)cols + eps);
    } else {
        float q = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += 256) q += x[c] * x[c];
        rstd = 1.0f / sqrtf(block_sum256(q, red) / (float)cols + eps);
    }
    for (int64_t c0 = (int64_t)threadIdx.x * 8; c0 < cols_pad; c0 += 256 * 8) {
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t c = c0 + e;
            float y = 0.0f;
            if (c < cols) {
                if constexpr (NORM == NORM_ADALN)
                    y = (1.0f + a[c]) * ((x[c] - mean) * rstd) + b[c];
                else
                    y = a ? x[c] * rstd * a[c] : x[c] * rstd;
            }
            h[e] = bf16_rne(y);
        }
        *(uint4 *)(dst + r * ldd + c0) = pack8(h);
    }
}

// The same normalisation with the row held in registers (one read of X):
// thread t owns the 4-column groups t, t + 256, ... (J of them); cols % 4 == 0,
// cols <= 4 * 256 * J, src rows and the per-column vectors 16-byte aligned.  J
// is the smallest of 1, 2, 3, 4, 6, 8, 12, 16 that holds the row, so short rows
// keep few registers and many rows in flight.
constexpr int NORM_ROW_GROUPS = 16;  // rows up to 16384 columns

template <int NORM, int J>
__global__ void __launch_bounds__(256) norm_rows_f32_bf16_reg(const float *__restrict__ src, int64_t lds,
                                                              const float *__restrict__ a,
                                                              const float *__restrict__ b, float eps,
                                                              uint16_t *__restrict__ dst, int64_t ldd, int64_t cols,
                                                              int64_t cols_pad) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *x = src + r * lds;
    const int ng = (int)(cols >> 2);
    // Every load of this thread is issued before the first reduction: its groups
    // of the row and the same groups of the per-column vectors, at a clamped
    // (always valid) group; groups past the row are zeroed after.
    float4 v[J], av[J], bv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int gi = min((int)threadIdx.x + 256 * j, ng - 1);
        v[j] = *(const float4 *)(x + 4 * gi);
        av[j] = a ? *(const float4 *)(a + 4 * gi) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        if constexpr (NORM == NORM_ADALN) bv[j] = *(const float4 *)(b + 4 * gi);
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
        if ((int)threadIdx.x + 256 * j >= ng) v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        s += (NORM == NORM_ADALN) ? (v[j].x + v[j].y) + (v[j].z + v[j].w)
                                  : (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
    float mean = 0.0f, rstd;
    if constexpr (NORM == NORM_ADALN) {
        mean = block_sum256(s, red) / (float)cols;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if ((int)threadIdx.x + 256 * j < ng) {
                const float d0 = v[j].x - mean, d1 = v[j].y - mean, d2 = v[j].z - mean, d3 = v[j].w - mean;
                q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
        }
        rstd = 1.0f / sqrtf(block_sum256(q, red) / (float)cols + eps);
    } else {
        rstd = 1.0f / sqrtf(block_sum256(s, red) / (float)cols + eps);
    }
    uint16_t *d = dst + r * ldd;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int g = threadIdx.x + 256 * j;
        if (g < ng) {
            const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            const float sv[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
            float hv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (NORM == NORM_ADALN) {
                hv[0] = bv[j].x; hv[1] = bv[j].y; hv[2] = bv[j].z; hv[3] = bv[j].w;
            }
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y;
                if constexpr (NORM == NORM_ADALN)
                    y = (1.0f + sv[e]) * ((xv[e] - mean) * rstd) + hv[e];
                else
                    y = xv[e] * rstd * sv[e];
                h[e] = bf16_rne(y);
            }
            *(uint2 *)(d + 4 * g) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                               (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        }
    }
    // zero padding up to cols_pad (fewer than 8 columns: at most one group of 4)
    if (threadIdx.x < (cols_pad >> 2) - ng) *(uint2 *)(d + 4 * (ng + threadIdx.x)) = make_uint2(0u, 0u);
}

// The steps between the Q/K projections and attention, in place on fp32
// x [rows x D] (rows = tokens * heads, D = 64 * EPT): each head's RMSNorm
// (QNNRMSNorm over its D values, src/quicknncpu.pas:2159-2185: x * w[d] * rstd,
// rstd = 1 / sqrt(sum(x^2) / D + eps)), then the rotary embedding of token
// row / heads:
//  ROPE_INTERLEAVED: pairs (2k, 2k+1) with table column 2k, tables [tokens x D]
//                    (QNNApplyRoPE2D, src/quicknncpu.pas:2968-2992);
//  ROPE_HALF:        pairs (i, i + D/2) with column i, tables [tokens x D/2]
//                    (QNNApplyRoPE2, src/quicknncpu.pas:2892-2917).
// One wave per head row at a time, EPT consecutive values per lane: the sum of squares is
// a wave reduction; a pair's partner is in the same lane (interleaved, EPT 2),
// in lane l ^ 1 (interleaved, EPT 1) or in lane l ^ 32 (half).
enum { ROPE_NONE = 0, ROPE_INTERLEAVED = 1, ROPE_HALF = 2 };

// BF16OUT: the result goes to y [rows x D] (packed) as bf16 (nearest-even)
// instead of back into x, the Q/K operand staging of the fused attention entry.
// A 256-thread workgroup covers 4 * HNR_ROWS rows.
constexpr int HNR_ROWS = 4;
template <int EPT, int ROPE, bool NORM, bool BF16OUT = false>
__global__ void __launch_bounds__(256) head_norm_rope(float *__restrict__ x, int64_t rows, int heads,
                                                      const float *__restrict__ w, const float *__restrict__ ct,
                                                      const float *__restrict__ st, float eps,
                                                      uint16_t *__restrict__ y, int64_t ldx) {
    constexpr int D = 64 * EPT;
    const int lane = threadIdx.x & 63;
    // HNR_ROWS consecutive rows per wave, their loads issued together: one row's
    // 64 x EPT floats alone leave too few bytes in flight to stream at the HBM rate
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * HNR_ROWS;
    // token row / heads starts ldx floats after the previous one (heads * D:
    // packed); one division per wave, then the rows step through the heads
    float *vp[HNR_ROWS];
    int64_t toks[HNR_ROWS];
    {
        int64_t tok = row0 / heads;
        int hd = (int)(row0 - tok * heads);
#pragma unroll
        for (int i = 0; i < HNR_ROWS; ++i) {
            vp[i] = x + tok * ldx + hd * D + EPT * lane;
            toks[i] = tok;
            if (++hd == heads) {
                hd = 0;
                ++tok;
            }
        }
    }
    float wv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        if constexpr (NORM)
            wv[j] = w[EPT * lane + j];
        else
            wv[j] = 1.0f;  // unused: no norm (w may be null)
    }
    float e[HNR_ROWS][EPT];
    float tc = 0.0f, ts = 0.0f;  // the current token's rotary pair (interleaved, EPT 2)
#pragma unroll
    for (int i = 0; i < HNR_ROWS; ++i) {
        const int64_t row = row0 + i;
        const float *v = vp[i];
        if (row >= rows) {
#pragma unroll
            for (int j = 0; j < EPT; ++j) e[i][j] = 0.0f;
        } else if constexpr (EPT == 2) {
            const float2 t = *(const float2 *)v;
            e[i][0] = t.x;
            e[i][1] = t.y;
        } else {
            e[i][0] = v[0];
        }
    }
#pragma unroll
    for (int i = 0; i < HNR_ROWS; ++i) {
        const int64_t row = row0 + i;
        if (row >= rows) break;  // the whole wave
        float *v = vp[i];
        if constexpr (NORM) {
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < EPT; ++j) sq += e[i][j] * e[i][j];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
            const float rstd = 1.0f / sqrtf(sq / (float)D + eps);
#pragma unroll
            for (int j = 0; j < EPT; ++j) e[i][j] = e[i][j] * wv[j] * rstd;
        }
        if constexpr (ROPE != ROPE_NONE) {
            const int64_t tok = toks[i];
            if constexpr (ROPE == ROPE_INTERLEAVED) {
                if constexpr (EPT == 2) {
                    // the wave's rows are heads of one token but at a token boundary:
                    // its table pair is loaded once for them
                    if (i == 0 || tok != toks[i - 1]) {
                        tc = ct[tok * D + 2 * lane];
                        ts = st[tok * D + 2 * lane];
                    }
                    const float c = tc, sn = ts;
                    const float x0 = e[i][0], x1 = e[i][1];
                    e[i][0] = x0 * c - x1 * sn;
                    e[i][1] = x1 * c + x0 * sn;
                } else {
                    const float p = __shfl_xor(e[i][0], 1);
                    const int col = lane & ~1;
                    const float c = ct[tok * D + col], sn = st[tok * D + col];
                    e[i][0] = (lane & 1) ? e[i][0] * c + p * sn : e[i][0] * c - p * sn;
                }
            } else {
                constexpr int H = D / 2;
                const bool lo = lane < 32;
#pragma unroll
                for (int j = 0; j < EPT; ++j) {
                    const float p = __shfl_xor(e[i][j], 32);
                    const int col = EPT * (lane & 31) + j;  // column of the pair
                    const float c = ct[tok * H + col], sn = st[tok * H + col];
                    e[i][j] = lo ? e[i][j] * c - p * sn : p * sn + e[i][j] * c;
                }
            }
        }
        if constexpr (BF16OUT) {
            uint16_t *o = y + row * D + EPT * lane;
            if constexpr (EPT == 2)
                *(uint32_t *)o = (uint32_t)bf16_rne(e[i][0]) | ((uint32_t)bf16_rne(e[i][1]) << 16);
            else
                o[0] = bf16_rne(e[i][0]);
        } else if constexpr (EPT == 2) {
            *(float2 *)v = make_float2(e[i][0], e[i][1]);
        } else {
            v[0] = e[i][0];
        }
    }
}

// dst[r, c] = src[r, c] (bf16) for c < cols, 0 up to cols_pad.  One thread per 8 outputs.
__global__ void __launch_bounds__(256) copy_rows_bf16(const uint16_t *__restrict__ src, int64_t lds,
                                                      uint16_t *__restrict__ dst, int64_t ldd, int64_t rows,
                                                      int64_t cols, int64_t cols_pad) {
    const int64_t per_row = cols_pad >> 3;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row;
    const int64_t c0 = (idx - r * per_row) << 3;
    const uint16_t *s = src + r * lds + c0;
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (c0 + e < cols) ? s[e] : (uint16_t)0;
    uint4 o;
    o.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
    o.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
    o.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
    o.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
    *(uint4 *)(dst + r * ldd + c0) = o;
}

// dst[c, s*rows_pad + r] = part_s(src[r, c]) : src [rows x cols] (ld lds) ->
// dst [cols x nseg*rows_pad] (ld ldd), parts as in cvt_rows_f32_bf16, zero for
// rows <= r < rows_pad.  64x64 tiles through LDS.
template <typename SrcT>
__global__ void __launch_bounds__(256) transpose_to_bf16(const SrcT *__restrict__ src, int64_t lds,
                                                         uint16_t *__restrict__ dst, int64_t ldd, int64_t rows,
                                                         int64_t cols, int64_t rows_pad, int nseg, int lo_mask) {
    __shared__ float tile[64][65];
    const int64_t r0 = (int64_t)blockIdx.y * 64;
    const int64_t c0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;  // 0..3
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        float v = 0.0f;
        if (r < rows && c < cols) {
            if constexpr (sizeof(SrcT) == 4)
                v = (float)src[r * lds + c];
            else
                v = __uint_as_float((uint32_t)src[r * lds + c] << 16);
        }
        tile[i][tx] = v;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows_pad) {
            uint16_t hi, lo;
            bf16_split(tile[tx][i], hi, lo);
            for (int sg = 0; sg < nseg; ++sg) dst[c * ldd + sg * rows_pad + r] = ((lo_mask >> sg) & 1) ? lo : hi;
        }
    }
}

// dst[c, r] = bf16(src[r, c]) for a [rows x cols] source with cols % 64 == 0,
// 16-byte aligned rows (lds % 8 for bf16, % 4 for fp32), into [cols x rows_pad]
// with rows_pad % 64 == 0 (zeros past rows): 64x64 tiles, 16-byte loads and
// stores on both sides, the transpose itself through LDS.
template <typename SrcT>
__global__ void __launch_bounds__(256) transpose64_to_bf16(const SrcT *__restrict__ src, int64_t lds,
                                                           uint16_t *__restrict__ dst, int64_t ldd, int64_t rows,
                                                           int64_t rows_pad) {
    constexpr int PITCH = 64 + 8;  // u16 per LDS row
    __shared__ __attribute__((aligned(16))) uint16_t tile[64 * PITCH];
    const int64_t r0 = (int64_t)blockIdx.y * 64;
    const int64_t c0 = (int64_t)blockIdx.x * 64;
    const int tid = threadIdx.x;
    if constexpr (sizeof(SrcT) == 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + 256 * i, row = q >> 3, cc = q & 7;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r0 + row < rows) v = *(const uint4 *)(src + (r0 + row) * lds + c0 + 8 * cc);
            *(uint4 *)(tile + row * PITCH + 8 * cc) = v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + 256 * i, row = q >> 4, cc = q & 15;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r0 + row < rows) v = *(const float4 *)(src + (r0 + row) * lds + c0 + 4 * cc);
            uint16_t *t = tile + row * PITCH + 4 * cc;
            t[0] = bf16_rne(v.x);
            t[1] = bf16_rne(v.y);
            t[2] = bf16_rne(v.z);
            t[3] = bf16_rne(v.w);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = tid + 256 * i, oc = q >> 3, rr = q & 7;
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = tile[(8 * rr + e) * PITCH + oc];
        *(uint4 *)(dst + (c0 + oc) * ldd + r0 + 8 * rr) = pack8(h);
    }
}

// The patch matrix of a convolution, pixel-major: col[p][k] = bf16(src[ic][ih][iw])
// with ih = oh*stride - pad + kr, iw = ow*stride - pad + kc (0 outside the
// image), for the output pixel p = (oh - oh0)*outW + ow of output rows
// [oh0, oh0 + npix/outW) and k = (ic*kH + kr)*kW + kc < K; columns K..ldc-1 are
// zero.  It is the transpose of QNNConv2d's column buffer
// (src/quicknncpu.pas:2063-2110), so that the GEMM reads both operands with K
// contiguous.  A 512-thread workgroup makes an (IM2COL_PG * 64)-pixel x 64-k
// block: wave w gathers k = 64*blockIdx.y + 8w .. +7 for IM2COL_PG groups of 64
// consecutive pixels (one per lane, so reads along an image row coalesce; every
// group's loads are issued before the first is used) into an LDS tile, then the
// block is written out row by row, eight lanes per 128-byte row segment.  src
// is one image [C x H x W], fp32 or bf16; ldc % 64 == 0 and col 16-byte aligned; grid
// (ceil(npix / (64 * IM2COL_PG)), ldc / 64).
constexpr int IM2COL_PG = 4;

// Filter columns from the reference's order (k = ic * taps + tap, the
// im2col order above) to tap-major (k = tap * C + ic), the order of the
// implicit convolution's k-tiles: dst [rows x C*taps] (pitch C*taps) from src
// [rows x lds]; total = rows * C * taps.
__global__ void __launch_bounds__(256) conv_filter_tap_major(const uint16_t *__restrict__ src, int64_t lds,
                                                             uint16_t *__restrict__ dst, int C, int taps,
                                                             int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t K = (int64_t)C * taps;
    const int64_t o = i / K;
    const int k = (int)(i - o * K);
    const int t = k / C, c = k - t * C;
    dst[i] = src[o * lds + (int64_t)c * taps + t];
}
template <typename SrcT>
__global__ void __launch_bounds__(512) im2col_bf16(const SrcT *__restrict__ src, uint16_t *__restrict__ col, int H,
                                                   int W, int kH, int kW, int stride, int pad, int outW, int oh0,
                                                   int64_t npix, int K, int64_t ldc) {
    constexpr int PITCH = 72;  // bf16 per LDS row: 64 + 8, so 16-byte writes of 64 rows spread over the banks
    constexpr int ROWS = 64 * IM2COL_PG;
    __shared__ __attribute__((aligned(16))) uint16_t tile[ROWS * PITCH];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t p0 = (int64_t)blockIdx.x * ROWS;
    const int k0 = (int)blockIdx.y * 64 + wave * 8;
    float v[IM2COL_PG][8];
    if (k0 < K) {
        const int khw = kH * kW;
        const int ic0 = k0 / khw;
        const int r0 = k0 - ic0 * khw;
        const int kr0 = r0 / kW, kc0 = r0 - (r0 / kW) * kW;
        // the group's first pixel; the others follow by 64 along the row (wrapping to the next rows)
        const int64_t pl = p0 + lane;
        int oh = oh0 + (int)(pl / outW), ow = (int)(pl % outW);
#pragma unroll
        for (int g = 0; g < IM2COL_PG; ++g) {
            const bool in = p0 + g * 64 + lane < npix;
            const int ih0 = oh * stride - pad, iw0 = ow * stride - pad;
            int ic = ic0, kr = kr0, kc = kc0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int ih = ih0 + kr, iw = iw0 + kc;
                v[g][e] = (in && k0 + e < K && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                              ? image_value(src, ((int64_t)ic * H + ih) * W + iw)
                              : 0.0f;
                if (++kc == kW) {
                    kc = 0;
                    if (++kr == kH) {
                        kr = 0;
                        ++ic;
                    }
                }
            }
            ow += 64;
            while (ow >= outW) {
                ow -= outW;
                ++oh;
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < IM2COL_PG; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[g][e] = 0.0f;
    }
#pragma unroll
    for (int g = 0; g < IM2COL_PG; ++g) {
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = bf16_rne(v[g][e]);
        *(uint4 *)(tile + (g * 64 + lane) * PITCH + wave * 8) = pack8(h);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < IM2COL_PG; ++i) {
        const int row = i * 64 + (threadIdx.x >> 3), c = threadIdx.x & 7;
        if (p0 + row < npix)
            *(uint4 *)(col + (p0 + row) * ldc + (int64_t)blockIdx.y * 64 + c * 8) =
                *(const uint4 *)(tile + row * PITCH + c * 8);
    }
}

// A 3x3, stride-1 convolution with few output channels (the VAE's conv_out,
// 128 -> 3), computed directly: the im2col path would write a patch matrix
// 9 * in_ch times larger than the image for a GEMM whose M is 3.  A 256-thread
// workgroup makes a CT_TH x CT_TW output tile of one image (4 consecutive
// pixels of one row per thread) for all OC (>= n_oc) output channels.  Input
// channels go CT_CC at a time through an LDS tile of the (CT_TH + 2) x
// (CT_TW + 2) input window, each value rounded to bf16 (RNE) as the patch
// matrix rounds it (a bf16 image, rounded by the host, is used as it is) and
// stored as bf16 pairs of channels (2p, 2p + 1); the
// filter's bf16 values (the weight handle's rows, [out_ch x in_ch*9] in the
// reference's (ic, kh, kw) order, row pitch ldw) are paired the same way, OC
// consecutive per tap so each tap's are one broadcast read.  v_dot2_f32_bf16
// then multiplies a pair and adds both products to the fp32 sum: results
// match the im2col path but for the summation order.  The loads of chunk
// c + 1 (image and filter) are issued before the multiplies of chunk c and
// written to LDS after them: the kernel streams the image at the rate of its
// loads in flight, not of one row's latency at a time.
// grid (ceil(outW / CT_TW), ceil(outH / CT_TH), batch).
constexpr int CT_TH = 16, CT_TW = 64, CT_CC = 8;
template <int OC, typename SrcT>
__global__ void __launch_bounds__(256) conv3x3_thin(const SrcT *__restrict__ src, const uint16_t *__restrict__ filt,
                                                    int64_t ldw, const float *__restrict__ bias,
                                                    float *__restrict__ dst, int C, int H, int W, int pad, int n_oc,
                                                    int outH, int outW) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    constexpr int CP = CT_CC / 2;                                     // channel pairs per chunk
    constexpr int TR = CT_TH + 2, TC = CT_TW + 2, PITCH = CT_TW + 4;  // PITCH: 16-byte aligned rows
    constexpr int RPW = CP * TR / 4;                                  // window row pairs per wave and chunk
    constexpr int NH = CP * TR * (TC - 64);                           // halo pairs (columns 64..TC-1) per chunk
    constexpr int HPT = (NH + 255) / 256;                             // of them per thread
    constexpr int NW = CP * 9 * OC;                                   // filter pairs per chunk
    constexpr int WPT = (NW + 255) / 256;                             // of them per thread
    static_assert(RPW * 4 == CP * TR && TC - 64 == 2 && CT_CC % 2 == 0, "window rows split evenly over the waves");
    __shared__ __attribute__((aligned(16))) uint32_t tile[CP][TR][PITCH];
    __shared__ __attribute__((aligned(16))) uint32_t wts[CP][9][OC];
    // wave-uniform row bookkeeping in scalar registers; a lane adds its column
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroup w of the dispatch runs on XCD w % 8.  The tiles are handed out
    // so that consecutive tiles (x fastest), which share their halo columns and
    // rows, run on one XCD and meet in its L2: the image's lines are fetched
    // once (1.05x the image at 1024x1024) instead of about twice.  The grid has
    // at most INT32_MAX workgroups (checked at launch).
    const int gx = gridDim.x, gxy = gx * gridDim.y, total = gxy * gridDim.z;
    const int wid = blockIdx.x + gx * (blockIdx.y + gridDim.y * blockIdx.z);
    const int per = total >> 3, rem = total & 7, xcd = wid & 7, local = wid >> 3;
    const int L = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    const int b = L / gxy, by = (L - b * gxy) / gx, bx = L - b * gxy - by * gx;
    const int oh0 = by * CT_TH, ow0 = bx * CT_TW;
    const SrcT *img = src + (int64_t)b * C * H * W;
    const int64_t plane = (int64_t)H * W;
    const int ty = tid >> 4, tx = (tid & 15) * 4;
    const int iw = ow0 - pad + lane;
    const bool cin = (unsigned)iw < (unsigned)W;
    float v[RPW][2], v2[HPT][2];
    uint32_t fw[WPT];
    // the two channels' values at one window position (zero outside the image or past C)
    auto pair_at = [&](int ic, int ih, int iwp, bool ok, float (&out)[2]) {
        const bool rin = ok && ic < C && (unsigned)ih < (unsigned)H;
        const SrcT *rp = img + (rin ? ((int64_t)ic * H + ih) * W + iwp : 0);
        out[0] = rin ? image_value(rp, 0) : 0.f;
        out[1] = rin && ic + 1 < C ? image_value(rp, plane) : 0.f;
    };
    // issue chunk c0's loads into v (window columns 0..63 of channels 2p and
    // 2p + 1, one row pair per wave and step), v2 (the two halo columns, spread
    // over all threads) and fw
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = wave + 4 * i;
            const int cp = row / TR, r = row - cp * TR;
            pair_at(c0 + 2 * cp, oh0 - pad + r, iw, cin, v[i]);
        }
#pragma unroll
        for (int i = 0; i < HPT; ++i) {
            const int e = tid + 256 * i;  // (window row pair, halo column)
            const int row = e >> 1, cp = row / TR, r = row - cp * TR;
            const int iwh = ow0 - pad + 64 + (e & 1);
            pair_at(c0 + 2 * cp, oh0 - pad + r, iwh, e < NH && (unsigned)iwh < (unsigned)W, v2[i]);
        }
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int e = tid + 256 * i;  // (pair, tap, o)
            const int cp = e / (9 * OC), t = (e / OC) % 9, o = e % OC;
            const int ic = c0 + 2 * cp;
            const bool ok = e < NW && o < n_oc;
            const uint32_t lo = (ok && ic < C) ? filt[o * ldw + ic * 9 + t] : 0u;
            const uint32_t hi = (ok && ic + 1 < C) ? filt[o * ldw + (ic + 1) * 9 + t] : 0u;
            fw[i] = lo | (hi << 16);
        }
    };
    // two fp32 values -> their bf16 pair (RNE), the first in the low half
    auto packed = [](const float (&x)[2]) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x[0], x[1]}, bf16x2_t));
    };
    float acc[OC][4];
#pragma unroll
    for (int o = 0; o < OC; ++o)
#pragma unroll
        for (int x = 0; x < 4; ++x) acc[o][x] = 0.f;
    load(0);
    for (int c0 = 0; c0 < C; c0 += CT_CC) {
        __syncthreads();  // every wave is done with the previous chunk
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = wave + 4 * i;
            const int cp = row / TR, r = row - cp * TR;
            tile[cp][r][lane] = packed(v[i]);
        }
#pragma unroll
        for (int i = 0; i < HPT; ++i) {
            const int e = tid + 256 * i;
            const int row = e >> 1, cp = row / TR, r = row - cp * TR;
            if (e < NH) tile[cp][r][64 + (e & 1)] = packed(v2[i]);
        }
#pragma unroll
        for (int i = 0; i < WPT; ++i)
            if (tid + 256 * i < NW) (&wts[0][0][0])[tid + 256 * i] = fw[i];
        __syncthreads();
        if (c0 + CT_CC < C) load(c0 + CT_CC);  // in flight under this chunk's multiplies
#pragma unroll
        for (int cp = 0; cp < CP; ++cp) {  // pairs past C hold zeros
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const uint32_t *rp = &tile[cp][ty + kh][tx];
                const uint4 a = *(const uint4 *)rp;
                const uint2 c = *(const uint2 *)(rp + 4);
                const uint32_t x[6] = {a.x, a.y, a.z, a.w, c.x, c.y};
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    uint32_t wv[OC];
                    if constexpr (OC % 4 == 0) {
#pragma unroll
                        for (int o = 0; o < OC; o += 4) *(uint4 *)&wv[o] = *(const uint4 *)&wts[cp][kh * 3 + kw][o];
                    } else {
#pragma unroll
                        for (int o = 0; o < OC; ++o) wv[o] = wts[cp][kh * 3 + kw][o];
                    }
#pragma unroll
                    for (int o = 0; o < OC; ++o)
#pragma unroll
                        for (int px = 0; px < 4; ++px)
                            acc[o][px] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x[px + kw]),
                                                                          __builtin_bit_cast(bf16x2_t, wv[o]),
                                                                          acc[o][px], false);
                }
            }
        }
    }
    const int oh = oh0 + ty, ow = ow0 + tx;
    if (oh >= outH) return;
#pragma unroll
    for (int o = 0; o < OC; ++o) {
        if (o >= n_oc) break;
        const float bv = bias ? bias[o] : 0.f;
        float *drow = dst + (((int64_t)b * n_oc + o) * outH + oh) * outW;
        if (ow + 3 < outW && (((uintptr_t)(drow + ow)) & 15) == 0) {
            *(float4 *)(drow + ow) = make_float4(acc[o][0] + bv, acc[o][1] + bv, acc[o][2] + bv, acc[o][3] + bv);
        } else {
#pragma unroll
            for (int px = 0; px < 4; ++px)
                if (ow + px < outW) drow[ow + px] = acc[o][px] + bv;
        }
    }
}

// dst[i] = src[i] for n16 16-byte words, grid-stride (device-to-device copy of
// resident buffers; also the reference kernel of known traffic, 2 x bytes).
__global__ void __launch_bounds__(256) copy_words16(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                    int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace inv
