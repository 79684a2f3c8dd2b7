// gemm_kernel.hpp -- bf16 "NT" GEMM for gfx950 (CDNA4) on MFMA 32x32x16.
//
//   Y[m, n] = epilogue( alpha * sum_k X[m, k] * W[n, k]  (+ bias[n])  (+ beta * C[m, n]) )
//
// X [M x K] and W [N x K] are bf16, row-major, K contiguous (the layout of the
// reference's QNNLinear: cblas_gemm(RowMajor, NoTrans, Trans, ...),
// src/quicknncpu.pas:1807-1828).  Accumulation is fp32 in the matrix cores.
//
// Mapping onto the hardware
//  * The MFMA A operand is the W tile (rows n) and the B operand is the X tile
//    (rows m), so the 32x32 accumulator of a lane holds 4 consecutive n for one
//    m: the epilogue writes Y with one 16-byte store per 4 outputs.
//  * Global -> LDS uses buffer_load_dwordx4 ... lds (no VGPR staging).  Each
//    workgroup addresses its W and X row panels through a buffer resource whose
//    size ends at the last valid row, so rows past M or N read as zero; chunks
//    past K are given an out-of-range offset and also read as zero.  K must be
//    a multiple of 8 and rows 16-byte aligned (the host pads otherwise).
//  * LDS holds each tile as rows of 64 bf16 (8 chunks of 16 B); chunk c of row
//    r is stored in slot c ^ key(r) (row_slot_key), so the rows read by
//    consecutive lanes of a ds_read_b128 fall in different bank groups.
//  * Two LDS stages: the loads of k-tile t+1 run while k-tile t is multiplied.
//  * Workgroups are remapped so that the tiles resident on one XCD (hardware
//    dispatches workgroup b to XCD b % 8) form a compact block of the output,
//    which keeps the shared X and W panels in that XCD's L2.
//  * Split-K: each (tile, split) workgroup multiplies a K range; all but the
//    last to finish park fp32 partials in a workspace; the last one sums the
//    partials in split order (deterministic), applies the epilogue and resets
//    the tile counter for the next call.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace inv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char_t;

enum EpiKind { EPI_NONE = 0, EPI_SILU = 1, EPI_GELU = 2 };
enum OutKind { OUT_F32 = 0, OUT_BF16 = 1 };

struct GemmParams {
    const uint16_t *W;  // [N x ldw] bf16
    const uint16_t *X;  // [M x ldx] bf16
    void *Y;            // [M x ldy] f32 or bf16
    const float *bias;  // [N] or null
    const float *Cin;   // [M x ldc] f32, read when beta != 0
    int64_t ldw, ldx, ldy, ldc;
    int M, N, K;  // K: the reduction length of X (and of W unless it wraps)
    int w_seg_tiles, Kw;  // W wraps every w_seg_tiles k-tiles (0: no wrap); Kw: valid K of W
    int tiles_m, tiles_n, group_m;
    int ksplit, kt_per_split;  // K tiles per split
    float alpha, beta;
    int has_bias, vec_store;
    int swizzle;  // LDS slot permutation: 0 -> row & 7, 1 -> (row + row/8) & 7
    float *partial;       // split-K workspace: [tiles][ksplit][threads][acc regs]
    unsigned *counters;   // split-K arrival counters, one per tile, zero between calls
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int EPI>
__device__ __forceinline__ float epilogue_op(float v) {
    if constexpr (EPI == EPI_SILU) {
        return v / (1.0f + expf(-v));
    } else if constexpr (EPI == EPI_GELU) {
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
    } else {
        return v;
    }
}

// s_waitcnt with vmcnt(n) and no wait on the other counters (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup id -> output tile, XCD-aware and grouped along m.
__device__ __forceinline__ void tile_coords(int bid, int ntiles, int tiles_m, int group_m, int &tm, int &tn) {
    // Undo the round-robin XCD dispatch: consecutive logical ids share an XCD.
    const int per = ntiles >> 3, rem = ntiles & 7;
    const int xcd = bid & 7, local = bid >> 3;
    int L = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    // Grouped order: group_m tile rows, walked column by column.
    const int tiles_n = ntiles / tiles_m;
    const int group_size = group_m * tiles_n;
    const int g = L / group_size;
    const int first_m = g * group_m;
    const int gm = min(group_m, tiles_m - first_m);
    const int r = L - g * group_size;
    tm = first_m + r % gm;
    tn = r / gm;
}

template <int TN, int TM, int WN, int WM>
struct TileCfg {
    static constexpr int BK = 64;
    static constexpr int NWAVES = WN * WM;
    static constexpr int NTHREADS = NWAVES * 64;
    static constexpr int WTN = TN / WN;
    static constexpr int WTM = TM / WM;
    static constexpr int FN = WTN / 32;
    static constexpr int FM = WTM / 32;
    static constexpr int A_BYTES = TN * BK * 2;
    static constexpr int B_BYTES = TM * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
    static constexpr int A_LOADS = TN * 8 / NTHREADS;
    static constexpr int B_LOADS = TM * 8 / NTHREADS;
    static constexpr int ACC_REGS = FN * FM * 16;
    static_assert(TN % (WN * 32) == 0 && TM % (WM * 32) == 0, "wave tile must be a multiple of 32");
    static_assert((TN * 8) % NTHREADS == 0 && (TM * 8) % NTHREADS == 0, "loads must divide evenly");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
};

#if defined(__HIP_DEVICE_COMPILE__)
// Global -> LDS copies of one k-tile: A_LOADS + B_LOADS buffer_load_dwordx4
// ... lds per lane.  Lane l of wave w writes 16 bytes at LDS position
// (i * NTHREADS + w * 64 + l) * 16 of the stage; `kadd` is the k offset in
// bytes, or 0x80000000 to make every lane read out of range (zeros).
template <class C>
__device__ __forceinline__ void issue_tile_loads(__amdgpu_buffer_rsrc_t rsw, __amdgpu_buffer_rsrc_t rsx,
                                                 lds_char_t *stage, int wave, uint32_t a_base, uint32_t a_step,
                                                 uint32_t b_base, uint32_t b_step, uint32_t kadd_a,
                                                 uint32_t kadd_b) {
    lds_char_t *sa = stage + wave * 1024;
    lds_char_t *sb = sa + C::A_BYTES;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, sa + i * C::NTHREADS * 16, 16, a_base + i * a_step + kadd_a,
                                                 0, 0, 0);
#pragma unroll
    for (int i = 0; i < C::B_LOADS; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsx, sb + i * C::NTHREADS * 16, 16, b_base + i * b_step + kadd_b,
                                                 0, 0, 0);
}

// Per-row key of the LDS slot permutation: chunk c of row r lives in slot
// c ^ key(r).  key = r & 7 spreads any 8 consecutive rows over the 8 16-byte
// slots of a 128-byte row (conflict-free when 8 lanes share 32 banks); key =
// (r + r/8) & 7 also spreads the even and the odd rows of any aligned 16-row
// window (conflict-free when 16 lanes share 64 banks).  Depends on r mod 16 only.
__device__ __forceinline__ int row_slot_key(int r, int mode) {
    return mode ? ((r + (r >> 3)) & 7) : (r & 7);
}

// Byte offset of k-tile `ktile` in a row, or an offset past every buffer
// (reads as zeros) when the chunk is not valid.
__device__ __forceinline__ uint32_t k_byte_offset(bool valid, int ktile) {
    return valid ? (uint32_t)(ktile * 64) * 2 : 0x80000000u;
}

// MFMA fragments of one 16-wide k substep: FN rows blocks of W, FM of X.
template <class C>
__device__ __forceinline__ void load_frags(const lds_char_t *sbase, int a_frag, int b_frag, int coff,
                                           bf16x8_t (&fa)[C::FN], bf16x8_t (&fb)[C::FM]) {
#pragma unroll
    for (int i = 0; i < C::FN; ++i) fa[i] = *(const bf16x8_t *)(sbase + a_frag + i * 32 * C::BK * 2 + coff);
#pragma unroll
    for (int j = 0; j < C::FM; ++j) fb[j] = *(const bf16x8_t *)(sbase + b_frag + j * 32 * C::BK * 2 + coff);
}

template <class C>
__device__ __forceinline__ void mfma_block(f32x16_t (&acc)[C::FN][C::FM], const bf16x8_t (&fa)[C::FN],
                                           const bf16x8_t (&fb)[C::FM]) {
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
}

#endif  // __HIP_DEVICE_COMPILE__

// The body is compiled only in the device pass: the host pass needs just the
// launch stub, and buffer-resource types do not exist for the host target.
template <int TN, int TM, int WN, int WM, int EPI, int OUT, bool SPLIT>
__global__ void __launch_bounds__(256, 1) gemm_nt_bf16_kernel(const GemmParams p) {
#if defined(__HIP_DEVICE_COMPILE__)
    using C = TileCfg<TN, TM, WN, WM>;
    constexpr int BK = C::BK;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave / WM;
    const int wm = wave % WM;

    const int ntiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    int split = 0;
    if constexpr (SPLIT) {
        split = bid % p.ksplit;
        bid = bid / p.ksplit;
    }
    int tm, tn;
    tile_coords(bid, ntiles, p.tiles_m, p.group_m, tm, tn);
    const int m0 = tm * TM;
    const int n0 = tn * TN;

    const int KT = (p.K + BK - 1) / BK;
    int kt_begin = 0, kt_end = KT;
    if constexpr (SPLIT) {
        kt_begin = split * p.kt_per_split;
        kt_end = min(KT, kt_begin + p.kt_per_split);
    }

    // Buffer resources covering exactly the valid rows of this tile's panels.
    const int rows_w = min(TN, p.N - n0);
    const int rows_x = min(TM, p.M - m0);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.W + (int64_t)n0 * p.ldw), 0, (int)((int64_t)rows_w * p.ldw * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.X + (int64_t)m0 * p.ldx), 0, (int)((int64_t)rows_x * p.ldx * 2), 0x00020000);

    // Per-lane global offsets.  Position q = i*NTHREADS + tid of the tile maps to
    // row q/8 and LDS slot q%8; the chunk loaded there is slot ^ (row & 7).  With
    // NTHREADS a multiple of 64 the chunk is the same for every i.
    const int ld_chunk = (tid & 7) ^ row_slot_key(tid >> 3, p.swizzle);
    const int ld_row = tid >> 3;
    const uint32_t a_base = (uint32_t)(ld_row * p.ldw * 2 + ld_chunk * 16);
    const uint32_t b_base = (uint32_t)(ld_row * p.ldx * 2 + ld_chunk * 16);
    constexpr int ROWS_PER_LOAD = C::NTHREADS / 8;
    const uint32_t a_step = (uint32_t)(ROWS_PER_LOAD * p.ldw * 2);
    const uint32_t b_step = (uint32_t)(ROWS_PER_LOAD * p.ldx * 2);

    lds_char_t *lds = (lds_char_t *)smem;

    f32x16_t acc[C::FN][C::FM];
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Fragment addressing: lane reads row (lane & 31) of each 32-row block,
    // logical chunk 2*kk + (lane >> 5), stored at slot chunk ^ (row & 7).
    const int frow = lane & 31;
    const int fh = lane >> 5;
    const int fsw = row_slot_key(frow, p.swizzle);
    const int a_frag = (wn * C::WTN + frow) * (BK * 2);
    const int b_frag = C::A_BYTES + (wm * C::WTM + frow) * (BK * 2);
    int coff[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) coff[kk] = (((2 * kk + fh) ^ fsw) * 16);

    // A k-tile at or past kt_end gets out-of-range offsets for every lane, so
    // its copy writes zeros and reads nothing; the prefetch of the next tile
    // is then unconditional and the loop body stays one basic block.
    // W may wrap along K (split-precision passes reuse the resident weight):
    // its k-tile index runs modulo w_seg_tiles, tracked incrementally.
    int ktw = p.w_seg_tiles ? kt_begin % p.w_seg_tiles : kt_begin;
    {
        const bool in = kt_begin < kt_end;
        issue_tile_loads<C>(rsw, rsx, lds, wave, a_base, a_step, b_base, b_step,
                            k_byte_offset(in && ktw * BK + ld_chunk * 8 < p.Kw, ktw),
                            k_byte_offset(in && kt_begin * BK + ld_chunk * 8 < p.K, kt_begin));
    }

    for (int kt = kt_begin; kt < kt_end; ++kt) {
        const int stage = (kt - kt_begin) & 1;
        wait_vmcnt<0>();
        __syncthreads();
        {
            const int kn = kt + 1;
            ktw = (p.w_seg_tiles && ktw + 1 == p.w_seg_tiles) ? 0 : ktw + 1;
            const bool in = kn < kt_end;
            issue_tile_loads<C>(rsw, rsx, lds + (stage ^ 1) * C::STAGE_BYTES, wave, a_base, a_step, b_base, b_step,
                                k_byte_offset(in && ktw * BK + ld_chunk * 8 < p.Kw, ktw),
                                k_byte_offset(in && kn * BK + ld_chunk * 8 < p.K, kn));
        }

        const lds_char_t *sbase = lds + stage * C::STAGE_BYTES;
        bf16x8_t fa0[C::FN], fb0[C::FM], fa1[C::FN], fb1[C::FM], fa2[C::FN], fb2[C::FM], fa3[C::FN], fb3[C::FM];
        load_frags<C>(sbase, a_frag, b_frag, coff[0], fa0, fb0);
        load_frags<C>(sbase, a_frag, b_frag, coff[1], fa1, fb1);
        mfma_block<C>(acc, fa0, fb0);
        load_frags<C>(sbase, a_frag, b_frag, coff[2], fa2, fb2);
        mfma_block<C>(acc, fa1, fb1);
        load_frags<C>(sbase, a_frag, b_frag, coff[3], fa3, fb3);
        mfma_block<C>(acc, fa2, fb2);
        mfma_block<C>(acc, fa3, fb3);
        // Schedule: the fragments of substeps 0 and 1 first, then each group of
        // MFMAs interleaved with the fragment reads two substeps ahead.
        constexpr int NF = C::FN + C::FM;  // ds_reads per substep
        constexpr int NM = C::FN * C::FM;  // MFMAs per substep
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NF, 0);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, NM / NF > 0 ? NM / NF : 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * NM, 0);
    }
    // The final (all out-of-range) prefetch still writes LDS; let it land
    // before the workgroup can retire.
    wait_vmcnt<0>();

    if constexpr (SPLIT) {
        // Park this split's partial sums, then let the last arriving split finish.
        float *mine = p.partial + ((int64_t)bid * p.ksplit + split) * (C::NTHREADS * C::ACC_REGS);
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
#pragma unroll
            for (int j = 0; j < C::FM; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    *(f32x4_t *)(mine + ((((i * C::FM + j) * 4 + g) * C::NTHREADS + tid) * 4)) = v;
                }
        __shared__ unsigned s_last;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (tid == 0) {
            unsigned prev = __hip_atomic_fetch_add(&p.counters[bid], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            s_last = (prev == (unsigned)(p.ksplit - 1)) ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // Sum the partials in split order so the result does not depend on
        // which split arrived last.
        const float *base = p.partial + (int64_t)bid * p.ksplit * (C::NTHREADS * C::ACC_REGS);
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
#pragma unroll
            for (int j = 0; j < C::FM; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4_t s = {0.f, 0.f, 0.f, 0.f};
                    for (int sp = 0; sp < p.ksplit; ++sp) {
                        f32x4_t v;
                        if (sp == split) {
                            v = f32x4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                        acc[i][j][4 * g + 3]};
                        } else {
                            v = __builtin_nontemporal_load(
                                (const f32x4_t *)(base + (int64_t)sp * (C::NTHREADS * C::ACC_REGS) +
                                                  ((((i * C::FM + j) * 4 + g) * C::NTHREADS + tid) * 4)));
                        }
                        s += v;
                    }
                    acc[i][j][4 * g] = s[0];
                    acc[i][j][4 * g + 1] = s[1];
                    acc[i][j][4 * g + 2] = s[2];
                    acc[i][j][4 * g + 3] = s[3];
                }
        if (tid == 0) p.counters[bid] = 0u;  // ready for the next call
    }

    // Epilogue: lane holds D[n = 8g + 4h + e][m = lane & 31] of each 32x32 block.
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * C::WTN + i * 32 + 8 * g + 4 * fh;
            float bv[4] = {0.f, 0.f, 0.f, 0.f};
            if (p.has_bias) {
                if (n + 3 < p.N) {
                    f32x4_t t = *(const f32x4_t *)(p.bias + n);  // bias is 16-byte aligned, N % 4 == 0 here
                    bv[0] = t[0]; bv[1] = t[1]; bv[2] = t[2]; bv[3] = t[3];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[e] = (n + e < p.N) ? p.bias[n + e] : 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < C::FM; ++j) {
                const int m = m0 + wm * C::WTM + j * 32 + frow;
                if (m >= p.M) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = p.alpha * acc[i][j][4 * g + e];
                if (p.beta != 0.0f) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) v[e] += p.beta * p.Cin[(int64_t)m * p.ldc + n + e];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = epilogue_op<EPI>(v[e] + bv[e]);
                if constexpr (OUT == OUT_F32) {
                    float *y = (float *)p.Y + (int64_t)m * p.ldy + n;
                    if (p.vec_store && n + 3 < p.N) {
                        *(f32x4_t *)y = f32x4_t{v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < p.N) y[e] = v[e];
                    }
                } else {
                    uint16_t *y = (uint16_t *)p.Y + (int64_t)m * p.ldy + n;
                    if (p.vec_store && n + 3 < p.N) {
                        uint2 packed;
                        packed.x = (uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16);
                        packed.y = (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16);
                        *(uint2 *)y = packed;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < p.N) y[e] = f32_to_bf16_rne(v[e]);
                    }
                }
            }
        }
    }
#endif  // __HIP_DEVICE_COMPILE__
}

}  // namespace inv
