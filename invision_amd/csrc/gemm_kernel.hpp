// gemm_kernel.hpp -- bf16 "NT" GEMM for gfx950 (CDNA4) on MFMA 32x32x16.
//
//   Y[m, n] = epilogue( alpha * sum_k X[m, k] * W[n, k]  (+ bias[n]) ) (* colscale[n])  (+ beta * C[m, n])
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
//    past K get an out-of-range offset and also read as zero.  K must be a
//    multiple of 8 and rows 16-byte aligned (the host pads otherwise).
//  * LDS holds each k-tile as rows of BK bf16 (BK/8 chunks of 16 B); chunk c of
//    row r sits in slot c ^ key(r), chosen so that the 16 rows read by any 16
//    consecutive lanes of a ds_read_b128 cover all 64 banks (gfx950 serves a
//    b128 read 16 lanes at a time).
//  * An NST-stage LDS ring: k-tile t+NST-1 is copied while t is multiplied, so
//    a copy has NST-2 k-tiles of MFMA time to land.  One barrier per k-tile.
//  * Fragments are double-buffered in registers: the reads for the next
//    16-wide substep (including the first substep of the next k-tile) are
//    issued under the MFMAs of the current one, so the matrix cores do not wait
//    for LDS after the barrier.
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

#include <type_traits>
#include <utility>

namespace inv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char_t;

// EPI_SWIGLU: the weight holds gate and up rows interleaved in 128-row blocks
// (a 256-row tile = 128 gate rows, then the 128 up rows of the same outputs);
// Y[m][f] = silu(gate + bias) * (up + bias), Y is nout columns wide.
// EPI_ROWBIAS: no activation; p.row_bias[m] is added to row m (a convolution's
// output channel).  Staged epilogue only.
enum EpiKind { EPI_NONE = 0, EPI_SILU = 1, EPI_GELU = 2, EPI_SWIGLU = 3, EPI_ROWBIAS = 4 };
enum OutKind { OUT_F32 = 0, OUT_BF16 = 1 };

struct GemmParams {
    const uint16_t *W;  // [N x ldw] bf16
    const uint16_t *X;  // [M x ldx] bf16
    void *Y;            // [M x ldy] f32 or bf16
    const float *bias;  // [N] or null
    const float *Cin;   // [M x ldc] f32, read when beta != 0
    int64_t ldw, ldx, ldy, ldc;
    int M, N, K;          // K: the reduction length of X (and of W unless it wraps)
    int w_seg_k, Kw;      // W wraps every w_seg_k columns (a multiple of 64; 0: no wrap); Kw: valid K of W
    int tiles_m, tiles_n, group_m;
    int ksplit, kt_per_split;  // split-K: splits, K tiles per split; stream-K: ksplit = persistent grid size
    int sk_dp_tiles;           // stream-K: tiles done one per workgroup (whole rounds) before the balanced phase
    int tile_base, tile_count; // tile grid / split-K: tiles tile_base .. +tile_count-1 of the grouped order (count 0: all)
    float alpha, beta;
    int has_bias, vec_store;
    int nout;             // EPI_SWIGLU: output columns (N = its padded gate+up row count)
    const float *colscale;  // [N] or null: Y = epi(alpha*acc + bias) * colscale[n] (+ beta*C)
    const float *row_bias;  // EPI_ROWBIAS: [M], added to row m with the bias
    float *partial;       // split/stream-K partial sums
    unsigned *counters;   // arrival counters, one per tile, zero between calls
    int ws_cached;        // 0: partial/counters are uncached memory; 1: ordinary (cached) device memory
    // Implicit convolution (the gather instantiations): W is an NHWC bf16 image
    // [cv_H x cv_W x cv_C] and row n of the A operand is output pixel n of the
    // band starting at output row cv_oh0 ((cv_oh0 + n / cv_outW, n % cv_outW));
    // k = ((kh * cv_kW + kw) * cv_C + ic), so a 64-wide k-tile is 64 channels of
    // one filter tap (cv_C % 64 == 0; cv_taps = kH * kW <= 31).  Taps outside
    // the image read zeros.  The image is below 2 GiB (32-bit offsets).
    int cv_H, cv_W, cv_C, cv_outW, cv_kW, cv_taps, cv_stride, cv_pad, cv_oh0;
};

// A unit's arrival at its shared tile (thread 0, after a barrier that follows
// every thread's partial stores and their vmcnt drain); returns how many units
// arrived before it.
//  Uncached workspace: stores bypass every L2 and are in memory once
//  acknowledged, and the loads that read them are issued after this atomic
//  has returned, so a relaxed agent-scope atomic suffices.
//  Cached workspace: a partial may sit dirty in the writer XCD's L2 while the
//  reader runs on another XCD, so the arrival is an acquire-release RMW at
//  agent scope: its release half writes this XCD's L2 back before the
//  increment (cumulative over the workgroup's stores through the barrier), its
//  acquire half invalidates this XCD's caches before the last arriver reads
//  the other units' partials.
__device__ __forceinline__ unsigned tile_arrive(const GemmParams &p, int tile) {
    if (p.ws_cached)
        return __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    return __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Two fp32 values to packed bf16 (low half = a) with v_cvt_pk_bf16_f32:
// round to nearest, ties to even -- bit-identical to f32_to_bf16_rne on every
// bf16 value combined with the low halves 0x0000/0x7FFF/0x8000/0x8001/0xFFFF,
// NaNs and denormals included (checked on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// The epilogue's transcendental functions on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each) instead of the correctly rounded
// library expf / division / erff, whose range reduction and Newton steps cost
// several times more VALU work than the whole rest of the epilogue.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// x * sigmoid(x): a few ulp from the exact value; 0 for x -> -inf, x for x -> +inf.
__device__ __forceinline__ float silu(float x) { return x * rcp_fast(1.0f + exp_fast(-x)); }

// 0.5 x (1 + erf(x / sqrt 2)) with erfc from Abramowitz & Stegun 7.1.26
// (Handbook of Mathematical Functions, |error of erf| <= 1.5e-7):
// erfc(z) ~ t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2), t = 1 / (1 + p z), z >= 0.
// For x < 0 the factor 1 + erf is erfc(|z|) itself, so no cancellation.
__device__ __forceinline__ float gelu_erf(float x) {
    const float z = fabsf(x) * 0.70710678118654752f;
    const float t = rcp_fast(fmaf(0.3275911f, z, 1.0f));
    const float poly =
        t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f), 0.254829592f);
    const float q = poly * exp_fast(-z * z);  // erfc(z)
    return 0.5f * x * (x >= 0.0f ? 2.0f - q : q);
}

template <int EPI>
__device__ __forceinline__ float epilogue_op(float v) {
    if constexpr (EPI == EPI_SILU) {
        return silu(v);
    } else if constexpr (EPI == EPI_GELU) {
        return gelu_erf(v);
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

// Hardware dispatches workgroup b to XCD b % 8.  xcd_remap turns the
// dispatch index into a logical index whose consecutive values share an XCD,
// so that neighbouring tiles (which share X and W panels) meet in one L2.
__device__ __forceinline__ int xcd_remap(int bid, int count) {
    const int per = count >> 3, rem = count & 7;
    const int xcd = bid & 7, local = bid >> 3;
    return (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Logical tile index -> (tm, tn): group_m tile rows, walked column by column.
__device__ __forceinline__ void grouped_tile(int L, int tiles_m, int tiles_n, int group_m, int &tm, int &tn) {
    const int group_size = group_m * tiles_n;
    const int g = L / group_size;
    const int first_m = g * group_m;
    const int gm = min(group_m, tiles_m - first_m);
    const int r = L - g * group_size;
    tm = first_m + r % gm;
    tn = r / gm;
}

// Tile configuration: TN x TM output tile (W rows x X rows), WN x WM waves,
// BK-wide k-tiles, NST LDS stages.
template <int TN_, int TM_, int WN_, int WM_, int BK_, int NST_>
struct TileCfg {
    static constexpr bool REG_STAGED = false;
    static constexpr int BH = 32;  // MFMA block: v_mfma_f32_32x32x16_bf16
    typedef f32x16_t acc_t;
    static constexpr int TN = TN_, TM = TM_, WN = WN_, WM = WM_, BK = BK_, NST = NST_;
    static constexpr int NWAVES = WN * WM;
    static constexpr int NTHREADS = NWAVES * 64;
    static constexpr int WTN = TN / WN;
    static constexpr int WTM = TM / WM;
    static constexpr int FN = WTN / 32;
    static constexpr int FM = WTM / 32;
    static constexpr int SLOTS = BK / 8;      // 16-byte chunks per LDS row
    static constexpr int ROWB = BK * 2;       // bytes per LDS row
    static constexpr int KSUB = BK / 16;      // MFMA k-substeps per k-tile
    static constexpr int A_BYTES = TN * ROWB;
    static constexpr int B_BYTES = TM * ROWB;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = NST * STAGE_BYTES;
    static constexpr int A_LOADS = TN * SLOTS / NTHREADS;
    static constexpr int B_LOADS = TM * SLOTS / NTHREADS;
    static constexpr int LOADS = A_LOADS + B_LOADS;  // buffer_load_dwordx4 per thread per k-tile
    static constexpr int ACC_REGS = FN * FM * 16;
    static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
    static_assert(NST >= 3, "the ring needs the current, the next and one loading stage");
    static_assert(TN % (WN * 32) == 0 && TM % (WM * 32) == 0, "wave tile must be a multiple of 32");
    static_assert((TN * SLOTS) % NTHREADS == 0 && (TM * SLOTS) % NTHREADS == 0, "copies must divide evenly");
    static_assert((NTHREADS / SLOTS) % 16 == 0, "copy rows must advance in multiples of 16");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    static_assert(KSUB % 2 == 0, "register double-buffering alternates over an even substep count");
    // The staged epilogue reads rows of WTN floats with WTN/4 lanes each, so a
    // whole number of rows must fill a wave.
    static constexpr bool STAGED_EPI = NWAVES * 32 * (WTN + 4) * 4 <= LDS_BYTES && 64 % (WTN / 4) == 0;
    static constexpr bool SWIGLU_OK = STAGED_EPI && TN == 256 && WN == 2;  // wave columns = gate | up
};

// Register-staged configuration: TN x TM tile, WN x WM waves, 64-wide k-tiles
// in two LDS buffers filled by ds_write from NREG (1 or 2) register stages of
// global prefetch (see mainloop_rs); MFMA fragments are read PF substeps ahead.
template <int TN_, int TM_, int WN_, int WM_, int NREG_ = 2, int PF_ = 1>
struct RsCfg {
    static constexpr bool REG_STAGED = true;
    static constexpr bool ASINGLE = false;
    static constexpr int BH = 32;  // MFMA block: v_mfma_f32_32x32x16_bf16
    typedef f32x16_t acc_t;
    static constexpr int TN = TN_, TM = TM_, WN = WN_, WM = WM_, BK = 64, NST = 2, NREG = NREG_;
    static constexpr int PF = PF_;  // fragment reads run PF 16-wide substeps ahead of the MFMAs
    static constexpr int NWAVES = WN * WM;
    static constexpr int NTHREADS = NWAVES * 64;
    static constexpr int WTN = TN / WN;
    static constexpr int WTM = TM / WM;
    static constexpr int FN = WTN / 32;
    static constexpr int FM = WTM / 32;
    static constexpr int SLOTS = 8;
    static constexpr int ROWB = 128;
    static constexpr int KSUB = 4;
    static constexpr int A_BYTES = TN * ROWB;
    static constexpr int B_BYTES = TM * ROWB;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
    static constexpr int A_LOADS = TN * SLOTS / NTHREADS;
    static constexpr int B_LOADS = TM * SLOTS / NTHREADS;
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr int ACC_REGS = FN * FM * 16;
    static_assert(TN % (WN * 32) == 0 && TM % (WM * 32) == 0, "wave tile must be a multiple of 32");
    static_assert((TN * SLOTS) % NTHREADS == 0 && (TM * SLOTS) % NTHREADS == 0, "copies must divide evenly");
    static_assert((NTHREADS / SLOTS) % 16 == 0, "copy rows must advance in multiples of 16");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    static_assert(NREG == 1 || NREG == 2, "one or two register stages");
    static_assert(PF == 1 || PF == 2, "fragment prefetch distance 1 or 2 substeps");
    // The staged epilogue reads rows of WTN floats with WTN/4 lanes each, so a
    // whole number of rows must fill a wave.
    static constexpr bool STAGED_EPI = NWAVES * 32 * (WTN + 4) * 4 <= LDS_BYTES && 64 % (WTN / 4) == 0;
    static constexpr bool SWIGLU_OK = STAGED_EPI && TN == 256 && WN == 2;  // wave columns = gate | up
    static_assert(NREG * LOADS - 1 < 64, "vmcnt holds at most 63 outstanding loads");
};

// Register-staged configuration on v_mfma_f32_16x16x32_bf16: 16-row MFMA
// blocks, so a wave tile may be any multiple of 16 (e.g. 128 x 112, whose 224
// accumulator registers leave room that a 128 x 128 tile of 16x16 blocks does
// not).  64-wide k-tiles as RsCfg, each two 32-wide substeps; fragments one
// substep ahead (two register sets).  MFMA blocks of 16 rows give twice the
// operand reads per FLOP of 32x32x16 but a quarter of the accumulator traffic.
//  ASINGLE: the W (A operand) fragments are single-buffered: A fragment i of
//  the next substep is read into the same registers right after the last MFMA
//  of this substep that uses it (i-major order: A[i] is used by FM consecutive
//  MFMAs), while the X fragments, used by every MFMA row, stay double-buffered.
//  That frees FN*4 registers, enough for a second register stage of global
//  prefetch.
template <int TN_, int TM_, int WN_, int WM_, int NREG_ = 1, bool ASINGLE_ = false>
struct Rs16Cfg {
    static constexpr bool REG_STAGED = true;
    static constexpr int BH = 16;  // MFMA block: v_mfma_f32_16x16x32_bf16
    typedef f32x4_t acc_t;
    static constexpr int TN = TN_, TM = TM_, WN = WN_, WM = WM_, BK = 64, NST = 2, NREG = NREG_;
    static constexpr int PF = 1;
    static constexpr bool ASINGLE = ASINGLE_;
    static constexpr int NWAVES = WN * WM;
    static constexpr int NTHREADS = NWAVES * 64;
    static constexpr int WTN = TN / WN;
    static constexpr int WTM = TM / WM;
    static constexpr int FN = WTN / 16;
    static constexpr int FM = WTM / 16;
    static constexpr int SLOTS = 8;
    static constexpr int ROWB = 128;
    static constexpr int KSUB = 2;
    static constexpr int A_BYTES = TN * ROWB;
    static constexpr int B_BYTES = TM * ROWB;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
    static constexpr int A_LOADS = TN * SLOTS / NTHREADS;
    static constexpr int B_LOADS = TM * SLOTS / NTHREADS;
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr int ACC_REGS = FN * FM * 4;
    static_assert(TN % (WN * 16) == 0 && TM % (WM * 16) == 0, "wave tile must be a multiple of 16");
    static_assert((TN * SLOTS) % NTHREADS == 0 && (TM * SLOTS) % NTHREADS == 0, "copies must divide evenly");
    static_assert((NTHREADS / SLOTS) % 16 == 0, "copy rows must advance in multiples of 16");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    static_assert(NREG == 1 || NREG == 2, "one or two register stages");
    static_assert(NREG * LOADS - 1 < 64, "vmcnt holds at most 63 outstanding loads");
    static constexpr bool STAGED_EPI = NWAVES * BH * (WTN + 4) * 4 <= LDS_BYTES && 64 % (WTN / 4) == 0;
    static constexpr bool SWIGLU_OK = STAGED_EPI && TN == 256 && WN == 2;
    static_assert(STAGED_EPI, "16x16 blocks have only the staged epilogue");
};

#if defined(__HIP_DEVICE_COMPILE__)

// LDS slot key of row r (depends on r mod 16 only, so the copy side and the
// fragment side can both compute it from their low row bits); chunk c of row r
// is stored in slot c ^ key(r).
//  8 slots (128-byte rows): key = (r >> 1) & 7.  Measured on gfx950 with the
//    SQ_LDS_BANK_CONFLICT counter over ds_read_b128 of both fragment shapes
//    (32x32x16: rows lane % 32, chunk lane / 32; 16x16x32: rows lane % 16,
//    chunk lane / 16): no conflict cycles for either.  (r + ((r >> 3) & 1)) & 7
//    is conflict-free for the first shape only, r & 7 for the second only.
//  4 slots (64-byte rows): rows r, r+4, r+8, r+12 get 4 different slots.
template <int SLOTS>
__device__ __forceinline__ int slot_key(int r) {
    if constexpr (SLOTS == 8)
        return (r >> 1) & 7;
    else
        return (r >> 2) & 3;
}

// Byte offset of k-tile `ktile` within a row, or an offset past every buffer
// (reads as zeros) when the chunk is not valid.
template <int BK>
__device__ __forceinline__ uint32_t k_byte_offset(bool valid, int ktile) {
    return valid ? (uint32_t)(ktile * BK) * 2 : 0x80000000u;
}

// Global -> LDS copies of one k-tile: A_LOADS + B_LOADS buffer_load_dwordx4
// ... lds per lane.  Lane l of wave w writes 16 bytes at LDS position
// (i * NTHREADS + w * 64 + l) * 16 of the stage.
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

// MFMA fragments of one 16-wide k substep: FN row blocks of W, FM of X.
template <class C>
__device__ __forceinline__ void load_frags(const lds_char_t *stage, int a_frag, int b_frag, int coff,
                                           bf16x8_t (&fa)[C::FN], bf16x8_t (&fb)[C::FM]) {
#pragma unroll
    for (int i = 0; i < C::FN; ++i) fa[i] = *(const bf16x8_t *)(stage + a_frag + i * 32 * C::ROWB + coff);
#pragma unroll
    for (int j = 0; j < C::FM; ++j) fb[j] = *(const bf16x8_t *)(stage + b_frag + j * 32 * C::ROWB + coff);
}

// One MFMA of the configuration's block shape: acc += A . B^T over 16 (32x32
// blocks) or 32 (16x16 blocks) k.
template <class C>
__device__ __forceinline__ void mfma_step(typename C::acc_t &acc, const bf16x8_t &a, const bf16x8_t &b) {
    if constexpr (C::BH == 32)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    else
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
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

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// One global->LDS copy (the idx-th of the LOADS copies of a k-tile).
template <class C, int IDX>
__device__ __forceinline__ void issue_copy(__amdgpu_buffer_rsrc_t rsw, __amdgpu_buffer_rsrc_t rsx, lds_char_t *dst,
                                           uint32_t a_base, uint32_t a_step, uint32_t b_base, uint32_t b_step,
                                           uint32_t kadd_a, uint32_t kadd_b) {
    if constexpr (IDX < C::A_LOADS)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, dst + IDX * C::NTHREADS * 16, 16, a_base + IDX * a_step + kadd_a,
                                                 0, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsx, dst + C::A_BYTES + (IDX - C::A_LOADS) * C::NTHREADS * 16, 16,
                                                 b_base + (IDX - C::A_LOADS) * b_step + kadd_b, 0, 0, 0);
}

// Position (in MFMA steps of a k-tile) after which copy i is issued: the
// The fragment read issued at step r of a substep, for the next substep: A
// fragment i as i >= 0, B fragment j as -1 - j.  Reads go in the order the next
// substep's MFMAs (i-major) first use them -- A0, B0 .. B(FM-1), A1 .. A(FN-1) --
// so each has most of a substep of MFMAs to land before it is needed.
#ifndef INV_READ_FIRST_USE
#define INV_READ_FIRST_USE 1
#endif
template <class C>
constexpr int frag_read(int r) {
    if constexpr (!INV_READ_FIRST_USE) return r < C::FN ? r : -1 - (r - C::FN);
    if (r == 0) return 0;
    if (r <= C::FM) return -r;  // B fragment r - 1
    return r - C::FM;
}

// The MFMA step after which copy i of a k-tile is issued.  Early issue (one
// copy per MFMA from the first step) gives each load the full NST-2 k-tiles
// to land; the spread form distributes them evenly over the k-tile.
#ifndef INV_COPY_SPREAD
#define INV_COPY_SPREAD 0
#endif
template <class C>
constexpr int copy_step(int i) {
    constexpr int T = C::KSUB * C::FN * C::FM;
    if constexpr (INV_COPY_SPREAD) return ((2 * i + 1) * T) / (2 * C::LOADS);
    return C::LOADS <= T ? i : (i * T) / C::LOADS;
}
#endif  // __HIP_DEVICE_COMPILE__

enum GridMode { GRID_TILES = 0, GRID_SPLITK = 1, GRID_STREAMK = 2 };
// Launch mode only: a tile grid whose A operand is gathered from an NHWC image
// (implicit convolution; per-row bias epilogue, fp32 output).
constexpr int LAUNCH_GATHER = 3;

#if defined(__HIP_DEVICE_COMPILE__)

// How a work unit's accumulators become output: directly (the unit is a whole
// tile), or through the partial-sum workspace when several units share a tile
// (split-K: ksplit equal K ranges; stream-K: the ranges cut by the persistent
// workgroups' shares of the global k-iteration space).
struct UnitFix {
    int tile;     // tile id (counter index)
    int rel_tile; // stream-K: tile index within the balanced phase
    int nseg;     // units sharing the tile (1: direct)
    int my_seg;   // this unit's position among them, in K order
    int g_first;  // stream-K: workgroup owning segment 0
    int G, KT;    // stream-K: grid size, k-tiles per tile
    int64_t I;    // stream-K: total k-iterations
};

// Start of stream-K workgroup g's share of [0, I).
__device__ __forceinline__ int64_t sk_start(int64_t g, int64_t I, int64_t G) { return g * I / G; }

// Workspace slot of segment `seg` of a shared tile.  Split-K: one slot per
// (tile, split).  Stream-K: each workgroup owns two slots, one for the first
// and one for the last unit of its share (only those two can be partial).
template <int MODE, class C>
__device__ __forceinline__ float *unit_slot(const GemmParams &p, const UnitFix &f, int seg) {
    constexpr int64_t SZ = (int64_t)C::NTHREADS * C::ACC_REGS;
    if constexpr (MODE == GRID_SPLITK) {
        return p.partial + ((int64_t)(f.tile - p.tile_base) * f.nseg + seg) * SZ;
    } else {
        const int64_t g = f.g_first + seg;
        const bool starts_before = sk_start(g, f.I, f.G) < (int64_t)f.rel_tile * f.KT;
        return p.partial + (2 * g + (starts_before ? 1 : 0)) * SZ;
    }
}

// The LDS-ring main loop: direct global->LDS copies into an NST-stage ring,
// k-tiles [kt_begin, kt_end) accumulated into acc.
template <class C>
__device__ __forceinline__ void mainloop_ring(const GemmParams &p, lds_char_t *lds, __amdgpu_buffer_rsrc_t rsw,
                                              __amdgpu_buffer_rsrc_t rsx, int kt_begin, int kt_end,
                                              f32x16_t (&acc)[C::FN][C::FM]) {
    constexpr int BK = C::BK;
    constexpr int NST = C::NST;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave / C::WM;
    const int wm = wave % C::WM;

    // Copy-side lane constants: position q = i*NTHREADS + tid of a tile is row
    // q / SLOTS, slot q % SLOTS, and holds chunk slot ^ key(row); the row
    // advances by NTHREADS/SLOTS (a multiple of 16) per i, so the chunk is the
    // same for every i.
    const int ld_row = tid / C::SLOTS;
    const int ld_chunk = (tid % C::SLOTS) ^ slot_key<C::SLOTS>(ld_row);
    const uint32_t a_base = (uint32_t)(ld_row * p.ldw * 2 + ld_chunk * 16);
    const uint32_t b_base = (uint32_t)(ld_row * p.ldx * 2 + ld_chunk * 16);
    constexpr int ROWS_PER_LOAD = C::NTHREADS / C::SLOTS;
    const uint32_t a_step = (uint32_t)(ROWS_PER_LOAD * p.ldw * 2);
    const uint32_t b_step = (uint32_t)(ROWS_PER_LOAD * p.ldx * 2);

    // Fragment-side lane constants: lane reads row (lane & 31) of each 32-row
    // block, logical chunk 2*kk + (lane >> 5), stored at slot chunk ^ key(row).
    const int frow = lane & 31;
    const int fh = lane >> 5;
    const int fkey = slot_key<C::SLOTS>(frow);
    const int a_frag = (wn * C::WTN + frow) * C::ROWB;
    const int b_frag = C::A_BYTES + (wm * C::WTM + frow) * C::ROWB;
    int coff[C::KSUB];
#pragma unroll
    for (int kk = 0; kk < C::KSUB; ++kk) coff[kk] = ((2 * kk + fh) ^ fkey) * 16;

    // K-tile cursors.  The copy of a k-tile at or past kt_end gets out-of-range
    // offsets for every lane: it writes zeros and reads nothing, which keeps the
    // ring uniform (every iteration issues exactly one k-tile of copies).
    // W may wrap along K (split-precision passes reuse the resident weight):
    // its k-tile index runs modulo the segment length, tracked incrementally.
    const int wseg = p.w_seg_k / BK;  // W k-tiles per wrap segment (0: no wrap)
    int load_kt = kt_begin;
    int load_ktw = wseg ? kt_begin % wseg : kt_begin;

    // Prologue: k-tiles 0 .. NST-2 in flight; wait for the first, read its
    // first substep.
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) {
        const bool in = load_kt < kt_end;
        issue_tile_loads<C>(rsw, rsx, lds + s * C::STAGE_BYTES, wave, a_base, a_step, b_base, b_step,
                            k_byte_offset<BK>(in && load_ktw * BK + ld_chunk * 8 < p.Kw, load_ktw),
                            k_byte_offset<BK>(in && load_kt * BK + ld_chunk * 8 < p.K, load_kt));
        ++load_kt;
        load_ktw = (wseg && load_ktw + 1 == wseg) ? 0 : load_ktw + 1;
    }
    wait_vmcnt<(NST - 2) * C::LOADS>();
    __syncthreads();

    bf16x8_t fa0[C::FN], fb0[C::FM], fa1[C::FN], fb1[C::FM];
    load_frags<C>(lds, a_frag, b_frag, coff[0], fa0, fb0);

    int stage = 0;
    for (int kt = kt_begin; kt < kt_end; ++kt) {
        // k-tiles t+1 .. t+NST-2 are in flight; t+1 must have landed, everywhere.
        wait_vmcnt<(NST - 3) * C::LOADS>();
        __syncthreads();
        // The stage of t-1 is free now (every wave passed the barrier after
        // finishing t-1): this k-tile's copies fill it with k-tile t+NST-1.
        const int load_stage = (stage == 0) ? NST - 1 : stage - 1;
        lds_char_t *cdst = lds + load_stage * C::STAGE_BYTES + wave * 1024;
        const bool in = load_kt < kt_end;
        const uint32_t kadd_a = k_byte_offset<BK>(in && load_ktw * BK + ld_chunk * 8 < p.Kw, load_ktw);
        const uint32_t kadd_b = k_byte_offset<BK>(in && load_kt * BK + ld_chunk * 8 < p.K, load_kt);
        ++load_kt;
        load_ktw = (wseg && load_ktw + 1 == wseg) ? 0 : load_ktw + 1;
        const lds_char_t *cur = lds + stage * C::STAGE_BYTES;
        const int next_stage = (stage + 1 == NST) ? 0 : stage + 1;
        const lds_char_t *nxt = lds + next_stage * C::STAGE_BYTES;

        // The k-tile as a fixed instruction order: step q of substep ks is one
        // MFMA of substep ks, one fragment read of substep ks+1 (or of substep 0
        // of the next k-tile), and a copy if one is due; sched_barrier pins it.
        static_for<C::KSUB>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            bf16x8_t(&ca)[C::FN] = (ks % 2 == 0) ? fa0 : fa1;
            bf16x8_t(&cb)[C::FM] = (ks % 2 == 0) ? fb0 : fb1;
            bf16x8_t(&na)[C::FN] = (ks % 2 == 0) ? fa1 : fa0;
            bf16x8_t(&nb)[C::FM] = (ks % 2 == 0) ? fb1 : fb0;
            const lds_char_t *rs = (ks + 1 < C::KSUB) ? cur : nxt;
            const int rc = coff[(ks + 1) % C::KSUB];
            static_for<C::FN * C::FM>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                constexpr int i = q / C::FM, j = q % C::FM;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ca[i], cb[j], acc[i][j], 0, 0, 0);
                if constexpr (q < C::FN + C::FM) {
                    constexpr int fr = frag_read<C>(q);
                    if constexpr (fr >= 0)
                        na[fr] = *(const bf16x8_t *)(rs + a_frag + fr * 32 * C::ROWB + rc);
                    else
                        nb[-1 - fr] = *(const bf16x8_t *)(rs + b_frag + (-1 - fr) * 32 * C::ROWB + rc);
                }
                // every copy whose slot is this step (several when LOADS exceeds the MFMA count)
                static_for<C::LOADS>([&](auto cc) {
                    constexpr int ci = decltype(cc)::value;
                    if constexpr (copy_step<C>(ci) == ks * C::FN * C::FM + q)
                        issue_copy<C, ci>(rsw, rsx, cdst, a_base, a_step, b_base, b_step, kadd_a, kadd_b);
                });
                __builtin_amdgcn_sched_barrier(0);
            });
            // reads left over when a substep has more fragments than MFMAs
            static_for<(C::FN + C::FM > C::FN * C::FM) ? C::FN + C::FM - C::FN * C::FM : 0>([&](auto rc2) {
                constexpr int fr = frag_read<C>(C::FN * C::FM + decltype(rc2)::value);
                if constexpr (fr >= 0)
                    na[fr] = *(const bf16x8_t *)(rs + a_frag + fr * 32 * C::ROWB + rc);
                else
                    nb[-1 - fr] = *(const bf16x8_t *)(rs + b_frag + (-1 - fr) * 32 * C::ROWB + rc);
            });
        });
        stage = next_stage;
    }
    // The copies of the k-tiles past the end still write LDS; let them land
    // before the ring is reused or the workgroup retires.
    wait_vmcnt<0>();
}

// The register-staged main loop (RsCfg): 64-wide k-tiles, two LDS buffers.
// K-tile t (counted from kt_begin) is loaded into registers during iteration
// t-1-NREG, written to LDS buffer t % 2 during iteration t-1 and multiplied in
// iteration t, so each global load has NREG k-tiles of MFMA time to land; each
// wave's loads cover whole 128-byte lines (8 lanes per row).  Per iteration,
// for every copy chunk c: wait until chunk c of tile t+1 has landed
// (NREG*LOADS-1 younger loads may be outstanding), ds_write it, and reuse its
// registers for chunk c of tile t+1+NREG.  One barrier per iteration, early in
// the last substep: it publishes tile t+1's LDS buffer and retires every read
// of tile t's, so the next iteration may overwrite it.
template <class C, bool GATHER = false>
__device__ __forceinline__ void mainloop_rs(const GemmParams &p, lds_char_t *lds, __amdgpu_buffer_rsrc_t rsw,
                                            __amdgpu_buffer_rsrc_t rsx, int kt_begin, int kt_end,
                                            typename C::acc_t (&acc)[C::FN][C::FM], int n0 = 0) {
    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
    constexpr int BK = C::BK, ROWB = C::ROWB, SLOTS = C::SLOTS;
    constexpr int AL = C::A_LOADS, L = C::LOADS;
    constexpr int RPL = C::NTHREADS / SLOTS;  // rows covered by one copy chunk
    constexpr int T = C::FN * C::FM;         // MFMAs per substep
    constexpr int NR = C::FN + C::FM;        // fragment reads per substep
    // MFMA block geometry: a lane reads 16 bytes (8 k) of row lane % BH of each
    // block; the 64 / BH lane groups take consecutive 8-k chunks, so a substep
    // covers CPS chunks (16 k for 32x32x16, 32 k for 16x16x32).
    constexpr int BH = C::BH;
    constexpr int CPS = 64 / BH;
    static_assert(C::KSUB * CPS == SLOTS, "the substeps cover the 64-wide k-tile");
    constexpr int BAR = 1;                   // MFMA step of the last substep after which the barrier sits
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave / C::WM;
    const int wm = wave % C::WM;

    // Copy side: lane reads global chunk ld_chunk (k offset 8 * ld_chunk) of
    // rows ld_row + RPL*i and stores it at slot ld_chunk ^ key(row); the key
    // depends on the row mod 16 only, so it is the same for every i.
    const int ld_row = tid / SLOTS;
    const int ld_chunk = tid % SLOTS;
    const int wr_off = ld_row * ROWB + ((ld_chunk ^ slot_key<SLOTS>(ld_row)) * 16);
    const uint32_t a_base = (uint32_t)(ld_row * p.ldw * 2 + ld_chunk * 16);
    const uint32_t b_base = (uint32_t)(ld_row * p.ldx * 2 + ld_chunk * 16);
    const uint32_t a_step = (uint32_t)(RPL * p.ldw * 2);
    const uint32_t b_step = (uint32_t)(RPL * p.ldx * 2);

    // Fragment side: lane reads row (lane % BH) of each block, logical chunk
    // CPS*kk + lane / BH, stored at slot chunk ^ key(row) (the key depends on
    // the row mod 16, the same for every block).
    const int frow = lane & (BH - 1);
    const int fh = lane / BH;
    const int fkey = slot_key<SLOTS>(frow);
    const int a_frag = (wn * C::WTN + frow) * ROWB;
    const int b_frag = C::A_BYTES + (wm * C::WTM + frow) * ROWB;
    int coff[C::KSUB];
#pragma unroll
    for (int kk = 0; kk < C::KSUB; ++kk) coff[kk] = ((CPS * kk + fh) ^ fkey) * 16;

    const int wseg = p.w_seg_k / BK;
    int load_kt = kt_begin;
    int load_ktw = wseg ? kt_begin % wseg : kt_begin;
    // Gather: for each A copy chunk, the byte offset of its pixel's window
    // origin (ih0, iw0) plus the chunk's 16 bytes, and a mask of the taps that
    // land inside the image (bit kh * cv_kW + kw; none for a pixel past N).
    // The next k-tile is tap g_tap (byte offset g_tapoff from the origin),
    // channel block g_cb; bit 31 is never set, so g_bit = 31 loads zeros.
    int g_base[GATHER ? AL : 1];
    unsigned g_mask[GATHER ? AL : 1];
    int g_cb = 0, g_tap = 0, g_kw = 0, g_tapoff = 0, g_bit = 0;
    if constexpr (GATHER) {
#pragma unroll
        for (int c = 0; c < AL; ++c) {
            const int n = n0 + ld_row + c * RPL;
            const int oh = p.cv_oh0 + n / p.cv_outW, ow = n % p.cv_outW;
            const int ih0 = oh * p.cv_stride - p.cv_pad, iw0 = ow * p.cv_stride - p.cv_pad;
            unsigned cols = 0, m = 0;
            for (int kw = 0; kw < p.cv_kW; ++kw) cols |= ((unsigned)(iw0 + kw) < (unsigned)p.cv_W) << kw;
            for (int kh = 0, t = 0; t < p.cv_taps; ++kh, t += p.cv_kW)
                if ((unsigned)(ih0 + kh) < (unsigned)p.cv_H) m |= cols << t;
            g_mask[c] = n < p.N ? m : 0u;
            g_base[c] = n < p.N ? (ih0 * p.cv_W + iw0) * p.cv_C * 2 + ld_chunk * 16 : 0;
        }
    }
    // Offsets of the next k-tile to load (out of range, i.e. zeros, past kt_end
    // or K).  Gather (tile grids, kt_begin = 0): ka is the tap's byte offset
    // from the window origin plus the channel block's, g_bit the tap's mask bit.
    auto next_kadd = [&](uint32_t &ka, uint32_t &kb) {
        const bool in = load_kt < kt_end;
        if constexpr (GATHER) {
            g_bit = in ? g_tap : 31;
            ka = (uint32_t)(g_tapoff + g_cb * BK * 2);
            if (++g_cb == p.cv_C / BK) {
                g_cb = 0;
                ++g_tap;
                if (++g_kw == p.cv_kW) {
                    g_kw = 0;
                    g_tapoff += (p.cv_W - p.cv_kW + 1) * p.cv_C * 2;
                } else {
                    g_tapoff += p.cv_C * 2;
                }
            }
        } else {
            ka = k_byte_offset<BK>(in && load_ktw * BK + ld_chunk * 8 < p.Kw, load_ktw);
        }
        kb = k_byte_offset<BK>(in && load_kt * BK + ld_chunk * 8 < p.K, load_kt);
        ++load_kt;
        load_ktw = (wseg && load_ktw + 1 == wseg) ? 0 : load_ktw + 1;
    };
    auto gload = [&](int cidx, uint32_t ka, uint32_t kb) -> u32x4_t {
        if (cidx < AL) {
            if constexpr (GATHER) {
                const uint32_t off = ((g_mask[cidx] >> g_bit) & 1u) ? (uint32_t)g_base[cidx] + ka : 0x80000000u;
                return __builtin_amdgcn_raw_buffer_load_b128(rsw, off, 0, 0);
            }
            return __builtin_amdgcn_raw_buffer_load_b128(rsw, a_base + cidx * a_step + ka, 0, 0);
        }
        return __builtin_amdgcn_raw_buffer_load_b128(rsx, b_base + (cidx - AL) * b_step + kb, 0, 0);
    };
    auto lds_chunk = [&](lds_char_t *buf, int cidx) -> u32x4_t * {
        return (u32x4_t *)(buf + (cidx < AL ? 0 : C::A_BYTES) + wr_off + (cidx < AL ? cidx : cidx - AL) * RPL * ROWB);
    };

    u32x4_t R0[L], R1[C::NREG == 2 ? L : 1];
    lds_char_t *buf0 = lds;
    lds_char_t *buf1 = lds + C::STAGE_BYTES;

    // Prologue: tile 0 to LDS buffer 0; the next NREG tiles in registers
    // (tile 1 in R1 and tile 2 in R0 with two stages, tile 1 in R0 with one).
    {
        uint32_t ka, kb;
        next_kadd(ka, kb);
#pragma unroll
        for (int c = 0; c < L; ++c) R0[c] = gload(c, ka, kb);
        if constexpr (C::NREG == 2) {
            next_kadd(ka, kb);
#pragma unroll
            for (int c = 0; c < L; ++c) R1[c] = gload(c, ka, kb);
        }
        next_kadd(ka, kb);
#pragma unroll
        for (int c = 0; c < L; ++c) {
            *lds_chunk(buf0, c) = R0[c];
            R0[c] = gload(c, ka, kb);
        }
    }
    __syncthreads();

    // Fragment buffers: the reads for substep s+PF are issued under the MFMAs
    // of substep s (PF = 1: two buffers alternating; PF = 2: one per substep).
    constexpr int PF = C::PF;
    constexpr int NB = (PF == 1) ? 2 : C::KSUB;
    constexpr bool AS = C::ASINGLE;
    static_assert(!AS || PF == 1, "single-buffered A fragments are read one substep ahead");
    constexpr int NBA = AS ? 1 : NB;
    bf16x8_t fa[NBA][C::FN], fb[NB][C::FM];
    static_for<PF>([&](auto sc) {
        constexpr int s0 = decltype(sc)::value;
#pragma unroll
        for (int i = 0; i < C::FN; ++i) fa[s0][i] = *(const bf16x8_t *)(buf0 + a_frag + i * BH * ROWB + coff[s0]);
#pragma unroll
        for (int j = 0; j < C::FM; ++j) fb[s0][j] = *(const bf16x8_t *)(buf0 + b_frag + j * BH * ROWB + coff[s0]);
    });
    // The barrier precedes the first read of the next tile (substep KSUB-PF);
    // the ds_writes of the next tile all come before it.
    constexpr int BSUB = C::KSUB - PF;

    // One iteration: multiply the tile in `cur` while moving register stage R
    // (tile t+1) into `nxt` and refilling R with tile t+1+NREG.
    auto iteration = [&](const lds_char_t *cur, lds_char_t *nxt, u32x4_t(&R)[L]) {
        uint32_t ka, kb;
        next_kadd(ka, kb);
        static_for<C::KSUB>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            constexpr int cb_i = ks % NB;               // buffer of this substep
            constexpr int rd = ks + PF;                 // substep whose fragments are read now
            constexpr int nb_i = rd % NB;
            const lds_char_t *rs = (rd < C::KSUB) ? cur : nxt;
            const int rc = coff[rd % C::KSUB];
            static_for<T>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                constexpr int i = q / C::FM, j = q % C::FM;
                mfma_step<C>(acc[i][j], fa[AS ? 0 : cb_i][i], fb[cb_i][j]);
                if constexpr (ks == BSUB && q == BAR) __syncthreads();
                if constexpr (AS && j == C::FM - 1) {
                    // the last use of A fragment i in this substep: read the next
                    // substep's into the same registers (after the barrier in the
                    // last substep, as i * FM + FM - 1 > BAR)
                    static_assert(!(ks == BSUB) || C::FM - 1 > BAR, "A reads of the next tile follow the barrier");
                    fa[0][i] = *(const bf16x8_t *)(rs + a_frag + i * BH * ROWB + rc);
                }
                // fragment reads for substep rd (the X fragments only, with AS)
                static_for<NR>([&](auto rc2) {
                    constexpr int r = decltype(rc2)::value;
                    constexpr int at = (ks == BSUB) ? BAR + 1 + (r * (T - BAR - 1)) / NR : (r * T) / NR;
                    if constexpr (at == q) {
                        constexpr int fr = frag_read<C>(r);
                        if constexpr (fr >= 0) {
                            if constexpr (!AS) fa[nb_i][fr] = *(const bf16x8_t *)(rs + a_frag + fr * BH * ROWB + rc);
                        } else {
                            fb[nb_i][-1 - fr] = *(const bf16x8_t *)(rs + b_frag + (-1 - fr) * BH * ROWB + rc);
                        }
                    }
                });
                // copy chunks: ds_write tile t+1, reload the registers with tile t+1+NREG
                if constexpr (ks < BSUB) {
                    static_for<L>([&](auto cc) {
                        constexpr int cidx = decltype(cc)::value;
                        constexpr int at = ((2 * cidx + 1) * BSUB * T) / (2 * L);
                        if constexpr (at == ks * T + q) {
                            wait_vmcnt<C::NREG * L - 1>();
                            *lds_chunk(nxt, cidx) = R[cidx];
                            R[cidx] = gload(cidx, ka, kb);
                        }
                    });
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    };

    const int n = kt_end - kt_begin;
    if constexpr (C::NREG == 2) {
        // The register stage alternates, so iterations go in pairs.
        int t = 0;
        for (; t + 1 < n; t += 2) {
            iteration(buf0, buf1, R1);
            iteration(buf1, buf0, R0);
        }
        if (t < n) iteration(buf0, buf1, R1);
    } else {
        lds_char_t *cur = buf0, *nxt = buf1;
        for (int t = 0; t < n; ++t) {
            iteration(cur, nxt, R0);
            lds_char_t *tmp = cur;
            cur = nxt;
            nxt = tmp;
        }
    }
    wait_vmcnt<0>();
}

// Epilogue through LDS.  The MFMA accumulator layout gives each lane 4
// consecutive n of one row m, so direct stores write 32 bytes into each of 32
// rows per instruction.  Instead, each wave writes one 32-row block of its
// accumulators (times alpha) to its own LDS region, rows padded by 16 bytes
// (conflict-free for the 16-lane phases of ds_write_b128), and reads them back
// row-major: WTN/4 lanes per row, so every store covers whole row segments of
// 4*WTN (fp32) or 2*WTN (bf16) bytes.  beta*C, bias and the activation are
// applied on the row-major side, where their loads are contiguous too.
// BETA is a template parameter so that the common beta == 0 path has no loads
// among the stores: loads and stores share vmcnt, and a wait for a load that
// may have been issued also waits for every store before it.
// Requires the ring to be idle (a barrier first) and NWAVES*32*(WTN+4)*4 bytes.
//
// Shared tiles (split-K / stream-K) go through the same row loop:
//  SK_PUBLISH: the staged rows (alpha * acc) are written to the unit's
//              workspace slot instead of Y, no epilogue;
//  SK_FINISH:  the rows are the sum, in unit (K) order, of every unit's slot
//              (this unit's own included), then the epilogue as usual.
// A slot holds each wave's 32-row blocks row-major: float index
// ((wave * FM + j) * 32 + row) * WTN + col, so both sides move whole rows and
// the accumulators are never touched by VALU adds (which would need them in
// VGPRs next to the main loop's registers).
enum { SK_NONE = 0, SK_PUBLISH = 1, SK_FINISH = 2 };

// Stage block column j of a wave's accumulators (every i) as BH rows of WTN
// floats (times alpha) at st: lane holds D[n][m = frow] for 4 consecutive n,
// at n = 8g + 4*fh (32x32 blocks, g = 0..3) or 4*fh (16x16 blocks).
template <class C>
__device__ __forceinline__ void stage_block(__attribute__((address_space(3))) float *st,
                                            const typename C::acc_t (&acc)[C::FN][C::FM], int j, int lane,
                                            float alpha) {
    constexpr int SROW = C::WTN + 4;
    const int frow = lane & (C::BH - 1);
    const int fh = lane / C::BH;
    typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
        if constexpr (C::BH == 32) {
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *(lds_f32x4_t *)(st + frow * SROW + i * 32 + 8 * g + 4 * fh) =
                    f32x4_t{alpha * acc[i][j][4 * g], alpha * acc[i][j][4 * g + 1], alpha * acc[i][j][4 * g + 2],
                            alpha * acc[i][j][4 * g + 3]};
        } else {
            *(lds_f32x4_t *)(st + frow * SROW + i * 16 + 4 * fh) =
                f32x4_t{alpha * acc[i][j][0], alpha * acc[i][j][1], alpha * acc[i][j][2], alpha * acc[i][j][3]};
        }
    }
}

template <class C, int EPI, int OUT, bool BETA, int SKM = SK_NONE, int MODE = 0>
__device__ __forceinline__ void store_tile_staged(const GemmParams &p, lds_char_t *lds,
                                                  const typename C::acc_t (&acc)[C::FN][C::FM], int m0, int n0,
                                                  int wn, int wm, int lane, int wave, const UnitFix *fix = nullptr,
                                                  float *slot = nullptr) {
    typedef __attribute__((address_space(3))) float lds_float_t;
    constexpr int BH = C::BH;              // rows of an MFMA block (32 or 16)
    constexpr int SROW = C::WTN + 4;       // staged row pitch in floats
    constexpr int LPR = C::WTN / 4;        // lanes per row on the read side
    constexpr int RPI = 64 / LPR;          // rows per read instruction
    static_assert(LPR * RPI == 64 && BH % RPI == 0, "whole rows per wave-wide read");
    lds_float_t *st = (lds_float_t *)lds + wave * BH * SROW;
    const int col = (lane % LPR) * 4;
    const int rsub = lane / LPR;
    const int n = n0 + wn * C::WTN + col;
    const bool nvec = p.vec_store && n + 3 < p.N;
    float bv[4] = {0.f, 0.f, 0.f, 0.f}, sc[4] = {1.f, 1.f, 1.f, 1.f};
    if (SKM != SK_PUBLISH && p.has_bias) {
        if (n + 3 < p.N) {
            const f32x4_t t = *(const f32x4_t *)(p.bias + n);  // bias is 16-byte aligned, n % 4 == 0
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = t[e];
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = (n + e < p.N) ? p.bias[n + e] : 0.f;
        }
    }
    if (SKM != SK_PUBLISH && p.colscale) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = (n + e < p.N) ? p.colscale[n + e] : 0.f;
    }
    // EPI_ROWBIAS: the bias of every row this lane stores, loaded here so
    // that no load sits among the stores.
    constexpr int NIT = BH / RPI;
    constexpr bool RB = EPI == EPI_ROWBIAS;
    float rb[RB ? C::FM : 1][RB ? NIT : 1];
    if constexpr (RB) {
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int m = m0 + wm * C::WTM + j * BH + it * RPI + rsub;
                rb[j][it] = (SKM != SK_PUBLISH && m < p.M) ? p.row_bias[m] : 0.f;
            }
    }

    // The bias has landed before the first store: a later wait for it would
    // also wait for every store issued before it.
    wait_vmcnt<0>();
    __syncthreads();  // every wave has finished with the ring
#pragma unroll
    for (int j = 0; j < C::FM; ++j) {
        f32x4_t t[NIT];
        const int64_t slot_off = ((int64_t)(wave * C::FM + j) * BH + rsub) * C::WTN + col;
        if constexpr (SKM == SK_FINISH) {
            for (int sp = 0; sp < fix->nseg; ++sp) {
                const float *src = unit_slot<MODE, C>(p, *fix, sp) + slot_off;
                f32x4_t u[NIT];
#pragma unroll
                for (int it = 0; it < NIT; ++it)
                    u[it] = __builtin_nontemporal_load((const f32x4_t *)(src + it * RPI * C::WTN));
#pragma unroll
                for (int it = 0; it < NIT; ++it) t[it] = (sp == 0) ? u[it] : t[it] + u[it];
            }
        } else {
            stage_block<C>(st, acc, j, lane, p.alpha);
            // LDS operations of one wave execute in order: the reads below see the
            // writes above, and the next block's writes follow these reads.  All
            // reads (and C loads) of the block are issued before any store, so the
            // stores are never behind a wait.
#pragma unroll
            for (int it = 0; it < NIT; ++it)
                t[it] = *(const __attribute__((address_space(3))) f32x4_t *)(st + (it * RPI + rsub) * SROW + col);
        }
        if constexpr (SKM == SK_PUBLISH) {
#pragma unroll
            for (int it = 0; it < NIT; ++it) *(f32x4_t *)(slot + slot_off + it * RPI * C::WTN) = t[it];
            continue;
        }
        if constexpr (RB) {
#pragma unroll
            for (int it = 0; it < NIT; ++it) t[it] += rb[j][it];
        }
        const int mrow = m0 + wm * C::WTM + j * BH + rsub;  // row of it = 0; it adds RPI rows
        if (nvec && mrow + (NIT - 1) * RPI < p.M) {
            // every row of this lane in range, 16-byte aligned: no branches
            f32x4_t cv[BETA ? NIT : 1];
            if constexpr (BETA) {
#pragma unroll
                for (int it = 0; it < NIT; ++it)
                    cv[it] = *(const f32x4_t *)(p.Cin + (int64_t)(mrow + it * RPI) * p.ldc + n);
            }
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = epilogue_op<EPI>(t[it][e] + bv[e]) * sc[e];
                    if constexpr (BETA) v[e] += p.beta * cv[it][e];
                }
                const int64_t off = (int64_t)(mrow + it * RPI) * p.ldy + n;
                if constexpr (OUT == OUT_F32) {
                    *reinterpret_cast<f32x4_t *>((float *)p.Y + off) = f32x4_t{v[0], v[1], v[2], v[3]};
                } else {
                    u32x2_t packed;
                    packed[0] = pack_bf16x2(v[0], v[1]);
                    packed[1] = pack_bf16x2(v[2], v[3]);
                    *reinterpret_cast<u32x2_t *>((uint16_t *)p.Y + off) = packed;
                }
            }
        } else {
            // edge tiles and unaligned outputs: element-wise bounds
            for (int it = 0; it < NIT; ++it) {
                const int m = mrow + it * RPI;
                if (m >= p.M) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = epilogue_op<EPI>(t[it][e] + bv[e]) * sc[e];
                if constexpr (BETA) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) v[e] += p.beta * p.Cin[(int64_t)m * p.ldc + n + e];
                }
                if constexpr (OUT == OUT_F32) {
                    float *y = (float *)p.Y + (int64_t)m * p.ldy + n;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) y[e] = v[e];
                } else {
                    uint16_t *y = (uint16_t *)p.Y + (int64_t)m * p.ldy + n;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) y[e] = f32_to_bf16_rne(v[e]);
                }
            }
        }
    }
}

// Direct epilogue (configurations whose LDS cannot hold the staging area).
// Lane holds D[n = 8g + 4*fh + e][m = frow] of each 32x32 block; for each (i, j)
// a lane's four g stores cover 32 bytes of row m and the two lane halves the
// row's whole 128-byte segment, issued back to back so the L2 merges them.
template <class C, int EPI, int OUT, bool BETA>
__device__ __forceinline__ void store_tile_direct(const GemmParams &p, const f32x16_t (&acc)[C::FN][C::FM], int m0,
                                                  int n0, int wn, int wm, int lane) {
    const int frow = lane & 31;
    const int fh = lane >> 5;
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
        const int nb = n0 + wn * C::WTN + i * 32 + 4 * fh;
        float bv[4][4], sc[4][4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = nb + 8 * g;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bv[g][e] = 0.f;
                sc[g][e] = p.colscale ? ((n + e < p.N) ? p.colscale[n + e] : 0.f) : 1.f;
            }
            if (p.has_bias) {
                if (n + 3 < p.N) {
                    f32x4_t t = *(const f32x4_t *)(p.bias + n);  // bias is 16-byte aligned, n % 4 == 0
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[g][e] = t[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[g][e] = (n + e < p.N) ? p.bias[n + e] : 0.f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < C::FM; ++j) {
            const int m = m0 + wm * C::WTM + j * 32 + frow;
            if (m >= p.M) continue;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = nb + 8 * g;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = epilogue_op<EPI>(p.alpha * acc[i][j][4 * g + e] + bv[g][e]) * sc[g][e];
                if constexpr (BETA) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) v[e] += p.beta * p.Cin[(int64_t)m * p.ldc + n + e];
                }
                if constexpr (OUT == OUT_F32) {
                    float *y = (float *)p.Y + (int64_t)m * p.ldy + n;
                    if (p.vec_store && n + 3 < p.N) {
                        *reinterpret_cast<f32x4_t *>(y) = f32x4_t{v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < p.N) y[e] = v[e];
                    }
                } else {
                    uint16_t *y = (uint16_t *)p.Y + (int64_t)m * p.ldy + n;
                    if (p.vec_store && n + 3 < p.N) {
                        u32x2_t packed;
                        packed[0] = pack_bf16x2(v[0], v[1]);
                        packed[1] = pack_bf16x2(v[2], v[3]);
                        *reinterpret_cast<u32x2_t *>(y) = packed;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < p.N) y[e] = f32_to_bf16_rne(v[e]);
                    }
                }
            }
        }
    }
}

// SwiGLU epilogue (QNNSiluMul over two projections, src/quicknncpu.pas:2404-
// 2418, fused).  Wave column wn = 0 holds the gate rows of the tile, wn = 1 the
// up rows of the same outputs: both stage each 32-row block in LDS, then each
// wave of the pair finishes half of the block's rows,
//   Y[m][f] = silu(alpha*gate + bg) * (alpha*up + bu),  f = n0/2 + col,
// with the exact SiLU v / (1 + exp(-v)).  Needs SWIGLU_OK and beta == 0.
template <class C, int OUT>
__device__ __forceinline__ void store_tile_swiglu(const GemmParams &p, lds_char_t *lds,
                                                  const typename C::acc_t (&acc)[C::FN][C::FM], int m0, int n0,
                                                  int wn, int wm, int lane, int wave) {
    static_assert(C::SWIGLU_OK, "SwiGLU needs 256-row tiles split over two wave columns");
    typedef __attribute__((address_space(3))) float lds_float_t;
    constexpr int BH = C::BH;
    constexpr int SROW = C::WTN + 4;
    constexpr int LPR = C::WTN / 4;   // 32 lanes per staged row
    constexpr int RPI = 64 / LPR;     // 2 rows per read instruction
    constexpr int HALF = BH / 2;      // rows of a block finished by each wave of the pair
    constexpr int NIT = HALF / RPI;
    lds_float_t *own = (lds_float_t *)lds + wave * BH * SROW;
    const lds_float_t *gst = (const lds_float_t *)lds + (0 * C::WM + wm) * BH * SROW;  // gate wave of this row band
    const lds_float_t *ust = (const lds_float_t *)lds + (1 * C::WM + wm) * BH * SROW;  // up wave
    const int col = (lane % LPR) * 4;
    const int rsub = lane / LPR;
    const int f = n0 / 2 + col;  // output column
    const bool fvec = p.vec_store && f + 3 < p.nout;
    float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.has_bias) {  // interleaved like the rows: gate bias at n0 + col, up bias at n0 + 128 + col
        const f32x4_t g4 = *(const f32x4_t *)(p.bias + n0 + col);
        const f32x4_t u4 = *(const f32x4_t *)(p.bias + n0 + C::WTN + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            bg[e] = g4[e];
            bu[e] = u4[e];
        }
    }
    wait_vmcnt<0>();
    __syncthreads();  // every wave has finished with the ring
#pragma unroll
    for (int j = 0; j < C::FM; ++j) {
        stage_block<C>(own, acc, j, lane, p.alpha);
        __syncthreads();  // the pair's gate and up blocks are both staged
        f32x4_t gv[NIT], uv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int r = wn * HALF + it * RPI + rsub;
            gv[it] = *(const __attribute__((address_space(3))) f32x4_t *)(gst + r * SROW + col);
            uv[it] = *(const __attribute__((address_space(3))) f32x4_t *)(ust + r * SROW + col);
        }
        const int mrow = m0 + wm * C::WTM + j * BH + wn * HALF + rsub;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int m = mrow + it * RPI;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float gt = gv[it][e] + bg[e];
                v[e] = silu(gt) * (uv[it][e] + bu[e]);
            }
            if (m >= p.M) continue;
            const int64_t off = (int64_t)m * p.ldy + f;
            if (fvec) {
                if constexpr (OUT == OUT_F32)
                    *reinterpret_cast<f32x4_t *>((float *)p.Y + off) = f32x4_t{v[0], v[1], v[2], v[3]};
                else
                    *reinterpret_cast<u32x2_t *>((uint16_t *)p.Y + off) =
                        u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
                for (int e = 0; e < 4; ++e) {
                    if (f + e >= p.nout) break;
                    if constexpr (OUT == OUT_F32)
                        ((float *)p.Y)[off + e] = v[e];
                    else
                        ((uint16_t *)p.Y)[off + e] = f32_to_bf16_rne(v[e]);
                }
            }
        }
        __syncthreads();  // both waves have read the block before the next one is staged
    }
}

// One work unit: output tile (tm, tn), k-tiles [kt_begin, kt_end).
template <class C, int EPI, int OUT, int MODE, bool GATHER = false>
__device__ __forceinline__ void gemm_unit(const GemmParams &p, char *smem, int tm, int tn, int kt_begin, int kt_end,
                                          const UnitFix &fix) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave / C::WM;
    const int wm = wave % C::WM;
    const int m0 = tm * C::TM;
    const int n0 = tn * C::TN;

    // Buffer resources covering exactly the valid rows of this tile's panels.
    const int rows_w = min(C::TN, p.N - n0);
    const int rows_x = min(C::TM, p.M - m0);
    // gather: the whole NHWC image (an input pixel may belong to any output row of the tile)
    const __amdgpu_buffer_rsrc_t rsw =
        GATHER ? __builtin_amdgcn_make_buffer_rsrc((void *)p.W, 0, (int)((int64_t)p.cv_H * p.cv_W * p.cv_C * 2),
                                                   0x00020000)
               : __builtin_amdgcn_make_buffer_rsrc((void *)(p.W + (int64_t)n0 * p.ldw), 0,
                                                   (int)((int64_t)rows_w * p.ldw * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.X + (int64_t)m0 * p.ldx), 0, (int)((int64_t)rows_x * p.ldx * 2), 0x00020000);

    lds_char_t *lds = (lds_char_t *)smem;

    typename C::acc_t acc[C::FN][C::FM];
    constexpr int ACC_ELEMS = C::BH * C::BH / 64;  // accumulator registers per block and lane
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
#pragma unroll
            for (int r = 0; r < ACC_ELEMS; ++r) acc[i][j][r] = 0.0f;

    if constexpr (C::REG_STAGED)
        mainloop_rs<C, GATHER>(p, lds, rsw, rsx, kt_begin, kt_end, acc, n0);
    else
        mainloop_ring<C>(p, lds, rsw, rsx, kt_begin, kt_end, acc);


    if constexpr (MODE != GRID_TILES && C::STAGED_EPI && EPI != EPI_SWIGLU) {
        if (fix.nseg > 1) {
            // Park this unit's partial rows; the last arriving unit of the tile
            // sums every unit's rows in K order and finishes the tile.
            store_tile_staged<C, EPI, OUT, false, SK_PUBLISH, MODE>(p, lds, acc, m0, n0, wn, wm, lane, wave, &fix,
                                                                    unit_slot<MODE, C>(p, fix, fix.my_seg));
            // The slot stores are acknowledged before the arrival (tile_arrive).
            wait_vmcnt<0>();
            volatile __attribute__((address_space(3))) unsigned *s_last =
                (volatile __attribute__((address_space(3))) unsigned *)lds;
            __syncthreads();  // every wave's staging reads and slot stores are done
            if (tid == 0) {
                const unsigned prev = tile_arrive(p, fix.tile);
                *s_last = (prev == (unsigned)(fix.nseg - 1)) ? 1u : 0u;
            }
            __syncthreads();
            const bool last = *s_last != 0;
            __syncthreads();  // everyone has read the flag before the ring is reused
            if (!last) return;
            if (p.beta != 0.0f)
                store_tile_staged<C, EPI, OUT, true, SK_FINISH, MODE>(p, lds, acc, m0, n0, wn, wm, lane, wave, &fix);
            else
                store_tile_staged<C, EPI, OUT, false, SK_FINISH, MODE>(p, lds, acc, m0, n0, wn, wm, lane, wave, &fix);
            if (tid == 0)  // ready for the next call
                __hip_atomic_store(&p.counters[fix.tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    } else if constexpr (MODE != GRID_TILES && C::BH == 32) {
        if (fix.nseg > 1) {
            // Park this unit's partial sums, then let the last arriving unit of
            // the tile finish it.
            float *mine = unit_slot<MODE, C>(p, fix, fix.my_seg);
#pragma unroll
            for (int i = 0; i < C::FN; ++i)
#pragma unroll
                for (int j = 0; j < C::FM; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                     acc[i][j][4 * g + 3]};
                        *(f32x4_t *)(mine + ((((i * C::FM + j) * 4 + g) * C::NTHREADS + tid) * 4)) = v;
                    }
            // The partial stores are acknowledged before the arrival (tile_arrive).
            wait_vmcnt<0>();
            // The flag lives in the (now idle) ring: the barrier below completes
            // every wave's LDS reads and partial stores before thread 0 acts.
            volatile __attribute__((address_space(3))) unsigned *s_last =
                (volatile __attribute__((address_space(3))) unsigned *)lds;
            __syncthreads();
            if (tid == 0) {
                const unsigned prev = tile_arrive(p, fix.tile);
                *s_last = (prev == (unsigned)(fix.nseg - 1)) ? 1u : 0u;
            }
            __syncthreads();
            const bool last = *s_last != 0;
            __syncthreads();  // everyone has read the flag before the ring is reused
            if (!last) return;
            // Sum the partials in K order (this unit's own included, read back)
            // so the result does not depend on which unit arrived last.  The
            // segment loop is outermost so each segment's loads issue together.
            // Plain loads: the barrier above orders them after the counter, and
            // each slot is uncached and written once per launch.
            for (int sp = 0; sp < fix.nseg; ++sp) {
                const float *src = unit_slot<MODE, C>(p, fix, sp);
#pragma unroll
                for (int i = 0; i < C::FN; ++i) {
                    // one fragment row at a time: FM*4 loads in flight, then the adds
                    f32x4_t v[C::FM * 4];
#pragma unroll
                    for (int q = 0; q < C::FM * 4; ++q)
                        v[q] = __builtin_nontemporal_load(
                            (const f32x4_t *)(src + (((i * C::FM * 4 + q) * C::NTHREADS + tid) * 4)));
#pragma unroll
                    for (int q = 0; q < C::FM * 4; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[i][q >> 2][4 * (q & 3) + e] =
                                (sp == 0) ? v[q][e] : acc[i][q >> 2][4 * (q & 3) + e] + v[q][e];
                }
            }
            if (tid == 0)  // ready for the next call
                __hip_atomic_store(&p.counters[fix.tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    if constexpr (EPI == EPI_SWIGLU) {
        store_tile_swiglu<C, OUT>(p, lds, acc, m0, n0, wn, wm, lane, wave);
    } else if constexpr (C::STAGED_EPI) {
        if (p.beta != 0.0f)
            store_tile_staged<C, EPI, OUT, true>(p, lds, acc, m0, n0, wn, wm, lane, wave);
        else
            store_tile_staged<C, EPI, OUT, false>(p, lds, acc, m0, n0, wn, wm, lane, wave);
    } else if (p.beta != 0.0f) {
        store_tile_direct<C, EPI, OUT, true>(p, acc, m0, n0, wn, wm, lane);
    } else {
        store_tile_direct<C, EPI, OUT, false>(p, acc, m0, n0, wn, wm, lane);
    }
}

#endif  // __HIP_DEVICE_COMPILE__

// The body is compiled only in the device pass: the host pass needs just the
// launch stub, and buffer-resource types do not exist for the host target.
//  GRID_TILES:   one workgroup per output tile (tiles tile_base ..
//                tile_base + tile_count - 1 of the grouped order when
//                tile_count > 0).
//  GRID_SPLITK:  ksplit workgroups per tile (of the same range), equal K ranges.
//  GRID_STREAMK: a persistent grid of G workgroups.  The first sk_dp_tiles
//                tiles (whole rounds) go one per workgroup; then workgroup g
//                takes k-iterations [g*I/G, (g+1)*I/G) of the I = (remaining
//                tiles) * KT, in tile order, so every workgroup ends together.
template <class C, int EPI, int OUT, int MODE, bool GATHER = false>
__global__ void __launch_bounds__(C::NTHREADS, 1) gemm_nt_bf16_kernel(const GemmParams p) {
    static_assert(!GATHER || (C::REG_STAGED && MODE == GRID_TILES), "the gather loader is register-staged, tiles only");
#if defined(__HIP_DEVICE_COMPILE__)
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const int ntiles = p.tiles_m * p.tiles_n;
    const int nt = p.tile_count > 0 ? p.tile_count : ntiles;  // tiles of this launch, from p.tile_base
    const int KT = (p.K + C::BK - 1) / C::BK;
    int tm, tn;
    if constexpr (MODE == GRID_TILES) {
        grouped_tile(p.tile_base + xcd_remap(blockIdx.x, nt), p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        UnitFix fix{};
        fix.nseg = 1;
        gemm_unit<C, EPI, OUT, MODE, GATHER>(p, smem, tm, tn, 0, KT, fix);
    } else if constexpr (MODE == GRID_SPLITK) {
        // Logical units in split-major order, remapped so that consecutive ones
        // share an XCD: the m-tiles of one n-tile and one K range then run on one
        // XCD and its L2 fetches their W panel slice once.
        const int L = xcd_remap(blockIdx.x, nt * p.ksplit);
        const int split = L / nt;
        const int tile = p.tile_base + (L - split * nt);
        grouped_tile(tile, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        UnitFix fix{};
        fix.tile = tile;
        fix.nseg = p.ksplit;
        fix.my_seg = split;
        const int kt_begin = split * p.kt_per_split;
        gemm_unit<C, EPI, OUT, MODE>(p, smem, tm, tn, kt_begin, min(KT, kt_begin + p.kt_per_split), fix);
    } else {
        const int G = gridDim.x;
        const int g = xcd_remap(blockIdx.x, G);
        // Whole rounds first, one tile per workgroup (compact in L2, no
        // partial sums), then the remaining tiles' k-iterations in equal
        // shares.  One loop with one call site keeps a single copy of the unit
        // body (two copies spill registers).
        const int t0 = p.sk_dp_tiles;
        const int64_t I = (int64_t)(ntiles - t0) * KT;
        int dp_tile = g;
        int64_t it = sk_start(g, I, G);
        const int64_t end = sk_start(g + 1, I, G);
        while (true) {
            UnitFix fix{};
            int tile, klo, khi;
            if (dp_tile < t0) {
                tile = dp_tile;
                klo = 0;
                khi = KT;
                fix.nseg = 1;
                dp_tile += G;
            } else if (it < end) {
                const int rt = (int)(it / KT);  // tile index within the balanced phase
                tile = t0 + rt;
                klo = (int)(it - (int64_t)rt * KT);
                khi = (int)min((int64_t)KT, (int64_t)klo + (end - it));
                it += khi - klo;
                fix.tile = tile;
                fix.rel_tile = rt;
                fix.G = G;
                fix.KT = KT;
                fix.I = I;
                // Workgroups whose shares meet this tile: the first is the one
                // whose share contains iteration rt*KT, the last the one
                // containing (rt+1)*KT - 1 (largest g with g*I/G <= x is
                // ceil((x+1)G/I) - 1).
                const int64_t x0 = (int64_t)rt * KT, x1 = (int64_t)(rt + 1) * KT - 1;
                const int g_first = (int)(((x0 + 1) * G + I - 1) / I - 1);
                const int g_last = (int)(((x1 + 1) * G + I - 1) / I - 1);
                fix.g_first = g_first;
                fix.nseg = g_last - g_first + 1;
                fix.my_seg = g - g_first;
            } else {
                break;
            }
            grouped_tile(tile, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
            gemm_unit<C, EPI, OUT, MODE>(p, smem, tm, tn, klo, khi, fix);
            __syncthreads();  // the next unit's prologue overwrites the ring
        }
    }
#endif  // __HIP_DEVICE_COMPILE__
}

}  // namespace inv
