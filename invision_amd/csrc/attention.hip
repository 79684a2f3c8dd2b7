// attention.hip -- attention forward on MI355X (gfx950):
//   O[q, h] = sum_j softmax_j(scale * Q[q, h] . K[j, g]) V[j, g],  g = h / (heads / kv_heads)
// for the reference's [tokens x heads*head_dim] layout, one pass over K and V
// with the running max / running sum of the online softmax (the algorithm of
// TQNNSingleOPS.QNNFlashAttentionHeadTiled, src/quicknncpu.pas:2662-2761, on
// MFMA tiles instead of per-row axpy).
//
// Workgroup: 4 waves, 128 queries of one head (32 per wave); key tiles of 64
// staged in LDS (double-buffered, filled one tile ahead by direct
// buffer_load ... lds copies) and shared by the 4 waves; two workgroups per CU,
// so one's softmax VALU work overlaps the other's MFMAs.
// Short sequences (KS = 2): a grid of 128-query blocks leaves CUs idle, and a
// block walks its keys one tile after another, so the block with the most keys
// sets the time.  There the workgroup takes 64 queries, and its 4 waves form
// two key groups of 2 waves: group g takes key tiles g, g + 2, ..., each group
// with its own double buffer, and group 1 hands its running max, sum and O to
// group 0 through LDS at the end, which merges them as the online softmax
// merges tiles.  Twice the workgroups, half the tiles in sequence.
//
// Per wave and key tile, with v_mfma_f32_32x32x16_bf16 (D[n][m] = sum_k A[n][k] B[m][k],
// lane l holding A[l%32][8*(l/32) .. +7] and B[l%32][8*(l/32) .. +7], and output
// register r of lane l at n = 8*(r/4) + 4*(l/32) + r%4, m = l%32):
//  S^T = K Q^T:  A = K-tile rows (keys), B = the wave's Q rows (held in registers
//                for the whole kernel), k = head_dim.  Each lane then holds the
//                scores of ONE query (m = l%32) for 16 keys per 32-key block, so
//                the row max and row sum are lane-local plus one exchange with
//                lane l^32.
//  O^T += V^T P^T: A = V^T (head_dim rows), B = P (bf16) straight from the
//                score registers, k = keys.  For that, the B fragment's 8 k-slots
//                of lane l must be the keys the lane holds; the K tile is stored
//                with rows 4-7 and 8-11 of every 16-row group swapped (`quadswap`),
//                which makes a lane's 8 consecutive score registers exactly keys
//                16c + 8*(l/32) + 0..7, the keys its V^T fragment covers.  No
//                cross-lane shuffle of P is needed.  V stays in the reference's
//                layout (key rows, as K) in HBM and LDS; its V^T fragments come
//                from two ds_read_b64_tr_b16 (4 keys each), so no transposed copy
//                of V is made.
// Softmax runs in the exp2 domain: exp(scale*s - m) = exp2(s*scale*log2e - m'),
// on the hardware exp2; P is rounded to bf16 (nearest-even) for the second MFMA,
// and the row sum is taken over those same bf16 weights (v_dot2_f32_bf16).
#include "attention.hpp"

#include <type_traits>

namespace inv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_t;

#if defined(__HIP_DEVICE_COMPILE__)

// Slot key of a 128-byte LDS row (8 slots of 16 bytes): 16 consecutive rows read
// at one logical slot land on 16 different 16-byte bank groups.
__device__ __forceinline__ int key8(int r) { return (r + ((r >> 3) & 1)) & 7; }

// Physical 16-byte slot of chunk c in row r of a K tile (D/8 chunks per row).
template <int D>
__device__ __forceinline__ int k_slot(int r, int c) {
    if constexpr (D == 128)
        return c ^ (r & 15);  // 256-byte rows: one bank window each
    else
        return c ^ key8(r);
}

// K-tile row r holds key quadswap(r) of the tile: rows 4-7 and 8-11 of every
// 16-row group trade places (an involution).
__device__ __forceinline__ int quadswap(int r) { return (((r >> 2) ^ (r >> 3)) & 1) ? (r ^ 12) : r; }

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// V tile rows (keys) hold D/8 chunks of 16 bytes; chunk c of key row r sits in
// slot c ^ v_swz(r).  The P.V fragments are read with ds_read_b64_tr_b16 from
// 4 key rows at a time (keys 4j..4j+3): the key bits the XOR uses spread each
// read's 8 rows x 4 chunks over every bank in the minimum two passes.
template <int D>
__device__ __forceinline__ int v_swz(int r) {
    if constexpr (D == 128)
        return 4 * (r & 3);
    else
        return 4 * ((r >> 1) & 1);
}

// Hardware dispatches workgroup b to XCD b % 8: the logical index whose
// consecutive values share an XCD, so the query blocks of one head meet its K
// and V in one L2.
__device__ __forceinline__ int xcd_order(int bid, int count) {
    const int per = count >> 3, rem = count & 7;
    const int xcd = bid & 7, local = bid >> 3;
    return (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

#endif  // __HIP_DEVICE_COMPILE__

// The body exists only in the device pass; the host pass needs the launch stub
// (buffer-resource types do not exist for the host target).
// Two workgroups per CU with one key group; with two, each workgroup's stage
// buffers fill most of the LDS and it runs alone.
template <int D, bool CAUSAL, int OUT, int KS>
__global__ void __launch_bounds__(256, KS == 1 ? 2 : 1) attn_fwd_kernel(const AttnParams p) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int WQ = 4 / KS;             // query waves per key group
    constexpr int BQ = 32 * WQ, BK = kAttnBlockK;
    constexpr int NT = 64 * WQ;            // threads of one key group
    static_assert((KS == 1 || KS == 2) && BK == 64, "one or two key groups, 64-key tiles");
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    constexpr int KROW = D * 2;            // bytes per K-tile row
    constexpr int K_BYTES = BK * KROW;     // K tile
    constexpr int V_BYTES = BK * KROW;     // V tile: key rows, as K
    constexpr int STAGE = K_BYTES + V_BYTES;
    constexpr int KCH = D / 8;             // 16-byte chunks per K row
    constexpr int KIT = BK * KCH / NT;     // K copies per thread per tile
    constexpr int VIT = BK * KCH / NT;     // V copies per thread per tile
    constexpr int NC = D / 16;             // 16-wide head_dim steps of S
    constexpr int ND = D / 32;             // 32-row head_dim blocks of O
    constexpr int NX = ND * 16 + 2;        // KS = 2: floats per lane handed from group 1 to group 0
    static_assert(KS == 1 || WQ * NX * 64 * 4 <= KS * 2 * STAGE, "the hand-off fits in the stage buffers");
    __shared__ __attribute__((aligned(1024))) char smem[KS * 2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS copy bases stay scalar
    const int kg = wave / WQ, wq = wave % WQ;                   // key group, query wave within it
    const int gtid = tid % NT;                                  // thread within the key group
    lds_t *lds = (lds_t *)smem + kg * 2 * STAGE;                // the group's double buffer
    const int lq = lane & 31, lh = lane >> 5;
    // 1-D grid of heads x query blocks; causal blocks run longest first.
    const int nqb = (p.seq_q + BQ - 1) / BQ;
    const int L = xcd_order(blockIdx.x, nqb * p.heads);
    const int head = L / nqb;
    const int qb = CAUSAL ? nqb - 1 - L % nqb : L % nqb;
    const int kvh = head / (p.heads / p.kv_heads);
    const int q0 = qb * BQ;
    const int my_q = q0 + wq * 32 + lq;

    // This wave's Q rows as the B operand of S^T = K Q^T (zero past seq_q).
    bf16x8_t qf[NC];
    {
        const bool ok = my_q < p.seq_q;
        const uint16_t *qrow = p.Q + (int64_t)(ok ? my_q : 0) * p.ldq + head * D + 8 * lh;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const u32x4_t v = ok ? *(const u32x4_t *)(qrow + 16 * c) : u32x4_t{0u, 0u, 0u, 0u};
            qf[c] = __builtin_bit_cast(bf16x8_t, v);
        }
    }

    // K and V rows of kv head kvh: the buffer ranges end with key seq_k - 1, so
    // the rows of a partial last tile read as zeros.
    const __amdgpu_buffer_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.K + kvh * D), 0, (int)(((int64_t)(p.seq_k - 1) * p.ldk + D) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.V + kvh * D), 0, (int)(((int64_t)(p.seq_k - 1) * p.ldv + D) * 2), 0x00020000);

    // Global -> LDS copies (buffer_load ... lds): copy i of group thread gtid fills
    // the 16-byte LDS slot i*NT + gtid of its tile, so each thread fetches the chunk
    // that belongs there -- the swizzle and the K row order live in these
    // global offsets.  K slot s: row n = s / KCH holds key quadswap(n), physical
    // chunk s % KCH holds logical chunk (s % KCH) ^ swizzle(n).  V slot s: row
    // n = s / KCH holds key n, physical chunk s % KCH logical chunk (s % KCH) ^ v_swz(n).
    uint32_t k_goff[KIT], v_goff[VIT];
#pragma unroll
    for (int i = 0; i < KIT; ++i) {
        const int sl = i * NT + gtid, n = sl / KCH;
        k_goff[i] = (uint32_t)(quadswap(n) * p.ldk * 2 + k_slot<D>(n, sl % KCH) * 16);
    }
#pragma unroll
    for (int i = 0; i < VIT; ++i) {
        const int sl = i * NT + gtid, n = sl / KCH;
        v_goff[i] = (uint32_t)(n * p.ldv * 2 + ((sl % KCH) ^ v_swz<D>(n)) * 16);
    }
    const uint32_t k_tile_step = (uint32_t)(BK * p.ldk * 2), v_tile_step = (uint32_t)(BK * p.ldv * 2);
    auto load_tile = [&](int kt, lds_t *st) {
        lds_t *wk = st + wq * 64 * 16;
#pragma unroll
        for (int i = 0; i < KIT; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsk, wk + i * NT * 16, 16, k_goff[i] + kt * k_tile_step, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < VIT; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsv, wk + K_BYTES + i * NT * 16, 16, v_goff[i] + kt * v_tile_step,
                                                     0, 0, 0);
    };

    // Key tiles this block needs: all of them, or (causal) up to the last key
    // visible to its last query.
    int nkt = (p.seq_k + BK - 1) / BK;
    if constexpr (CAUSAL) {
        const int last = min(p.seq_k - 1, q0 + BQ - 1 + p.causal_offset);
        nkt = last < 0 ? 0 : last / BK + 1;
    }

    f32x16_t o[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
    // Running max (log2 domain) and this lane's partial running sum.  The max is
    // only moved when a score exceeds it by more than 2^8 (or on the first
    // tile): exp2 values then stay below 256, and O is rescaled on few tiles.
    float m_run = -__builtin_inff(), l_run = 0.f;
    const float sl2 = p.scale_log2;
    constexpr float kSlack = 8.0f;

    // Fragment addresses within a stage.
    int k_frag[2][NC];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int n = 32 * b + lq;
            k_frag[b][c] = n * KROW + k_slot<D>(n, 2 * c + lh) * 16;
        }
    // P.V's A operand (V^T: row d = lq of head_dim block i, keys 16*kc4 + 8*lh
    // + 0..7) through two ds_read_b64_tr_b16.  In each 16-lane group (lanes
    // 16*gq .. +15) output lane j receives element j % 4 of source lanes j/4,
    // j/4 + 4, j/4 + 8, j/4 + 12; so source lane sq points at key row
    // 8*(gq/2) + sq/4 (+4 for the second read), head_dim 32*i + 16*(gq%2) +
    // 4*(sq%4) .. +3, and lane j gets 4 consecutive keys of head_dim 32*i +
    // 16*(gq%2) + j.  The row's swizzle depends on key bits the per-lane part
    // fixes, so v_addr[i] plus the key block's row offset is the whole address.
    int v_addr[ND];
    {
        const int gq = lane >> 4, sq = lane & 15;
        const int row = 8 * (gq >> 1) + (sq >> 2);
        const int cc = 2 * (gq & 1) + ((sq & 3) >> 1);  // chunk within the 32-wide block
        const int swz = v_swz<D>(row) >> 2;              // v_swz is 4 * swz for these rows
#pragma unroll
        for (int i = 0; i < ND; ++i) v_addr[i] = K_BYTES + row * KROW + 8 * (sq & 1) + 16 * (4 * (i ^ swz) + cc);
    }

    if (kg < nkt) load_tile(kg, lds);  // the group's first tile
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): it is in LDS
    __syncthreads();

    // One key tile; EDGE tiles (a partial last tile, or keys after some
    // query's diagonal) mask scores, the others carry no masking code at all.
    // PAR is the buffer holding tile kt when it is known at compile time (the
    // unmasked loop runs two tiles per trip), so LDS addresses are a register
    // plus an immediate offset; -1: it follows kt at run time (edge tiles; the
    // group's j-th tile, kt = KS*j + kg, sits in buffer j & 1).
    auto step = [&](int kt, auto edge_c, auto par_c) {
        constexpr bool EDGE = decltype(edge_c)::value;
        constexpr int PAR = decltype(par_c)::value;
        const int par = PAR < 0 ? ((kt / KS) & 1) : PAR;
        const lds_t *cur = lds + par * STAGE;
        if (kt + KS < nkt) load_tile(kt + KS, lds + (1 - par) * STAGE);

        // S^T for 64 keys: two 32-key blocks whose MFMAs alternate (no back-to-back
        // accumulator chain); K fragments are read two head_dim steps ahead.
        auto read_k = [&](int c, bf16x8_t (&f)[2]) {
#pragma unroll
            for (int b = 0; b < 2; ++b) f[b] = *(const __attribute__((address_space(3))) bf16x8_t *)(cur + k_frag[b][c]);
        };
        f32x16_t s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[b][r] = 0.f;
        bf16x8_t kf[3][2];
        read_k(0, kf[0]);
        read_k(1, kf[1]);
        // Raised issue priority while this wave feeds the matrix core: the
        // other workgroup's wave on the SIMD then runs its softmax in the gaps
        // instead of competing with the MFMA issue.
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (c + 2 < NC) read_k(c + 2, kf[(c + 2) % 3]);
#pragma unroll
            for (int b = 0; b < 2; ++b) s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c % 3][b], qf[c], s[b], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);

        // The first V^T fragments: their LDS latency hides under the softmax.
        auto read_v = [&](int kc4, bf16x8_t (&f)[ND]) {
            typedef short s16x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const lds_t *a = cur + v_addr[i] + 16 * kc4 * KROW;
                const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t *)a);
                const s16x4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t *)(a + 4 * KROW));
                f[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        };
        bf16x8_t vf[2][ND];
        read_v(0, vf[0]);

        // Keys past seq_k, and (causal) after the query's diagonal, do not exist.
        // With a key mask every tile is an edge tile: bit k of `keep` says key
        // kt*BK + k is kept.  Lane half lh holds the tile's keys 16*g + 8*lh +
        // (0..7) (g = 2b + r/8, the K rows being quadswapped), so after a shift
        // by 8*lh each score's bit sits at a compile-time position.
        if constexpr (EDGE) {
            const int vis = CAUSAL ? min(p.seq_k - 1, my_q + p.causal_offset) : p.seq_k - 1;
            uint64_t keep = ~0ull;
            if (p.key_mask) {
                const int kk = kt * BK + lane;
                keep = __builtin_amdgcn_ballot_w64(kk < p.seq_k && p.key_mask[kk] != 0) >> (8 * lh);
            }
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt * BK + quadswap(32 * b + 8 * (r >> 2) + 4 * lh + (r & 3));
                    const bool kept = (keep >> (16 * (2 * b + (r >> 3)) + (r & 7))) & 1u;
                    if (key > vis || !kept) s[b][r] = -__builtin_inff();
                }
        }

        // Online softmax for this lane's query (the other half of its keys is in lane ^ 32).
        float mx = -__builtin_inff();
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32)) * sl2;
        const bool grow = mx > m_run + kSlack;
        if (__builtin_amdgcn_ballot_w64(grow)) {  // some query's max moved: rescale (alpha = 1 elsewhere)
            // (the empty volatile asm pins this block as a branch, skipped on most
            // tiles, rather than 64 multiplies executed on every one)
            asm volatile("" ::: "memory");
            const float m_new = grow ? mx : m_run;
            // 0 on the first tile, 1 where the max stays; a row that has seen no
            // key yet (m_new = -inf) keeps its zero sums (-inf - -inf would be NaN)
            const float alpha = (m_new == -__builtin_inff()) ? 1.0f : exp2_hw(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < ND; ++i) o[i] *= alpha;
            m_run = m_new;
        }
        const float m_use = (m_run == -__builtin_inff()) ? 0.f : m_run;  // no key seen yet
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[b][r] = exp2_hw(fmaf(s[b][r], sl2, -m_use));

        // O^T += V^T P^T over the 4 chunks of 16 keys, V^T fragments one chunk ahead.
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kc4 = 0; kc4 < 4; ++kc4) {
            if (kc4 + 1 < 4) read_v(kc4 + 1, vf[(kc4 + 1) & 1]);
            const int b = kc4 >> 1, c2 = kc4 & 1;
            const f32x8_t pv = {s[b][8 * c2 + 0], s[b][8 * c2 + 1], s[b][8 * c2 + 2], s[b][8 * c2 + 3],
                                s[b][8 * c2 + 4], s[b][8 * c2 + 5], s[b][8 * c2 + 6], s[b][8 * c2 + 7]};
            const bf16x8_t pf = __builtin_convertvector(pv, bf16x8_t);
#pragma unroll
            for (int i = 0; i < ND; ++i) o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[kc4 & 1][i], pf, o[i], 0, 0, 0);
            // the row sum of the same bf16 weights the MFMA multiplies, two per dot2
            typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
            const bf16x2_t one2 = {(__bf16)1.0f, (__bf16)1.0f};
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 0, 1), one2, l_run, false);
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 2, 3), one2, l_run, false);
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 4, 5), one2, l_run, false);
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 6, 7), one2, l_run, false);
        }

        __builtin_amdgcn_s_setprio(0);
        // The next tile has landed in the other buffer, and every wave is done
        // reading this one, before it is refilled.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
    };
    // Tiles before n_full need no mask for any query of this block.
    int n_full = p.seq_k / BK;
    if constexpr (CAUSAL) n_full = min(n_full, max(0, (q0 + p.causal_offset + 1) / BK));
    n_full = p.key_mask ? 0 : min(n_full, nkt);
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using PR = std::integral_constant<int, -1>;
    if constexpr (KS == 1) {
        int kt = 0;
        for (; kt + 1 < n_full; kt += 2) {
            step(kt, std::false_type{}, P0{});
            step(kt + 1, std::false_type{}, P1{});
        }
        if (kt < n_full) step(kt++, std::false_type{}, P0{});
        for (; kt < nkt; ++kt) step(kt, std::true_type{}, PR{});
    } else {
        // Both groups take the same number of turns, so every wave meets the
        // same barriers; a group whose tiles ran out waits out the last turn.
        const int turns = (nkt + KS - 1) / KS;
        for (int j = 0; j < turns; ++j) {
            const int kt = KS * j + kg;
            if (kt < n_full) {
                step(kt, std::false_type{}, PR{});
            } else if (kt < nkt) {
                step(kt, std::true_type{}, PR{});
            } else {
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
            }
        }
        // Group 1 hands its state to group 0 (same query wave, same lane); the
        // stage buffers are free: every load has landed and every wave has
        // passed the last turn's barrier.
        float *xch = (float *)smem + wq * NX * 64 + lane;
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < ND; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) xch[(16 * i + r) * 64] = o[i][r];
            xch[(NX - 2) * 64] = m_run;
            xch[(NX - 1) * 64] = l_run;
        }
        __syncthreads();
        if (kg == 1) return;
        // exp2(m_g - m) weighs each group's sums (zero for a group that saw no key)
        const float m1 = xch[(NX - 2) * 64], l1 = xch[(NX - 1) * 64];
        const float mn = fmaxf(m_run, m1);
        const float a0 = (m_run == -__builtin_inff()) ? 0.f : exp2_hw(m_run - mn);
        const float a1 = (m1 == -__builtin_inff()) ? 0.f : exp2_hw(m1 - mn);
        l_run = l_run * a0 + l1 * a1;
#pragma unroll
        for (int i = 0; i < ND; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[i][r] = o[i][r] * a0 + xch[(16 * i + r) * 64] * a1;
    }

    // Normalise and store this lane's query row: 4 consecutive head_dim values per register group.
    const float lt = l_run + __shfl_xor(l_run, 32);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (my_q < p.seq_q) {
#pragma unroll
        for (int i = 0; i < ND; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = 32 * i + 8 * j + 4 * lh;
                const f32x4_t v = {o[i][4 * j] * inv, o[i][4 * j + 1] * inv, o[i][4 * j + 2] * inv,
                                   o[i][4 * j + 3] * inv};
                const int64_t off = (int64_t)my_q * p.ldo + head * D + d;
                if constexpr (OUT == 0) {
                    *(f32x4_t *)((float *)p.O + off) = v;
                } else {
                    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
                    *(u32x2_t *)((uint16_t *)p.O + off) =
                        __builtin_bit_cast(u32x2_t, __builtin_convertvector(v, bf16x4_t));
                }
            }
    }
#endif  // __HIP_DEVICE_COMPILE__
}

template <int D, bool CAUSAL, int OUT, int KS>
hipError_t launch4(const AttnParams &p, hipStream_t s) {
    constexpr int BQ = 128 / KS;
    const dim3 grid((unsigned)(((p.seq_q + BQ - 1) / BQ) * p.heads));
    hipLaunchKernelGGL((attn_fwd_kernel<D, CAUSAL, OUT, KS>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <int D, bool CAUSAL, int OUT>
hipError_t launch3(const AttnParams &p, int key_groups, hipStream_t s) {
    return key_groups == 2 ? launch4<D, CAUSAL, OUT, 2>(p, s) : launch4<D, CAUSAL, OUT, 1>(p, s);
}

template <int D>
hipError_t launch2(const AttnParams &p, bool causal, int out, int key_groups, hipStream_t s) {
    if (causal) return out ? launch3<D, true, 1>(p, key_groups, s) : launch3<D, true, 0>(p, key_groups, s);
    return out ? launch3<D, false, 1>(p, key_groups, s) : launch3<D, false, 0>(p, key_groups, s);
}

}  // namespace

hipError_t attention_launch(const AttnParams &p, int D, bool causal, int out, int key_groups, hipStream_t stream) {
    if (key_groups != 1 && key_groups != 2) return hipErrorInvalidValue;
    if (D == 128) return launch2<128>(p, causal, out, key_groups, stream);
    if (D == 64) return launch2<64>(p, causal, out, key_groups, stream);
    return hipErrorInvalidValue;
}

}  // namespace inv
