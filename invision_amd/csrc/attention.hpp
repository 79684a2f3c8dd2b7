// attention.hpp -- parameters and launcher of the attention forward kernel
// (attention.hip): O = softmax(scale * Q . K^T) . V per head, the computation
// of TQNNSingleOPS.QNNFlashAttention (src/quicknncpu.pas:2763) and of the
// per-head cblas_gemm + QNNSoftmaxRows + cblas_gemm sequences
// (src/quicknn_transformers.pas:1150-1311, 2228-2271; src/quicknn_qwen3.pas:727-769).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace inv {

// Row-major operands in the reference's [tokens x heads*head_dim] layout, all bf16
// except O.  Head h reads kv head h / (heads / kv_heads) (grouped-query attention).
struct AttnParams {
    const uint16_t *Q;   // [seq_q x ldq], head h at columns h*D .. h*D+D-1
    const uint16_t *K;   // [seq_k x ldk], kv head g at columns g*D ..
    const uint16_t *V;   // [seq_k x ldv], kv head g at columns g*D .. (as K)
    void *O;             // [seq_q x ldo], fp32 or bf16
    int64_t ldq, ldk, ldv, ldo;
    int seq_q, seq_k, heads, kv_heads;
    float scale_log2;    // scale * log2(e): scores enter exp2 directly
    int causal_offset;   // causal: key j is visible to query i iff j <= i + causal_offset
    const int32_t *key_mask;  // null, or [seq_k]: key j hidden from every query where key_mask[j] == 0
};

// D: 64 or 128; causal: mask keys after the query's diagonal; out: 0 fp32, 1 bf16;
// key_groups: 1 (128 queries per workgroup, 4 waves over every key tile) or 2
// (64 queries per workgroup, two pairs of waves over alternate key tiles: for
// grids of 128-query blocks that do not fill the chip).
hipError_t attention_launch(const AttnParams &p, int D, bool causal, int out, int key_groups, hipStream_t stream);

constexpr int kAttnBlockQ = 128;  // queries per workgroup with one key group (4 waves x 32)
constexpr int kAttnBlockK = 64;   // keys per tile

}  // namespace inv
