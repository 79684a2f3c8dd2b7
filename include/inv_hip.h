/*
 * inv_hip.h -- C ABI of libinvision_hip.so, the MI355X (gfx950) backend for
 * hshatti/Invision's dense linear layer  Y = X . W^T (+bias) (+SiLU/GELU).
 *
 * Plain C: no C++ or HIP types cross this boundary.  Every entry point returns
 * an int status (INV_OK = 0) and never aborts; the message for the last
 * failure on the calling thread is inv_hip_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *  - the CBLAS slot  TQNNSingleOPS.cblas_sgemm   src/quicknncpu.pas:102-103
 *    (bound by LoadLibrary/getProcAddress at src/quicknncpu.pas:3967-3992),
 *    replaced by inv_hip_sgemm, same argument list and meaning;
 *  - the bf16 slot   TQNNSingleOPS.cblas_sbgemm  src/quicknncpu.pas:110-111,
 *    replaced by inv_hip_sbgemm;
 *  - QNNLinear / QNNLinearNoBias / QNNLinearNoBias_BF16 / QNNMatMulNT /
 *    QNNLINEAR_BF16_OR_F32  (src/quicknn_kernels.pas:216-223, 317;
 *    src/quicknncpu.pas:1773-1784, 1807-1847, 3062-3071), replaced by
 *    inv_hip_linear on a device-resident weight handle;
 *  - the bf16 weight source  TSafeTensorFile.getTensorDataMemBlockBF16
 *    (src/safetensor.pas:650-683), whose mmap pointer feeds
 *    inv_hip_weight_upload once, instead of the per-call widening at
 *    src/quicknncpu.pas:1842-1844; the safetensors reader itself
 *    (src/safetensor.pas:466-513, 584-683) by inv_hip_weight_load_safetensors;
 *  - ffnSwigluForward's gate/up projections + QNNSiluMul
 *    (src/quicknn_transformers.pas:1331-1334) by INV_EPI_SWIGLU, and the
 *    projection + QNNGatedAdd (src/quicknncpu.pas:853-859) by
 *    inv_hip_linear_gated_add;
 *  - QNNFlashAttention and the per-head attention loops
 *    (src/quicknncpu.pas:2763; src/quicknn_transformers.pas:1150-1311) by
 *    inv_hip_attention, and Qwen3's masked causal attention
 *    (src/quicknn_qwen3.pas:727-769) by inv_hip_attention_masked;
 *  - QNNAdaLN / QNNRMSNorm before a projection (src/quicknncpu.pas:3042-3060,
 *    2159-2198) by inv_hip_linear_norm;
 *  - the per-head QK RMSNorm and rotary embedding before attention
 *    (QNNQKRMSNorm + QNNApplyRoPE2D, QNNHeadRSMNorm + QNNApplyRoPE3;
 *    src/quicknncpu.pas:2209-2246, 2892-2992) by inv_hip_head_norm_rope, or
 *    fused into attention's operand staging by inv_hip_attention_qk_norm_rope;
 *  - the VAE's QNNConv2d (src/quicknncpu.pas:1958-2124) by inv_hip_conv2d.
 */
#ifndef INV_HIP_H
#define INV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INV_HIP_ABI_VERSION 1

/* ---- status codes ------------------------------------------------------- */
#define INV_OK               0
#define INV_ERR_ARG          1  /* bad pointer, shape, leading dimension or enum   */
#define INV_ERR_UNSUPPORTED  2  /* valid but not implemented (e.g. ColMajor)        */
#define INV_ERR_NO_DEVICE    3  /* no gfx950 device visible                         */
#define INV_ERR_OOM          4  /* device or pinned-host allocation failed          */
#define INV_ERR_HIP          5  /* a HIP runtime call failed                        */
#define INV_ERR_NOT_INIT     6  /* inv_hip_init has not succeeded                   */

/* ---- element types: the reference's TQNNDataType values
 *      (src/quicknn_common.pas:77-98: dtF16 = 1, dtBf16 = 2, dtF32 = 3) ------ */
#define INV_DT_F16  1 /* safetensors weights only */
#define INV_DT_BF16 2
#define INV_DT_F32  3

/* ---- CBLAS enums: src/quicknn_common.pas:55-58 -------------------------- */
#define INV_CBLAS_ROW_MAJOR 101
#define INV_CBLAS_COL_MAJOR 102
#define INV_CBLAS_NO_TRANS  111
#define INV_CBLAS_TRANS     112

/* ---- epilogues fused into the GEMM's store ------------------------------- */
#define INV_EPI_NONE      0 /* Y = acc (+bias)                                            */
#define INV_EPI_SILU      1 /* Y = silu(acc + bias) = v * rcp(1 + exp2(-v log2 e)), hw ops */
#define INV_EPI_GELU_ERF  2 /* Y = 0.5 v (1 + erf(v / sqrt 2)); the reference has no GELU */
#define INV_EPI_SWIGLU    3 /* gate/up weight only (inv_hip_weight_upload_gate_up):
                               Y = silu(X.Wg^T + bg) * (X.Wu^T + bu), SiLU as above -- the two
                               projections and QNNSiluMul of ffnSwigluForward
                               (src/quicknn_transformers.pas:1331-1334, src/quicknncpu.pas:
                               2404-2418) in one GEMM; Y has F columns */

/* ---- flags for inv_hip_linear -------------------------------------------- */
#define INV_FLAG_DEVICE_PTRS 0x1 /* X, Y and bias are device pointers (inv_hip_malloc) */
#define INV_FLAG_ASYNC       0x2 /* with DEVICE_PTRS: return without waiting; call
                                    inv_hip_synchronize before reading Y            */
#define INV_FLAG_PRECISE     0x4 /* fp32 X is split into bf16 hi + lo and both halves
                                    are multiplied (2 MFMA passes): the result then
                                    matches the reference's fp32-activation GEMM to
                                    ~1e-5 instead of ~1.5e-3 (no effect for bf16 X)   */

/* ---- precision of the CBLAS fp32 slot (inv_hip_set_sgemm_precision) ----- */
#define INV_PREC_BF16     0 /* A and B rounded to bf16: 1 MFMA pass                      */
#define INV_PREC_SPLIT_A  1 /* A split hi + lo, B rounded: 2 passes (exact for bf16 B)    */
#define INV_PREC_SPLIT_AB 2 /* both split, A.B ~ AhBh + AlBh + AhBl: 3 passes (default),
                               relative error ~2^-16, the accuracy an fp32 slot expects */

typedef struct inv_weight_s *inv_weight_t; /* opaque device-resident weight */

/* ---- lifetime ------------------------------------------------------------- */
/* Select device `device` (ordinal among visible devices), check it is gfx950,
 * create the library stream.  Returns INV_ERR_NO_DEVICE when there is none, so
 * the caller keeps its CPU GEMM bound (src/quicknncpu.pas:3951-3955).  With
 * INV_HIP_ALLOC_LIMIT_MB set in the environment, the device memory the library
 * allocates from then on (workspaces, weights, inv_hip_malloc) is capped at
 * that many MiB: a call that would pass the cap returns INV_ERR_OOM, as one
 * whose hipMalloc fails does. */
int inv_hip_init(int device);
/* Free every weight, workspace and the stream (src/quicknncpu.pas:4073-4086). */
int inv_hip_shutdown(void);
/* Message for the last failing call on this thread ("" if none). */
const char *inv_hip_last_error(void);
int inv_hip_abi_version(void);
/* Name, compute-unit count and peak engine clock of the selected device. */
int inv_hip_device_info(char *name, size_t name_len, int *cu_count, int *clock_khz);

/* ---- weights -------------------------------------------------------------- */
/* Copy W[N x K] bf16 (row-major, leading dimension K, e.g. the mmap pointer
 * from getTensorDataMemBlockBF16) and an optional fp32 bias[N] to the device
 * once.  The host buffer may be read-only; it is not retained. */
int inv_hip_weight_upload(const uint16_t *w_bf16, int64_t N, int64_t K, const float *bias,
                          inv_weight_t *out);
/* Same from fp32 weights (getTensorDataMemBlock, src/safetensor.pas:584-647):
 * each value is rounded to bf16, ties to even (exact for widened bf16). */
int inv_hip_weight_upload_f32(const float *w_f32, int64_t N, int64_t K, const float *bias,
                              inv_weight_t *out);
/* A gate/up pair for INV_EPI_SWIGLU: gate and up are [F x K] bf16 (FLUX2's
 * fused linear_in [2F x K] is gate = ptr, up = ptr + F*K, as
 * src/quicknn_transformers.pas:595-597 splits it; Qwen3 and Z-Image hold them
 * as separate tensors).  Biases optional (fp32 [F] each).  Stored interleaved
 * in 128-row blocks so that one output tile holds matching gate and up rows. */
int inv_hip_weight_upload_gate_up(const uint16_t *gate_bf16, const uint16_t *up_bf16, int64_t F, int64_t K,
                                  const float *gate_bias, const float *up_bias, inv_weight_t *out);
int inv_hip_weight_free(inv_weight_t w);

/* ---- weights from .safetensors files --------------------------------------
 * The file format the reference reads its weights from (TSafeTensorFile,
 * src/safetensor.pas:466-513): u64 little-endian header length, a JSON header
 * {name: {dtype, shape, data_offsets [begin, end) from the data block}}, data.
 * The same checks as the reference: header length below the file size, every
 * tensor inside the file, and (in addition) byte size = product(shape) * dtype
 * size for F32/BF16/F16. */
#define INV_ST_MAX_DIMS 8
#define INV_ST_GATE_UP  0x2 /* the tensor is a fused [2F x K] gate|up weight (and the
                               bias, if any, [2F]): load it as a gate/up pair for
                               INV_EPI_SWIGLU (N of the handle = F) */
#define INV_ST_TRUNCATE 0x1 /* F32/F16 -> bf16 by truncation (u16 = u32 >> 16), the
                               reference's SingleToBF16 (src/quicknn_common.pas:
                               2010-2027) as getTensorDataMemBlockBF16 applies it
                               (src/safetensor.pas:675); default: ties to even */
/* Metadata of tensor `name` (no device needed): dtype as INV_DT_* (-1 for
 * other dtypes), rank, up to INV_ST_MAX_DIMS dimensions, and the byte offset
 * of its data in the file.  Replaces TSafeTensorFile.find + the tensor record
 * (src/safetensor.pas:491-507). */
int inv_hip_safetensors_info(const char *path, const char *name, int *dtype, int *ndim, int64_t *shape,
                             int64_t *data_offset);
/* Upload the 2-D weight `name` ([N x K], PyTorch Linear layout) of a
 * .safetensors file, with an optional 1-D bias `bias_name` (NULL: none; any
 * of F32/BF16/F16, widened to fp32).  BF16 weights go from the read-only file
 * mapping straight to the device, as getTensorDataMemBlockBF16 hands the mmap
 * pointer over (src/safetensor.pas:650-683); F32 and F16 are rounded to bf16
 * (ties to even, or truncated with INV_ST_TRUNCATE).  The file is unmapped on
 * return. */
int inv_hip_weight_load_safetensors(const char *path, const char *name, const char *bias_name, int flags,
                                    inv_weight_t *out);
/* N and K of a handle. */
int inv_hip_weight_shape(inv_weight_t w, int64_t *N, int64_t *K);

/* ---- the device weight cache ---------------------------------------------- */
/* The reference re-reads and re-widens every block's weights from the mapped
 * file on every sampler step and frees them afterwards
 * (src/quicknn_transformers.pas:1581-1602, src/quicknn_qwen3.pas:1087-1091,
 * through getTensorDataMemBlock, src/safetensor.pas:584-683).
 * inv_hip_weight_cache_get returns the resident handle of (file, tensor, bias
 * tensor, flags) -- the file identified by device, inode, size and
 * modification time, so a rewritten file is loaded again -- uploading it on
 * the first request only (as inv_hip_weight_load_safetensors).  Each get holds
 * one reference; inv_hip_weight_free on the handle releases it and leaves the
 * weight resident.  With a budget (bytes; 0 = unlimited, the default), the
 * least recently used unreferenced weights are evicted while the cache holds
 * more; referenced ones never are.  inv_hip_weight_cache_clear frees every
 * unreferenced entry and detaches the rest (freed by their last release).
 * stats: entries, resident bytes, hits, misses and bytes uploaded so far. */
int inv_hip_weight_cache_get(const char *path, const char *name, const char *bias_name, int flags,
                             inv_weight_t *out);
int inv_hip_weight_cache_set_budget(int64_t bytes);
int inv_hip_weight_cache_clear(void);
int inv_hip_weight_cache_stats(int64_t *entries, int64_t *bytes, int64_t *hits, int64_t *misses,
                               int64_t *uploaded_bytes);

/* ---- the linear layer ----------------------------------------------------- */
/* Y[M x N] = epilogue(X[M x K] . W^T + bias), row-major, leading dims K and N.
 *  X: fp32 (rounded to bf16, ties to even, on the device) or bf16.
 *  Y: fp32 or bf16 (rounded to nearest even from the fp32 accumulator).
 *  bias: NULL -> the handle's uploaded bias if it has one, else none.
 *  Accumulation is fp32 in the MFMA units.  Host pointers by default (copied
 *  in and out, synchronous); INV_FLAG_DEVICE_PTRS for resident buffers. */
int inv_hip_linear(const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y,
                   int y_dtype, int64_t M, int64_t K, int64_t N, int epilogue, int flags);

/* Gated residual projection: Y[m][n] += gate[n] * (X . W^T + bias)[m][n].
 * Replaces the QNNLINEAR_BF16_OR_F32 projection followed by QNNGatedAdd
 * (src/quicknn_transformers.pas:1432-1438, 1447, 1456, 1528-1529;
 * QNNGatedAdd src/quicknncpu.pas:853-859, QNNAccMul 1752-1758) with one GEMM
 * whose epilogue scales each column by the gate and adds it into the fp32
 * residual stream Y [M x N] in place; the projection is never stored.
 * gate: [N] fp32, or NULL for a plain residual add (Y += X . W^T + bias).
 * bias, X dtypes and flags as for inv_hip_linear; gate/up weights are
 * rejected.  With host pointers Y is copied in, updated and copied back. */
int inv_hip_linear_gated_add(const void *X, int x_dtype, inv_weight_t W, const float *bias,
                             const float *gate, float *Y, int64_t M, int64_t K, int64_t N, int flags);

/* ---- normalised projections ------------------------------------------------ */
#define INV_NORM_ADALN 1 /* (1 + scale[k]) * (x - mean) / sqrt(var + eps) + shift[k], population
                            variance over the row: QNNAdaLN (src/quicknncpu.pas:3042-3060)    */
#define INV_NORM_RMS   2 /* x * weight[k] / sqrt(mean(x^2) + eps); weight may be NULL:
                            QNNRMSNorm (src/quicknncpu.pas:2159-2185)                          */
/* Y = epilogue(norm(X) . W^T + bias) for the fp32 residual stream X [M x K]:
 * replaces QNNAdaLN (or QNNRMSNorm) into a scratch activation followed by the
 * projection (e.g. src/quicknn_transformers.pas:1400-1404, 1440-1441).  The
 * normalisation runs while X is rounded into the GEMM's bf16 operand, so it
 * costs the same one pass over X as the plain fp32 path, and the normalised
 * activation is never stored.  norm_scale / norm_shift are [K] fp32 (AdaLN:
 * both required; RMS: weight or NULL, shift NULL).  The reference uses
 * EPSILON = 1e-6 (src/quicknn_common.pas:51) whatever eps its callers pass;
 * give 1e-6 to match.  flags: INV_FLAG_DEVICE_PTRS (X, Y, bias and the norm
 * vectors on the device), INV_FLAG_ASYNC. */
int inv_hip_linear_norm(const float *X, int norm, const float *norm_scale, const float *norm_shift,
                        float eps, inv_weight_t W, const float *bias, void *Y, int y_dtype, int64_t M,
                        int64_t K, int64_t N, int epilogue, int flags);

/* ---- attention ------------------------------------------------------------ */
#define INV_ATTN_CAUSAL 0x100 /* key j is visible to query i iff j <= i + (seq_k - seq_q) */
/* O = softmax(scale * Q . K^T) . V for every head, in the reference's
 * [tokens x heads*head_dim] layout: Q [seq_q x heads*head_dim], K and V
 * [seq_k x kv_heads*head_dim], O [seq_q x heads*head_dim], all row-major; head h
 * uses kv head h / (heads / kv_heads).
 * Replaces TQNNSingleOPS.QNNFlashAttention(dst, Q, K, V, heads, seq_q, seq_k,
 * head_dim, scale) (src/quicknncpu.pas:2763, reached via src/quicknn_kernels.pas:
 * 1655-1663; its callers pass heads first, src/quicknn_transformers.pas:1203,
 * 1301-1302) and the per-head cblas_gemm + QNNSoftmaxRows + cblas_gemm loops of
 * multiHeadForward / jointAttentionForward (src/quicknn_transformers.pas:
 * 1150-1311), Z-Image's attentionForward (:2228-2271) and, with kv_heads < heads
 * and INV_ATTN_CAUSAL, Qwen3's grouped causal attention (src/quicknn_qwen3.pas:
 * 727-769).  The [seq_q x seq_k] score matrix is never stored.
 *  in_dtype: INV_DT_F32 (rounded to bf16, nearest-even, on the device) or
 *  INV_DT_BF16, for Q, K and V alike; out_dtype INV_DT_F32 or INV_DT_BF16.
 *  head_dim 64 or 128 (else INV_ERR_UNSUPPORTED); heads a multiple of kv_heads;
 *  scale > 0.  Scores accumulate in fp32; the softmax weights are rounded to
 *  bf16 for the P.V product, which accumulates in fp32.
 *  flags: INV_FLAG_DEVICE_PTRS, INV_FLAG_ASYNC, INV_ATTN_CAUSAL. */
int inv_hip_attention(const void *Q, const void *K, const void *V, void *O, int in_dtype,
                      int out_dtype, int64_t heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                      int64_t head_dim, float scale, int flags);

/* inv_hip_attention with the key mask of Qwen3's attention: key j is hidden
 * from every query where key_mask[j] == 0 (seq_k int32 entries, host or device
 * per INV_FLAG_DEVICE_PTRS; null: no mask).  Replaces the mask argument of
 * QNNMatTriangularFill(seq_len, scores, -inf, attention_mask) before
 * QNNSoftmaxRows (src/quicknn_qwen3.pas:753-754; src/quicknncpu.pas:
 * 3017-3028), which with INV_ATTN_CAUSAL and seq_q == seq_k is the same mask;
 * the encoder's padding to 512 tokens sets it (src/quicknn_qwen3.pas:
 * 1136-1140, 293-303).  A query that sees no key gets zeros (the reference's
 * softmax gives NaN there). */
int inv_hip_attention_masked(const void *Q, const void *K, const void *V, void *O, int in_dtype,
                             int out_dtype, int64_t heads, int64_t kv_heads, int64_t seq_q,
                             int64_t seq_k, int64_t head_dim, float scale, const int32_t *key_mask,
                             int flags);

/* ---- between the Q/K projections and attention ---------------------------- */
#define INV_ROPE_NONE        0
#define INV_ROPE_INTERLEAVED 1 /* pairs (2k, 2k+1), tables [seq x head_dim], column 2k */
#define INV_ROPE_HALF        2 /* pairs (i, i + head_dim/2), tables [seq x head_dim/2], column i */

/* In place on X [seq x heads*head_dim] (fp32, row-major): each head's RMSNorm
 * with norm_weight [head_dim] (null: none; rstd = 1/sqrt(mean(x^2) + 1e-6),
 * x * w * rstd), then the rotary embedding of token s from row s of the tables
 * (INV_ROPE_NONE: none).  Replaces, in one pass over X:
 *  - FLUX2: QNNQKRMSNorm then QNNApplyRoPE2D (src/quicknn_transformers.pas:
 *    1405-1408, 1415-1422; src/quicknncpu.pas:2209-2246, 2968-2992), called
 *    once for Q and once for K with INV_ROPE_INTERLEAVED;
 *  - Qwen3: QNNHeadRSMNorm then QNNApplyRoPE3 (src/quicknn_qwen3.pas:718-723,
 *    223-230; src/quicknncpu.pas:2892-2917) with INV_ROPE_HALF.
 * head_dim 64 or 128 (else INV_ERR_UNSUPPORTED).  flags: INV_FLAG_DEVICE_PTRS
 * (X, weight and tables on the device), INV_FLAG_ASYNC. */
int inv_hip_head_norm_rope(float *X, int64_t seq, int64_t heads, int64_t head_dim,
                           const float *norm_weight, int rope, const float *cos_table,
                           const float *sin_table, int flags);

/* inv_hip_attention_masked on fp32 Q and K with each head's RMSNorm and the
 * rotary embedding applied while they are staged for the MFMA (one read of
 * each, no separate pass): the FLUX2 and Qwen3 sequence of
 * inv_hip_head_norm_rope on Q, on K, then attention, in one call.
 * q_/k_norm_weight [head_dim] or null; rope as for inv_hip_head_norm_rope with
 * per-token tables for Q (seq_q rows) and K (seq_k rows; for FLUX2's joint
 * attention the text rows then the image rows, like K itself); key_mask as for
 * inv_hip_attention_masked.  Q, K, V fp32 (host or device per
 * INV_FLAG_DEVICE_PTRS), each row-major with a token stride ldq/ldk/ldv in
 * elements (0: packed, heads*head_dim), so the three thirds of a fused QKV
 * projection's output are read in place (ld = 3*hidden); O is packed.  No
 * counterpart in the reference as one call. */
int inv_hip_attention_qk_norm_rope(const float *Q, int64_t ldq, const float *K, int64_t ldk,
                                   const float *V, int64_t ldv, void *O, int out_dtype, int64_t heads,
                                   int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                                   float scale,
                                   const float *q_norm_weight, const float *k_norm_weight, int rope,
                                   const float *q_cos, const float *q_sin, const float *k_cos,
                                   const float *k_sin, const int32_t *key_mask, int flags);

/* ---- convolution (the VAE) ------------------------------------------------ */
/* TQNNSingleOPS.QNNConv2d (src/quicknncpu.pas:176-177, 1958-2124; reached
 * through QNNConv2d, src/quicknn_kernels.pas:990-1006, from the VAE's ResNet,
 * attention, down/up-sampling and in/out convolutions, src/quicknn_vae.pas:
 * 174-184, 269-310, 402-456, 556-627): dst [batch x out_ch x outH x outW] =
 * conv(src [batch x in_ch x H x W]) + bias[out_ch], NCHW fp32, zero padding,
 * outH = (H + 2*padding - kH)/stride + 1 (QNNConv2DShape,
 * src/quicknn_kernels.pas:984-987), likewise outW.  weight is a handle of the
 * reference's [out_ch x in_ch*kH*kW] fp32 filter (inv_hip_weight_upload_f32,
 * N = out_ch, K = in_ch*kH*kW); bias [out_ch] (null: the handle's, if any).
 * The image is rounded to bf16 (RNE) into a patch matrix and multiplied with
 * fp32 accumulation; an fp32 filter was rounded to bf16 by its upload too.
 * Normwise deviation from the fp32 convolution: 1.5e-3 to 2.1e-3 with a
 * bf16-exact filter, 2.2e-3 to 3.2e-3 with an fp32 one (the two roundings).
 * The output follows the convolution's definition; the reference's default
 * im2col loop differs from it for stride-1 shapes with padding != (kW-1)/2 and
 * for 1x1 filters with stride or padding (src/quicknncpu.pas:2063-2110).
 * flags: INV_FLAG_DEVICE_PTRS (src, dst, bias on the device), INV_FLAG_ASYNC. */
int inv_hip_conv2d(const float *src, inv_weight_t weight, const float *bias, float *dst, int64_t in_ch,
                   int64_t out_ch, int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t stride,
                   int64_t padding, int64_t batch, int flags);

/* ---- the CBLAS slots ------------------------------------------------------ */
/* Exactly the signature of TQNNSingleOPS.cblas_sgemm (src/quicknncpu.pas:
 * 102-103): C = alpha * op(A) . op(B) + beta * C on host fp32 arrays, RowMajor
 * or ColMajor, every NoTrans/Trans combination.  A and B are converted to bf16
 * on the device per the slot's precision mode (default INV_PREC_SPLIT_AB) and
 * multiplied with fp32 accumulation; beta == 0 does not read C (BLAS
 * semantics).  Returns a status; the slot's callers ignore it, so the binding
 * checks the status itself. */
int inv_hip_sgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                  const float *A, int64_t lda, const float *B, int64_t ldb, float beta, float *C,
                  int64_t ldc);
/* TQNNSingleOPS.cblas_sbgemm (src/quicknncpu.pas:110-111): bf16 A and B
 * (exact in one MFMA pass). */
int inv_hip_sbgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                   const uint16_t *A, int64_t lda, const uint16_t *B, int64_t ldb, float beta, float *C,
                   int64_t ldc);

/* Precision of inv_hip_sgemm for subsequent calls (INV_PREC_*).  No
 * counterpart in the reference, whose fp32 slot is always fp32. */
int inv_hip_set_sgemm_precision(int mode);

/* ---- device memory and timing, for callers that keep activations resident */
int inv_hip_malloc(void **ptr, size_t bytes);
int inv_hip_free(void *ptr);
int inv_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int inv_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
/* Device-to-device copy on the library stream (a 16-byte-word copy kernel when
 * both pointers and the size are 16-byte granular). */
int inv_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int inv_hip_memset(void *dst, int value, size_t bytes);
int inv_hip_synchronize(void);
/* HIP events recorded on the library stream: start, then stop -> elapsed ms. */
int inv_hip_timer_start(void);
int inv_hip_timer_stop(float *ms);

/* ---- statistics (the per-op accumulator of src/nopmetrics.pas:30-72) ------- */
/* Number of inv_hip_linear/sgemm/sbgemm calls and the summed GPU time of their
 * GEMM kernels in ms (HIP events, only while enabled). */
int inv_hip_stats_enable(int enable);
int inv_hip_stats(int64_t *calls, double *gemm_ms, double *flops);
int inv_hip_stats_reset(void);

/* ---- linear layer without allocation -------------------------------------- */
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): inv_hip_linear with the same arguments, results and
 * kernels, on device pointers only (flags must hold INV_FLAG_DEVICE_PTRS;
 * INV_FLAG_ASYNC and INV_FLAG_PRECISE as for inv_hip_linear), that calls no
 * hipMalloc, hipFree or allocating routine.  Its scratch memory (activations
 * staged to bf16, a misaligned bias, split-K partial sums and counters) is a
 * static device array of INV_NOALLOC_SCRATCH_BYTES, one per GPU, kept until
 * the process ends and shared by every call on that GPU: calls run in order on
 * the library stream, so they never overlap; work that would need more scratch
 * returns INV_ERR_UNSUPPORTED (e.g. fp32 activations above 2^25 elements). */
#define INV_NOALLOC_SCRATCH_BYTES (64u << 20)
int inv_hip_linear_noalloc(const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y, int y_dtype,
                           int64_t M, int64_t K, int64_t N, int epilogue, int flags);

/* ---- the reference's sampler, for synthetic inputs (host only) ----------- */
/* src/quicknn_sample.pas:212-276: xoshiro256** seeded by SplitMix64
 * (rng_seed), uniform singles from 53-bit draws (rand), Box-Muller normals
 * (random_normal).  The stream is per calling thread.  inv_hip_sample_randn draws
 * n normals in order, each times sigma, rounded to bf16 (RNE, kept as fp32
 * values) when round_bf16 is non-zero.  Need no device and no inv_hip_init. */
int inv_hip_sample_seed(uint64_t seed);
int inv_hip_sample_randn(float *dst, int64_t n, float sigma, int round_bf16);

#ifdef __cplusplus
}
#endif
#endif /* INV_HIP_H */
