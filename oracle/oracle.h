/*
 * oracle.h -- CPU restatement of hshatti/Invision's dense linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product library (libinvision_hip.so)
 * never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  How each one is
 * pinned (known-answer vectors, the reference's own sgemm2.cpp built under
 * oracle/_ref, closed forms, brute force) is listed in tests/test_oracle.py.
 */
#ifndef INV_ORACLE_H
#define INV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- RNG: src/quicknn_sample.pas:212-276 ---------------------------------- */
void     orc_rng_seed(uint64_t seed);              /* SplitMix64 -> 4 state words   */
void     orc_rng_set_state(const uint64_t s[4]);   /* for known-answer tests        */
void     orc_rng_get_state(uint64_t s[4]);
uint64_t orc_xoshiro256ss(void);                   /* xoshiro256**                   */
float    orc_rand(void);                           /* (x >> 11) * 2^-53 -> single    */
float    orc_random_normal(void);                  /* Box-Muller, cos branch only    */
void     orc_randn(float *dst, int64_t n);         /* randn(dst, N)                  */
/* Draw n normals, scale by sigma, optionally round to bf16 (RNE) in place. */
void     orc_randn_scaled(float *dst, int64_t n, float sigma, int round_bf16);

/* ---- bf16: src/quicknn_common.pas:1991-2027 ------------------------------- */
void     orc_bf16_to_f32(const uint16_t *src, float *dst, int64_t n);      /* exact <<16   */
void     orc_f32_to_bf16_trunc(const float *src, uint16_t *dst, int64_t n); /* ref: >>16    */
void     orc_f32_to_bf16_rne(const float *src, uint16_t *dst, int64_t n);   /* build: RNE   */

/* ---- GEMM: src/quicknncpu.pas:1176-1496 (qgemm -> gemm_nn/nt/tn) ----------
 * CBLAS semantics of the reference slot (quicknncpu.pas:102-103), RowMajor
 * only.  order/trans use the reference enum values (quicknn_common.pas:55-58).
 * Returns 0, or -1 for an unsupported combination (the reference asserts).
 * nthreads <= 0 uses every OpenMP thread. */
int orc_qgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K,
              float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
              float beta, float *C, int64_t ldc, int nthreads);
/* Same arithmetic as orc_qgemm's NT path, but scalar (no AVX2) with the same
 * 8-lane FMA association; used to show the AVX2 path is bit-identical. */
int orc_gemm_nt_scalar(int64_t M, int64_t N, int64_t K, float alpha,
                       const float *A, int64_t lda, const float *B, int64_t ldb,
                       float beta, float *C, int64_t ldc);

/* fp64 gold: C[m,n] = sum_k A[m,k]*B[n,k] accumulated in double. */
void orc_gemm_nt_f64(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
                     const float *B, int64_t ldb, double *C, int64_t ldc, int nthreads);

/* ---- linear layer: src/quicknncpu.pas:1807-1847, 3062-3071 ----------------
 * QNNLinear / QNNLinearNoBias / QNNLinearNoBias_BF16:
 *   Y[M,N] = X[M,K] . widen(W_bf16)[N,K]^T  (+ bias[N] per row), then epilogue.
 * epilogue: 0 none, 1 SiLU (exact expf), 2 GELU (erf form), 3 SiLU as the
 * reference's sSiLU_avx2 computes it (polynomial exp2, exact reciprocal). */
int orc_linear_bf16w(const float *X, const uint16_t *W, const float *bias, float *Y,
                     int64_t M, int64_t K, int64_t N, int epilogue, int nthreads);

/* ---- epilogue ops: src/ops_avx2.inc:22-35, 267-376; quicknncpu.pas:305-330, 2372-2418 */
float orc_silu_exact(float x);
float orc_gelu_erf(float x);
/* sSiLU_avx2(N, src, up, outSigmoid, dst) with vrcpps replaced by 1/x. */
void  orc_silu_qnn(int64_t n, const float *src, const float *up, float *out_sigmoid, float *dst);
float orc_fast_exp(float x);

/* ---- CBLAS-shaped epilogue helpers used by the tests ---------------------- */
void orc_add_bias_rows(float *Y, const float *bias, int64_t M, int64_t N); /* QNNAddInplace per row */
void orc_apply_epilogue(float *Y, int64_t n, int epilogue);
/* QNNGatedAdd (quicknncpu.pas:853-859): dst[i][j] += gate[j] * proj[i][j]. */
void orc_gated_add(float *dst, const float *gate, const float *proj, int64_t seq, int64_t hidden);

/* ---- attention: src/quicknn_transformers.pas:1150-1311, 2228-2271;
 *      src/quicknn_qwen3.pas:727-769; src/quicknncpu.pas:2421-2500, 2763 ------
 * Q [seq_q x heads*d], K/V [seq_k x kv_heads*d], O [seq_q x heads*d]; head h uses
 * kv head h / (heads / kv_heads); causal: key j visible to query i iff
 * j <= i + seq_k - seq_q; key_mask (nullable, seq_k entries): key j hidden
 * from every query where key_mask[j] == 0 (QNNMatTriangularFill's mask,
 * quicknncpu.pas:3017-3028).  orc_attention_f64 gives a query with no visible
 * key zeros; orc_attention_qnn follows the reference (NaN there). */
int orc_attention_f64(const float *Q, const float *K, const float *V, double *O, int64_t heads,
                      int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t d, double scale, int causal,
                      const int32_t *key_mask, int nthreads);
int orc_attention_qnn(const float *Q, const float *K, const float *V, float *O, int64_t heads,
                      int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t d, float scale, int causal,
                      const int32_t *key_mask, int nthreads);
/* sSoftmax_avx2 (ops_avx2.inc:552-760) with an exact 1/sum in place of rcpss. */
void orc_softmax_qnn(float *x, int64_t n);

/* ---- rotary position embedding of Q or K, in place, x [seq x heads*d] ------
 * orc_rope_interleaved: QNNApplyRoPE2D (quicknncpu.pas:2968-2992), FLUX2's:
 *   pairs (2k, 2k+1) rotated by cos/sin[s*d + 2k] (tables [seq x d]);
 * orc_rope_half: QNNApplyRoPE3 -> QNNApplyRoPE2 (quicknncpu.pas:2892-2917),
 *   Qwen3's: pairs (i, i + d/2) rotated by cos/sin[s*d/2 + i] (tables [seq x d/2]). */
void orc_rope_interleaved(float *x, const float *cos_t, const float *sin_t, int64_t seq, int64_t heads, int64_t d);
void orc_rope_half(float *x, const float *cos_t, const float *sin_t, int64_t seq, int64_t heads, int64_t d);

/* ---- QNNAdaLN (quicknncpu.pas:3042-3060), QNNRMSNormRows (:2159-2198) ---- */
void orc_adaln(float *dst, const float *src, const float *shift, const float *scale, int64_t seq, int64_t hidden);
void orc_rmsnorm_rows(float *dst, const float *src, const float *weight, int64_t rows, int64_t dim);

/* ---- QNNConv2d (quicknncpu.pas:1958-2124) ---------------------------------- */
/* The direct convolution the reference states as its loop form
 * (quicknncpu.pas:2020-2039), accumulated in double: dst[b][oc][oh][ow] =
 * bias[oc] + sum over ic, kr, kc of src[b][ic][oh*stride - pad + kr][ow*stride
 * - pad + kc] (zero outside the image) * w[oc][(ic*kH + kr)*kW + kc].  NCHW;
 * outH/outW as QNNConv2DShape (quicknn_kernels.pas:984-987); bias may be null. */
void orc_conv2d_f64(const float *src, const float *w, const float *bias, double *dst, int64_t in_ch,
                    int64_t out_ch, int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t stride,
                    int64_t pad, int64_t batch);

int orc_has_avx2(void);
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
