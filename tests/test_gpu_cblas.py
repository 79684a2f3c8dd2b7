"""The CBLAS slots (inv_hip_sgemm / inv_hip_sbgemm) and the reference operator
mirror (QNNLinear & co.) against the oracle's qgemm (marked gpu).

The HIP path rounds A and B to bf16 (ties to even) and accumulates in fp32, so
the tight comparison feeds the oracle the same rounded operands; the
north-star comparison uses the fp32 operands as the reference would.
"""
import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, round_bf16

pytestmark = pytest.mark.gpu

NT, T = hip.CblasNoTrans, hip.CblasTrans


def rnd(shape, seed, scale=1.0):
    oracle.rng_seed(seed)
    return oracle.randn_scaled(shape, scale, False)


def oracle_gemm(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C0, ldc):
    """qgemm, with the TT case (which the reference rejects) done as NT on A^T."""
    C = C0.copy()
    if ta == T and tb == T:
        At = np.ascontiguousarray(A[:K, :M].T) if A.ndim == 2 else None
        oracle.qgemm(NT, T, M, N, K, alpha, At, K, B, ldb, beta, C, ldc)
    else:
        oracle.qgemm(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc)
    return C


@pytest.mark.parametrize("ta", [NT, T])
@pytest.mark.parametrize("tb", [NT, T])
@pytest.mark.parametrize("M,N,K", [(37, 53, 129), (256, 128, 512), (5, 300, 64)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.75, -0.5)])
def test_sgemm_all_transposes(hiplib, ta, tb, M, N, K, alpha, beta):
    # Default precision (INV_PREC_SPLIT_AB): fp32-slot accuracy.
    A = rnd((K, M) if ta == T else (M, K), 1)
    B = rnd((N, K) if tb == T else (K, N), 2, 0.05)
    lda, ldb = A.shape[1], B.shape[1]
    C0 = rnd((M, N), 3)
    C = C0.copy()
    q.cblas_gemm(hip.CblasRowMajor, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, N)
    want_ref = oracle_gemm(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C0, N)
    err = oracle.normwise_err(C, want_ref)
    print(f"  split-AB sgemm vs fp32 qgemm: {err:.3e}", flush=True)
    assert err <= 5e-5


@pytest.mark.parametrize("mode", [hip.INV_PREC_BF16, hip.INV_PREC_SPLIT_A, hip.INV_PREC_SPLIT_AB])
def test_sgemm_precision_modes(hiplib, mode):
    M, N, K = 96, 160, 384
    A = rnd((M, K), 21)
    B = rnd((N, K), 22, 0.05)
    C = np.zeros((M, N), np.float32)
    q.set_sgemm_precision(mode)
    try:
        q.cblas_gemm(hip.CblasRowMajor, NT, T, M, N, K, 1.0, A, K, B, K, 0.0, C, N)
    finally:
        q.set_sgemm_precision(hip.INV_PREC_SPLIT_AB)
    ref32 = oracle_gemm(NT, T, M, N, K, 1.0, A, K, B, K, 0.0, np.zeros((M, N), np.float32), N)
    if mode == hip.INV_PREC_BF16:
        tight = oracle_gemm(NT, T, M, N, K, 1.0, round_bf16(A), K, round_bf16(B), K, 0.0, np.zeros_like(C), N)
        assert oracle.normwise_err(C, tight) <= 2e-5
        assert oracle.normwise_err(C, ref32) <= 4e-3  # both operands rounded: twice the linear budget
    elif mode == hip.INV_PREC_SPLIT_A:
        tight = oracle_gemm(NT, T, M, N, K, 1.0, A, K, round_bf16(B), K, 0.0, np.zeros_like(C), N)
        assert oracle.normwise_err(C, tight) <= 5e-5
    else:
        assert oracle.normwise_err(C, ref32) <= 5e-5


def test_sgemm_leading_dimensions_and_untouched_padding(hiplib):
    M, N, K = 40, 24, 72
    lda, ldb, ldc = 80, 100, 33
    A = rnd((M, lda), 4)
    B = rnd((N, ldb), 5, 0.05)
    C = np.full((M, ldc), 7.0, np.float32)
    q.cblas_gemm(hip.CblasRowMajor, NT, T, M, N, K, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    want = A[:, :K].astype(np.float64) @ B[:, :K].astype(np.float64).T
    assert oracle.normwise_err(C[:, :N], want) <= 5e-5
    assert np.all(C[:, N:] == 7.0)  # bytes between rows are not written


def test_sgemm_col_major(hiplib):
    M, N, K = 33, 45, 96
    A = rnd((K, M), 6)   # col-major M x K  == row-major K x M
    B = rnd((N, K), 7)   # col-major K x N  == row-major N x K
    Ccm = np.zeros((N, M), np.float32)  # col-major M x N, ldc = M
    q.cblas_gemm(hip.CblasColMajor, NT, NT, M, N, K, 1.0, A, M, B, K, 0.0, Ccm, M)
    want = A.T.astype(np.float64) @ B.T.astype(np.float64)
    assert oracle.normwise_err(Ccm.T, want) <= 5e-5


def test_sgemm_k_zero_scales_c(hiplib):
    C = np.ones((4, 5), np.float32)
    A = np.zeros((4, 1), np.float32)
    B = np.zeros((1, 5), np.float32)
    q.cblas_gemm(hip.CblasRowMajor, NT, NT, 4, 5, 0, 1.0, A, 1, B, 5, 3.0, C, 5)
    np.testing.assert_array_equal(C, np.full((4, 5), 3.0, np.float32))


def test_sbgemm_bf16_operands(hiplib):
    M, N, K = 64, 80, 200
    A = as_bf16_bits(rnd((M, K), 8))
    B = as_bf16_bits(rnd((N, K), 9, 0.02))
    C = np.zeros((M, N), np.float32)
    q.cblas_sbgemm(hip.CblasRowMajor, NT, T, M, N, K, 1.0, A, K, B, K, 0.0, C, N)
    want = oracle.linear_bf16w(oracle.bf16_to_f32(A), B)
    assert oracle.normwise_err(C, want) <= 2e-5


def test_sgemm_bad_arguments(hiplib):
    lib = hip.load()
    A = np.zeros((4, 4), np.float32)
    assert lib.inv_hip_sgemm(999, NT, T, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, A.ctypes.data,
                             4) == hip.INV_ERR_ARG
    assert lib.inv_hip_sgemm(101, 115, T, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, A.ctypes.data,
                             4) == hip.INV_ERR_ARG
    assert lib.inv_hip_sgemm(101, NT, T, 4, 4, 4, 1.0, A.ctypes.data, 2, A.ctypes.data, 4, 0.0, A.ctypes.data,
                             4) == hip.INV_ERR_ARG
    assert lib.inv_hip_sgemm(101, NT, T, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, A.ctypes.data,
                             3) == hip.INV_ERR_ARG


# ------------------------------------------------ the reference operator mirror

def test_qnnlinear_family_matches_oracle(hiplib):
    M, K, N = 48, 160, 96
    X = rnd((M, K), 10)
    Wf = round_bf16(rnd((N, K), 11, 0.02))
    Wb = as_bf16_bits(Wf)
    b = rnd((N,), 12, 0.01)
    ref_nb = oracle.linear_bf16w(round_bf16(X), Wb)
    ref_b = oracle.linear_bf16w(round_bf16(X), Wb, b)

    y = np.zeros((M, N), np.float32)
    q.QNNLinear(y, X, Wf, b, M, K, N)
    assert oracle.normwise_err(y, ref_b) <= 2e-5
    q.QNNLinear(y, X, Wf, None, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    q.QNNLinearNoBias(y, X, Wf, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    q.QNNLinearNoBias_BF16(y, X, Wb, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    q.QNNLINEAR_BF16_OR_F32(y, X, None, Wb, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    q.QNNLINEAR_BF16_OR_F32(y, X, Wf, None, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    with q.Weight(Wb) as w:  # resident weight, the intended path
        q.QNNLinearNoBias(y, X, w, M, K, N)
    assert oracle.normwise_err(y, ref_nb) <= 2e-5
    c = np.zeros((M, N), np.float32)
    q.QNNMatMulNT(c, X, Wf, M, K, N)  # the fp32 CBLAS slot: ~fp32 accuracy
    assert oracle.normwise_err(c, oracle.linear_bf16w(X, Wb)) <= 5e-5


def test_qnnmatmul_nn_tn(hiplib):
    M, K, N = 30, 70, 50
    A = rnd((M, K), 13)
    B = rnd((K, N), 14)
    C = np.zeros((M, N), np.float32)
    q.QNNMatMulNN(C, A, B, M, K, N)
    want = A.astype(np.float64) @ B.astype(np.float64)
    assert oracle.normwise_err(C, want) <= 5e-5


def test_reference_assertions_are_kept(hiplib):
    y = np.zeros((2, 2), np.float32)
    with pytest.raises(AssertionError, match="out of bound"):
        q.QNNMatMulNT(y, np.zeros(3, np.float32), np.zeros(4, np.float32), 2, 2, 2)
    with pytest.raises(AssertionError, match="no weight"):
        q.QNNLINEAR_BF16_OR_F32(y, np.zeros((2, 2), np.float32), None, None, 2, 2, 2)
