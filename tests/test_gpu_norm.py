"""Normalised projections: Y = epi(norm(X) . W^T + b) with the AdaLN or RMS
normalisation applied while the fp32 X is rounded into the GEMM's bf16 operand
(QNNAdaLN src/quicknncpu.pas:3042-3060 then the projection,
src/quicknn_transformers.pas:1400-1404, 1440-1441; QNNRMSNorm :2159-2185).

Tolerances, normwise:
  - 2e-3 against the reference's fp32 chain (oracle norm, fp32 activations):
    the single bf16 rounding of the normalised X, as for any fp32-X linear;
  - 1e-3 against the same library's unfused path (oracle norm -> inv_hip_linear)
    and against the oracle on the bf16-rounded oracle norm: the GPU's tree sums
    and the oracle's sequential sums give means and 1/std that differ in the last
    bits, which moves a normalised element across a bf16 rounding boundary now
    and then (one such flip moves an output by ~1e-4 of max|Y|; 3e-4 measured at
    300x1024x520).  A missing (1 + scale), a sample variance or a wrong row each
    move the result by far more (the oracle tests plant them).
The modulation vectors are drawn N(0, 0.1), the size an AdaLN modulation layer
produces; X ~ 2 N(0, 1) + 0.5.
"""
import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import bf16_bits_to_f32, round_bf16

TOL_REF = 2e-3
TOL_SAME = 1e-3


def gen(seed, M, K, N):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 2.0, False) + np.float32(0.5)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b = oracle.randn_scaled((N,), 0.01, False)
    shift = oracle.randn_scaled((K,), 0.1, False)
    scale = oracle.randn_scaled((K,), 0.1, False)
    return X.astype(np.float32), W, b, shift, scale


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(300, 1024, 520), (64, 3072, 256), (1, 1536, 130), (257, 200, 96),
                                   (40, 1036, 96),   # K % 8 == 4: one zero-padded group of 4 columns
                                   (33, 77, 64),     # K % 4 != 0: the multi-pass kernel
                                   (16, 5120, 64), (8, 8192, 64), (4, 12288, 32), (4, 16384, 64)])
                                   # 6, 8, 12 and 16 register groups per thread
def test_adaln_linear_matches_oracle(hiplib, M, K, N):
    X, W, b, shift, scale = gen(81, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear_norm(X, "adaln", w, scale, shift)
        Xn = oracle.adaln(X, shift, scale)
        y_unfused = q.linear(Xn, w)
    ref32 = oracle.linear_bf16w(Xn, W, b)
    ref_r = oracle.linear_bf16w(round_bf16(Xn), W, b)
    e32, er, eu = (oracle.normwise_err(y, r) for r in (ref32, ref_r, y_unfused))
    print(f"  normwise err: fp32 chain {e32:.3e}, bf16-rounded oracle norm {er:.3e}, unfused {eu:.3e}", flush=True)
    assert np.all(np.isfinite(y))
    assert er <= TOL_SAME and eu <= TOL_SAME
    if K >= 1024:
        assert e32 <= TOL_REF


@pytest.mark.gpu
@pytest.mark.parametrize("weighted", [True, False])
def test_rms_linear_matches_oracle(hiplib, weighted):
    M, K, N = 200, 2560, 384
    X, W, b, _, scale = gen(82, M, K, N)
    wt = (np.float32(1.0) + scale).astype(np.float32) if weighted else None
    with q.Weight(W) as w:
        y = q.linear_norm(X, "rms", w, wt)
    Xn = oracle.rmsnorm_rows(X, wt)
    assert oracle.normwise_err(y, oracle.linear_bf16w(round_bf16(Xn), W)) <= TOL_SAME
    assert oracle.normwise_err(y, oracle.linear_bf16w(Xn, W)) <= TOL_REF


@pytest.mark.gpu
def test_adaln_with_silu_and_bf16_output(hiplib):
    M, K, N = 128, 1024, 512
    X, W, b, shift, scale = gen(83, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear_norm(X, "adaln", w, scale, shift, epilogue="silu", out_dtype="bf16")
    ref = oracle.linear_bf16w(round_bf16(oracle.adaln(X, shift, scale)), W, b, oracle.EPI_SILU)
    assert oracle.normwise_err(bf16_bits_to_f32(y), ref) <= TOL_SAME + 2.0 ** -8


@pytest.mark.gpu
def test_device_pointers_match_host_path(hiplib):
    M, K, N = 150, 768, 320
    X, W, b, shift, scale = gen(84, M, K, N)
    with q.Weight(W, b) as w:
        y_host = q.linear_norm(X, "adaln", w, scale, shift)
        xd, sd, hd = (q.DeviceArray.from_host(a, "f32") for a in (X, scale, shift))
        yd = q.DeviceArray((M, N), "f32")
        hip.call("inv_hip_linear_norm", xd.ptr, hip.INV_NORM_ADALN, sd.ptr, hd.ptr, q.EPSILON, w.handle, None, yd.ptr,
                 hip.INV_DT_F32, M, K, N, hip.INV_EPI_NONE, hip.INV_FLAG_DEVICE_PTRS)
        np.testing.assert_array_equal(yd.to_host(), y_host)
        # modulation vectors at a 4-byte (not 16-byte) offset into device memory
        sh = np.concatenate([np.zeros(1, np.float32), scale]), np.concatenate([np.zeros(1, np.float32), shift])
        sd1, hd1 = (q.DeviceArray.from_host(a, "f32") for a in sh)
        yd.free()
        yd = q.DeviceArray((M, N), "f32")
        hip.call("inv_hip_linear_norm", xd.ptr, hip.INV_NORM_ADALN, sd1.ptr + 4, hd1.ptr + 4, q.EPSILON, w.handle,
                 None, yd.ptr, hip.INV_DT_F32, M, K, N, hip.INV_EPI_NONE, hip.INV_FLAG_DEVICE_PTRS)
        np.testing.assert_array_equal(yd.to_host(), y_host)
        for a in (xd, sd, hd, yd, sd1, hd1):
            a.free()


@pytest.mark.gpu
def test_qnn_adaln_linear_mirror(hiplib):
    seq, hidden, out = 256, 1024, 512
    X, W, _, shift, scale = gen(85, seq, hidden, out)
    dst = np.zeros((seq, out), np.float32)
    q.QNNAdaLNLinear(dst, X, shift, scale, None, W, seq, hidden, out)
    ref = oracle.linear_bf16w(oracle.adaln(X, shift, scale), W)
    assert oracle.normwise_err(dst, ref) <= TOL_REF


@pytest.mark.gpu
def test_norm_argument_errors(hiplib):
    X, W, b, shift, scale = gen(86, 8, 64, 64)
    lib = hip.load()
    y = np.zeros((8, 64), np.float32)
    with q.Weight(W) as w:
        def call(norm, sc, sh, flags=0, eps=1e-6):
            return lib.inv_hip_linear_norm(X.ctypes.data, norm, sc.ctypes.data if sc is not None else None,
                                           sh.ctypes.data if sh is not None else None, eps, w.handle, None,
                                           y.ctypes.data, hip.INV_DT_F32, 8, 64, 64, 0, flags)
        assert call(hip.INV_NORM_ADALN, scale, None) == hip.INV_ERR_ARG and "scale and shift" in hip.last_error()
        assert call(hip.INV_NORM_RMS, scale, shift) == hip.INV_ERR_ARG and "no shift" in hip.last_error()
        assert call(7, scale, shift) == hip.INV_ERR_ARG and "bad norm" in hip.last_error()
        assert call(hip.INV_NORM_RMS, scale, None, eps=-1.0) == hip.INV_ERR_ARG
        assert call(hip.INV_NORM_RMS, scale, None, flags=hip.INV_FLAG_PRECISE) == hip.INV_ERR_UNSUPPORTED
    assert not np.any(y)
