"""Gated residual projection: Y += gate[n] * (X.W^T + b) in one GEMM (the
projection and QNNGatedAdd of the double- and single-stream blocks,
src/quicknn_transformers.pas:1432-1438, 1447, 1456, 1528-1529; QNNGatedAdd
src/quicknncpu.pas:853-859).

The oracle computes the projection (linear_bf16w on the same bf16-rounded X)
and then QNNGatedAdd on the CPU; the error is taken on the update Y - Y0, so a
large residual cannot hide a wrong projection."""
import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, round_bf16

TOL_TIGHT = 2e-5  # fp32 accumulation over bf16 operands, vs the oracle's own fp32 sum


def gen(seed, M, K, N, bias=True, gate=True):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 1.0, False)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b = oracle.randn_scaled((N,), 0.01, False) if bias else None
    g = oracle.randn_scaled((N,), 0.5, False) if gate else None
    Y0 = oracle.randn_scaled((M, N), 1.0, False)
    return X, W, b, g, Y0


def oracle_gated(Y0, Xr, W, b, g):
    proj = oracle.linear_bf16w(Xr, W, b, oracle.EPI_NONE)
    gate = g if g is not None else np.ones(W.shape[0], np.float32)
    return oracle.gated_add(Y0, gate, proj)


def update_err(Y, Y0, ref):
    return oracle.normwise_err(Y.astype(np.float64) - Y0, ref.astype(np.float64) - Y0)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,bias,gate", [(300, 1000, 520, True, True), (64, 512, 256, False, True),
                                             (1, 256, 130, True, True), (129, 72, 136, True, False),
                                             (2048, 3072, 3072, True, True)])
def test_gated_add_matches_oracle(hiplib, M, K, N, bias, gate):
    X, W, b, g, Y0 = gen(31, M, K, N, bias, gate)
    with q.Weight(W) as w:
        Y = q.linear_gated_add(Y0.copy(), as_bf16_bits(X), w, g, b)
    ref = oracle_gated(Y0, round_bf16(X), W, b, g)
    err = update_err(Y, Y0, ref)
    print(f"  normwise err of the update vs oracle {err:.3e}", flush=True)
    assert np.all(np.isfinite(Y))
    assert err <= TOL_TIGHT


@pytest.mark.gpu
def test_gated_add_equals_projection_then_gated_add(hiplib):
    """Fused against the unfused path through the same library (the
    projection stored, then the reference's elementwise QNNGatedAdd)."""
    M, K, N = 200, 640, 384
    X, W, b, g, Y0 = gen(32, M, K, N)
    Xb = as_bf16_bits(X)
    with q.Weight(W, b) as w:
        Y = q.linear_gated_add(Y0.copy(), Xb, w, g)  # the handle's bias
        proj = q.linear(Xb, w)
    ref = oracle.gated_add(Y0, g, proj)
    # one fused multiply-add against a rounded product: an ulp of Y at most
    np.testing.assert_allclose(Y, ref, rtol=0, atol=4 * np.finfo(np.float32).eps * np.max(np.abs(ref)))


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [0, 2, 3, 4, 5, 8, 16, 17, 18])
@pytest.mark.parametrize("grid", ["tiles", "splitk3", "streamk37"])
def test_gated_add_every_tile_and_grid_mode(hiplib, monkeypatch, cfg, grid):
    """The residual is read once, by the unit that writes the tile, in every grid mode."""
    modes = {"tiles": {"INV_HIP_MODE": "0"}, "splitk3": {"INV_HIP_MODE": "1", "INV_HIP_KSPLIT": "3"},
             "streamk37": {"INV_HIP_MODE": "2", "INV_HIP_SK_GRID": "37"}}
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    for k, v in modes[grid].items():
        monkeypatch.setenv(k, v)
    M, K, N = 300, 1000, 520
    X, W, b, g, Y0 = gen(33, M, K, N)
    with q.Weight(W, b) as w:
        Y = q.linear_gated_add(Y0.copy(), as_bf16_bits(X), w, g)
    assert update_err(Y, Y0, oracle_gated(Y0, round_bf16(X), W, b, g)) <= TOL_TIGHT


@pytest.mark.gpu
def test_gated_add_resident_buffers_accumulate(hiplib):
    """Device pointers, Y updated in place twice: Y0 + 2 * gate * proj."""
    M, K, N = 257, 384, 264
    X, W, b, g, Y0 = gen(34, M, K, N)
    with q.Weight(W, b) as w:
        xd = q.DeviceArray.from_host(as_bf16_bits(X), "bf16")
        yd = q.DeviceArray.from_host(Y0, "f32")
        gd = q.DeviceArray.from_host(g, "f32")
        q.linear_gated_add_device(xd, w, yd, M, gate=gd)
        q.linear_gated_add_device(xd, w, yd, M, gate=gd, asynchronous=True)
        hip.call("inv_hip_synchronize")
        Y = yd.to_host()
        for d in (xd, yd, gd):
            d.free()
    proj = oracle.linear_bf16w(round_bf16(X), W, b)
    ref = oracle.gated_add(oracle.gated_add(Y0, g, proj), g, proj)
    assert update_err(Y, Y0, ref) <= TOL_TIGHT


@pytest.mark.gpu
def test_gated_add_precise_fp32_x(hiplib):
    M, K, N = 96, 700, 200
    X, W, b, g, Y0 = gen(35, M, K, N)
    with q.Weight(W) as w:
        Y = q.linear_gated_add(Y0.copy(), X, w, g, b, precise=True)
    ref = oracle_gated(Y0, X.astype(np.float32), W, b, g)  # fp32 X, no rounding
    assert update_err(Y, Y0, ref) <= TOL_TIGHT


@pytest.mark.gpu
def test_qnn_linear_gated_add_mirror(hiplib):
    """QNNLINEAR_BF16_OR_F32 + QNNGatedAdd as one call, fp32 activations."""
    seq, din, dout = 77, 320, 192
    X, W, _, g, Y0 = gen(36, seq, din, dout, bias=False)
    dst = Y0.copy()
    q.QNNLinearGatedAdd(dst, X, None, W, g, seq, din, dout)
    assert update_err(dst, Y0, oracle_gated(Y0, round_bf16(X), W, None, g)) <= TOL_TIGHT
    with pytest.raises(AssertionError, match="no weight"):
        q.QNNLinearGatedAdd(dst, X, None, None, g, seq, din, dout)


@pytest.mark.gpu
def test_gated_add_argument_errors(hiplib):
    X, W, b, g, Y0 = gen(37, 8, 64, 128)
    with q.Weight.gate_up(W, W) as wgu:
        with pytest.raises(hip.HipError, match="no gated-add form"):
            q.linear_gated_add(np.zeros((8, 128), np.float32), as_bf16_bits(X), wgu, g)
    with q.Weight(W) as w:
        with pytest.raises(ValueError, match="gate must have"):
            q.linear_gated_add(Y0.copy(), as_bf16_bits(X), w, g[:5])
        lib = hip.load()
        Y = Y0.copy()
        rc = lib.inv_hip_linear_gated_add(None, hip.INV_DT_BF16, w.handle, None, None, Y.ctypes.data, 8, 64, 128, 0)
        assert rc == hip.INV_ERR_ARG and "X or Y is null" in hip.last_error()
        Xb = as_bf16_bits(X)
        rc = lib.inv_hip_linear_gated_add(Xb.ctypes.data, hip.INV_DT_BF16, w.handle, None, None, Y.ctypes.data, 8,
                                          64, 127, 0)
        assert rc == hip.INV_ERR_ARG and "shape mismatch" in hip.last_error()
        np.testing.assert_array_equal(Y, Y0)  # untouched on error


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [8, 13, 15, 16, 17, 18])
@pytest.mark.parametrize("grid", [{"INV_HIP_MODE": "1", "INV_HIP_KSPLIT": "3"},
                                  {"INV_HIP_MODE": "2", "INV_HIP_SK_GRID": "37"}], ids=["splitk3", "streamk37"])
def test_gated_add_with_shared_tiles(hiplib, monkeypatch, cfg, grid):
    """Tiles whose K range is shared by several workgroups: the last one sums
    the parked partial rows, then applies bias, gate and the residual add."""
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    for k, v in grid.items():
        monkeypatch.setenv(k, v)
    M, K, N = 300, 1000, 520
    X, W, b, g, Y0 = gen(33, M, K, N)
    with q.Weight(W) as w:
        Y = q.linear_gated_add(Y0.copy(), as_bf16_bits(X), w, g, b)
        Y2 = q.linear_gated_add(Y0.copy(), as_bf16_bits(X), w, g, b)
    assert update_err(Y, Y0, oracle_gated(Y0, round_bf16(X), W, b, g)) <= TOL_TIGHT
    np.testing.assert_array_equal(Y, Y2)
