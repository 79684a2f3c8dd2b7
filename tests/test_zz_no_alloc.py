"""inv_hip_linear_noalloc (the linear layer that allocates nothing, its scratch a
static device array) against inv_hip_linear on the same device pointers: the
same kernels run, so the outputs are bit-identical.  Two calls in a row per
case, the second with fewer rows, so a scratch left dirty by the first call
(staged activations, split-K counters and partials) would show."""
import ctypes

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits

pytestmark = pytest.mark.gpu

DEV = hip.INV_FLAG_DEVICE_PTRS

# (name, M, K, N, x dtype, y dtype, epilogue, flags, bias)
CASES = [
    ("c2_bf16_in_place", 4608, 3072, 9216, "bf16", "f32", hip.INV_EPI_NONE, 0, True),
    ("fp32_x_staged_silu_bf16_out", 640, 1024, 1536, "f32", "bf16", hip.INV_EPI_SILU, 0, True),
    ("c4_down_split_k", 512, 9728, 2560, "bf16", "f32", hip.INV_EPI_NONE, 0, False),
    ("c1_split_k_fp32_x", 256, 3072, 3072, "f32", "f32", hip.INV_EPI_NONE, 0, True),
    ("ragged_k_gelu", 300, 1000, 700, "bf16", "f32", hip.INV_EPI_GELU_ERF, 0, True),
    ("precise_split_x", 384, 2048, 1024, "f32", "f32", hip.INV_EPI_NONE, hip.INV_FLAG_PRECISE, True),
]


def _gen(seed, M, K, N):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 1.0, False)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b = oracle.randn_scaled((N,), 0.01, False)
    return X, W, b


def _run(fn, x, w, bias_d, y, M, K, N, xdt, ydt, epi, flags):
    hip.call(fn, x.ptr, x.inv_dtype, w.handle, bias_d.ptr if bias_d is not None else None, y.ptr, y.inv_dtype,
             M, K, N, epi, DEV | flags)
    return y.to_host()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_linear_twice(hiplib, case):
    name, M, K, N, xdt, ydt, epi, flags, has_bias = case
    X, W, b = _gen(31, M, K, N)
    Xin = as_bf16_bits(X) if xdt == "bf16" else X
    with q.Weight(W) as w:
        bd = q.DeviceArray.from_host(b, "f32") if has_bias else None
        for call, rows in enumerate((M, max(1, M // 3 + 5))):
            print(f"  {name}: call {call + 1}, M={rows}", flush=True)
            xd = q.DeviceArray.from_host(np.ascontiguousarray(Xin[:rows]), xdt)
            y_ref = q.DeviceArray((rows, N), ydt)
            y_na = q.DeviceArray((rows, N), ydt)
            ref = _run("inv_hip_linear", xd, w, bd, y_ref, rows, K, N, xdt, ydt, epi, flags)
            got = _run("inv_hip_linear_noalloc", xd, w, bd, y_na, rows, K, N, xdt, ydt, epi, flags)
            assert np.all(np.isfinite(got.astype(np.float32) if ydt == "f32" else got))
            np.testing.assert_array_equal(got, ref)
            for d in (xd, y_ref, y_na):
                d.free()
        if bd is not None:
            bd.free()


def test_noalloc_split_tail(hiplib, monkeypatch):
    """The split tail (rounds of 12 tiles here: 24 whole tiles, 6 split two
    ways along K) through the static scratch, against inv_hip_linear, on two
    calls in a row (the second's 12 tiles: no tail)."""
    monkeypatch.setenv("INV_HIP_SPLIT_TAIL_SLOTS", "12")
    monkeypatch.setenv("INV_HIP_TILE_CFG", "16")
    M, K, N = 1100, 1024, 1300
    X, W, b = _gen(32, M, K, N)
    Xin = as_bf16_bits(X)
    with q.Weight(W) as w:
        bd = q.DeviceArray.from_host(b, "f32")
        for rows in (M, 400):
            xd = q.DeviceArray.from_host(np.ascontiguousarray(Xin[:rows]), "bf16")
            y_ref = q.DeviceArray((rows, N), "f32")
            y_na = q.DeviceArray((rows, N), "f32")
            ref = _run("inv_hip_linear", xd, w, bd, y_ref, rows, K, N, "bf16", "f32", hip.INV_EPI_NONE, 0)
            got = _run("inv_hip_linear_noalloc", xd, w, bd, y_na, rows, K, N, "bf16", "f32", hip.INV_EPI_NONE, 0)
            np.testing.assert_array_equal(got, ref)
            for d in (xd, y_ref, y_na):
                d.free()
        bd.free()


def test_noalloc_swiglu_and_misaligned_bias(hiplib):
    M, K, F = 700, 1536, 1024
    X, W, b = _gen(32, M, K, 2 * F)
    Xb = as_bf16_bits(X)
    with q.Weight.gate_up(W[:F], W[F:], b[:F], b[F:]) as wgu, q.Weight(W[:F]) as w:
        for rows in (M, 129):
            xd = q.DeviceArray.from_host(np.ascontiguousarray(Xb[:rows]), "bf16")
            ya, yb = q.DeviceArray((rows, F), "bf16"), q.DeviceArray((rows, F), "bf16")
            ref = _run("inv_hip_linear", xd, wgu, None, ya, rows, K, F, "bf16", "bf16", hip.INV_EPI_SWIGLU, 0)
            got = _run("inv_hip_linear_noalloc", xd, wgu, None, yb, rows, K, F, "bf16", "bf16", hip.INV_EPI_SWIGLU,
                       0)
            np.testing.assert_array_equal(got, ref)
            # a bias 4 bytes past a 16-byte boundary: staged into the scratch's bias area
            bias_buf = q.DeviceArray.from_host(np.concatenate([[0.0], b[:F]]).astype(np.float32), "f32")
            ya2, yb2 = q.DeviceArray((rows, F), "f32"), q.DeviceArray((rows, F), "f32")
            for fn, yy in (("inv_hip_linear", ya2), ("inv_hip_linear_noalloc", yb2)):
                hip.call(fn, xd.ptr, hip.INV_DT_BF16, w.handle, bias_buf.ptr + 4, yy.ptr, hip.INV_DT_F32, rows, K, F,
                         hip.INV_EPI_NONE, DEV)
            np.testing.assert_array_equal(yb2.to_host(), ya2.to_host())
            for d in (xd, ya, yb, bias_buf, ya2, yb2):
                d.free()


def test_noalloc_limits_and_errors(hiplib):
    lib = hip.load()
    X, W, _ = _gen(33, 16, 256, 64)
    with q.Weight(W) as w:
        xd = q.DeviceArray.from_host(X, "f32")
        yd = q.DeviceArray((16, 64), "f32")
        # host pointers are refused (they would need the bounce buffers)
        y = np.zeros((16, 64), np.float32)
        assert lib.inv_hip_linear_noalloc(X.ctypes.data, 3, w.handle, None, y.ctypes.data, 3, 16, 256, 64, 0,
                                          0) == hip.INV_ERR_ARG
        assert "DEVICE_PTRS" in hip.last_error()
        assert lib.inv_hip_linear_noalloc(xd.ptr, 3, w.handle, None, yd.ptr, 3, 16, 255, 64, 0, DEV) == hip.INV_ERR_ARG
        assert lib.inv_hip_linear_noalloc(xd.ptr, 3, w.handle, None, yd.ptr, 3, 0, 256, 64, 0, DEV) == hip.INV_OK
        xd.free()
        yd.free()
    # fp32 activations whose bf16 staging exceeds the scratch: a clear error, nothing launched
    M, K, N = 16384, 4096, 64
    X = np.zeros((M, K), np.float32)
    W = np.zeros((N, K), np.uint16)
    with q.Weight(W) as w:
        xd = q.DeviceArray.from_host(X, "f32")
        yd = q.DeviceArray((M, N), "f32")
        assert lib.inv_hip_linear_noalloc(xd.ptr, 3, w.handle, None, yd.ptr, 3, M, K, N, 0, DEV) == \
            hip.INV_ERR_UNSUPPORTED
        assert "scratch" in hip.last_error()
        xd.free()
        yd.free()
