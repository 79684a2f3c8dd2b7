"""inv_hip_conv2d against the oracle's direct convolution (QNNConv2d,
src/quicknncpu.pas:1958-2124; the VAE's call sites src/quicknn_vae.pas:174-184,
269-310, 402-456, 556-627).

The library rounds the fp32 image to bf16 (RNE) into its patch matrix; the
filters here are bf16-exact (as a bf16 checkpoint's are), except in
test_conv2d_fp32_filter_rounded_on_upload.  Tolerances, normwise
(max|d| / max|ref|):
  - 2e-5 against the oracle (float64 sums) on the bf16-rounded image: fp32
    accumulation order only;
  - 3e-3 against the oracle on the fp32 image: the single bf16 rounding of the
    image (1.5e-3 to 2.3e-3 measured on the CPU for these shapes).
"""
import os

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import round_bf16

TOL_BF16 = 2e-5
TOL_REF = 3e-3


def gen(seed, b, c, oc, H, W, kH, kW):
    oracle.rng_seed(seed)
    x = oracle.randn_scaled((b, c, H, W), 1.0, False).astype(np.float32)
    w = oracle.bf16_to_f32(oracle.f32_to_bf16_rne(oracle.randn_scaled((oc, c * kH * kW), 0.05, False)))
    bias = oracle.randn_scaled((oc,), 0.01, False).astype(np.float32)
    return x, np.ascontiguousarray(w, dtype=np.float32), bias


def check(y, x, w, bias, c, oc, H, W, kH, kW, s, p, b):
    ref_b = oracle.conv2d_f64(round_bf16(x), w, bias, c, oc, H, W, kH, kW, s, p, b)
    ref = oracle.conv2d_f64(x, w, bias, c, oc, H, W, kH, kW, s, p, b)
    assert y.shape == ref.shape
    e_b, e_r = oracle.normwise_err(y, ref_b), oracle.normwise_err(y, ref)
    print(f"[conv2d] b{b} c{c} oc{oc} {H}x{W} k{kH}x{kW} s{s} p{p}: {e_b:.3e} (bf16 image), {e_r:.3e} (fp32)")
    assert e_b <= TOL_BF16 and e_r <= TOL_REF


SHAPES = [
    (1, 3, 64, 32, 32, 3, 3, 1, 1),     # VAE conv_in: 3 channels, K = 27
    (1, 64, 64, 24, 20, 3, 3, 1, 1),    # ResNet conv
    (2, 32, 48, 16, 16, 1, 1, 1, 0),    # skip / attention 1x1, batch 2
    (1, 32, 32, 17, 17, 3, 3, 2, 0),    # downsample: stride 2 on the padded image
    (1, 64, 3, 32, 32, 3, 3, 1, 1),     # conv_out: 3 output channels (M = 3)
    (2, 24, 5, 19, 17, 3, 3, 2, 1),     # 5 output channels, stride 2 with padding, batch 2
    (1, 40, 1, 16, 16, 3, 3, 1, 2),     # one output channel, padding 2
    (1, 40, 2, 16, 16, 5, 5, 1, 2),     # two output channels, 5x5
    (1, 16, 40, 9, 11, 5, 3, 1, 2),     # ragged: kH != kW, odd sizes
    (1, 128, 128, 48, 40, 3, 3, 1, 1),  # K = 1152
    (1, 256, 96, 20, 24, 3, 3, 1, 1),   # K = 2304, out_ch not a multiple of 32
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,c,oc,H,W,kH,kW,s,p", SHAPES)
def test_conv2d_matches_oracle(hiplib, b, c, oc, H, W, kH, kW, s, p):
    x, w, bias = gen(11, b, c, oc, H, W, kH, kW)
    with q.Weight(w) as wt:
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    check(y, x, w, bias, c, oc, H, W, kH, kW, s, p, b)


# fp32 filters that are not bf16-exact (a VAE checkpoint in F32): the upload rounds the filter to
# bf16 as well as the image, two roundings whose combined normwise deviation from the fp32
# convolution measured 2.2e-3 to 3.2e-3 on the CPU over these shapes and seeds (largest at K = 27,
# the 3-channel conv_in); the image alone gives 1.5e-3 to 2.1e-3.
TOL_REF_F32_FILTER = 4e-3


@pytest.mark.gpu
@pytest.mark.parametrize("b,c,oc,H,W,kH,kW,s,p", [SHAPES[0], SHAPES[1], SHAPES[4], SHAPES[9], SHAPES[10]])
def test_conv2d_fp32_filter_rounded_on_upload(hiplib, b, c, oc, H, W, kH, kW, s, p):
    oracle.rng_seed(13)
    x = oracle.randn_scaled((b, c, H, W), 1.0, False).astype(np.float32)
    w = np.ascontiguousarray(oracle.randn_scaled((oc, c * kH * kW), 0.05, False), dtype=np.float32)
    bias = oracle.randn_scaled((oc,), 0.01, False).astype(np.float32)
    assert np.any(round_bf16(w) != w)  # the filter is not bf16-exact
    with q.Weight(w) as wt:  # inv_hip_weight_upload_f32: rounded to bf16, ties to even
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    both = oracle.conv2d_f64(round_bf16(x), round_bf16(w), bias, c, oc, H, W, kH, kW, s, p, b)
    ref = oracle.conv2d_f64(x, w, bias, c, oc, H, W, kH, kW, s, p, b)
    e_b, e_r = oracle.normwise_err(y, both), oracle.normwise_err(y, ref)
    print(f"[conv2d fp32 filter] {b, c, oc, H, W, kH, kW, s, p}: {e_b:.3e} (bf16 image and filter), "
          f"{e_r:.3e} (fp32)", flush=True)
    assert e_b <= TOL_BF16 and e_r <= TOL_REF_F32_FILTER


@pytest.mark.gpu
def test_conv2d_mirror_and_handle_bias(hiplib):
    b, c, oc, H, W, kH, kW, s, p = 1, 8, 16, 12, 10, 3, 3, 1, 1
    x, w, bias = gen(12, b, c, oc, H, W, kH, kW)
    dims = q.QNNConv2DShape(b, oc, H, W, kH, kW, p, s)
    dst = np.zeros(dims, np.float32)
    q.QNNConv2d(dst, x, w, bias, c, oc, H, W, kH, kW, s, p, b)  # host filter, uploaded for the call
    check(dst, x, w, bias, c, oc, H, W, kH, kW, s, p, b)
    with q.Weight(w, bias) as wt:  # the handle's bias when the call passes none
        y = q.conv2d(x, wt, None, c, oc, H, W, kH, kW, s, p, b)
    np.testing.assert_array_equal(y, dst)
    y0 = q.conv2d(x, w, None, c, oc, H, W, kH, kW, s, p, b)  # no bias at all
    check(y0, x, w, None, c, oc, H, W, kH, kW, s, p, b)


@pytest.mark.gpu
def test_conv2d_device_pointers_match_host(hiplib):
    b, c, oc, H, W, kH, kW, s, p = 2, 16, 24, 14, 18, 3, 3, 1, 1
    x, w, bias = gen(13, b, c, oc, H, W, kH, kW)
    dims = q.QNNConv2DShape(b, oc, H, W, kH, kW, p, s)
    with q.Weight(w) as wt:
        yh = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        xd = q.DeviceArray.from_host(x)
        bd = q.DeviceArray.from_host(bias)
        yd = q.DeviceArray(tuple(dims), "f32")
        try:
            q.conv2d_device(xd, wt, yd, c, oc, H, W, kH, kW, s, p, b, bias=bd)
            np.testing.assert_array_equal(yd.to_host(), yh)
        finally:
            for a in (xd, bd, yd):
                a.free()


# (path, b, c, oc, H, W, kH, kW, s, p): the direct kernel, the implicit GEMM (forced with
# INV_HIP_CONV_GATHER=2) and the patch matrix
HOST_ROUNDING_CASES = [
    ("direct", 1, 64, 3, 37, 70, 3, 3, 1, 1),
    ("gather", 1, 128, 128, 24, 40, 3, 3, 1, 1),
    ("patch", 2, 16, 24, 14, 18, 3, 3, 2, 1),
]


@pytest.mark.gpu
@pytest.mark.parametrize("path,b,c,oc,H,W,kH,kW,s,p", HOST_ROUNDING_CASES)
def test_conv2d_host_image_rounded_on_upload_matches_device(hiplib, monkeypatch, path, b, c, oc, H, W, kH, kW, s, p):
    """A host image goes up rounded to bf16 by the host; the device-pointer call
    rounds the same fp32 image on the device.  Image values sit at and around
    the bf16 rounding ties, so any difference in the rounding shows: the two
    results must be identical on every path."""
    rng = np.random.default_rng(c + oc)
    hi = rng.integers(0x3C00, 0x4100, size=(b, c, H, W), dtype=np.uint32)
    sign = rng.integers(0, 2, size=hi.shape, dtype=np.uint32) << np.uint32(31)
    low = rng.choice(np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32), size=hi.shape)
    x = np.ascontiguousarray(((hi << np.uint32(16)) | low | sign).view(np.float32))
    _, w, bias = gen(14, b, c, oc, H, W, kH, kW)
    monkeypatch.setenv("INV_HIP_CONV_GATHER", "2" if path == "gather" else "0")
    dims = q.QNNConv2DShape(b, oc, H, W, kH, kW, p, s)
    with q.Weight(w) as wt:
        yh = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        xd = q.DeviceArray.from_host(x)
        bd = q.DeviceArray.from_host(bias)
        yd = q.DeviceArray(tuple(dims), "f32")
        try:
            q.conv2d_device(xd, wt, yd, c, oc, H, W, kH, kW, s, p, b, bias=bd)
            y_dev = yd.to_host()
        finally:
            for a in (xd, bd, yd):
                a.free()
    print(f"[conv2d host rounding] {path}: host == device", flush=True)
    np.testing.assert_array_equal(yh, y_dev)
    ref_b = oracle.conv2d_f64(round_bf16(x), w, bias, c, oc, H, W, kH, kW, s, p, b)
    assert oracle.normwise_err(yh, ref_b) <= TOL_BF16


@pytest.mark.gpu
def test_conv2d_patch_gemm_with_a_split_tail(hiplib, monkeypatch):
    """The patch-matrix GEMM with its per-channel row bias, run as whole tiles
    plus a split tail (rounds of 12 tiles forced): the split tiles' finishing
    unit adds the row bias; against the plain grid and the oracle.  4608 pixels
    make 18 tiles of 256 (x 96 channels): 12 whole, 6 split."""
    b, c, oc, H, W, kH, kW, s, p = 1, 128, 96, 72, 64, 3, 3, 1, 1
    x, w, bias = gen(15, b, c, oc, H, W, kH, kW)
    monkeypatch.setenv("INV_HIP_CONV_GATHER", "0")
    monkeypatch.setenv("INV_HIP_TILE_CFG", "16")
    with q.Weight(w) as wt:
        monkeypatch.setenv("INV_HIP_SPLIT_TAIL_SLOTS", "12")
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        monkeypatch.delenv("INV_HIP_SPLIT_TAIL_SLOTS")
        y_plain = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    assert not np.array_equal(y, y_plain)  # the split tiles sum their K halves in another order
    assert oracle.normwise_err(y, y_plain) <= 1e-6
    check(y, x, w, bias, c, oc, H, W, kH, kW, s, p, b)


@pytest.mark.gpu
def test_conv2d_row_chunks_match_one_pass(hiplib):
    # A patch-matrix cap of 1 MiB splits the 64x56 output into bands of rows;
    # every band is a GEMM over its own pixels, so the result is identical.
    b, c, oc, H, W, kH, kW, s, p = 1, 32, 40, 64, 56, 3, 3, 1, 1
    x, w, bias = gen(14, b, c, oc, H, W, kH, kW)
    with q.Weight(w) as wt:
        one = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        os.environ["INV_HIP_CONV_COL_MB"] = "1"
        try:
            banded = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        finally:
            del os.environ["INV_HIP_CONV_COL_MB"]
    np.testing.assert_array_equal(banded, one)
    check(banded, x, w, bias, c, oc, H, W, kH, kW, s, p, b)


@pytest.mark.gpu
def test_conv2d_errors(hiplib):
    x, w, bias = gen(15, 1, 4, 8, 6, 6, 3, 3)
    with q.Weight(w) as wt:
        with pytest.raises(hip.HipError) as e:  # filter is 8 x 36, call asks 8 x 4*1*1
            q.conv2d(x, wt, bias, 4, 8, 6, 6, 1, 1, 1, 0)
        assert e.value.code == hip.INV_ERR_ARG
        with pytest.raises(AssertionError, match="empty output"):  # 7x7 kernel on a 6x6 image, no padding
            q.conv2d(x, np.zeros((8, 4 * 49), np.float32), None, 4, 8, 6, 6, 7, 7, 1, 0)
        with pytest.raises(hip.HipError) as e:  # the same through the C-ABI
            hip.call("inv_hip_conv2d", x.ctypes.data, wt.handle, None, x.ctypes.data, 4, 8, 6, 6, 7, 7, 1, 0, 1, 0)
        assert e.value.code == hip.INV_ERR_ARG
        dst = np.zeros((1, 8, 6, 5), np.float32)  # one column short
        with pytest.raises(AssertionError, match="Incorrect destination size"):
            q.QNNConv2d(dst, x, wt, bias, 4, 8, 6, 6, 3, 3, 1, 1)
        with pytest.raises(hip.HipError):
            hip.call("inv_hip_conv2d", x.ctypes.data, wt.handle, None, dst.ctypes.data, 4, 8, 6, 6, 3, 3, 0, 1, 1, 0)
        # batch 0 is a no-op
        hip.call("inv_hip_conv2d", None, wt.handle, None, None, 4, 8, 6, 6, 3, 3, 1, 1, 0, 0)


# The direct kernel for 3x3 stride-1 convolutions with at most 8 output channels (conv_out):
# ragged tiles (H, W not multiples of 16 x 64), input channels not a multiple of 8, batch 2,
# padding 0, 1 and 2, 1 to 8 output channels (the 3-, 4- and 8-channel instantiations).
DIRECT_SHAPES = [
    (1, 13, 3, 37, 70, 1),
    (2, 16, 8, 20, 129, 1),
    (1, 24, 5, 33, 65, 0),
    (1, 9, 1, 17, 17, 2),
    (1, 16, 4, 23, 40, 1),
    (1, 128, 3, 64, 128, 1),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,c,oc,H,W,p", DIRECT_SHAPES)
def test_conv2d_direct_thin_output(hiplib, monkeypatch, b, c, oc, H, W, p):
    x, w, bias = gen(14, b, c, oc, H, W, 3, 3)
    with q.Weight(w) as wt:
        y = q.conv2d(x, wt, bias, c, oc, H, W, 3, 3, 1, p, b)
        monkeypatch.setenv("INV_HIP_CONV_DIRECT", "0")  # the im2col + GEMM path on the same inputs
        y_gemm = q.conv2d(x, wt, bias, c, oc, H, W, 3, 3, 1, p, b)
    check(y, x, w, bias, c, oc, H, W, 3, 3, 1, p, b)
    # the same bf16 products summed in another order
    assert oracle.normwise_err(y, y_gemm) <= 1e-5


# The implicit GEMM (in_ch a multiple of 64, at least 64 output channels): each k-tile is 64
# channels of one filter tap gathered from an NHWC bf16 copy of the image, the filter reordered
# tap-major.  INV_HIP_CONV_GATHER=2 takes it at sizes where the patch-matrix path would otherwise
# run (too few tiles), and =0 gives that path on the same inputs.  Shapes: 256x128 tiles (up to
# 128 output channels), 256x256 and 256x224 tiles (more), ragged pixel counts, batch 2, stride 2
# without padding (the VAE's downsample), 1x1 (skip connections), a 5x3 filter with padding 2.
GATHER_SHAPES = [
    (1, 64, 128, 24, 20, 3, 3, 1, 1, None),
    (2, 128, 96, 19, 23, 3, 3, 1, 1, None),
    (1, 64, 256, 17, 17, 3, 3, 2, 0, None),
    (1, 128, 320, 16, 20, 1, 1, 1, 0, None),
    (1, 64, 200, 9, 11, 5, 3, 1, 2, None),
    (1, 192, 512, 12, 12, 3, 3, 1, 1, None),
    (1, 128, 512, 13, 14, 3, 3, 1, 1, 16),
    (1, 64, 448, 15, 9, 3, 3, 1, 1, 9),
    (3, 64, 64, 7, 5, 3, 3, 1, 1, None),     # the smallest channel counts, batch 3
    (1, 64, 128, 2, 3, 3, 3, 1, 1, None),    # an image smaller than the window: most taps outside
    (1, 128, 256, 21, 18, 3, 3, 2, 1, None), # stride 2 with padding
    (1, 64, 96, 11, 13, 1, 1, 2, 0, None),   # 1x1 at stride 2 (forced: 1x1 takes the patch path by default)
    (2, 128, 320, 21, 18, 3, 3, 2, 1, 13),   # 256x128 tiles over ragged out_ch, stride 2, batch 2
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,c,oc,H,W,kH,kW,s,p,cfg", GATHER_SHAPES)
def test_conv2d_implicit_gemm(hiplib, monkeypatch, b, c, oc, H, W, kH, kW, s, p, cfg):
    x, w, bias = gen(16, b, c, oc, H, W, kH, kW)
    with q.Weight(w) as wt:
        monkeypatch.setenv("INV_HIP_CONV_GATHER", "2")
        if cfg is not None:
            monkeypatch.setenv("INV_HIP_CONV_GATHER_CFG", str(cfg))
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
        y_nobias = q.conv2d(x, wt, None, c, oc, H, W, kH, kW, s, p, b)
        monkeypatch.setenv("INV_HIP_CONV_GATHER", "0")
        y_col = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    check(y, x, w, bias, c, oc, H, W, kH, kW, s, p, b)
    check(y_nobias, x, w, None, c, oc, H, W, kH, kW, s, p, b)
    # the same bf16 products summed in another order (tap-major against channel-major)
    assert oracle.normwise_err(y, y_col) <= 1e-5


@pytest.mark.gpu
def test_conv2d_implicit_gemm_at_size(hiplib):
    # 128 -> 128 channels at 192x192: 144 tiles of 256x128, the default choice (no override)
    b, c, oc, H, W, kH, kW, s, p = 1, 128, 128, 192, 192, 3, 3, 1, 1
    x, w, bias = gen(17, b, c, oc, H, W, kH, kW)
    with q.Weight(w) as wt:
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    check(y, x, w, bias, c, oc, H, W, kH, kW, s, p, b)
