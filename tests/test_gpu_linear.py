"""GPU parity of libinvision_hip.so against the CPU oracle (marked gpu).

Parity rule: normwise max|y - r| / max|r| <= 2e-3 against
the reference's linear layer as it computes it (fp32 activations), and, to
catch kernel bugs, <= 2e-5 against the oracle fed the same bf16-rounded
activations the HIP path uses (round to nearest even).  Full-size shapes are
checked on a seeded sample of rows (rows of X . W^T only depend on the same
rows of X, so the sample is exact), plus determinism and finiteness of the
whole output.

Inputs: the reference RNG restated (quicknn_sample.pas:212-276), drawn in the
order X ~ N(0,1), W ~ N(0,0.02) (bf16), bias ~ N(0,0.01).
"""
import os

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

pytestmark = pytest.mark.gpu

TOL_REF = 2e-3    # vs the reference's fp32-activation linear (north star), K >= 1024
TOL_TIGHT = 2e-5  # vs the oracle on the same bf16-rounded activations
TOL_BF16_OUT = 2.0 ** -8 + TOL_TIGHT  # bf16 output: half an ulp is up to 2^-8 of the value


def gen(seed, M, K, N, x_scale=1.0, w_scale=0.02, b_scale=0.01):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), x_scale, False)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), w_scale, False))
    b = oracle.randn_scaled((N,), b_scale, False)
    return X, W, b


EPI_ORACLE = {"none": oracle.EPI_NONE, "silu": oracle.EPI_SILU, "gelu": oracle.EPI_GELU}


def oracle_linear(X, W, b, epi="none", rows=None):
    Xr = X if rows is None else X[rows]
    return oracle.linear_bf16w(Xr, W, b, EPI_ORACLE[epi])


def check(y, X, W, b, epi="none", rows=None, tight=TOL_TIGHT, ref_tol=TOL_REF):
    """Tight check against the oracle on bf16-rounded X, and the north-star
    check against the fp32-X reference.  The latter is asserted for K >= 1024
    (every workload shape has K >= 2560): rounding X to bf16 costs ~1.5e-3 at
    K = 3072 but can exceed 2e-3 when a handful of products make up each
    output; small-K shapes assert it on the INV_FLAG_PRECISE path instead."""
    ys = y if rows is None else y[rows]
    r_tight = oracle_linear(round_bf16(X), W, b, epi, rows)
    e_tight = oracle.normwise_err(ys, r_tight)
    r_ref = oracle_linear(X, W, b, epi, rows)
    e_ref = oracle.normwise_err(ys, r_ref)
    print(f"  normwise err: vs bf16-X oracle {e_tight:.3e} (tol {tight}), vs fp32-X reference {e_ref:.3e} "
          f"(tol {ref_tol} for K >= 1024)", flush=True)
    assert np.all(np.isfinite(ys))
    assert e_tight <= tight
    if X.shape[1] >= 1024:
        assert e_ref <= ref_tol
    return e_tight, e_ref


def sample_rows(M, n=48, seed=0):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(n, M), replace=False)]))
    return rows


# ------------------------------------------------------------ small & ragged

SMALL = [
    (1, 8, 8), (2, 16, 4), (3, 24, 5), (5, 7, 3), (17, 19, 23), (31, 64, 33), (33, 96, 130), (64, 128, 64),
    (65, 200, 257), (128, 64, 300), (129, 1000, 96), (250, 72, 510), (257, 256, 257), (300, 40, 1024),
]


@pytest.mark.parametrize("M,K,N", SMALL)
def test_linear_small_ragged_shapes(hiplib, M, K, N):
    X, W, b = gen(1000 + M + K + N, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(X, w)
        yp = q.linear(X, w, precise=True)
    check(y, X, W, b)
    # The split-X path meets the reference bar at every K.
    assert oracle.normwise_err(yp, oracle_linear(X, W, b)) <= TOL_REF


@pytest.mark.parametrize("epi", ["none", "silu", "gelu"])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_linear_epilogues_and_output_types(hiplib, epi, out):
    M, K, N = 200, 320, 264
    X, W, b = gen(7, M, K, N)
    with q.Weight(W) as w:
        y = q.linear(X, w, bias=b, epilogue=epi, out_dtype=out)
    if out == "f32":
        check(y, X, W, b, epi)
    else:
        yf = bf16_bits_to_f32(y)
        ref = oracle_linear(round_bf16(X), W, b, epi)
        # bf16 output: each element is within half a bf16 ulp of the fp32 result
        assert oracle.normwise_err(yf, ref) <= TOL_BF16_OUT
        same = np.mean(y == oracle.f32_to_bf16_rne(ref))
        print(f"  bf16 outputs equal to RNE(oracle): {same:.5f}", flush=True)
        assert same > 0.999


def test_golden_linear_fixtures(hiplib):
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "linear_small.npz"), allow_pickle=False)
    epi_name = {oracle.EPI_NONE: "none", oracle.EPI_SILU: "silu", oracle.EPI_GELU: "gelu"}
    for i, (M, K, N, has_bias, epi) in enumerate(fx["cases"]):
        X, W, b, Y = fx[f"X{i}"], fx[f"W{i}"], fx[f"b{i}"], fx[f"Y{i}"]
        with q.Weight(W) as w:
            y = q.linear(X, w, bias=b if has_bias else None, epilogue=epi_name[int(epi)])
        # X in the fixture is already bf16-exact: only accumulation order differs.
        assert oracle.normwise_err(y, Y) <= TOL_TIGHT, i


@pytest.mark.parametrize("M,K,N", [(64, 200, 96), (300, 1000, 520), (4608, 3072, 256)])
def test_precise_flag_matches_fp32_activation_reference(hiplib, M, K, N):
    # INV_FLAG_PRECISE: X = Xh + Xl, two MFMA passes over the resident W.
    X, W, b = gen(14, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(X, w, precise=True)
        y1 = q.linear(X, w)
    rows = sample_rows(M, 64)
    e = oracle.normwise_err(y[rows], oracle_linear(X, W, b, rows=rows))
    e1 = oracle.normwise_err(y1[rows], oracle_linear(X, W, b, rows=rows))
    print(f"  vs fp32-X reference: precise {e:.3e}, default {e1:.3e}", flush=True)
    assert e <= 3e-5 and e < e1


def test_bf16_activations_in(hiplib):
    M, K, N = 96, 256, 192
    X, W, b = gen(8, M, K, N)
    with q.Weight(W, b) as w:
        y16 = q.linear(as_bf16_bits(X), w)
        y32 = q.linear(X, w)
    np.testing.assert_array_equal(y16, y32)  # fp32 X is rounded RNE on the device


def test_weight_upload_from_fp32_rounds_rne(hiplib):
    M, K, N = 64, 136, 72
    X, W, b = gen(9, M, K, N)
    Wf = bf16_bits_to_f32(W)  # widened bf16: exact in fp32, so rounding is the identity
    with q.Weight(Wf, b) as w32, q.Weight(W, b) as w16:
        np.testing.assert_array_equal(q.linear(X, w32), q.linear(X, w16))
    # A general fp32 weight is rounded to nearest even on upload.
    oracle.rng_seed(99)
    Wg = oracle.randn_scaled((N, K), 0.02, False)
    with q.Weight(Wg, b) as wg, q.Weight(as_bf16_bits(Wg), b) as wr:
        np.testing.assert_array_equal(q.linear(X, wg), q.linear(X, wr))


# ------------------------------------------------------------ tiles, split-K

GRID_MODES = {  # INV_HIP_MODE / INV_HIP_KSPLIT / INV_HIP_SK_GRID
    "tiles": {"INV_HIP_MODE": "0"},
    "splitk3": {"INV_HIP_MODE": "1", "INV_HIP_KSPLIT": "3"},
    "streamk256": {"INV_HIP_MODE": "2", "INV_HIP_SK_GRID": "256"},
    "streamk37": {"INV_HIP_MODE": "2", "INV_HIP_SK_GRID": "37"},
}


ALL_CFGS = list(range(19))  # INV_GEMM_NUM_CONFIGS in invision_amd/csrc/gemm_configs.hpp
REG_STAGED_CFGS = [8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18]  # 11-14, 16, 18: unequal W and X copy-chunk counts


@pytest.mark.parametrize("cfg", ALL_CFGS)
@pytest.mark.parametrize("grid", sorted(GRID_MODES))
def test_every_tile_shape_and_grid_mode(hiplib, monkeypatch, cfg, grid):
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    for k, v in GRID_MODES[grid].items():
        monkeypatch.setenv(k, v)
    M, K, N = 300, 1000, 520
    X, W, b = gen(10, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(X, w, epilogue="silu")
        y2 = q.linear(X, w, epilogue="silu")
    check(y, X, W, b, "silu")
    np.testing.assert_array_equal(y, y2)  # deterministic, counters reset


@pytest.mark.parametrize("cfg", [8, 13, 15, 16, 17, 18])
@pytest.mark.parametrize("grid", ["splitk3", "streamk37"])
def test_shared_tiles_bf16_out_and_gelu(hiplib, monkeypatch, cfg, grid):
    """Split- and stream-K tiles with the bf16 output and GELU epilogue."""
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    for k, v in GRID_MODES[grid].items():
        monkeypatch.setenv(k, v)
    M, K, N = 300, 1000, 520
    X, W, b = gen(17, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(X, w, epilogue="gelu", out_dtype="bf16")
    check(bf16_bits_to_f32(y), X, W, b, "gelu", tight=TOL_TIGHT + 2.0 ** -8, ref_tol=TOL_REF + 2.0 ** -8)


# Split tail: the tile grid's whole rounds as tiles, then the last round's tiles split two ways
# along K.  INV_HIP_SPLIT_TAIL_SLOTS=12 makes rounds of 12 tiles, so the 30 tiles of these
# products run as 24 whole tiles and 6 split ones (12 workgroups of half the K loop).
@pytest.mark.parametrize("cfg", [16, 17, 18])
@pytest.mark.parametrize("epi,ydt", [("none", "f32"), ("silu", "bf16"), ("gelu", "f32")])
def test_split_tail_matches_plain_grid_and_oracle(hiplib, monkeypatch, cfg, epi, ydt):
    M, K, N = (900 if cfg == 18 else 1100), 1024, 1300  # 5 x 6 tiles of 224, 256 or 192 X rows
    X, W, b = gen(23, M, K, N)
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
    monkeypatch.setenv("INV_HIP_SPLIT_TAIL_SLOTS", "12")
    with q.Weight(W, b) as w:
        y = q.linear(X, w, epilogue=epi, out_dtype=ydt)
        y2 = q.linear(X, w, epilogue=epi, out_dtype=ydt)
        monkeypatch.setenv("INV_HIP_SPLIT_TAIL", "0")
        y_plain = q.linear(X, w, epilogue=epi, out_dtype=ydt)
    np.testing.assert_array_equal(y, y2)  # deterministic, counters reset
    f = (lambda a: bf16_bits_to_f32(a)) if ydt == "bf16" else (lambda a: a)
    if ydt == "f32":  # the split tiles sum their two K halves in another order than one loop
        assert not np.array_equal(y, y_plain)
    assert oracle.normwise_err(f(y), f(y_plain)) <= (2.0 ** -8 if ydt == "bf16" else 1e-6)
    extra = 2.0 ** -8 if ydt == "bf16" else 0.0
    check(f(y), X, W, b, epi, tight=TOL_TIGHT + extra, ref_tol=TOL_REF + extra)


def test_split_tail_accumulate(hiplib, monkeypatch):
    """Y += gate * (X W^T + b) (beta = 1, Y read in place): the whole tiles and
    the split tiles each read and write only their own rows and columns."""
    M, K, N = 1100, 1024, 1300
    X, W, b = gen(24, M, K, N)
    rng = np.random.default_rng(24)
    Y0 = rng.standard_normal((M, N)).astype(np.float32)
    gate = (rng.standard_normal(N) * 0.5).astype(np.float32)
    monkeypatch.setenv("INV_HIP_TILE_CFG", "16")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
    monkeypatch.setenv("INV_HIP_SPLIT_TAIL_SLOTS", "12")
    with q.Weight(W, b) as w:
        y = Y0.copy()
        q.linear_gated_add(y, X, w, gate)
        monkeypatch.setenv("INV_HIP_SPLIT_TAIL", "0")
        y_plain = Y0.copy()
        q.linear_gated_add(y_plain, X, w, gate)
    assert oracle.normwise_err(y - Y0, y_plain - Y0) <= 1e-6
    ref = gate * oracle.linear_bf16w(round_bf16(X), W, b, oracle.EPI_NONE)
    assert oracle.normwise_err(y - Y0, ref) <= TOL_TIGHT


@pytest.mark.parametrize("cfg", REG_STAGED_CFGS)
@pytest.mark.parametrize("K", [8, 64, 128, 200, 576, 1000, 3072])
def test_register_staged_k_tile_counts(hiplib, monkeypatch, cfg, K):
    """One, two, odd, even and ragged numbers of 64-wide k-tiles (the main loop
    runs two k-tiles per trip and a single one for an odd remainder)."""
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    monkeypatch.setenv("INV_HIP_MODE", "0")
    M, N = 300, 520
    X, W, b = gen(16, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(as_bf16_bits(X), w)
    check(y, X, W, b)


@pytest.mark.parametrize("M,K,N", [(4608, 3072, 9216), (512, 9728, 2560), (777, 1304, 1000)])
def test_stream_k_matches_one_workgroup_per_tile(hiplib, monkeypatch, M, K, N):
    X, W, b = gen(15, M, K, N)
    Xb = as_bf16_bits(X)
    with q.Weight(W, b) as w:
        monkeypatch.setenv("INV_HIP_MODE", "0")
        y0 = q.linear(Xb, w)
        monkeypatch.setenv("INV_HIP_MODE", "2")
        y1 = q.linear(Xb, w)
    # same products, different association across the K split: rounding-level
    assert oracle.normwise_err(y1, y0) < 5e-6
    check(y1, X, W, b, rows=sample_rows(M, 24))


def test_split_k_result_independent_of_split_count(hiplib, monkeypatch):
    M, K, N = 256, 2048, 384
    X, W, b = gen(11, M, K, N)
    outs = []
    with q.Weight(W, b) as w:
        for ks in (1, 2, 4, 8):
            monkeypatch.setenv("INV_HIP_MODE", "1")
            monkeypatch.setenv("INV_HIP_KSPLIT", str(ks))
            monkeypatch.setenv("INV_HIP_TILE_CFG", "3")
            outs.append(q.linear(X, w))
    for o in outs[1:]:
        assert oracle.normwise_err(o, outs[0]) < 1e-6


# ------------------------------------------------------------ workload shapes

def test_c1_single_linear_with_bias(hiplib):
    # X fp32 [256 x 3072], W [3072 x 3072], bias, fp32 out, seed 0.
    M, K, N = 256, 3072, 3072
    X, W, b = gen(0, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(X, w)
    check(y, X, W, b)


def test_c2_fused_qkv_metric_shape(hiplib):
    # 4608 x 3072 x 9216, bf16 X, fp32 out: the headline shape.
    M, K, N = 4608, 3072, 9216
    X, W, b = gen(0, M, K, N)
    Xb = as_bf16_bits(X)
    with q.Weight(W, b) as w:
        y = q.linear(Xb, w)
        y2 = q.linear(Xb, w)
    assert np.all(np.isfinite(y))
    np.testing.assert_array_equal(y, y2)
    rows = sample_rows(M)
    check(y, X, W, b, rows=rows)


def test_c3_mlp_up_silu_then_down(hiplib):
    M, K, F = 4608, 3072, 9216
    oracle.rng_seed(0)
    X = oracle.randn_scaled((M, K), 1.0, False)
    Wu = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    bu = oracle.randn_scaled((F,), 0.01, False)
    Wd = oracle.f32_to_bf16_rne(oracle.randn_scaled((K, F), 0.02, False))
    bd = oracle.randn_scaled((K,), 0.01, False)
    with q.Weight(Wu, bu) as wu, q.Weight(Wd, bd) as wd:
        xd = q.DeviceArray.from_host(as_bf16_bits(X))
        hd = q.DeviceArray((M, F), "bf16")
        yd = q.DeviceArray((M, K), "f32")
        q.linear_device(xd, wu, hd, M, epilogue="silu")
        q.linear_device(hd, wd, yd, M)
        y = yd.to_host()
        H = hd.to_host()
        for d in (xd, hd, yd):
            d.free()
    rows = sample_rows(M, 32)
    Xr = round_bf16(X[rows])
    H_ref = oracle.linear_bf16w(Xr, Wu, bu, oracle.EPI_SILU)
    e_h = oracle.normwise_err(bf16_bits_to_f32(H[rows]), H_ref)
    # The down projection on the device's own bf16 H (an H element whose fp32
    # sum sits near a bf16 tie may round one ulp apart from the oracle's).
    Y_ref = oracle.linear_bf16w(bf16_bits_to_f32(H[rows]), Wd, bd)
    e_y = oracle.normwise_err(y[rows], Y_ref)
    # The reference's chain keeps X and H in fp32; this one rounds both to bf16,
    # and each rounded activation contributes up to TOL_REF.
    H_f = oracle.linear_bf16w(X[rows], Wu, bu, oracle.EPI_SILU)
    Y_f = oracle.linear_bf16w(H_f, Wd, bd)
    e_ref = oracle.normwise_err(y[rows], Y_f)
    print(f"  H err {e_h:.3e}, Y err (on device H) {e_y:.3e}, Y err vs fp32 reference chain {e_ref:.3e}", flush=True)
    assert e_h <= TOL_BF16_OUT and e_y <= TOL_TIGHT and e_ref <= 2 * TOL_REF


def test_c3_chain_with_fp32_h_and_split_activations(hiplib):
    """c3 as the reference runs it, X and H in fp32: the up projection writes fp32 H, and
    both projections take INV_FLAG_PRECISE (each activation split into bf16 hi + lo, two MFMA
    passes over the resident bf16 weights).  Against the reference's fp32 chain this leaves only
    the lo part's own rounding (about 2^-16 relative) and the fp32 summation order, so the chain
    is held to the single-GEMM bar TOL_REF with room to spare (measured ~1e-5)."""
    M, K, F = 4608, 3072, 9216
    oracle.rng_seed(0)
    X = oracle.randn_scaled((M, K), 1.0, False)
    Wu = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    bu = oracle.randn_scaled((F,), 0.01, False)
    Wd = oracle.f32_to_bf16_rne(oracle.randn_scaled((K, F), 0.02, False))
    bd = oracle.randn_scaled((K,), 0.01, False)
    with q.Weight(Wu, bu) as wu, q.Weight(Wd, bd) as wd:
        xd = q.DeviceArray.from_host(np.ascontiguousarray(X, dtype=np.float32))
        hd = q.DeviceArray((M, F), "f32")
        yd = q.DeviceArray((M, K), "f32")
        q.linear_device(xd, wu, hd, M, epilogue="silu", precise=True)
        q.linear_device(hd, wd, yd, M, precise=True)
        y = yd.to_host()
        for d in (xd, hd, yd):
            d.free()
    rows = sample_rows(M, 32)
    H_f = oracle.linear_bf16w(X[rows], Wu, bu, oracle.EPI_SILU)
    Y_f = oracle.linear_bf16w(H_f, Wd, bd)
    e_ref = oracle.normwise_err(y[rows], Y_f)
    print(f"  Y err vs the fp32 reference chain, fp32 H and split activations: {e_ref:.3e}", flush=True)
    assert e_ref <= TOL_REF / 10


@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_c4_qwen3_small_m_split_k(hiplib, which):
    M = 512
    K, N = (2560, 9728) if which == "gate_up" else (9728, 2560)
    X, W, _ = gen(4, M, K, N)
    with q.Weight(W) as w:
        y = q.linear(as_bf16_bits(X), w)
        y2 = q.linear(as_bf16_bits(X), w)
    np.testing.assert_array_equal(y, y2)
    check(y, X, W, None, rows=sample_rows(M, 64))


def test_c5_adaln_modulation_m2(hiplib):
    M, K, N = 2, 3840, 6 * 3840
    X, W, b = gen(5, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(as_bf16_bits(X), w)
    check(y, X, W, b)


def test_c5_zimage_qkv_batched_cfg(hiplib):
    M, K, N = 2 * 4608, 3840, 11520
    X, W, b = gen(6, M, K, N)
    with q.Weight(W, b) as w:
        y = q.linear(as_bf16_bits(X), w)
    check(y, X, W, b, rows=sample_rows(M, 32))


@pytest.mark.parametrize("which", ["out", "mlp_up", "mlp_down"])
def test_c5_zimage_block_projections_batched_cfg(hiplib, which):
    """The rest of a Z-Image block's GEMMs over 2 CFG branches (M = 2 x 4608): the attention
    out-projection [3840 x 3840] and the MLP up [15360 x 3840] / down [3840 x 15360]
    (src/quicknn_transformers.pas:2272, 2286-2295), with bias, bf16 X, fp32 Y; sampled rows
    against the oracle plus a bit-for-bit repeat."""
    M = 2 * 4608
    K, N = {"out": (3840, 3840), "mlp_up": (3840, 15360), "mlp_down": (15360, 3840)}[which]
    X, W, b = gen(7, M, K, N)
    Xb = as_bf16_bits(X)
    with q.Weight(W, b) as w:
        xd = q.DeviceArray.from_host(Xb, "bf16")
        yd = q.DeviceArray((M, N), "f32")
        q.linear_device(xd, w, yd, M)
        y = yd.to_host()
        q.linear_device(xd, w, yd, M)
        np.testing.assert_array_equal(yd.to_host(), y)
        xd.free()
        yd.free()
    check(y, X, W, b, rows=sample_rows(M, 32))


# ------------------------------------------------------------ device pointers

def test_device_pointer_path_matches_host_path(hiplib):
    M, K, N = 333, 512, 640
    X, W, b = gen(12, M, K, N)
    with q.Weight(W, b) as w:
        y_host = q.linear(X, w)
        xd = q.DeviceArray.from_host(X, "f32")
        yd = q.DeviceArray((M, N), "f32")
        q.linear_device(xd, w, yd, M, asynchronous=True)
        hip.call("inv_hip_synchronize")
        np.testing.assert_array_equal(yd.to_host(), y_host)
        bd = q.DeviceArray.from_host(b, "f32")
        with q.Weight(W) as w_nobias:
            q.linear_device(xd, w_nobias, yd, M, bias=bd)
        np.testing.assert_array_equal(yd.to_host(), y_host)
        for d in (xd, yd, bd):
            d.free()


# ------------------------------------------------------------ errors

def test_error_paths_return_status_not_abort(hiplib):
    lib = hip.load()
    X, W, b = gen(13, 8, 16, 8)
    with q.Weight(W) as w:
        y = np.zeros((8, 8), np.float32)
        assert lib.inv_hip_linear(X.ctypes.data, 3, w.handle, None, y.ctypes.data, 3, 8, 17, 8, 0, 0) == hip.INV_ERR_ARG
        assert "mismatch" in hip.last_error()
        assert lib.inv_hip_linear(X.ctypes.data, 9, w.handle, None, y.ctypes.data, 3, 8, 16, 8, 0, 0) == hip.INV_ERR_ARG
        assert lib.inv_hip_linear(X.ctypes.data, 3, w.handle, None, y.ctypes.data, 3, 8, 16, 8, 7, 0) == hip.INV_ERR_ARG
        assert lib.inv_hip_linear(None, 3, w.handle, None, y.ctypes.data, 3, 8, 16, 8, 0, 0) == hip.INV_ERR_ARG
        assert lib.inv_hip_linear(X.ctypes.data, 3, w.handle, None, y.ctypes.data, 3, 8, 16, 8, 0, 2) == hip.INV_ERR_ARG
        stale = w.handle
    assert lib.inv_hip_linear(X.ctypes.data, 3, stale, None, y.ctypes.data, 3, 8, 16, 8, 0, 0) == hip.INV_ERR_ARG
    assert "unknown weight" in hip.last_error()
    # M = 0 is a no-op
    with q.Weight(W) as w:
        assert lib.inv_hip_linear(X.ctypes.data, 3, w.handle, None, y.ctypes.data, 3, 0, 16, 8, 0, 0) == hip.INV_OK


# ------------------------------------------------------------ failure handling

def test_allocation_cap_returns_oom_from_every_entry_point(hiplib, monkeypatch):
    """INV_HIP_ALLOC_LIMIT_MB caps what the library allocates after inv_hip_init: the linear layer,
    attention and convolution entry points report INV_ERR_OOM (with the cap in the message) where
    their staging would pass it, and nothing is left half-done (the reference's bind-time fallback,
    src/quicknncpu.pas:3951-3980, needs a clean status to fall back on)."""
    import ctypes
    lib = hip.load()
    q.shutdown()
    monkeypatch.setenv("INV_HIP_ALLOC_LIMIT_MB", "48")
    try:
        q.init()
        X, W, b = gen(41, 64, 256, 128)
        with q.Weight(W, b) as w:  # small: under the cap
            y = q.linear(X, w)
            check(y, X, W, b)
        # fp32 X of 8192 x 4096 needs a 64 MiB bf16 operand (rounded on the host): refused
        M, K = 8192, 4096
        Xb = np.zeros((M, K), np.float32)
        Wb = np.zeros((16, K), np.uint16)
        with q.Weight(Wb) as w:
            Y = np.zeros((M, 16), np.float32)
            rc = lib.inv_hip_linear(Xb.ctypes.data, hip.INV_DT_F32, w.handle, None, Y.ctypes.data, hip.INV_DT_F32,
                                    M, K, 16, 0, 0)
            assert rc == hip.INV_ERR_OOM and "INV_HIP_ALLOC_LIMIT_MB" in hip.last_error(), hip.last_error()
        # attention over 8192 tokens x 16 heads x 128 needs ~3 x 32 MiB of staged operands
        S, H, D = 8192, 16, 128
        Q = np.zeros((S, H * D), np.float32)
        O = np.zeros((S, H * D), np.float32)
        rc = lib.inv_hip_attention(Q.ctypes.data, Q.ctypes.data, Q.ctypes.data, O.ctypes.data, hip.INV_DT_F32,
                                   hip.INV_DT_F32, H, H, S, S, D, ctypes.c_float(0.088), 0)
        assert rc == hip.INV_ERR_OOM and "INV_HIP_ALLOC_LIMIT_MB" in hip.last_error(), hip.last_error()
        # a convolution whose patch matrix (64 x 9 x 512 x 512 x 2 bytes) passes the cap
        cin, cout, HW = 64, 8, 512
        with q.Weight(np.zeros((cout, cin * 9), np.float32)) as wc:
            img = np.zeros((1, cin, HW, HW), np.float32)
            out = np.zeros((1, cout, HW, HW), np.float32)
            rc = lib.inv_hip_conv2d(img.ctypes.data, wc.handle, None, out.ctypes.data, cin, cout, HW, HW, 3, 3, 1, 1,
                                    1, 0)
            assert rc == hip.INV_ERR_OOM and "INV_HIP_ALLOC_LIMIT_MB" in hip.last_error(), hip.last_error()
        # a weight past the cap, and a device buffer past it
        h = ctypes.c_void_p()
        big = np.zeros((8192, 4096), np.uint16)  # 64 MiB
        assert lib.inv_hip_weight_upload(big.ctypes.data, 8192, 4096, None, ctypes.byref(h)) == hip.INV_ERR_OOM
        p = ctypes.c_void_p()
        assert lib.inv_hip_malloc(ctypes.byref(p), 64 << 20) == hip.INV_ERR_OOM
        # the library still works within the cap
        with q.Weight(W, b) as w:
            np.testing.assert_array_equal(q.linear(X, w), y)
    finally:
        q.shutdown()
        monkeypatch.delenv("INV_HIP_ALLOC_LIMIT_MB")
        q.init()


def test_concurrent_calls_are_serialized_and_correct(hiplib):
    """Two host threads calling inv_hip_linear on shared weight handles at once (the reference's
    shared workspace is not safe under concurrency, src/quicknncpu.pas:117, 1842-1844): every call
    returns the same result as a sequential call, and none fails."""
    import threading
    X1, W1, b1 = gen(42, 300, 1000, 520)
    X2, W2, b2 = gen(43, 640, 2048, 1536)
    with q.Weight(W1, b1) as w1, q.Weight(W2, b2) as w2:
        ref1, ref2 = q.linear(X1, w1), q.linear(X2, w2, epilogue="silu")
        errors, results = [], {}

        def worker(tag, x, w, epi, ref, n):
            try:
                for i in range(n):
                    y = q.linear(x, w, epilogue=epi)
                    if not np.array_equal(y, ref):
                        errors.append(f"{tag} call {i}: result differs")
                results[tag] = n
            except Exception as e:  # noqa: BLE001 - reported below
                errors.append(f"{tag}: {e}")

        threads = [threading.Thread(target=worker, args=("a", X1, w1, "none", ref1, 25)),
                   threading.Thread(target=worker, args=("b", X2, w2, "silu", ref2, 25)),
                   threading.Thread(target=worker, args=("c", X1, w1, "none", ref1, 25))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a worker did not finish"
        assert not errors, errors
        assert results == {"a": 25, "b": 25, "c": 25}
