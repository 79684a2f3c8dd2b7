"""Fused SwiGLU projection: Y = silu(X.Wg^T + bg) * (X.Wu^T + bu) in one GEMM
(the two QNNLINEAR calls and QNNSiluMul of ffnSwigluForward,
src/quicknn_transformers.pas:1331-1334; QNNSiluMul src/quicknncpu.pas:2404-2418)."""
import json
import os

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

TOL_TIGHT = 2e-5          # vs the oracle on the same bf16-rounded X (fp32 accumulation, libm exp)
TOL_BF16_OUT = 2.0 ** -8 + TOL_TIGHT


def gen(seed, M, K, F, bias=True):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 1.0, False)
    Wg = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    Wu = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    bg = oracle.randn_scaled((F,), 0.01, False) if bias else None
    bu = oracle.randn_scaled((F,), 0.01, False) if bias else None
    return X, Wg, Wu, bg, bu


def oracle_swiglu(Xr, Wg, Wu, bg, bu):
    """silu(gate) * up from the oracle's linear layer (pinned) and its exact SiLU."""
    g = oracle.linear_bf16w(Xr, Wg, bg, oracle.EPI_SILU).astype(np.float64)
    u = oracle.linear_bf16w(Xr, Wu, bu, oracle.EPI_NONE).astype(np.float64)
    return g * u


def sample_rows(M, n):
    return np.unique(np.linspace(0, M - 1, num=min(M, n)).astype(int))


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,F,bias", [(300, 1000, 520, True), (64, 512, 256, False), (1, 256, 128, True),
                                        (129, 72, 130, True), (1024, 3072, 1536, True)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_swiglu_matches_oracle(hiplib, M, K, F, bias, out):
    X, Wg, Wu, bg, bu = gen(21, M, K, F, bias)
    with q.Weight.gate_up(Wg, Wu, bg, bu) as w:
        assert (w.N, w.K) == (F, K)
        y = q.linear(as_bf16_bits(X), w, epilogue="swiglu", out_dtype=out)
    yf = bf16_bits_to_f32(y) if out == "bf16" else y
    rows = sample_rows(M, 48)
    ref = oracle_swiglu(round_bf16(X[rows]), Wg, Wu, bg, bu)
    err = oracle.normwise_err(yf[rows], ref)
    print(f"  normwise err vs oracle {err:.3e}", flush=True)
    assert np.all(np.isfinite(yf))
    assert err <= (TOL_BF16_OUT if out == "bf16" else TOL_TIGHT)


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [2, 8, 16, 17, 18])
def test_swiglu_on_every_swiglu_tile(hiplib, monkeypatch, cfg):
    """The SwiGLU epilogue on each tile configuration that splits into gate | up wave columns:
    32x32 MFMA blocks (2, 8) and 16x16 blocks (16: a 16-row block finished 8 rows per wave)."""
    monkeypatch.setenv("INV_HIP_TILE_CFG", str(cfg))
    M, K, F = 333, 1000, 520
    X, Wg, Wu, bg, bu = gen(23, M, K, F, True)
    with q.Weight.gate_up(Wg, Wu, bg, bu) as w:
        y = q.linear(as_bf16_bits(X), w, epilogue="swiglu", out_dtype="f32")
    rows = sample_rows(M, 64)
    err = oracle.normwise_err(y[rows], oracle_swiglu(round_bf16(X[rows]), Wg, Wu, bg, bu))
    print(f"  cfg {cfg}: normwise err vs oracle {err:.3e}", flush=True)
    assert np.all(np.isfinite(y)) and err <= TOL_TIGHT


@pytest.mark.gpu
def test_swiglu_equals_two_projections_and_silu_mul(hiplib):
    """The fused result against the unfused path through the same library."""
    M, K, F = 200, 640, 384
    X, Wg, Wu, bg, bu = gen(22, M, K, F)
    Xb = as_bf16_bits(X)
    with q.Weight.gate_up(Wg, Wu, bg, bu) as w, q.Weight(Wg, bg) as wg, q.Weight(Wu, bu) as wu:
        y = q.linear(Xb, w, epilogue="swiglu")
        g = q.linear(Xb, wg).astype(np.float64)
        u = q.linear(Xb, wu).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    assert oracle.normwise_err(y, ref) <= 1e-6


@pytest.mark.gpu
def test_swiglu_deviation_from_reference_silu_is_its_approximation(hiplib):
    """The reference's sSiLU_avx2 gated form (restated as orc_silu_qnn) differs by
    its exp approximation only: the documented ~1.7e-3, not more."""
    M, K, F = 64, 1024, 256
    X, Wg, Wu, bg, bu = gen(23, M, K, F)
    with q.Weight.gate_up(Wg, Wu, bg, bu) as w:
        y = q.linear(as_bf16_bits(X), w, epilogue="swiglu")
    Xr = round_bf16(X)
    g = oracle.linear_bf16w(Xr, Wg, bg, oracle.EPI_NONE)
    u = oracle.linear_bf16w(Xr, Wu, bu, oracle.EPI_NONE)
    ref_qnn = oracle.silu_qnn(g, u)[1]
    err = oracle.normwise_err(y, ref_qnn)
    print(f"  vs the reference's approximate SiLU: {err:.3e}", flush=True)
    assert 1e-5 < err < 3e-3


@pytest.mark.gpu
def test_swiglu_precise_fp32_x(hiplib):
    M, K, F = 96, 700, 200
    X, Wg, Wu, bg, bu = gen(24, M, K, F)
    with q.Weight.gate_up(Wg, Wu, bg, bu) as w:
        y = q.linear(X, w, epilogue="swiglu", precise=True)
    ref = oracle_swiglu(X.astype(np.float32), Wg, Wu, bg, bu)  # fp32 X, no rounding
    assert oracle.normwise_err(y, ref) <= 2e-5


@pytest.mark.gpu
def test_swiglu_argument_errors(hiplib):
    X, Wg, Wu, bg, bu = gen(25, 8, 64, 128)
    with q.Weight.gate_up(Wg, Wu) as w, q.Weight(Wg) as plain:
        with pytest.raises(hip.HipError, match="needs INV_EPI_SWIGLU"):
            q.linear(as_bf16_bits(X), w)
        with pytest.raises(hip.HipError, match="needs a gate/up weight"):
            q.linear(as_bf16_bits(X), plain, epilogue="swiglu")
        with pytest.raises(hip.HipError, match="takes its biases at upload"):
            q.linear(as_bf16_bits(X), w, bias=np.zeros(128, np.float32), epilogue="swiglu")


@pytest.mark.gpu
def test_swiglu_from_fused_safetensors_tensor(hiplib, tmp_path):
    """FLUX2's linear_in: one [2F x K] tensor, gate rows first (src/quicknn_transformers.pas:595-597)."""
    M, K, F = 40, 96, 160
    X, Wg, Wu, bg, bu = gen(26, M, K, F)
    fused = np.concatenate([Wg, Wu]).astype("<u2")
    b = np.concatenate([bg, bu]).astype("<f4")
    hdr = {"linear_in.weight": {"dtype": "BF16", "shape": [2 * F, K], "data_offsets": [0, fused.nbytes]},
           "linear_in.bias": {"dtype": "F32", "shape": [2 * F], "data_offsets": [fused.nbytes, fused.nbytes + b.nbytes]}}
    hj = json.dumps(hdr).encode()
    path = os.path.join(tmp_path, "ffn.safetensors")
    with open(path, "wb") as f:
        f.write(len(hj).to_bytes(8, "little") + hj + fused.tobytes() + b.tobytes())
    with q.Weight.from_safetensors(path, "linear_in.weight", "linear_in.bias", gate_up=True) as wf, \
            q.Weight.gate_up(Wg, Wu, bg, bu) as wa:
        Xb = as_bf16_bits(X)
        np.testing.assert_array_equal(q.linear(Xb, wf, epilogue="swiglu"), q.linear(Xb, wa, epilogue="swiglu"))
