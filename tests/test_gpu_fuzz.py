"""Seeded fuzz of inv_hip_linear against the oracle (marked gpu): random shapes across every
tile choice (M from 1 to 1100: the W-streaming, ring, split-K and register-staged tiles; N and
K ragged, K not a multiple of 8), each epilogue, with and without bias, fp32 or bf16 X and Y,
host or device pointers.  Each case is small enough for the float64 oracle over all rows.

Tolerances as in test_gpu_linear.py: 2e-5 normwise against the oracle on the same bf16-rounded X
(fp32 accumulation order only); bf16 outputs add half an ulp, 2^-8.
"""
import numpy as np
import pytest

import oracle
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

pytestmark = pytest.mark.gpu

TOL_TIGHT = 2e-5
TOL_BF16_OUT = 2.0 ** -8 + TOL_TIGHT
EPI = {"none": oracle.EPI_NONE, "silu": oracle.EPI_SILU, "gelu": oracle.EPI_GELU}


def cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 2, 7, 31, 32, 33, 64, 65, 127, 200, 256, 257, 511, 700, 1100]))
        N = int(rng.integers(1, 1300))
        K = int(rng.integers(1, 2100))
        out.append((i, M, K, N, str(rng.choice(list(EPI))), bool(rng.integers(2)), str(rng.choice(["f32", "bf16"])),
                    str(rng.choice(["f32", "bf16"])), bool(rng.integers(2))))
    return out


@pytest.mark.parametrize("case,M,K,N,epi,bias,xdt,ydt,device", cases())
def test_linear_fuzz(hiplib, case, M, K, N, epi, bias, xdt, ydt, device):
    oracle.rng_seed(100 + case)
    X = oracle.randn_scaled((M, K), 1.0, False)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b = oracle.randn_scaled((N,), 0.01, False) if bias else None
    Xin = X.astype(np.float32) if xdt == "f32" else as_bf16_bits(X)
    with q.Weight(W, b) as w:
        if device:
            xd = q.DeviceArray.from_host(Xin, xdt)
            yd = q.DeviceArray((M, N), ydt)
            try:
                q.linear_device(xd, w, yd, M, epilogue=epi)
                y = yd.to_host()
            finally:
                xd.free()
                yd.free()
        else:
            y = q.linear(Xin, w, epilogue=epi, out_dtype=ydt)
    yf = bf16_bits_to_f32(y) if ydt == "bf16" else y
    ref = oracle.linear_bf16w(round_bf16(X), W, b, EPI[epi])
    e = oracle.normwise_err(yf, ref)
    print(f"  case {case}: {M}x{K}x{N} {epi} bias={bias} X {xdt} Y {ydt} device={device}: {e:.3e}", flush=True)
    assert yf.shape == (M, N) and np.all(np.isfinite(yf))
    assert e <= (TOL_BF16_OUT if ydt == "bf16" else TOL_TIGHT)
