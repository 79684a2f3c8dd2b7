"""Seeded fuzz of inv_hip_conv2d against the fp64 oracle (marked gpu): random channel counts
(multiples of 64 among them, so the implicit GEMM takes part; 1 to 8 output channels for the
direct kernel), image sizes, square and non-square filters, strides 1 and 2, paddings 0 to 2 and
batches 1 to 3, each through the library's own choice of path and, where it applies, the forced
implicit GEMM (INV_HIP_CONV_GATHER=2).

Tolerance as in test_gpu_conv.py: 2e-5 normwise against the oracle on the bf16-rounded image (the
filters are bf16-exact; fp32 accumulation order only).
"""
import numpy as np
import pytest

import oracle
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import round_bf16

pytestmark = pytest.mark.gpu

TOL = 2e-5


def cases(n=20, seed=11):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        c = int(rng.choice([3, 8, 13, 64, 128, 192]))
        oc = int(rng.choice([1, 3, 5, 8, 64, 96, 128, 256]))
        kH, kW = (3, 3) if rng.random() < 0.6 else (int(rng.choice([1, 3, 5])), int(rng.choice([1, 3])))
        s = int(rng.choice([1, 1, 2]))
        p = int(rng.integers(0, 3))
        H, W = int(rng.integers(max(kH, 2), 40)), int(rng.integers(max(kW, 2), 70))
        out.append((i, int(rng.integers(1, 4)), c, oc, H, W, kH, kW, s, p, bool(rng.integers(2))))
    return out


@pytest.mark.parametrize("case,b,c,oc,H,W,kH,kW,s,p,force_gather", cases())
def test_conv2d_fuzz(hiplib, monkeypatch, case, b, c, oc, H, W, kH, kW, s, p, force_gather):
    if force_gather:
        monkeypatch.setenv("INV_HIP_CONV_GATHER", "2")
    oracle.rng_seed(300 + case)
    x = oracle.randn_scaled((b, c, H, W), 1.0, False).astype(np.float32)
    w = oracle.bf16_to_f32(oracle.f32_to_bf16_rne(oracle.randn_scaled((oc, c * kH * kW), 0.05, False)))
    w = np.ascontiguousarray(w, dtype=np.float32)
    bias = oracle.randn_scaled((oc,), 0.01, False).astype(np.float32)
    with q.Weight(w) as wt:
        y = q.conv2d(x, wt, bias, c, oc, H, W, kH, kW, s, p, b)
    ref = oracle.conv2d_f64(round_bf16(x), w, bias, c, oc, H, W, kH, kW, s, p, b)
    e = oracle.normwise_err(y, ref)
    print(f"  case {case}: b{b} c{c} oc{oc} {H}x{W} k{kH}x{kW} s{s} p{p} gather={force_gather}: {e:.3e}", flush=True)
    assert y.shape == ref.shape and np.all(np.isfinite(y))
    assert e <= TOL
