"""Seeded fuzz of inv_hip_attention against the fp64 oracle (marked gpu): random head counts and
kv-head groupings, ragged query and key lengths (seq_q > seq_k with causal included), head_dim 64
and 128, causal or not, an optional key mask (key 0 kept), fp32 or bf16 inputs and outputs, and
both workgroup shapes (INV_HIP_ATTN_KEY_GROUPS 1 and 2).

Tolerance as in test_gpu_attention.py: 4e-3 normwise against the oracle on the same bf16-rounded
Q, K, V (the softmax weights are rounded to bf16 for the P.V product), plus 2^-8 for bf16 outputs.
Queries that see no key are zeros (checked separately), so the oracle comparison covers the rest.
"""
import math

import numpy as np
import pytest

import oracle
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

pytestmark = pytest.mark.gpu

TOL = 4e-3
TOL_BF16_OUT = 2.0 ** -8


def cases(n=24, seed=7):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kvh = int(rng.choice([1, 2, 3]))
        heads = kvh * int(rng.choice([1, 2, 4]))
        out.append((i, heads, kvh, int(rng.integers(1, 400)), int(rng.integers(1, 400)), int(rng.choice([64, 128])),
                    bool(rng.integers(2)), bool(rng.integers(2)), str(rng.choice(["f32", "bf16"])),
                    str(rng.choice(["f32", "bf16"])), int(rng.choice([1, 2]))))
    return out


@pytest.mark.parametrize("case,heads,kvh,sq,sk,d,causal,masked,xdt,odt,kg", cases())
def test_attention_fuzz(hiplib, monkeypatch, case, heads, kvh, sq, sk, d, causal, masked, xdt, odt, kg):
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(kg))
    oracle.rng_seed(200 + case)
    Q = oracle.randn_scaled((sq, heads * d), 1.0, False)
    K = oracle.randn_scaled((sk, kvh * d), 1.0, False)
    V = oracle.randn_scaled((sk, kvh * d), 1.0, False)
    mask = None
    if masked:
        mask = (np.random.default_rng(case).random(sk) < 0.7).astype(np.int32)
        mask[0] = 1
    ins = (Q, K, V) if xdt == "f32" else tuple(as_bf16_bits(a) for a in (Q, K, V))
    scale = 1.0 / math.sqrt(d)
    O = q.attention(*ins, heads=heads, head_dim=d, kv_heads=kvh, scale=scale, causal=causal, out_dtype=odt,
                    key_mask=mask)
    Of = bf16_bits_to_f32(O) if odt == "bf16" else O
    assert Of.shape == (sq, heads * d) and np.all(np.isfinite(Of))
    # causal with seq_q > seq_k: the first seq_q - seq_k queries see no key and are zero
    first = max(0, sq - sk) if causal else 0
    assert not np.any(Of[:first])
    if first == sq:
        return
    ref = oracle.attention_f64(round_bf16(Q), round_bf16(K), round_bf16(V), heads, kvh, d, scale, causal,
                               key_mask=mask)
    e = oracle.normwise_err(Of[first:], ref[first:])
    print(f"  case {case}: heads {heads}/{kvh} {sq}x{sk} d{d} causal={causal} mask={masked} {xdt}->{odt} "
          f"key groups {kg}: {e:.3e}", flush=True)
    assert e <= TOL + (TOL_BF16_OUT if odt == "bf16" else 0.0)
