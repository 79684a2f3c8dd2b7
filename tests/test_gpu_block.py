"""One FLUX2 double-block image stream through the library, against the
oracle's chain of the reference's steps (src/quicknn_transformers.pas:
1400-1460): AdaLN -> Q/K/V projection -> QK RMSNorm + 2-D RoPE -> attention ->
output projection and gated residual add -> AdaLN -> SwiGLU MLP -> gated
residual add.  The library path: inv_hip_linear_norm (AdaLN fused into the QKV
GEMM's operand staging), inv_hip_attention_qk_norm_rope, inv_hip_linear_gated_add,
inv_hip_linear_norm with the gate/up weight and the SwiGLU epilogue,
inv_hip_linear_gated_add.

The oracle chain rounds to bf16 exactly where the library does (each GEMM's
activation operand, attention's Q, K and V), so what remains is accumulation
order and the bf16 softmax weights: the residual update is asserted to 5e-3
normwise (measured 1.7e-3), the attention output to the attention bound 4e-3 (measured 1.3e-3).
"""
import math

import numpy as np
import pytest

import oracle
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import round_bf16


def gen(seed, seq, hidden, F, d):
    oracle.rng_seed(seed)
    r = lambda shape, s: oracle.randn_scaled(shape, s, False).astype(np.float32)
    w = lambda shape: oracle.f32_to_bf16_rne(oracle.randn_scaled(shape, 0.03, False))
    x = r((seq, hidden), 1.0)
    mod = {k: r((hidden,), 0.1) for k in ("shift1", "scale1", "gate1", "shift2", "scale2", "gate2")}
    Wqkv, Wo, Wg, Wu, Wd = w((3 * hidden, hidden)), w((hidden, hidden)), w((F, hidden)), w((F, hidden)), w((hidden, F))
    bo, bd = r((hidden,), 0.01), r((hidden,), 0.01)
    qw, kw = (np.float32(1.0) + r((d,), 0.1) for _ in range(2))
    th = np.random.default_rng(seed).uniform(-np.pi, np.pi, (seq, d // 2)).repeat(2, axis=1)
    return x, mod, (Wqkv, Wo, Wg, Wu, Wd, bo, bd, qw, kw), (np.cos(th).astype(np.float32), np.sin(th).astype(np.float32))


@pytest.mark.gpu
def test_flux2_double_block_image_stream(hiplib):
    seq, heads, d, F = 256, 4, 128, 1024
    hidden = heads * d
    x, m, (Wqkv, Wo, Wg, Wu, Wd, bo, bd, qw, kw), (ct, st) = gen(120, seq, hidden, F, d)
    scale = 1.0 / math.sqrt(d)

    # ---- the library
    y = x.copy()
    with q.Weight(Wqkv) as wqkv, q.Weight(Wo, bo) as wo, q.Weight.gate_up(Wg, Wu) as wgu, q.Weight(Wd, bd) as wd:
        qkv = q.linear_norm(y, "adaln", wqkv, m["scale1"], m["shift1"])
        Q, K, V = (np.ascontiguousarray(qkv[:, i * hidden:(i + 1) * hidden]) for i in range(3))
        attn = q.attention_qk_norm_rope(Q, K, V, heads, d, q_norm_weight=qw, k_norm_weight=kw, rope="interleaved",
                                        q_cos=ct, q_sin=st, k_cos=ct, k_sin=st)
        q.linear_gated_add(y, attn, wo, m["gate1"])
        h = q.linear_norm(y, "adaln", wgu, m["scale2"], m["shift2"], epilogue="swiglu")
        q.linear_gated_add(y, h, wd, m["gate2"])

    # ---- the oracle chain, rounding where the library rounds
    xn = oracle.adaln(x, m["shift1"], m["scale1"])
    qkv_r = oracle.linear_bf16w(round_bf16(xn), Wqkv)
    Qr, Kr, Vr = (qkv_r[:, i * hidden:(i + 1) * hidden] for i in range(3))
    Qp = oracle.rope(oracle.head_rmsnorm(Qr, qw, heads, d), ct, st, heads, d, "interleaved")
    Kp = oracle.rope(oracle.head_rmsnorm(Kr, kw, heads, d), ct, st, heads, d, "interleaved")
    attn_r = oracle.attention_f64(round_bf16(Qp), round_bf16(Kp), round_bf16(Vr), heads, heads, d, scale)
    attn_r = attn_r.astype(np.float32)
    x1 = oracle.gated_add(x, m["gate1"], oracle.linear_bf16w(round_bf16(attn_r), Wo, bo))
    xn2 = round_bf16(oracle.adaln(x1, m["shift2"], m["scale2"]))
    h_r = (oracle.linear_bf16w(xn2, Wg, None, oracle.EPI_SILU).astype(np.float64) *
           oracle.linear_bf16w(xn2, Wu).astype(np.float64)).astype(np.float32)
    x2 = oracle.gated_add(x1, m["gate2"], oracle.linear_bf16w(round_bf16(h_r), Wd, bd))

    e_attn = oracle.normwise_err(attn, attn_r)
    e_upd = oracle.normwise_err(y.astype(np.float64) - x, x2.astype(np.float64) - x)
    print(f"  normwise err: attention {e_attn:.3e}, block update {e_upd:.3e}", flush=True)
    assert np.all(np.isfinite(y))
    assert e_attn <= 4e-3
    assert e_upd <= 5e-3
