"""Per-head RMSNorm and rotary embedding between the Q/K projections and
attention: inv_hip_head_norm_rope against the oracle (QNNQKRMSNorm /
QNNHeadRSMNorm, src/quicknncpu.pas:2209-2246, src/quicknn_qwen3.pas:223-230;
QNNApplyRoPE2D, src/quicknncpu.pas:2968-2992; QNNApplyRoPE3 -> QNNApplyRoPE2,
:2892-2917).

Everything is fp32 on both sides; the GPU's sum of squares is a wave tree
instead of a sequential sum and the products may fuse, so the bound is 1e-5
normwise (measured ~1e-7).  A wrong pairing, the opposite rotation or a norm
over the whole row miss it by orders of magnitude (the oracle tests plant them).
"""
import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q

TOL = 1e-5


def tables(seq, width, seed):
    th = np.random.default_rng(seed).uniform(-np.pi, np.pi, (seq, width))
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)


def gen(seed, seq, heads, d, mode):
    oracle.rng_seed(seed)
    x = oracle.randn_scaled((seq, heads * d), 2.0, False).astype(np.float32)
    w = (np.float32(1.0) + oracle.randn_scaled((d,), 0.1, False)).astype(np.float32)
    width = d if mode == "interleaved" else d // 2
    c, s = tables(seq, width, seed + 1)
    return x, w, c, s


def reference(x, w, c, s, heads, d, mode):
    y = oracle.head_rmsnorm(x, w, heads, d) if w is not None else x
    return oracle.rope(y, c, s, heads, d, mode) if mode is not None else y


@pytest.mark.gpu
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("mode,norm", [("interleaved", True), ("half", True), (None, True), ("interleaved", False),
                                       ("half", False)])
def test_head_norm_rope_matches_oracle(hiplib, d, mode, norm):
    seq, heads = 37, 5
    x, w, c, s = gen(90, seq, heads, d, mode or "half")
    w = w if norm else None
    y = x.copy()
    q.head_norm_rope(y, heads, d, w, mode, c, s)
    ref = reference(x, w, c, s, heads, d, mode)
    assert oracle.normwise_err(y, ref) <= TOL


@pytest.mark.gpu
def test_flux2_joint_sequence_qk(hiplib):
    """FLUX2-Klein-4B: 4096 image + 512 text tokens, 24 heads of 128, QK norm
    then the interleaved (2-D axes) rotary embedding."""
    seq, heads, d = 4608, 24, 128
    x, w, c, s = gen(91, seq, heads, d, "interleaved")
    y = x.copy()
    q.head_norm_rope(y, heads, d, w, "interleaved", c, s)
    rows = np.unique(np.linspace(0, seq - 1, 40).astype(int))
    ref = reference(x[rows], w, c[rows], s[rows], heads, d, "interleaved")
    assert oracle.normwise_err(y[rows], ref) <= TOL


@pytest.mark.gpu
def test_qwen3_mirrors(hiplib):
    """Qwen3-4B: 512 tokens, 32 query heads and 8 kv heads of 128; the mirrors
    of the reference's calls, argument for argument."""
    seq, hq, hk, d = 512, 32, 8, 128
    Q, wq, c, s = gen(92, seq, hq, d, "half")
    K, wk, _, _ = gen(93, seq, hk, d, "half")
    Qn, Kn = np.empty_like(Q), np.empty_like(K)
    q.QNNHeadRSMNorm(Qn, Q, wq, seq, hq, d)
    q.QNNHeadRSMNorm(Kn, K, wk, seq, hk, d)
    q.QNNApplyRoPE3(Qn, c, s, seq, hq, d)
    q.QNNApplyRoPE3(Kn, c, s, seq, hk, d)
    assert oracle.normwise_err(Qn, reference(Q, wq, c, s, hq, d, "half")) <= TOL
    assert oracle.normwise_err(Kn, reference(K, wk, c, s, hk, d, "half")) <= TOL


@pytest.mark.gpu
def test_flux2_mirrors(hiplib):
    seq, heads, d = 300, 6, 128
    Q, wq, c, s = gen(94, seq, heads, d, "interleaved")
    K, wk, _, _ = gen(95, seq, heads, d, "interleaved")
    Qg, Kg = Q.copy(), K.copy()
    q.QNNQKRMSNorm(Qg, Kg, wq, wk, seq, heads, d)
    q.QNNApplyRoPE2D(Qg, c, s, seq, heads, d, 32)
    q.QNNApplyRoPE2D(Kg, c, s, seq, heads, d, 32)
    assert oracle.normwise_err(Qg, reference(Q, wq, c, s, heads, d, "interleaved")) <= TOL
    assert oracle.normwise_err(Kg, reference(K, wk, c, s, heads, d, "interleaved")) <= TOL


@pytest.mark.gpu
def test_device_pointers_match_host_path(hiplib):
    seq, heads, d = 129, 3, 64
    x, w, c, s = gen(96, seq, heads, d, "interleaved")
    y = x.copy()
    q.head_norm_rope(y, heads, d, w, "interleaved", c, s)
    xd, wd, cd, sd = (q.DeviceArray.from_host(a, "f32") for a in (x, w, c, s))
    hip.call("inv_hip_head_norm_rope", xd.ptr, seq, heads, d, wd.ptr, hip.INV_ROPE_INTERLEAVED, cd.ptr, sd.ptr,
             hip.INV_FLAG_DEVICE_PTRS)
    np.testing.assert_array_equal(xd.to_host(), y)
    for a in (xd, wd, cd, sd):
        a.free()


@pytest.mark.gpu
def test_head_norm_rope_argument_errors(hiplib):
    lib = hip.load()
    x = np.zeros((4, 96), np.float32)
    c = np.ones((4, 48), np.float32)
    w = np.ones(48, np.float32)
    assert lib.inv_hip_head_norm_rope(x.ctypes.data, 4, 2, 48, w.ctypes.data, 0, None, None, 0) == \
        hip.INV_ERR_UNSUPPORTED and "head_dim" in hip.last_error()
    x = np.zeros((4, 128), np.float32)
    assert lib.inv_hip_head_norm_rope(x.ctypes.data, 4, 2, 64, None, hip.INV_ROPE_HALF, None, None, 0) == \
        hip.INV_ERR_ARG and "tables" in hip.last_error()
    assert lib.inv_hip_head_norm_rope(x.ctypes.data, 4, 2, 64, None, 7, c.ctypes.data, c.ctypes.data, 0) == \
        hip.INV_ERR_ARG and "rope mode" in hip.last_error()
    assert lib.inv_hip_head_norm_rope(x.ctypes.data, 4, 2, 64, None, 0, None, None, 0) == hip.INV_OK  # nothing to do


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,sq,sk,d,mode,causal", [
    (24, 24, 300, 428, 128, "interleaved", False),   # FLUX2-like joint: image queries over text + image keys
    (32, 8, 257, 257, 128, "half", True),            # Qwen3: grouped kv heads, causal
    (4, 2, 70, 90, 64, "interleaved", True),
])
def test_fused_qk_prep_attention_equals_the_two_steps(hiplib, heads, kv_heads, sq, sk, d, mode, causal):
    """One call (norm + rotary applied while Q and K are staged) gives bit for bit
    what head_norm_rope on Q and K followed by attention gives, and matches the
    oracle's norm -> rotary -> attention chain."""
    import math
    Q, wq, qc, qs = gen(97, sq, heads, d, mode)
    K, wk, kc, ks = gen(98, sk, kv_heads, d, mode)
    V, _, _, _ = gen(99, sk, kv_heads, d, mode)
    fused = q.attention_qk_norm_rope(Q, K, V, heads, d, kv_heads, causal=causal, q_norm_weight=wq,
                                     k_norm_weight=wk, rope=mode, q_cos=qc, q_sin=qs, k_cos=kc, k_sin=ks)
    Qs, Ks = Q.copy(), K.copy()
    q.head_norm_rope(Qs, heads, d, wq, mode, qc, qs)
    q.head_norm_rope(Ks, kv_heads, d, wk, mode, kc, ks)
    two = q.attention(Qs, Ks, V, heads=heads, head_dim=d, kv_heads=kv_heads, causal=causal)
    np.testing.assert_array_equal(fused, two)
    Qo = reference(Q, wq, qc, qs, heads, d, mode)
    Ko = reference(K, wk, kc, ks, kv_heads, d, mode)
    from invision_amd.bf16 import round_bf16
    r64 = oracle.attention_f64(round_bf16(Qo), round_bf16(Ko), round_bf16(V), heads, kv_heads, d, 1.0 / math.sqrt(d),
                               causal)
    assert oracle.normwise_err(fused, r64) <= 4e-3


@pytest.mark.gpu
def test_fused_attention_reads_a_fused_qkv_in_place(hiplib):
    """Q, K and V as the three thirds of one [seq x 3*hidden] projection output
    (token stride 3*hidden) give exactly the packed-operand result."""
    seq, heads, d = 200, 3, 64
    hidden = heads * d
    qkv, wq, c, s = gen(100, seq, 3 * heads, d, "interleaved")
    wk = wq[::-1].copy()
    Q, K, V = (np.ascontiguousarray(qkv[:, i * hidden:(i + 1) * hidden]) for i in range(3))
    packed = q.attention_qk_norm_rope(Q, K, V, heads, d, q_norm_weight=wq, k_norm_weight=wk, rope="interleaved",
                                      q_cos=c, q_sin=s, k_cos=c, k_sin=s, causal=True)
    O = np.empty((seq, hidden), np.float32)
    base = qkv.ctypes.data
    hip.call("inv_hip_attention_qk_norm_rope", base, 3 * hidden, base + hidden * 4, 3 * hidden, base + 2 * hidden * 4,
             3 * hidden, O.ctypes.data, hip.INV_DT_F32, heads, heads, seq, seq, d, 1.0 / np.sqrt(d), wq.ctypes.data,
             wk.ctypes.data, hip.INV_ROPE_INTERLEAVED, c.ctypes.data, s.ctypes.data, c.ctypes.data, s.ctypes.data,
             None, hip.INV_ATTN_CAUSAL)
    np.testing.assert_array_equal(O, packed)
    lib = hip.load()
    assert lib.inv_hip_attention_qk_norm_rope(base, hidden - 1, base, 0, base, 0, O.ctypes.data, hip.INV_DT_F32,
                                              heads, heads, seq, seq, d, 0.125, None, None, 0, None, None, None,
                                              None, None, 0) == hip.INV_ERR_ARG
