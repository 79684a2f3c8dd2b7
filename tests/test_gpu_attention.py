"""Attention forward: inv_hip_attention against the oracle.

The reference computes O = softmax(scale * Q.K^T) V per head in fp32
(src/quicknn_transformers.pas:1150-1311, 2228-2271; src/quicknn_qwen3.pas:
727-769; QNNFlashAttention src/quicknncpu.pas:2763).  The GPU path rounds Q, K
and V to bf16 (nearest-even), accumulates scores in fp32 and rounds the softmax
weights to bf16 for the P.V product (fp32 accumulate).  Tolerances, normwise
(max|err| / max|ref|):
  - 4e-3 against the fp64 oracle on the same bf16-rounded Q, K, V (the bf16
    weights alone measure ~1-1.7e-3 in a CPU emulation of the kernel's rounding);
  - 1.5e-2 against the reference's fp32 path on the unrounded inputs (adds the
    bf16 rounding of Q, K and V: ~4-8e-3 measured the same way);
  - bf16 outputs add their own rounding, 2^-8 relative.
"""
import math

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

TOL_BF16_IN = 4e-3
# Workgroup shapes: 1 = 128 queries, 4 waves over every key tile; 2 = 64 queries, two pairs of
# waves over alternate key tiles whose softmax states merge at the end (the default where the
# 128-query grid has fewer blocks than the chip has CUs, i.e. for most shapes here).
KEY_GROUPS = [1, 2]
TOL_REF = 1.5e-2
TOL_BF16_OUT = 2.0 ** -8


def gen(seed, sq, sk, heads, kv_heads, d):
    oracle.rng_seed(seed)
    Q = oracle.randn_scaled((sq, heads * d), 1.0, False)
    K = oracle.randn_scaled((sk, kv_heads * d), 1.0, False)
    V = oracle.randn_scaled((sk, kv_heads * d), 1.0, False)
    return Q, K, V


def check(O, Q, K, V, heads, kv_heads, d, scale, causal, out="f32", rows=None, ref_path=True, key_mask=None):
    Of = bf16_bits_to_f32(O) if out == "bf16" else O
    if rows is not None:
        Of, Q = Of[rows], Q[rows]
        assert not causal
    Qr, Kr, Vr = round_bf16(Q), round_bf16(K), round_bf16(V)
    r64 = oracle.attention_f64(Qr, Kr, Vr, heads, kv_heads, d, scale, causal, key_mask=key_mask)
    e = oracle.normwise_err(Of, r64)
    extra = TOL_BF16_OUT if out == "bf16" else 0.0
    msg = f"  normwise err: vs oracle on bf16 inputs {e:.3e}"
    if ref_path:
        rq = oracle.attention_qnn(Q, K, V, heads, kv_heads, d, scale, causal, key_mask=key_mask)
        e_ref = oracle.normwise_err(Of, rq)
        msg += f", vs the reference's fp32 path {e_ref:.3e}"
    print(msg, flush=True)
    assert np.all(np.isfinite(Of))
    assert e <= TOL_BF16_IN + extra
    if ref_path:
        assert e_ref <= TOL_REF + extra


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,sq,sk,d,causal", [
    (2, 2, 128, 128, 128, False),
    (3, 3, 200, 333, 128, False),   # ragged query block and key tile
    (2, 2, 384, 512, 128, False),   # joint attention: image queries over text + image keys
    (4, 2, 130, 130, 64, True),     # grouped kv heads, causal
    (8, 2, 257, 257, 128, True),
    (2, 1, 77, 300, 64, False),
    (1, 1, 1, 1, 128, False),
    (2, 2, 5, 70, 64, True),        # causal with more keys than queries (offset 65)
])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("key_groups", KEY_GROUPS)
def test_attention_matches_oracle(hiplib, monkeypatch, heads, kv_heads, sq, sk, d, causal, dtype, key_groups):
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(key_groups))
    Q, K, V = gen(61, sq, sk, heads, kv_heads, d)
    scale = 1.0 / math.sqrt(d)
    ins = (Q, K, V) if dtype == "f32" else tuple(as_bf16_bits(a) for a in (Q, K, V))
    O = q.attention(*ins, heads=heads, head_dim=d, kv_heads=kv_heads, scale=scale, causal=causal)
    check(O, Q, K, V, heads, kv_heads, d, scale, causal)


@pytest.mark.gpu
@pytest.mark.parametrize("d", [64, 128])
def test_attention_bf16_output_and_sharp_softmax(hiplib, d):
    """A larger scale concentrates the weights on few keys (the max-subtraction path)."""
    heads, sq, sk = 2, 160, 200
    Q, K, V = gen(62, sq, sk, heads, heads, d)
    scale = 4.0 / math.sqrt(d)
    O = q.attention(Q, K, V, heads=heads, head_dim=d, scale=scale, out_dtype="bf16")
    check(O, Q, K, V, heads, heads, d, scale, False, out="bf16")


@pytest.mark.gpu
def test_gqa_equals_repeated_kv_heads(hiplib):
    """Grouped kv heads read exactly what repeating each kv head per query head gives."""
    heads, kvh, d, sq, sk = 8, 2, 128, 150, 190
    Q, K, V = gen(63, sq, sk, heads, kvh, d)
    rep = lambda A: np.ascontiguousarray(np.concatenate([A[:, (h // 4) * d:(h // 4 + 1) * d] for h in range(heads)], 1))
    O1 = q.attention(Q, K, V, heads=heads, head_dim=d, kv_heads=kvh, causal=True)
    O2 = q.attention(Q, rep(K), rep(V), heads=heads, head_dim=d, kv_heads=heads, causal=True)
    np.testing.assert_array_equal(O1, O2)


@pytest.mark.gpu
def test_causal_rows_equal_their_prefix(hiplib):
    """Query i of a causal call equals a non-causal call over keys 0 .. i + offset."""
    heads, d, sq, sk = 2, 64, 100, 140
    Q, K, V = gen(64, sq, sk, heads, heads, d)
    O = q.attention(Q, K, V, heads=heads, head_dim=d, causal=True)
    for i in (0, 1, 63, 64, 65, 99):
        n = i + sk - sq + 1
        Oi = q.attention(np.ascontiguousarray(Q[i:i + 1]), np.ascontiguousarray(K[:n]), np.ascontiguousarray(V[:n]),
                         heads=heads, head_dim=d)
        assert oracle.normwise_err(O[i:i + 1], Oi) < 1e-6, i


@pytest.mark.gpu
def test_device_pointers_match_host_path(hiplib):
    heads, d, sq, sk = 3, 128, 140, 260
    Q, K, V = gen(65, sq, sk, heads, heads, d)
    ref = q.attention(Q, K, V, heads=heads, head_dim=d)
    qd, kd, vd = (q.DeviceArray.from_host(as_bf16_bits(a), "bf16") for a in (Q, K, V))
    od = q.DeviceArray((sq, heads * d), "f32")
    q.attention_device(qd, kd, vd, od, heads=heads, head_dim=d, asynchronous=True)
    hip.call("inv_hip_synchronize")
    np.testing.assert_array_equal(od.to_host(), ref)
    for a in (qd, kd, vd, od):
        a.free()


@pytest.mark.gpu
def test_qnn_flash_attention_mirror(hiplib):
    heads, d, sq, sk = 2, 128, 96, 96
    Q, K, V = gen(66, sq, sk, heads, heads, d)
    dst = np.zeros((sq, heads * d), np.float32)
    q.QNNFlashAttention(dst, Q, K, V, heads, sq, sk, d, 1.0 / math.sqrt(d))
    check(dst, Q, K, V, heads, heads, d, 1.0 / math.sqrt(d), False)
    with pytest.raises(AssertionError, match="out of bound"):
        q.QNNFlashAttention(dst, Q, K, V, heads, sq, sk + 1, d, 0.1)


@pytest.mark.gpu
def test_flux2_joint_attention_shape_sampled_rows(hiplib):
    """FLUX2-Klein-4B at 1024x1024: 24 heads of 128, 4096 image + 512 text tokens."""
    heads, d, sq, sk = 24, 128, 4608, 4608
    Q, K, V = gen(67, sq, sk, heads, heads, d)
    Qb, Kb, Vb = (as_bf16_bits(a) for a in (Q, K, V))
    O = q.attention(Qb, Kb, Vb, heads=heads, head_dim=d)
    rows = np.unique(np.linspace(0, sq - 1, 12).astype(int))
    check(O, Q, K, V, heads, heads, d, 1.0 / math.sqrt(d), False, rows=rows, ref_path=False)


@pytest.mark.gpu
def test_attention_argument_errors(hiplib):
    Q, K, V = gen(68, 8, 8, 2, 2, 64)
    lib = hip.load()
    O = np.zeros_like(Q)
    args = lambda **kw: dict(dict(heads=2, kv=2, sq=8, sk=8, d=64, scale=0.125, flags=0), **kw)

    def call(a):
        return lib.inv_hip_attention(Q.ctypes.data, K.ctypes.data, V.ctypes.data, O.ctypes.data, hip.INV_DT_F32,
                                     hip.INV_DT_F32, a["heads"], a["kv"], a["sq"], a["sk"], a["d"], a["scale"],
                                     a["flags"])
    assert call(args(d=96)) == hip.INV_ERR_UNSUPPORTED and "head_dim" in hip.last_error()
    assert call(args(heads=3, kv=2)) == hip.INV_ERR_ARG and "multiple of kv_heads" in hip.last_error()
    assert call(args(sk=0)) == hip.INV_ERR_ARG and "seq_k is 0" in hip.last_error()
    assert call(args(scale=0.0)) == hip.INV_ERR_ARG and "scale" in hip.last_error()
    assert call(args(flags=0x8)) == hip.INV_ERR_ARG and "unknown flags" in hip.last_error()
    assert call(args(sq=0)) == hip.INV_OK
    assert not np.any(O)  # nothing written on error or for zero queries


@pytest.mark.gpu
def test_stats_count_the_evaluated_pairs(hiplib):
    """The library's FLOP counter counts 4 * D FLOPs per evaluated query-key pair
    per head: every pair, or (causal) key j <= i + seq_k - seq_q for query i."""
    heads, d = 2, 64
    for sq, sk, causal in ((5, 70, True), (100, 40, True), (33, 77, False)):
        Q, K, V = gen(69, sq, sk, heads, heads, d)
        hip.call("inv_hip_stats_reset")
        hip.call("inv_hip_stats_enable", 1)
        try:
            q.attention(Q, K, V, heads=heads, head_dim=d, causal=causal)
        finally:
            hip.call("inv_hip_stats_enable", 0)
        pairs = sum(min(sk, max(0, i + sk - sq + 1)) for i in range(sq)) if causal else sq * sk
        assert q.stats()["flops"] == 4.0 * pairs * d * heads


# ------------------------------------------------------------ key mask --

@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,sq,sk,d,causal", [(2, 2, 200, 333, 128, False), (4, 2, 130, 130, 64, True),
                                                          (8, 2, 257, 257, 128, True), (2, 1, 77, 300, 64, False)])
@pytest.mark.parametrize("key_groups", KEY_GROUPS)
def test_key_mask_matches_oracle(hiplib, monkeypatch, heads, kv_heads, sq, sk, d, causal, key_groups):
    """Keys with mask 0 hidden from every query (QNNMatTriangularFill's mask,
    src/quicknncpu.pas:3017-3028): a random mask, key 0 kept so that no causal
    row is empty."""
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(key_groups))
    Q, K, V = gen(70, sq, sk, heads, kv_heads, d)
    mask = (np.random.default_rng(7).random(sk) < 0.7).astype(np.int32)
    mask[0] = 1
    O = q.attention(Q, K, V, heads=heads, head_dim=d, kv_heads=kv_heads, causal=causal, key_mask=mask)
    check(O, Q, K, V, heads, kv_heads, d, 1.0 / math.sqrt(d), causal, key_mask=mask)


@pytest.mark.gpu
def test_padding_mask_equals_the_unpadded_keys(hiplib):
    """Right padding (the Qwen3 encoder's, src/quicknn_qwen3.pas:293-303): masking
    keys n.. gives exactly the attention over the first n keys."""
    heads, d, sq, sk, n = 3, 128, 150, 300, 201
    Q, K, V = gen(71, sq, sk, heads, heads, d)
    mask = (np.arange(sk) < n).astype(np.int32)
    Om = q.attention(Q, K, V, heads=heads, head_dim=d, key_mask=mask)
    On = q.attention(Q, np.ascontiguousarray(K[:n]), np.ascontiguousarray(V[:n]), heads=heads, head_dim=d)
    np.testing.assert_array_equal(Om, On)


@pytest.mark.gpu
@pytest.mark.parametrize("key_groups", KEY_GROUPS)
def test_qwen3_encoder_shape_padded_prompt(hiplib, monkeypatch, key_groups):
    """Qwen3-4B text encoder: 32 query heads over 8 kv heads of 128, 512 tokens,
    causal, a 137-token prompt padded to 512 (padding queries see the prompt)."""
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(key_groups))
    heads, kvh, d, s, n = 32, 8, 128, 512, 137
    Q, K, V = gen(72, s, s, heads, kvh, d)
    mask = (np.arange(s) < n).astype(np.int32)
    O = q.attention(as_bf16_bits(Q), as_bf16_bits(K), as_bf16_bits(V), heads=heads, head_dim=d, kv_heads=kvh,
                    causal=True, key_mask=mask)
    check(O, Q, K, V, heads, kvh, d, 1.0 / math.sqrt(d), True, key_mask=mask)


@pytest.mark.gpu
def test_key_mask_device_pointers_and_empty_rows(hiplib):
    heads, d, sq, sk = 2, 64, 70, 90
    Q, K, V = gen(73, sq, sk, heads, heads, d)
    mask = (np.arange(sk) % 3 != 1).astype(np.int32)
    mask[:5] = 0  # causal queries 0..4 (offset 20: keys up to 24 visible) keep keys 5..
    ref = q.attention(Q, K, V, heads=heads, head_dim=d, causal=True, key_mask=mask)
    qd, kd, vd = (q.DeviceArray.from_host(as_bf16_bits(a), "bf16") for a in (Q, K, V))
    md = q.DeviceArray.from_host(mask)
    od = q.DeviceArray((sq, heads * d), "f32")
    q.attention_device(qd, kd, vd, od, heads=heads, head_dim=d, causal=True, key_mask=md)
    np.testing.assert_array_equal(od.to_host(), ref)
    # every key hidden: zeros (the reference's softmax gives NaN there)
    Oz = q.attention(Q, K, V, heads=heads, head_dim=d, key_mask=np.zeros(sk, np.int32))
    assert not np.any(Oz)
    lib = hip.load()
    bad = lib.inv_hip_attention_masked(qd.ptr, kd.ptr, vd.ptr, od.ptr, hip.INV_DT_BF16, hip.INV_DT_F32, heads, heads,
                                       sq, sk, d, 0.125, md.ptr + 2, hip.INV_FLAG_DEVICE_PTRS)
    assert bad == hip.INV_ERR_ARG and "key_mask" in hip.last_error()
    for a in (qd, kd, vd, md, od):
        a.free()


@pytest.mark.gpu
@pytest.mark.parametrize("key_groups", KEY_GROUPS)
def test_rows_without_keys_are_zero(hiplib, monkeypatch, key_groups):
    """Queries before the diagonal's start (seq_q > seq_k, causal) see no key and
    get zeros, also in waves whose other rows do see keys (their running max
    moves while these rows' stays at -inf), and with two key groups, where one
    group may see keys for a row and the other none."""
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(key_groups))
    heads, d, sq, sk = 2, 64, 300, 100
    Q, K, V = gen(75, sq, sk, heads, heads, d)
    O = q.attention(Q, K, V, heads=heads, head_dim=d, causal=True)
    empty = sq - sk  # query i sees keys up to i - 200
    assert np.all(np.isfinite(O))
    assert not np.any(O[:empty])
    check(O[empty:], Q[empty:], K, V, heads, heads, d, 1.0 / math.sqrt(d), True)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,sq,sk,d,causal", [(32, 8, 512, 512, 128, True), (3, 3, 200, 333, 64, False),
                                                          (2, 2, 64, 1, 128, False), (2, 2, 65, 70, 128, True)])
def test_key_groups_agree(hiplib, monkeypatch, heads, kv_heads, sq, sk, d, causal):
    """The two workgroup shapes against each other and the oracle: one key tile
    (sk = 1: group 1 idle), an odd number of tiles, causal blocks whose groups see
    different numbers of tiles.  They differ by more than summation order: each
    key group rounds its softmax weights to bf16 relative to its own running max,
    so the bound is the bf16-input tolerance."""
    Q, K, V = gen(76, sq, sk, heads, kv_heads, d)
    outs = []
    for kgrp in KEY_GROUPS:
        monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(kgrp))
        outs.append(q.attention(Q, K, V, heads=heads, head_dim=d, kv_heads=kv_heads, causal=causal))
    d12 = oracle.normwise_err(outs[1], outs[0])
    print(f"  one against two key groups: {d12:.3e}", flush=True)
    assert d12 <= TOL_BF16_IN
    check(outs[1], Q, K, V, heads, kv_heads, d, 1.0 / math.sqrt(d), causal)
