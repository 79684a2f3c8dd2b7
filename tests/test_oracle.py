"""Pin the CPU oracle before trusting it (CPU only).

Each restated reference function is checked against something it cannot
agree with by construction if it is wrong: published known-answer vectors, the
reference's own sgemm2.cpp (built under oracle/_ref), an independent library
(numpy float64), closed forms, exact bit identities, or brute force on tiny
inputs.  The last test plants mistakes in oracle inputs and shows the checks
catch them.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- RNG ------

def test_splitmix64_seed0_matches_published_outputs():
    # SplitMix64 from state 0: the first four outputs (Vigna's splitmix64.c),
    # which rng_seed stores as the xoshiro state (quicknn_sample.pas:239-251).
    oracle.rng_seed(0)
    assert oracle.rng_state() == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]


def test_xoshiro256ss_known_answer():
    # Published xoshiro256** outputs from state {1, 2, 3, 4}
    # (the rand_xoshiro crate's reference test vector).
    oracle.rng_set_state([1, 2, 3, 4])
    assert oracle.xoshiro256ss(10) == [
        11520, 0, 1509978240, 1215971899390074240, 1216172134540287360, 607988272756665600,
        16172922978634559625, 8476171486693032832, 10595114339597558777, 2904607092377533576]


def test_rand_is_top53_bits_rounded_to_single():
    oracle.rng_seed(7)
    raw = oracle.xoshiro256ss(64)
    oracle.rng_seed(7)
    got = np.array([oracle.lib().orc_rand() for _ in range(64)], dtype=np.float32)
    want = np.array([(r >> 11) / 9007199254740992.0 for r in raw], dtype=np.float64).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_box_muller_pairs_u1_then_u2_cos_branch():
    oracle.rng_seed(11)
    us = [oracle.lib().orc_rand() for _ in range(40)]
    oracle.rng_seed(11)
    z = oracle.randn(20)
    for i in range(20):
        u1, u2 = np.float32(us[2 * i]), np.float32(us[2 * i + 1])
        assert u1 != 0.0
        want = np.float32(math.sqrt(-2.0 * math.log(float(u1))) * math.cos(2.0 * math.pi * float(u2)))
        assert z[i] == want, (i, z[i], want)


def test_normal_moments():
    oracle.rng_seed(0)
    z = oracle.randn(1_000_000).astype(np.float64)
    assert abs(z.mean()) < 5e-3
    assert abs(z.var() - 1.0) < 1e-2
    assert abs(np.mean(z ** 3)) < 2e-2  # symmetric


def test_rng_fixture_self_consistency():
    with open(os.path.join(GOLDEN, "rng_seed0.json")) as f:
        fx = json.load(f)
    for seed, rec in fx.items():
        oracle.rng_seed(int(seed))
        assert [f"{s:016x}" for s in oracle.rng_state()] == rec["state_after_seed"]
        assert [f"{r:016x}" for r in oracle.xoshiro256ss(8)] == rec["xoshiro256ss"]
        oracle.rng_seed(int(seed))
        got = [f"{int(v):08x}" for v in oracle.randn(8).view(np.uint32)]
        assert got == rec["random_normal_f32"]


# ---------------------------------------------------------------- bf16 -----

def test_bf16_widening_is_shift_for_every_pattern():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(h)
    np.testing.assert_array_equal(f.view(np.uint32), h.astype(np.uint32) << 16)


def test_bf16_truncation_special_cases():
    u = np.array([0x3F80FFFF, 0x3F808000, 0xBF80FFFF, 0x7F800000, 0x7FC00001, 0x00000001], dtype=np.uint32)
    t = oracle.f32_to_bf16_trunc(u.view(np.float32))
    np.testing.assert_array_equal(t, np.array([0x3F80, 0x3F80, 0xBF80, 0x7F80, 0x7FC0, 0x0000], dtype=np.uint16))


def test_bf16_rne_every_midpoint_and_neighbours():
    # For every finite bf16 b (both signs), the fp32 midpoint between b and its
    # successor rounds to the one with an even last bit; one ulp of fp32 either
    # side rounds to the nearer one.
    b = np.arange(0, 0x7F7F, dtype=np.uint32)  # finite, successor finite
    for sign in (0, 0x8000):
        lo = (b | sign) << 16
        mid = lo + 0x8000
        r_mid = oracle.f32_to_bf16_rne(mid.view(np.float32)).astype(np.uint32)
        even = np.where((b & 1) == 0, b, b + 1) | sign
        np.testing.assert_array_equal(r_mid, even)
        np.testing.assert_array_equal(oracle.f32_to_bf16_rne((mid - 1).view(np.float32)), (b | sign).astype(np.uint16))
        np.testing.assert_array_equal(oracle.f32_to_bf16_rne((mid + 1).view(np.float32)),
                                      ((b + 1) | sign).astype(np.uint16))


def test_bf16_rne_specials():
    u = np.array([0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0x00000000, 0x80000000],
                 dtype=np.uint32)
    r = oracle.f32_to_bf16_rne(u.view(np.float32))
    assert r[0] == 0x7F80  # largest finite rounds to +inf
    assert r[1] == 0x7F80 and r[2] == 0xFF80
    assert (r[3] & 0x7F80) == 0x7F80 and (r[3] & 0x7F) != 0  # NaN stays NaN
    assert (r[4] & 0x7F80) == 0x7F80 and (r[4] & 0x7F) != 0  # signalling NaN stays NaN
    assert r[5] == 0 and r[6] == 0x8000


# ---------------------------------------------------------------- GEMM -----

def _rand(shape, seed, scale=1.0):
    oracle.rng_seed(seed)
    return oracle.randn_scaled(shape, scale, True)


TINY = [(1, 1, 1), (3, 5, 7), (9, 13, 17), (8, 8, 8), (17, 33, 130), (64, 31, 257), (12, 4, 40)]


@pytest.mark.parametrize("M,N,K", TINY)
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0), (-1.25, 1.0)])
def test_qgemm_nt_vs_fp64_brute_force(M, N, K, alpha, beta):
    A, B, C0 = _rand((M, K), 1), _rand((N, K), 2), _rand((M, N), 3)
    C = C0.copy()
    oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, M, N, K, alpha, A, K, B, K, beta, C, N)
    want = alpha * (A.astype(np.float64) @ B.astype(np.float64).T) + beta * C0.astype(np.float64)
    # fp32 accumulation: |err| <= K * 2^-24 * sum|a||b| (+ rounding of alpha, beta terms)
    bound = (K + 3) * 2.0 ** -24 * (abs(alpha) * (np.abs(A) @ np.abs(B).T) + abs(beta) * np.abs(C0)) + 1e-30
    assert np.all(np.abs(C - want) <= bound)


@pytest.mark.parametrize("M,N,K", TINY)
def test_qgemm_nn_tn_vs_numpy_float64(M, N, K):
    A, B = _rand((M, K), 4), _rand((K, N), 5)
    C = np.zeros((M, N), np.float32)
    oracle.qgemm(oracle.NO_TRANS, oracle.NO_TRANS, M, N, K, 1.0, A, K, B, N, 0.0, C, N)
    want = A.astype(np.float64) @ B.astype(np.float64)
    assert oracle.normwise_err(C, want) < 1e-5
    At = np.ascontiguousarray(A.T)  # [K x M]
    C2 = np.zeros((M, N), np.float32)
    oracle.qgemm(oracle.TRANS, oracle.NO_TRANS, M, N, K, 1.0, At, M, B, N, 0.0, C2, N)
    assert oracle.normwise_err(C2, want) < 1e-5


def test_qgemm_tt_is_rejected_like_the_reference():
    A = np.zeros((4, 4), np.float32)
    with pytest.raises(AssertionError):
        oracle.qgemm(oracle.TRANS, oracle.TRANS, 4, 4, 4, 1.0, A, 4, A, 4, 0.0, A.copy(), 4)


@pytest.mark.skipif(not oracle.lib().orc_has_avx2(), reason="host has no AVX2")
@pytest.mark.parametrize("M,N,K", [(9, 13, 17), (16, 24, 64), (33, 10, 131)])
def test_qgemm_avx2_bit_identical_to_scalar_association(M, N, K):
    A, B = _rand((M, K), 6), _rand((N, K), 7)
    C = np.zeros((M, N), np.float32)
    oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, M, N, K, 1.0, A, K, B, K, 0.0, C, N)
    np.testing.assert_array_equal(C, oracle.gemm_nt_scalar(A, B))


def test_gold_f64_matches_numpy_float64():
    A, B = _rand((37, 300), 8), _rand((29, 300), 9)
    g = oracle.gemm_nt_f64(A, B)
    np.testing.assert_allclose(g, A.astype(np.float64) @ B.astype(np.float64).T, rtol=1e-12, atol=1e-12)


def test_qgemm_matches_reference_sgemm2_fixtures():
    # C computed by the reference's own sgemm2.cpp (tests/golden/make_golden.py).
    fx = np.load(os.path.join(GOLDEN, "sgemm2_ref.npz"), allow_pickle=False)
    for i, (M, N, K) in enumerate(fx["shapes"]):
        A, B, C_ref = fx[f"A{i}"], fx[f"B{i}"], fx[f"C{i}"]
        C = np.zeros((M, N), np.float32)
        oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, int(M), int(N), int(K), 1.0, A, int(K), B, int(K), 0.0, C, int(N))
        assert oracle.normwise_err(C, C_ref) < 1e-6, (M, N, K)
        gold = A.astype(np.float64) @ B.astype(np.float64).T
        assert oracle.normwise_err(C_ref, gold) < 1e-6


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_qgemm_matches_reference_sgemm2_live():
    for seed, (M, N, K) in enumerate([(16, 24, 256), (20, 36, 1024), (8, 12, 384)]):
        A, B = _rand((M, K), 50 + seed), _rand((N, K), 60 + seed, 0.02)
        C = np.zeros((M, N), np.float32)
        oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, M, N, K, 1.0, A, K, B, K, 0.0, C, N)
        assert oracle.normwise_err(C, oracle.sgemm2_ref_nt(A, B)) < 1e-6


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_reference_sgemm2_skips_k_below_128():
    # Hazard recorded for the oracle choice: sgemm2.cpp never enters its K loop
    # when K < 128 (sgemm2.cpp:348-365), so it returns C untouched (zeros).
    A, B = _rand((4, 64), 70), _rand((8, 64), 71)
    assert np.all(oracle.sgemm2_ref_nt(A, B) == 0.0)
    C = np.zeros((4, 8), np.float32)
    oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, 4, 8, 64, 1.0, A, 64, B, 64, 0.0, C, 8)
    assert np.abs(C).max() > 0.0


# ----------------------------------------------------------- epilogue ops --

def test_silu_and_gelu_closed_forms():
    xs = np.linspace(-30, 30, 2001).astype(np.float32)
    for x in xs[::7]:
        s = oracle.lib().orc_silu_exact(float(x))
        assert s == np.float32(float(x) / (1.0 + math.exp(-float(x))))
        gl = oracle.lib().orc_gelu_erf(float(x))
        assert gl == np.float32(0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0))))


def test_fast_exp_close_to_exp():
    xs = np.linspace(-80, 80, 4001)
    rel = max(abs(oracle.lib().orc_fast_exp(float(x)) / math.exp(x) - 1.0) for x in xs)
    assert rel < 1e-5
    assert oracle.lib().orc_fast_exp(-90.0) == 0.0


def test_reference_silu_approximation_error_is_its_documented_size():
    # sSiLU_avx2's quadratic exp2 has max relative error ~1.72e-3 on exp(-x);
    # the restatement must show that size of error (not 0: it is not exact,
    # not larger: constants in the right places).
    x = np.linspace(-20, 20, 100001).astype(np.float32)
    sig, silu = oracle.silu_qnn(x)
    exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    rel = np.abs(sig / exact - 1.0)
    assert 1.0e-3 < rel.max() < 2.0e-3
    np.testing.assert_allclose(silu, sig * x, rtol=1e-6, atol=1e-30)
    # exp(-0) ~= C2 = 1.00172476 (the constant term of the polynomial)
    s0, _ = oracle.silu_qnn(np.zeros(1, np.float32))
    assert abs(float(s0[0]) - 1.0 / (1.0 + 1.00172476)) < 1e-7


def test_silu_qnn_gated_form():
    x = np.linspace(-5, 5, 101).astype(np.float32)
    up = np.linspace(2, -2, 101).astype(np.float32)
    sig, out = oracle.silu_qnn(x, up)
    np.testing.assert_allclose(out, sig * x * up, rtol=1e-6, atol=1e-30)


# --------------------------------------------------------------- linear ----

def test_linear_fixtures_against_closed_form():
    fx = np.load(os.path.join(GOLDEN, "linear_small.npz"), allow_pickle=False)
    for i, (M, K, N, has_bias, epi) in enumerate(fx["cases"]):
        X, W, b, Y = fx[f"X{i}"], fx[f"W{i}"], fx[f"b{i}"], fx[f"Y{i}"]
        got = oracle.linear_bf16w(X, W, b if has_bias else None, int(epi))
        assert oracle.normwise_err(got, Y) < 1e-6, i


def test_linear_bias_is_added_per_row():
    X, W = _rand((3, 16), 20), oracle.f32_to_bf16_rne(_rand((5, 16), 21))
    b = np.arange(5, dtype=np.float32)
    y0 = oracle.linear_bf16w(X, W)
    y1 = oracle.linear_bf16w(X, W, b)
    np.testing.assert_allclose(y1 - y0, np.broadcast_to(b, (3, 5)), rtol=0, atol=1e-5)


def test_gated_add_against_numpy_and_special_gates():
    d, pr = _rand((7, 33), 40), _rand((7, 33), 41)
    g = _rand((33,), 42)
    got = oracle.gated_add(d, g, pr)
    # numpy's fp32 ops round the product, then the sum: the loop's own order
    np.testing.assert_array_equal(got, d + (g[None, :] * pr))
    np.testing.assert_array_equal(oracle.gated_add(d, np.zeros(33, np.float32), pr), d)
    np.testing.assert_array_equal(oracle.gated_add(d, np.ones(33, np.float32), pr), d + pr)
    # the gate indexes columns, not rows: a row-indexed gate differs
    g_rows = np.resize(g, 7)
    assert not np.array_equal(got, d + g_rows[:, None] * pr)


# ------------------------------------------------------- normalisations ----

def test_adaln_and_rmsnorm_against_numpy_and_invariants():
    x = _rand((9, 300), 70, 2.0) + np.float32(0.5)
    sh, sc = _rand((300,), 71, 0.3), _rand((300,), 72, 0.3)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    ln = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(oracle.adaln(x, sh, sc), (1 + sc) * ln + sh, rtol=0, atol=2e-5)
    z = np.zeros(300, np.float32)
    y0 = oracle.adaln(x, z, z).astype(np.float64)
    np.testing.assert_allclose(y0.mean(1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y0.var(1), 1.0, atol=1e-4)
    # a per-row offset and a per-row positive scale leave the layer norm unchanged
    xs = (x * np.float32(3.0) + np.float32(7.0)).astype(np.float32)
    np.testing.assert_allclose(oracle.adaln(xs, sh, sc), oracle.adaln(x, sh, sc), rtol=0, atol=1e-4)
    w = _rand((300,), 73)
    rms = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(oracle.rmsnorm_rows(x, w), rms * w, rtol=0, atol=2e-5)
    np.testing.assert_allclose(oracle.rmsnorm_rows(x), rms, rtol=0, atol=2e-5)
    np.testing.assert_allclose(oracle.rmsnorm_rows(x * np.float32(5.0), w), oracle.rmsnorm_rows(x, w), atol=1e-5)
    # planted: sample variance (N-1) or a missing (1 + scale) are caught
    bad = (1 + sc) * ((x64 - mu) / np.sqrt(((x64 - mu) ** 2).sum(1, keepdims=True) / 299 + 1e-6)) + sh
    assert np.max(np.abs(oracle.adaln(x, sh, sc) - bad)) > 1e-4
    assert np.max(np.abs(oracle.adaln(x, sh, sc) - (sc * ln + sh))) > 1e-2


# ------------------------------------------------------------ attention ----

def _np_attention(Q, K, V, heads, kv_heads, d, scale, causal=False, key_mask=None):
    """numpy float64 softmax(QK^T)V per head: an independent statement (rows with
    no visible key are left out: callers avoid them)."""
    sq, sk = Q.shape[0], K.shape[0]
    O = np.zeros((sq, heads * d))
    for h in range(heads):
        g = h // (heads // kv_heads)
        S = Q[:, h * d:(h + 1) * d].astype(np.float64) @ K[:, g * d:(g + 1) * d].astype(np.float64).T * scale
        if causal:
            S[np.arange(sk)[None, :] > np.arange(sq)[:, None] + (sk - sq)] = -np.inf
        if key_mask is not None:
            S[:, np.asarray(key_mask) == 0] = -np.inf
        P = np.exp(S - S.max(axis=1, keepdims=True))
        O[:, h * d:(h + 1) * d] = (P / P.sum(axis=1, keepdims=True)) @ V[:, g * d:(g + 1) * d].astype(np.float64)
    return O


def _qkv(seed, sq, sk, heads, kv_heads, d):
    return (_rand((sq, heads * d), seed), _rand((sk, kv_heads * d), seed + 1), _rand((sk, kv_heads * d), seed + 2))


@pytest.mark.parametrize("heads,kv_heads,sq,sk,d,causal", [(2, 2, 5, 9, 16, False), (4, 2, 9, 9, 8, True),
                                                          (3, 1, 7, 12, 8, True), (1, 1, 1, 1, 4, False)])
def test_attention_f64_vs_numpy(heads, kv_heads, sq, sk, d, causal):
    Q, K, V = _qkv(50, sq, sk, heads, kv_heads, d)
    got = oracle.attention_f64(Q, K, V, heads, kv_heads, d, 0.3, causal)
    np.testing.assert_allclose(got, _np_attention(Q, K, V, heads, kv_heads, d, 0.3, causal), rtol=0, atol=1e-12)


def test_attention_invariants():
    h, d, sq, sk = 2, 8, 6, 10
    Q, K, V = _qkv(51, sq, sk, h, h, d)
    base = oracle.attention_f64(Q, K, V, h, h, d, 0.5)
    # every key holding the same value row: the output is that row
    Vc = np.tile(V[3:4], (sk, 1))
    np.testing.assert_allclose(oracle.attention_f64(Q, K, Vc, h, h, d, 0.5), np.tile(V[3:4], (sq, 1)), atol=1e-6)
    # one key: its value
    np.testing.assert_allclose(oracle.attention_f64(Q, K[:1], V[:1], h, h, d, 0.5), np.tile(V[:1], (sq, 1)), atol=1e-7)
    # all keys equal: uniform weights, the mean of V
    Ke = np.tile(K[:1], (sk, 1))
    np.testing.assert_allclose(oracle.attention_f64(Q, Ke, V, h, h, d, 0.5),
                               np.tile(V.astype(np.float64).mean(0, keepdims=True), (sq, 1)), atol=1e-6)
    # one vector added to every key shifts each query's scores by a constant
    u = _rand((1, h * d), 52)
    np.testing.assert_allclose(oracle.attention_f64(Q, (K + u).astype(np.float32), V, h, h, d, 0.5), base, atol=1e-5)
    # causal: query i sees exactly the keys up to i + (sk - sq)
    c = oracle.attention_f64(Q, K, V, h, h, d, 0.5, causal=True)
    for i in range(sq):
        n = i + sk - sq + 1
        np.testing.assert_allclose(c[i:i + 1], oracle.attention_f64(Q[i:i + 1], K[:n], V[:n], h, h, d, 0.5), atol=1e-12)
    # grouped kv heads equal the same kv heads repeated per query head
    Qg, Kg, Vg = _qkv(53, 5, 7, 4, 2, 8)
    rep = lambda A: np.concatenate([A[:, (j // 2) * 8:(j // 2 + 1) * 8] for j in range(4)], axis=1)
    np.testing.assert_allclose(oracle.attention_f64(Qg, Kg, Vg, 4, 2, 8, 0.4),
                               oracle.attention_f64(Qg, rep(Kg), rep(Vg), 4, 4, 8, 0.4), atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_key_mask(causal):
    """QNNMatTriangularFill's mask (quicknncpu.pas:3017-3028): a key with
    mask 0 is hidden from every query.  Pinned by the numpy statement, by
    removing the masked keys outright, and by the reference's fp32 path."""
    h, d, sq, sk = 2, 8, 9, 9
    Q, K, V = _qkv(56, sq, sk, h, h, d)
    mask = np.array([1, 1, 0, 1, 0, 0, 1, 1, 1], np.int32)
    got = oracle.attention_f64(Q, K, V, h, h, d, 0.5, causal, key_mask=mask)
    rows = slice(0, sq)
    np.testing.assert_allclose(got[rows], _np_attention(Q, K, V, h, h, d, 0.5, causal, mask)[rows], atol=1e-12)
    keep = np.flatnonzero(mask)
    if not causal:  # the masked keys removed: the same attention
        np.testing.assert_allclose(got, oracle.attention_f64(Q, K[keep], V[keep], h, h, d, 0.5), atol=1e-12)
    else:  # query i: the kept keys up to i
        for i in range(sq):
            vis = keep[keep <= i]
            np.testing.assert_allclose(got[i:i + 1], oracle.attention_f64(Q[i:i + 1], K[vis], V[vis], h, h, d, 0.5),
                                       atol=1e-12)
    assert oracle.normwise_err(oracle.attention_qnn(Q, K, V, h, h, d, 0.5, causal, key_mask=mask), got) < 1e-5
    # planted: the mask read inverted, or ignored
    assert oracle.normwise_err(oracle.attention_f64(Q, K, V, h, h, d, 0.5, causal, key_mask=1 - mask), got) > 4e-3
    assert oracle.normwise_err(oracle.attention_f64(Q, K, V, h, h, d, 0.5, causal), got) > 4e-3


def test_attention_query_with_no_visible_key():
    """Right-padded keys under a causal mask leave no row empty; a mask that hides
    every key of a query does: zeros in the fp64 oracle, NaN in the reference's
    softmax (its max is -inf)."""
    h, d = 1, 4
    Q, K, V = _qkv(57, 3, 3, h, h, d)
    mask = np.array([0, 1, 1], np.int32)
    o = oracle.attention_f64(Q, K, V, h, h, d, 0.5, True, key_mask=mask)
    assert np.all(o[0] == 0.0) and np.all(np.isfinite(o))
    r = oracle.attention_qnn(Q, K, V, h, h, d, 0.5, True, key_mask=mask)
    assert np.all(np.isnan(r[0])) and np.all(np.isfinite(r[1:]))


def test_softmax_qnn_is_the_softmax_within_its_polynomial():
    x = np.concatenate([np.linspace(-30, 5, 999), [-200.0, 3.0]]).astype(np.float32)
    got = oracle.softmax_qnn(x)
    e = np.exp(x.astype(np.float64) - x.max())
    ref = e / e.sum()
    assert abs(float(got.sum()) - 1.0) < 1e-5
    assert np.max(np.abs(got - ref) / np.maximum(ref, 1e-30)[None]) < 1e-5 or np.max(np.abs(got - ref)) < 1e-9
    # the clamp at -87.3: far-below-max inputs get ~exp(-87.3), not 0
    assert 0.0 < got[-2] < 1e-37
    # the restated reference path equals the closed form to fp32 rounding
    Q, K, V = _qkv(54, 6, 11, 2, 2, 16)
    assert oracle.normwise_err(oracle.attention_qnn(Q, K, V, 2, 2, 16, 0.25),
                               oracle.attention_f64(Q, K, V, 2, 2, 16, 0.25)) < 1e-5


def test_attention_checks_catch_planted_mistakes():
    """A wrong scale, a value row shifted by one key, a causal diagonal off by one
    and a wrong kv-head grouping each fail the attention parity bound (4e-3)."""
    h, d, sq, sk = 4, 16, 12, 12
    Q, K, V = _qkv(55, sq, sk, h, 2, d)
    good = oracle.attention_f64(Q, K, V, h, 2, d, 0.5, causal=True)
    assert oracle.normwise_err(oracle.attention_f64(Q, K, V, h, 2, d, 0.55, causal=True), good) > 4e-3
    Vr = np.ascontiguousarray(np.roll(V, 1, axis=0))
    assert oracle.normwise_err(oracle.attention_f64(Q, K, Vr, h, 2, d, 0.5, causal=True), good) > 4e-3
    # diagonal one key later: as if seq_k were one longer
    K1 = np.concatenate([K, K[-1:]]); V1 = np.concatenate([V, V[-1:]])
    assert oracle.normwise_err(oracle.attention_f64(Q, K1, V1, h, 2, d, 0.5, causal=True), good) > 4e-3
    # kv head g = h % kv_heads instead of h // (heads / kv_heads): query heads 1 and 2 trade kv heads
    perm = np.r_[0:d, 2 * d:3 * d, d:2 * d, 3 * d:4 * d]
    wrong = oracle.attention_f64(np.ascontiguousarray(Q[:, perm]), K, V, h, 2, d, 0.5, causal=True)[:, perm]
    assert oracle.normwise_err(wrong, good) > 4e-3


# ------------------------------------------------------- planted mistakes --

def test_checks_catch_planted_mistakes():
    """A wrong operand (transposed W, dropped bias, X not rounded the way the
    GPU path rounds it) must fail the parity metric used by the GPU tests."""
    X = _rand((16, 64), 30, 1.0)
    W = oracle.f32_to_bf16_rne(_rand((64, 64), 31, 0.02))
    b = _rand((64,), 32, 0.01)
    good = oracle.linear_bf16w(X, W, b)
    Wt = oracle.f32_to_bf16_rne(oracle.bf16_to_f32(W).T.copy())
    assert oracle.normwise_err(oracle.linear_bf16w(X, Wt, b), good) > 1e-2
    assert oracle.normwise_err(oracle.linear_bf16w(X, W, None), good) > 1e-3
    Xs = X.copy()
    Xs[:, 3] *= -1.0  # a sign error in one column of K
    assert oracle.normwise_err(oracle.linear_bf16w(Xs, W, b), good) > 1e-3
    Xo = np.ascontiguousarray(np.roll(X, 1, axis=1))  # k index off by one
    assert oracle.normwise_err(oracle.linear_bf16w(Xo, W, b), good) > 1e-2
    Wr = np.ascontiguousarray(np.roll(W, 1, axis=0))  # output row n off by one
    assert oracle.normwise_err(oracle.linear_bf16w(X, Wr, b), good) > 1e-2


# ------------------------------------------------- QK norm and rotary --

def _angles(seq, width, seed):
    th = np.random.default_rng(seed).uniform(-np.pi, np.pi, (seq, width))
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32), th


@pytest.mark.parametrize("mode", ["interleaved", "half"])
def test_rope_is_the_pairwise_complex_rotation(mode):
    """QNNApplyRoPE2D pairs (2k, 2k+1) with table column 2k; QNNApplyRoPE3 pairs
    (i, i + d/2) with column i.  Pinned by numpy complex products, the identity
    table, norm preservation and composition of angles."""
    seq, heads, d = 5, 3, 16
    x = _rand((seq, heads * d), 60)
    width = d if mode == "interleaved" else d // 2
    c, s, th = _angles(seq, width, 61)
    got = oracle.rope(x, c, s, heads, d, mode)
    xh = x.reshape(seq, heads, d).astype(np.float64)
    if mode == "interleaved":
        z = (xh[..., 0::2] + 1j * xh[..., 1::2]) * (c[:, None, 0::2] + 1j * s[:, None, 0::2])
        ref = np.empty_like(xh)
        ref[..., 0::2], ref[..., 1::2] = z.real, z.imag
    else:
        z = (xh[..., :d // 2] + 1j * xh[..., d // 2:]) * (c[:, None, :] + 1j * s[:, None, :])
        ref = np.concatenate([z.real, z.imag], axis=-1)
    np.testing.assert_allclose(got.reshape(seq, heads, d), ref, atol=1e-5)
    # identity table
    np.testing.assert_array_equal(oracle.rope(x, np.ones_like(c), np.zeros_like(s), heads, d, mode), x)
    # a rotation keeps each pair's length; two rotations add their angles
    pairs = lambda a: (a.reshape(seq, heads, d)[..., 0::2], a.reshape(seq, heads, d)[..., 1::2]) if mode == "interleaved" \
        else (a.reshape(seq, heads, d)[..., :d // 2], a.reshape(seq, heads, d)[..., d // 2:])
    (a0, a1), (b0, b1) = pairs(x.astype(np.float64)), pairs(got.astype(np.float64))
    np.testing.assert_allclose(a0 ** 2 + a1 ** 2, b0 ** 2 + b1 ** 2, rtol=1e-5, atol=1e-6)
    c2, s2 = np.cos(2 * th).astype(np.float32), np.sin(2 * th).astype(np.float32)
    np.testing.assert_allclose(oracle.rope(got, c, s, heads, d, mode), oracle.rope(x, c2, s2, heads, d, mode), atol=1e-5)
    # planted: the opposite rotation, or the other pairing, is far off
    assert np.max(np.abs(oracle.rope(x, c, -s, heads, d, mode) - got)) > 0.1
    if mode == "half":
        cw, sw = np.repeat(c, 2, axis=1), np.repeat(s, 2, axis=1)
        assert np.max(np.abs(oracle.rope(x, cw, sw, heads, d, "interleaved") - got)) > 0.1


def test_head_rmsnorm_normalises_each_head():
    """QNNQKRMSNorm / QNNHeadRSMNorm: each head's head_dim values over their own
    rms (EPSILON 1e-6), times the shared weight; not the whole row's rms."""
    seq, heads, d = 4, 3, 8
    x = _rand((seq, heads * d), 62) * np.float32(3.0)
    w = _rand((d,), 63)
    got = oracle.head_rmsnorm(x, w, heads, d)
    xh = x.reshape(seq, heads, d).astype(np.float64)
    ref = xh / np.sqrt((xh ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got.reshape(seq, heads, d), ref, rtol=1e-5, atol=1e-6)
    whole = oracle.rmsnorm_rows(x, np.tile(w, heads))
    assert np.max(np.abs(whole - got)) > 1e-2


# ---------------------------------------------------------- conv2d ----------

def _conv_im2col_f64(x, w, bias, kH, kW, stride, pad):
    """numpy float64 im2col + matmul: an independent formulation of QNNConv2d."""
    b, c, H, W = x.shape
    oc = w.shape[0]
    outH, outW = (H + 2 * pad - kH) // stride + 1, (W + 2 * pad - kW) // stride + 1
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    cols = np.empty((b, c, kH, kW, outH, outW))
    for kr in range(kH):
        for kc in range(kW):
            cols[:, :, kr, kc] = xp[:, :, kr:kr + stride * (outH - 1) + 1:stride, kc:kc + stride * (outW - 1) + 1:stride]
    y = np.einsum("ok,bkp->bop", w.astype(np.float64), cols.reshape(b, c * kH * kW, outH * outW))
    if bias is not None:
        y += bias.astype(np.float64)[None, :, None]
    return y.reshape(b, oc, outH, outW)


@pytest.mark.parametrize("b,c,oc,H,W,kH,kW,stride,pad", [
    (1, 3, 4, 7, 6, 3, 3, 1, 1),
    (2, 5, 3, 9, 8, 3, 3, 2, 0),
    (1, 4, 6, 8, 8, 1, 1, 1, 0),
    (1, 2, 3, 6, 7, 2, 3, 1, 2),
    (2, 3, 2, 5, 5, 5, 5, 1, 2),
])
def test_conv2d_matches_im2col_matmul(b, c, oc, H, W, kH, kW, stride, pad):
    rng = np.random.default_rng(b * 100 + c * 10 + kH)
    x = rng.standard_normal((b, c, H, W)).astype(np.float32)
    w = rng.standard_normal((oc, c * kH * kW)).astype(np.float32)
    bias = rng.standard_normal(oc).astype(np.float32)
    y = oracle.conv2d_f64(x, w, bias, c, oc, H, W, kH, kW, stride, pad, b)
    assert list(y.shape) == oracle.conv2d_shape(b, oc, H, W, kH, kW, pad, stride)
    np.testing.assert_allclose(y, _conv_im2col_f64(x, w, bias, kH, kW, stride, pad), rtol=1e-12, atol=1e-12)


def test_conv2d_pointwise_is_the_filter_matmul():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 6, 5, 4)).astype(np.float32)
    w = rng.standard_normal((3, 6)).astype(np.float32)
    y = oracle.conv2d_f64(x, w, None, 6, 3, 5, 4, 1, 1, 1, 0, 2)
    ref = np.matmul(w.astype(np.float64), x.astype(np.float64).reshape(2, 6, 20)).reshape(2, 3, 5, 4)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_conv2d_centred_delta_filter_reproduces_the_image():
    rng = np.random.default_rng(8)
    c = 3
    x = rng.standard_normal((1, c, 6, 5)).astype(np.float32)
    w = np.zeros((c, c, 3, 3), np.float32)
    for i in range(c):
        w[i, i, 1, 1] = 1.0
    y = oracle.conv2d_f64(x, w.reshape(c, -1), None, c, c, 6, 5, 3, 3, 1, 1, 1)
    np.testing.assert_array_equal(y, x.astype(np.float64))
    # shifted delta (kr=0, kc=2): y[oh][ow] = x[oh-1][ow+1], zero outside
    w[:] = 0
    w[0, 0, 0, 2] = 1.0
    y = oracle.conv2d_f64(x[:, :1], w[:1, :1].reshape(1, -1), None, 1, 1, 6, 5, 3, 3, 1, 1, 1)
    ref = np.zeros((6, 5))
    ref[1:, :4] = x[0, 0, :5, 1:]
    np.testing.assert_array_equal(y[0, 0], ref)


def test_conv2d_stride2_ones_filter_gives_block_sums():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 1, 8, 6)).astype(np.float32)
    y = oracle.conv2d_f64(x, np.ones((1, 4), np.float32), None, 1, 1, 8, 6, 2, 2, 2, 0, 1)
    ref = x.astype(np.float64).reshape(4, 2, 3, 2).sum(axis=(1, 3))
    np.testing.assert_allclose(y[0, 0], ref, rtol=1e-12, atol=1e-12)


def test_conv2d_zero_filter_gives_the_bias():
    bias = np.array([1.5, -2.0, 0.25], np.float32)
    y = oracle.conv2d_f64(np.ones((1, 2, 4, 4), np.float32), np.zeros((3, 18), np.float32), bias, 2, 3, 4, 4, 3, 3,
                          1, 1, 1)
    np.testing.assert_array_equal(y, np.broadcast_to(bias.astype(np.float64)[None, :, None, None], y.shape))


def test_conv2d_checks_catch_planted_mistakes():
    # A transposed filter (kr <-> kc) or a dropped padding offset must fail the
    # independent formulation.
    rng = np.random.default_rng(10)
    x = rng.standard_normal((1, 2, 6, 6)).astype(np.float32)
    w = rng.standard_normal((2, 2, 3, 3)).astype(np.float32)
    good = _conv_im2col_f64(x, w.reshape(2, -1), None, 3, 3, 1, 1)
    wrong_w = oracle.conv2d_f64(x, w.transpose(0, 1, 3, 2).reshape(2, -1), None, 2, 2, 6, 6, 3, 3, 1, 1, 1)
    assert np.abs(wrong_w - good).max() > 1e-3
    wrong_pad = oracle.conv2d_f64(np.pad(x, ((0, 0), (0, 0), (0, 2), (0, 2))), w.reshape(2, -1), None, 2, 2, 8, 8, 3,
                                  3, 1, 0, 1)
    assert np.abs(wrong_pad - good).max() > 1e-3
