"""Row-band pipeline of inv_hip_linear with host pointers (marked gpu).

With X and Y in host memory a product of at least two bands is uploaded,
multiplied and downloaded band by band on overlapping streams.  Every band runs
the tile choice of the whole product, so the banded call must give the same
bits as the serial pass (INV_HIP_HOST_PIPELINE=0) and as the device-pointer
call: bit-exact, for every epilogue, fp32 and bf16 X (16-byte granular rows
and not) and Y, with a ragged last band.  INV_HIP_HOST_BAND_MB=1 makes bands of
small products; the full-size product (4608 x 3072 x 9216) runs with the
default bands and is also checked against the oracle on sampled rows.  The
normalised (inv_hip_linear_norm) and accumulating (inv_hip_linear_gated_add)
entry points band the same way, and so does host-pointer attention over query
rows (bands of whole workgroup blocks: bit-exact against one launch).
"""
import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32, round_bf16

pytestmark = pytest.mark.gpu

TOL_TIGHT = 2e-5


def gen(seed, M, K, N):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 1.0, False)
    W = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b = oracle.randn_scaled((N,), 0.01, False)
    return X, W, b


def device_call(Xin, xdt, w, M, ydt, epi):
    xd = q.DeviceArray.from_host(Xin, xdt)
    yd = q.DeviceArray((M, w.N), ydt)
    try:
        q.linear_device(xd, w, yd, M, epilogue=epi)
        return yd.to_host()
    finally:
        xd.free()
        yd.free()


# (M, K, N, epilogue, bias, X dtype, Y dtype): 1 MiB bands
CASES = [
    (1100, 1000, 1000, "none", True, "f32", "f32"),
    (1100, 1000, 1000, "silu", False, "f32", "bf16"),
    (777, 1001, 1500, "gelu", True, "bf16", "f32"),    # bf16 rows of 2002 bytes: staged, then copied
    (1536, 512, 2048, "none", True, "bf16", "bf16"),   # bf16 rows land in the operand as they are
    (1025, 1900, 300, "silu", True, "f32", "f32"),     # the input side sets the band
]


@pytest.mark.parametrize("M,K,N,epi,bias,xdt,ydt", CASES)
def test_banded_equals_serial_and_device(hiplib, monkeypatch, M, K, N, epi, bias, xdt, ydt):
    X, W, b = gen(M + K + N, M, K, N)
    Xin = X.astype(np.float32) if xdt == "f32" else as_bf16_bits(X)
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")  # fails unless the call is banded
    with q.Weight(W, b if bias else None) as w:
        y_band = q.linear(Xin, w, epilogue=epi, out_dtype=ydt)
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
        y_serial = q.linear(Xin, w, epilogue=epi, out_dtype=ydt)
        y_dev = device_call(Xin, xdt, w, M, ydt, epi)
    print(f"  {M}x{K}x{N} {epi} bias={bias} X {xdt} Y {ydt}: banded == serial == device", flush=True)
    np.testing.assert_array_equal(y_band, y_serial)
    np.testing.assert_array_equal(y_band, y_dev)
    yf = bf16_bits_to_f32(y_band) if ydt == "bf16" else y_band
    ref = oracle.linear_bf16w(round_bf16(X), W, b if bias else None,
                              {"none": oracle.EPI_NONE, "silu": oracle.EPI_SILU, "gelu": oracle.EPI_GELU}[epi])
    assert oracle.normwise_err(yf, ref) <= (2.0 ** -8 + TOL_TIGHT if ydt == "bf16" else TOL_TIGHT)


def test_banded_swiglu_equals_serial(hiplib, monkeypatch):
    M, K, F = 900, 512, 640
    oracle.rng_seed(41)
    X = oracle.randn_scaled((M, K), 1.0, False)
    Wg = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    Wu = oracle.f32_to_bf16_rne(oracle.randn_scaled((F, K), 0.02, False))
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
    with q.Weight.gate_up(Wg, Wu) as w:
        y_band = q.linear(as_bf16_bits(X), w, epilogue="swiglu")
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
        y_serial = q.linear(as_bf16_bits(X), w, epilogue="swiglu")
    np.testing.assert_array_equal(y_band, y_serial)


def test_consecutive_banded_calls_and_interleaved_device_calls(hiplib, monkeypatch):
    """Bounce buffers and events are reused across calls: alternate banded host
    calls of different sizes with asynchronous device calls on the library stream."""
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    X, W, b = gen(5, 1300, 768, 1024)
    with q.Weight(W, b) as w:
        want = {m: device_call(X[:m].astype(np.float32), "f32", w, m, "f32", "none") for m in (1300, 600)}
        xd = q.DeviceArray.from_host(X.astype(np.float32), "f32")
        yd = q.DeviceArray((1300, 1024), "f32")
        try:
            for m in (1300, 600, 1300):
                q.linear_device(xd, w, yd, 1300, asynchronous=True)
                monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
                y = q.linear(X[:m].astype(np.float32), w)
                monkeypatch.delenv("INV_HIP_HOST_PIPELINE")
                np.testing.assert_array_equal(y, want[m])
            hip.call("inv_hip_synchronize")
            np.testing.assert_array_equal(yd.to_host(), want[1300])
        finally:
            xd.free()
            yd.free()


def test_full_size_projection_banded(hiplib, monkeypatch):
    """4608 x 3072 x 9216 with fp32 host X and Y (eleven bands of 448 rows,
    two 224-row tiles each): the same bits as the device-pointer call, and
    the oracle on sampled rows, band edges among them."""
    M, K, N = 4608, 3072, 9216
    X, W, b = gen(2, M, K, N)
    X32 = X.astype(np.float32)
    with q.Weight(W, b) as w:
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
        y = q.linear(X32, w)
        monkeypatch.delenv("INV_HIP_HOST_PIPELINE")
        y_dev = device_call(X32, "f32", w, M, "f32", "none")
    np.testing.assert_array_equal(y, y_dev)
    rows = np.unique(np.concatenate([[0, 447, 448, 4479, 4480, M - 1], np.random.default_rng(0).choice(M, 24, replace=False)]))
    e = oracle.normwise_err(y[rows], oracle.linear_bf16w(round_bf16(X[rows]), W, b, oracle.EPI_NONE))
    print(f"  sampled rows normwise err {e:.3e}", flush=True)
    assert e <= TOL_TIGHT


@pytest.mark.parametrize("norm,K", [("adaln", 1024), ("rms", 1024), ("adaln", 1001)])
def test_banded_linear_norm_equals_serial(hiplib, monkeypatch, norm, K):
    """inv_hip_linear_norm with host X and Y: each band normalises its own rows
    (K = 1001 takes the row kernel without register groups)."""
    M, N = 1100, 1000
    X, W, b = gen(K + 7, M, K, N)
    rng = np.random.default_rng(K)
    scale = (rng.standard_normal(K) * 0.3).astype(np.float32)
    shift = (rng.standard_normal(K) * 0.3).astype(np.float32) if norm == "adaln" else None
    X32 = X.astype(np.float32)
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
    with q.Weight(W, b) as w:
        y_band = q.linear_norm(X32, norm, w, scale, shift, epilogue="silu")
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
        y_serial = q.linear_norm(X32, norm, w, scale, shift, epilogue="silu")
    print(f"  {norm} {M}x{K}x{N}: banded == serial", flush=True)
    np.testing.assert_array_equal(y_band, y_serial)
    assert np.all(np.isfinite(y_band))


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_banded_gated_add_equals_serial_and_device(hiplib, monkeypatch, xdt):
    """inv_hip_linear_gated_add with host X and Y: a band's Y rows go up behind
    its X rows and are updated in place (Y += gate * (X W^T + b))."""
    M, K, N = 1300, 768, 1024
    X, W, b = gen(9, M, K, N)
    rng = np.random.default_rng(9)
    Y0 = rng.standard_normal((M, N)).astype(np.float32)
    gate = (rng.standard_normal(N) * 0.5).astype(np.float32)
    Xin = X.astype(np.float32) if xdt == "f32" else as_bf16_bits(X)
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    with q.Weight(W, b) as w:
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
        y_band = Y0.copy()
        q.linear_gated_add(y_band, Xin, w, gate)
        monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
        y_serial = Y0.copy()
        q.linear_gated_add(y_serial, Xin, w, gate)
        xd = q.DeviceArray.from_host(Xin, xdt)
        yd = q.DeviceArray.from_host(Y0, "f32")
        gd = q.DeviceArray.from_host(gate, "f32")
        try:
            q.linear_gated_add_device(xd, w, yd, M, gate=gd)
            y_dev = yd.to_host()
        finally:
            for d in (xd, yd, gd):
                d.free()
    np.testing.assert_array_equal(y_band, y_serial)
    np.testing.assert_array_equal(y_band, y_dev)
    ref = Y0.astype(np.float64) + gate * oracle.linear_bf16w(round_bf16(X), W, b, oracle.EPI_NONE)
    assert oracle.normwise_err(y_band - Y0, ref - Y0) <= TOL_TIGHT


def attn_gen(seed, sq, sk, heads, kv_heads, d):
    oracle.rng_seed(seed)
    Q = oracle.randn_scaled((sq, heads * d), 1.0, False)
    K = oracle.randn_scaled((sk, kv_heads * d), 1.0, False)
    V = oracle.randn_scaled((sk, kv_heads * d), 1.0, False)
    return Q, K, V


# (seq_q, seq_k, heads, kv_heads, head_dim, causal, key mask, Q/K/V dtype, O dtype, key groups):
# 1 MiB bands of 256 or 512 query rows, ragged last bands; causal with more keys
# than queries (the diagonal offset counts from each band's first row)
ATTN_CASES = [
    (1100, 1100, 8, 8, 128, False, False, "f32", "f32", 2),
    (1000, 1300, 8, 2, 128, True, False, "f32", "bf16", 2),
    (777, 777, 16, 16, 64, True, True, "bf16", "f32", 2),
    (1536, 600, 8, 4, 128, False, True, "bf16", "bf16", 1),
    (1300, 1400, 8, 4, 128, True, True, "f32", "f32", 1),
]


@pytest.mark.parametrize("sq,sk,heads,kvh,d,causal,masked,idt,odt,kg", ATTN_CASES)
def test_banded_attention_equals_serial_and_device(hiplib, monkeypatch, sq, sk, heads, kvh, d, causal, masked, idt,
                                                   odt, kg):
    """inv_hip_attention(_masked) with host Q and O: K and V go up whole, then
    query bands of whole workgroup blocks upload, run and download overlapped."""
    Q, K, V = attn_gen(sq + sk + d, sq, sk, heads, kvh, d)
    mask = None
    if masked:
        mask = (np.random.default_rng(sq).random(sk) < 0.7).astype(np.int32)
        mask[0] = 1
    cvt = (lambda a: a.astype(np.float32)) if idt == "f32" else as_bf16_bits
    Qh, Kh, Vh = cvt(Q), cvt(K), cvt(V)
    monkeypatch.setenv("INV_HIP_ATTN_KEY_GROUPS", str(kg))
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")  # fails unless the call is banded
    kw = dict(heads=heads, head_dim=d, kv_heads=kvh, causal=causal, out_dtype=odt, key_mask=mask)
    o_band = q.attention(Qh, Kh, Vh, **kw)
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
    o_serial = q.attention(Qh, Kh, Vh, **kw)
    devs = [q.DeviceArray.from_host(a, idt) for a in (Qh, Kh, Vh)]
    od = q.DeviceArray((sq, heads * d), odt)
    md = q.DeviceArray.from_host(mask, "i32") if masked else None
    try:
        q.attention_device(*devs, od, heads=heads, head_dim=d, kv_heads=kvh, causal=causal, key_mask=md)
        o_dev = od.to_host()
    finally:
        for a in devs + [od] + ([md] if md is not None else []):
            a.free()
    print(f"  {sq}x{sk} {heads}/{kvh} heads of {d} causal={causal} mask={masked} {idt}->{odt} key groups {kg}: "
          "banded == serial == device", flush=True)
    np.testing.assert_array_equal(o_band, o_serial)
    np.testing.assert_array_equal(o_band, o_dev)
    of = bf16_bits_to_f32(o_band) if odt == "bf16" else o_band
    ref = oracle.attention_f64(round_bf16(Q), round_bf16(K), round_bf16(V), heads, kvh, d, 1.0 / np.sqrt(d), causal,
                               key_mask=mask)
    assert oracle.normwise_err(of, ref) <= 4e-3 + (2.0 ** -8 if odt == "bf16" else 0.0)


def test_banded_causal_attention_with_fewer_keys_than_queries(hiplib, monkeypatch):
    """Causal, 700 keys for 1100 queries: queries 0..399 see no key (their rows
    are zero) and the first bands' diagonal offsets are negative."""
    sq, sk, heads, d = 1100, 700, 8, 128
    Q, K, V = attn_gen(31, sq, sk, heads, heads, d)
    kw = dict(heads=heads, head_dim=d, causal=True)
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
    o_band = q.attention(Q, K, V, **kw)
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "0")
    o_serial = q.attention(Q, K, V, **kw)
    devs = [q.DeviceArray.from_host(a, "f32") for a in (Q, K, V)]
    od = q.DeviceArray((sq, heads * d), "f32")
    try:
        q.attention_device(*devs, od, **kw)
        o_dev = od.to_host()
    finally:
        for a in devs + [od]:
            a.free()
    np.testing.assert_array_equal(o_band, o_serial)
    np.testing.assert_array_equal(o_band, o_dev)
    assert not np.any(o_band[: sq - sk])
    # the remaining queries see keys 0 .. i - (sq - sk): a causal call of sk queries over the same keys
    ref = oracle.attention_f64(round_bf16(Q[sq - sk:]), round_bf16(K), round_bf16(V), heads, heads, d,
                               1.0 / np.sqrt(d), True)
    assert oracle.normwise_err(o_band[sq - sk:], ref) <= 4e-3


def test_attention_not_banded_below_two_bands(hiplib, monkeypatch):
    """A query count that fits one band runs the one-pass path (PIPELINE=2 then
    reports the call as not banded)."""
    Q, K, V = attn_gen(5, 200, 200, 8, 8, 128)
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2")
    with pytest.raises(hip.HipError):
        q.attention(Q, K, V, heads=8, head_dim=128)
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "1")
    O = q.attention(Q, K, V, heads=8, head_dim=128)
    assert np.all(np.isfinite(O))


def tie_values(rng, shape):
    """fp32 values whose low half-words sit at and around the bf16 rounding ties
    (normal exponents from ~1e-9 to ~2e9, both signs)."""
    hi = rng.integers(0x3000, 0x4F00, size=shape, dtype=np.uint32)
    sign = rng.integers(0, 2, size=shape, dtype=np.uint32) << np.uint32(31)
    low = rng.choice(np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32), size=shape)
    return ((hi << np.uint32(16)) | low | sign).view(np.float32)


@pytest.mark.parametrize("path", ["serial", "banded"])
def test_host_rounding_is_the_device_rounding(hiplib, monkeypatch, path):
    """Host fp32 X is rounded to bf16 by the host on its way into the bounce
    buffers.  Through an identity weight Y is the rounded X itself: nearest
    even at every tie, as the oracle rounds and as the device-pointer call
    (rounded on the device) gives; a NaN makes its whole row NaN on both."""
    M, K = 2600, 512
    X = tie_values(np.random.default_rng(77), (M, K))
    X[0, 5] = np.nan
    W = oracle.f32_to_bf16_rne(np.eye(K, dtype=np.float32))
    monkeypatch.setenv("INV_HIP_HOST_BAND_MB", "1")
    monkeypatch.setenv("INV_HIP_HOST_PIPELINE", "2" if path == "banded" else "0")
    with q.Weight(W) as w:
        y = q.linear(X, w)
        y_dev = device_call(X, "f32", w, M, "f32", "none")
    np.testing.assert_array_equal(y, y_dev)
    assert np.all(np.isnan(y[0]))
    np.testing.assert_array_equal(y[1:], bf16_bits_to_f32(oracle.f32_to_bf16_rne(X[1:])))


def test_fp32_weight_rounded_on_upload_is_the_oracle_rounding(hiplib):
    """inv_hip_weight_upload_f32 rounds on the host (rows padded 1001 -> 1008):
    the same products as the weight rounded by the oracle and uploaded as bf16."""
    N, K, M = 300, 1001, 64
    rng = np.random.default_rng(78)
    W = tie_values(rng, (N, K))
    X = rng.standard_normal((M, K)).astype(np.float32)
    with q.Weight(W) as w32, q.Weight(oracle.f32_to_bf16_rne(W)) as w16:
        y32 = device_call(X, "f32", w32, M, "f32", "none")
        y16 = device_call(X, "f32", w16, M, "f32", "none")
    np.testing.assert_array_equal(y32, y16)


def test_host_rounding_of_few_wide_rows(hiplib):
    """Two rows of a million columns: the copy threads round column slices of
    every row (fewer rows than slices).  An fp32 weight and fp32 X of that shape,
    rounded by the host, give the products of the oracle-rounded bf16 weight and
    of X rounded on the device."""
    K = 1_000_003
    rng = np.random.default_rng(79)
    W = tie_values(rng, (2, K)) * np.float32(1e-3)
    X = tie_values(rng, (3, K)) * np.float32(1e-3)
    with q.Weight(W) as w32, q.Weight(oracle.f32_to_bf16_rne(W)) as w16:
        y_host = q.linear(X, w32)
        y_dev = device_call(X, "f32", w16, 3, "f32", "none")
    np.testing.assert_array_equal(y_host, y_dev)
    assert np.all(np.isfinite(y_host))
