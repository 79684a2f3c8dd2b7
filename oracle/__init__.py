"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference's
own C++ SGEMM built under oracle/_ref (when present).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never by the product (invision_amd/).

How each oracle function is pinned:
  * RNG (quicknn_sample.pas:212-276): SplitMix64 seed-0 and xoshiro256**
    state-[1,2,3,4] published known-answer outputs; Box-Muller against its
    closed form on the drawn uniforms; moments of 10^6 draws.
  * bf16 widening/truncation (quicknn_common.pas:1991-2027): exact bit
    identities and special values; RNE rounding: every bf16 midpoint.
  * qgemm NN/NT/TN (quicknncpu.pas:1176-1496): fp64 brute force on tiny and
    ragged shapes (K % 8 != 0), numpy's float64 matmul (an independent
    library), the reference's own sgemm2.cpp built under oracle/_ref, and the
    scalar restatement (bit-identical association order).
  * SiLU/GELU/fast_exp (ops_avx2.inc:22-35, 267-376; quicknncpu.pas:305-330):
    closed forms (math.exp / math.erf), the polynomial's value at fixed points,
    and the documented error bound of the reference approximation.
  * linear (quicknncpu.pas:1807-1847): closed form with bias.
  * gated add (quicknncpu.pas:853-859): numpy's fp32 elementwise product and
    sum (bit-exact), gate = 0 leaves dst unchanged, gate = 1 is dst + proj.
  * AdaLN / RMSNorm (quicknncpu.pas:3042-3060, 2159-2198): numpy float64
    layer and RMS norms; zero shift/scale rows have mean 0 and variance 1;
    invariance to a per-row offset (AdaLN) and to a per-row scale (both).
  * attention (quicknn_transformers.pas:1150-1311; quicknn_qwen3.pas:727-769):
    numpy float64 softmax(QK^T)V per head; invariants (constant V, one key,
    equal keys, a vector added to every key, the causal prefix); the restated
    AVX2 softmax against the exact softmax within its polynomial's error.
  * conv2d (quicknncpu.pas:1958-2124): numpy float64 im2col + matmul (an
    independent formulation); a 1x1 convolution is the matmul of the filter
    and the image; a centred delta filter with padding 1 reproduces the image;
    a 2x2 all-ones filter with stride 2 gives the 2x2 block sums; zero
    filters give the bias; the output shape is QNNConv2DShape's.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int64, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libsgemm2_ref.so")

ROW_MAJOR, NO_TRANS, TRANS = 101, 111, 112
EPI_NONE, EPI_SILU, EPI_GELU, EPI_SILU_QNN = 0, 1, 2, 3

_lib = None
_ref = None


def _build() -> None:
    subprocess.run(["make", "-C", HERE, "liboracle.so"], check=True, capture_output=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            _build()
        L = ctypes.CDLL(LIB)
        L.orc_rng_seed.argtypes = [c_uint64]
        L.orc_rng_set_state.argtypes = [POINTER(c_uint64)]
        L.orc_rng_get_state.argtypes = [POINTER(c_uint64)]
        L.orc_xoshiro256ss.restype = c_uint64
        L.orc_rand.restype = c_float
        L.orc_random_normal.restype = c_float
        L.orc_randn.argtypes = [c_void_p, c_int64]
        L.orc_randn_scaled.argtypes = [c_void_p, c_int64, c_float, c_int]
        for f in ("orc_bf16_to_f32", "orc_f32_to_bf16_trunc", "orc_f32_to_bf16_rne"):
            getattr(L, f).argtypes = [c_void_p, c_void_p, c_int64]
        L.orc_qgemm.restype = c_int
        L.orc_qgemm.argtypes = [c_int, c_int, c_int, c_int64, c_int64, c_int64, c_float, c_void_p, c_int64,
                                c_void_p, c_int64, c_float, c_void_p, c_int64, c_int]
        L.orc_gemm_nt_scalar.argtypes = [c_int64, c_int64, c_int64, c_float, c_void_p, c_int64, c_void_p, c_int64,
                                         c_float, c_void_p, c_int64]
        L.orc_gemm_nt_f64.argtypes = [c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                      c_int64, c_int]
        L.orc_linear_bf16w.restype = c_int
        L.orc_linear_bf16w.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int,
                                       c_int]
        L.orc_silu_exact.restype = c_float
        L.orc_silu_exact.argtypes = [c_float]
        L.orc_gelu_erf.restype = c_float
        L.orc_gelu_erf.argtypes = [c_float]
        L.orc_fast_exp.restype = c_float
        L.orc_fast_exp.argtypes = [c_float]
        L.orc_silu_qnn.argtypes = [c_int64, c_void_p, c_void_p, c_void_p, c_void_p]
        L.orc_apply_epilogue.argtypes = [c_void_p, c_int64, c_int]
        L.orc_gated_add.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int64]
        for f in (L.orc_attention_f64, L.orc_attention_qnn):
            f.restype = c_int
        L.orc_attention_f64.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_int64, ctypes.c_double, c_int, c_void_p, c_int]
        L.orc_attention_qnn.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_int64, c_float, c_int, c_void_p, c_int]
        L.orc_softmax_qnn.argtypes = [c_void_p, c_int64]
        L.orc_adaln.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64]
        L.orc_rmsnorm_rows.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int64]
        L.orc_conv2d_f64.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p] + [c_int64] * 9
        for f in (L.orc_rope_interleaved, L.orc_rope_half):
            f.restype = None
            f.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64]
        L.orc_add_bias_rows.argtypes = [c_void_p, c_void_p, c_int64, c_int64]
        L.orc_has_avx2.restype = c_int
        L.orc_max_threads.restype = c_int
        _lib = L
    return _lib


def ref_lib():
    """The reference's own sgemm2.cpp (cpp_sgemm export, sgemm2.cpp:530-547), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        R = ctypes.CDLL(REF_LIB)
        R.cpp_sgemm.restype = None
        R.cpp_sgemm.argtypes = [c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_int, c_void_p, c_int,
                                c_float, c_void_p, c_int, c_int, c_int]
        _ref = R
    return _ref


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- RNG -------------------------------------------------------------------

def rng_seed(seed: int) -> None:
    lib().orc_rng_seed(seed)


def rng_state() -> list[int]:
    s = (c_uint64 * 4)()
    lib().orc_rng_get_state(s)
    return list(s)


def rng_set_state(state) -> None:
    lib().orc_rng_set_state((c_uint64 * 4)(*state))


def xoshiro256ss(n: int) -> list[int]:
    return [lib().orc_xoshiro256ss() for _ in range(n)]


def randn(n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_randn(_p(out), n)
    return out


def randn_scaled(shape, sigma: float, round_bf16: bool) -> np.ndarray:
    """Draw prod(shape) normals from the current stream, times sigma, optionally bf16-rounded."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().orc_randn_scaled(_p(out), n, sigma, 1 if round_bf16 else 0)
    return out.reshape(shape)


# ---- bf16 ------------------------------------------------------------------

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32(_p(h), _p(out), h.size)
    return out


def f32_to_bf16_trunc(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_trunc(_p(x), _p(out), x.size)
    return out


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_rne(_p(x), _p(out), x.size)
    return out


# ---- GEMM / linear -----------------------------------------------------------

def qgemm(transA: int, transB: int, M: int, N: int, K: int, alpha: float, A: np.ndarray, lda: int, B: np.ndarray,
          ldb: int, beta: float, C: np.ndarray, ldc: int, nthreads: int = 0) -> None:
    """The reference's built-in CBLAS fallback (quicknncpu.pas:1398-1496), in place on C."""
    for a, nm in ((A, "A"), (B, "B"), (C, "C")):
        assert a.dtype == np.float32 and a.flags.c_contiguous, nm
    rc = lib().orc_qgemm(ROW_MAJOR, transA, transB, M, N, K, alpha, _p(A), lda, _p(B), ldb, beta, _p(C), ldc,
                         nthreads)
    if rc:
        raise AssertionError("ERROR : Operation is not supported using the provided arguments!")


def gemm_nt_scalar(A: np.ndarray, B: np.ndarray, alpha: float = 1.0) -> np.ndarray:
    M, K = A.shape
    N = B.shape[0]
    C = np.zeros((M, N), dtype=np.float32)
    lib().orc_gemm_nt_scalar(M, N, K, alpha, _p(A), K, _p(B), K, 0.0, _p(C), N)
    return C


def gemm_nt_f64(A: np.ndarray, B: np.ndarray, nthreads: int = 0) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm_nt_f64(M, N, K, _p(A), K, _p(B), K, _p(C), N, nthreads)
    return C


def linear_bf16w(X: np.ndarray, W_bf16: np.ndarray, bias=None, epilogue: int = EPI_NONE,
                 nthreads: int = 0) -> np.ndarray:
    """QNNLinear / QNNLinearNoBias_BF16 + epilogue (quicknncpu.pas:1807-1847): fp32 X, bf16 W."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    W_bf16 = np.ascontiguousarray(W_bf16, dtype=np.uint16)
    M, K = X.shape
    N = W_bf16.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    rc = lib().orc_linear_bf16w(_p(X), _p(W_bf16), _p(b) if b is not None else None, _p(Y), M, K, N, epilogue,
                                nthreads)
    if rc:
        raise MemoryError("oracle linear failed")
    return Y


def apply_epilogue(Y: np.ndarray, epilogue: int) -> np.ndarray:
    Y = np.ascontiguousarray(Y, dtype=np.float32).copy()
    lib().orc_apply_epilogue(_p(Y), Y.size, epilogue)
    return Y


def gated_add(dst: np.ndarray, gate: np.ndarray, proj: np.ndarray) -> np.ndarray:
    """QNNGatedAdd (quicknncpu.pas:853-859) on a copy of dst: dst + gate[j] * proj."""
    d = np.ascontiguousarray(dst, dtype=np.float32).copy()
    g = np.ascontiguousarray(gate, dtype=np.float32)
    pr = np.ascontiguousarray(proj, dtype=np.float32)
    seq, hidden = d.shape
    if pr.shape != d.shape or g.size != hidden:
        raise ValueError("gated_add: shapes")
    lib().orc_gated_add(_p(d), _p(g), _p(pr), seq, hidden)
    return d


def _attn_args(Q, K, V, heads, kv_heads, d):
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    seq_q, seq_k = Q.shape[0], K.shape[0]
    if Q.shape[1] != heads * d or K.shape[1] != kv_heads * d or V.shape != K.shape:
        raise ValueError("attention: shapes")
    return Q, K, V, seq_q, seq_k


def _key_mask(key_mask, seq_k):
    if key_mask is None:
        return None
    m = np.ascontiguousarray(key_mask, dtype=np.int32)
    if m.shape != (seq_k,):
        raise ValueError(f"key_mask needs {seq_k} entries, got shape {m.shape}")
    return m


def attention_f64(Q, K, V, heads: int, kv_heads: int, d: int, scale: float, causal: bool = False,
                  key_mask=None, nthreads: int = 0) -> np.ndarray:
    """softmax(scale * Q_h K_g^T) V_g per head in fp64 (the reference's attention
    loops, quicknn_transformers.pas:1150-1311; quicknn_qwen3.pas:727-769); keys
    with key_mask[j] == 0 are hidden (quicknncpu.pas:3017-3028); a query with no
    visible key gets zeros."""
    Q, K, V, seq_q, seq_k = _attn_args(Q, K, V, heads, kv_heads, d)
    m = _key_mask(key_mask, seq_k)
    O = np.empty((seq_q, heads * d), dtype=np.float64)
    rc = lib().orc_attention_f64(_p(Q), _p(K), _p(V), _p(O), heads, kv_heads, seq_q, seq_k, d, float(scale),
                                 int(causal), _p(m) if m is not None else None, nthreads)
    if rc:
        raise ValueError(f"oracle attention failed ({rc})")
    return O


def attention_qnn(Q, K, V, heads: int, kv_heads: int, d: int, scale: float, causal: bool = False,
                  key_mask=None, nthreads: int = 0) -> np.ndarray:
    """The reference's fp32 BLAS path with its AVX2 softmax (orc_attention_qnn)."""
    Q, K, V, seq_q, seq_k = _attn_args(Q, K, V, heads, kv_heads, d)
    m = _key_mask(key_mask, seq_k)
    O = np.empty((seq_q, heads * d), dtype=np.float32)
    rc = lib().orc_attention_qnn(_p(Q), _p(K), _p(V), _p(O), heads, kv_heads, seq_q, seq_k, d, float(scale),
                                 int(causal), _p(m) if m is not None else None, nthreads)
    if rc:
        raise ValueError(f"oracle attention failed ({rc})")
    return O


def softmax_qnn(x: np.ndarray) -> np.ndarray:
    """sSoftmax_avx2 restated (exact 1/sum) on a copy of a 1-D fp32 array."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_softmax_qnn(_p(y), y.size)
    return y


def adaln(x: np.ndarray, shift: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """QNNAdaLN (quicknncpu.pas:3042-3060): (1 + scale) * layernorm(x) + shift per row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    sh = np.ascontiguousarray(shift, dtype=np.float32)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    lib().orc_adaln(_p(y), _p(x), _p(sh), _p(sc), x.shape[0], x.shape[1])
    return y


def rmsnorm_rows(x: np.ndarray, weight=None) -> np.ndarray:
    """QNNRMSNormRows (quicknncpu.pas:2159-2198): x * weight / rms(x) per row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    w = np.ascontiguousarray(weight, dtype=np.float32) if weight is not None else None
    lib().orc_rmsnorm_rows(_p(y), _p(x), _p(w) if w is not None else None, x.shape[0], x.shape[1])
    return y


def rope(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray, heads: int, head_dim: int, mode: str) -> np.ndarray:
    """Rotary embedding on a copy of x [seq x heads*head_dim]: mode "interleaved"
    (QNNApplyRoPE2D, tables [seq x head_dim]) or "half" (QNNApplyRoPE3, tables
    [seq x head_dim/2])."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    seq = y.shape[0]
    width = head_dim if mode == "interleaved" else head_dim // 2
    if y.shape[1] != heads * head_dim or c.shape != (seq, width) or s.shape != (seq, width):
        raise ValueError("rope: shape mismatch")
    f = lib().orc_rope_interleaved if mode == "interleaved" else lib().orc_rope_half
    f(_p(y), _p(c), _p(s), seq, heads, head_dim)
    return y


def head_rmsnorm(x: np.ndarray, weight, heads: int, head_dim: int) -> np.ndarray:
    """Per-head RMSNorm (QNNQKRMSNorm, quicknncpu.pas:2209-2246; QNNHeadRSMNorm,
    quicknn_qwen3.pas:223-230): QNNRMSNorm over each head's head_dim values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return rmsnorm_rows(x.reshape(-1, head_dim), weight).reshape(x.shape)


def silu_qnn(x: np.ndarray, up=None):
    """sSiLU_avx2 restated: returns (sigmoid, silu[*up])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    sig = np.empty_like(x)
    dst = np.empty_like(x)
    u = np.ascontiguousarray(up, dtype=np.float32) if up is not None else None
    lib().orc_silu_qnn(x.size, _p(x), _p(u) if u is not None else None, _p(sig), _p(dst))
    return sig, dst


def sgemm2_ref_nt(A: np.ndarray, B: np.ndarray, alpha: float = 1.0) -> np.ndarray:
    """C = alpha * A . B^T through the reference's cpp_sgemm (sgemm2.cpp:530-547).

    Without -DEXEC the reference ignores beta (sgemm2.cpp:312-324), so C is
    zeroed first; it also skips K < 128 entirely (sgemm2.cpp:348-365)."""
    R = ref_lib()
    if R is None:
        raise FileNotFoundError("oracle/_ref/libsgemm2_ref.so is not built")
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    N = B.shape[0]
    C = np.zeros((M, N), dtype=np.float32)
    R.cpp_sgemm(NO_TRANS, TRANS, M, N, K, alpha, _p(A), K, _p(B), K, 0.0, _p(C), N, 0, M)
    return C


def conv2d_shape(batch: int, filters: int, H: int, W: int, kH: int, kW: int, padding: int, stride: int):
    """QNNConv2DShape (quicknn_kernels.pas:984-987)."""
    return [batch, filters, (H + 2 * padding - kH) // stride + 1, (W + 2 * padding - kW) // stride + 1]


def conv2d_f64(src: np.ndarray, weights: np.ndarray, bias, in_ch: int, out_ch: int, H: int, W: int, kH: int,
               kW: int, stride: int, padding: int, batch: int = 1) -> np.ndarray:
    """QNNConv2d (quicknncpu.pas:1958-2124) in its direct form, float64 sums:
    src [batch x in_ch x H x W], weights [out_ch x in_ch*kH*kW], bias [out_ch]
    or None; returns [batch x out_ch x outH x outW] float64."""
    x = np.ascontiguousarray(src, dtype=np.float32).reshape(batch, in_ch, H, W)
    w = np.ascontiguousarray(weights, dtype=np.float32).reshape(out_ch, in_ch * kH * kW)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    shape = conv2d_shape(batch, out_ch, H, W, kH, kW, padding, stride)
    y = np.empty(shape, dtype=np.float64)
    lib().orc_conv2d_f64(_p(x), _p(w), _p(b) if b is not None else None, _p(y), in_ch, out_ch, H, W, kH, kW,
                         stride, padding, batch)
    return y


def normwise_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the parity metric)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    if den == 0.0:
        return float(np.max(np.abs(y - ref))) if y.size else 0.0
    return float(np.max(np.abs(y - ref)) / den)
