"""Host-side mirror of the reference's linear-layer operators over libinvision_hip.so.

Same names, argument order and meaning as the reference's L2 entry points
(src/quicknn_kernels.pas:216-223, 317) and the CBLAS slot
(src/quicknncpu.pas:102-103); host arrays are numpy arrays written in place,
as TMemoryBlock storage is.  Bound violations raise AssertionError with the
reference's messages (src/quicknncpu.pas:1775-1777); library failures raise
HipError.  All arithmetic happens in the HIP library: this module only moves
arguments across the C ABI.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

from . import hip
from .bf16 import as_bf16_bits

_initialized = False


def init(device: int = 0) -> None:
    """inv_hip_init; idempotent."""
    global _initialized
    if not _initialized:
        hip.call("inv_hip_init", device)
        _initialized = True


def shutdown() -> None:
    global _initialized
    if _initialized:
        hip.call("inv_hip_shutdown")
        _initialized = False


def device_info() -> dict:
    init()
    name = ctypes.create_string_buffer(256)
    cus, clk = ctypes.c_int(), ctypes.c_int()
    hip.call("inv_hip_device_info", name, 256, ctypes.byref(cus), ctypes.byref(clk))
    return {"name": name.value.decode(), "cu_count": cus.value, "clock_khz": clk.value}


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def rng_seed(seed: int) -> None:
    """The reference's rng_seed (src/quicknn_sample.pas:239-251) for this thread's
    synthetic-input stream (inv_hip_sample_seed; host only, no device needed)."""
    hip.call("inv_hip_sample_seed", int(seed) & 0xFFFFFFFFFFFFFFFF)


def randn(shape, sigma: float = 1.0, round_bf16: bool = False) -> np.ndarray:
    """prod(shape) normals from this thread's stream in order, times sigma (the
    reference's randn/random_normal, src/quicknn_sample.pas:261-276), optionally
    rounded to bf16 values (RNE); float32."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    hip.call("inv_hip_sample_randn", _ptr(out), n, float(sigma), 1 if round_bf16 else 0)
    return out.reshape(shape)


def _check_host(a: np.ndarray, dtype, name: str) -> None:
    if not isinstance(a, np.ndarray):
        raise TypeError(f"{name} must be a numpy array")
    if a.dtype != dtype:
        raise TypeError(f"{name} must be {np.dtype(dtype).name}, got {a.dtype}")
    if not a.flags.c_contiguous:
        raise ValueError(f"{name} must be C-contiguous")


# ---------------------------------------------------------------------------
# Device memory
# ---------------------------------------------------------------------------

class DeviceArray:
    """A device buffer owned by the library (inv_hip_malloc)."""

    # i32: attention key masks (no element type of the GEMM paths)
    _DT = {"f32": (np.float32, 4, hip.INV_DT_F32), "bf16": (np.uint16, 2, hip.INV_DT_BF16), "i32": (np.int32, 4, None)}

    def __init__(self, shape, dtype: str = "f32"):
        init()
        if dtype not in self._DT:
            raise ValueError("dtype must be 'f32', 'bf16' or 'i32'")
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.np_dtype, self.itemsize, self.inv_dtype = self._DT[dtype]
        self.nbytes = int(np.prod(self.shape)) * self.itemsize
        p = ctypes.c_void_p()
        hip.call("inv_hip_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray, dtype: Optional[str] = None) -> "DeviceArray":
        if dtype is None:
            dtype = {np.dtype(np.uint16): "bf16", np.dtype(np.int32): "i32"}.get(a.dtype, "f32")
        d = cls(a.shape, dtype)
        d.copy_from(a)
        return d

    def copy_from(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.np_dtype)
        if a.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        hip.call("inv_hip_memcpy_h2d", self.ptr, _ptr(a), self.nbytes)

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.np_dtype)
        hip.call("inv_hip_memcpy_d2h", _ptr(out), self.ptr, self.nbytes)
        return out

    def fill_zero(self) -> None:
        hip.call("inv_hip_memset", self.ptr, 0, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            hip.call("inv_hip_free", self.ptr)
            self.ptr = None

    def __del__(self):  # best effort
        try:
            if self.ptr and _initialized:
                hip.load().inv_hip_free(self.ptr)
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Weights: uploaded once, device resident (the bf16 source is
# TSafeTensorFile.getTensorDataMemBlockBF16, src/safetensor.pas:650-683)
# ---------------------------------------------------------------------------

class Weight:
    """A device-resident [N x K] bf16 weight with an optional fp32 bias."""

    def __init__(self, w: np.ndarray, bias: Optional[np.ndarray] = None):
        init()
        if w.ndim != 2:
            raise ValueError("weight must be 2-D [out x in]")
        self.N, self.K = (int(s) for s in w.shape)
        b = None
        if bias is not None:
            b = np.ascontiguousarray(bias, dtype=np.float32)
            if b.shape != (self.N,):
                raise ValueError("bias must have shape (N,)")
        h = ctypes.c_void_p()
        bp = _ptr(b) if b is not None else None
        if w.dtype == np.uint16:
            w = np.ascontiguousarray(w)
            hip.call("inv_hip_weight_upload", _ptr(w), self.N, self.K, bp, ctypes.byref(h))
        elif w.dtype == np.float32:
            w = np.ascontiguousarray(w)
            hip.call("inv_hip_weight_upload_f32", _ptr(w), self.N, self.K, bp, ctypes.byref(h))
        else:
            raise TypeError("weight must be bf16 bits (uint16) or float32")
        self.handle = h.value
        self.has_bias = b is not None
        self.gated = False

    @classmethod
    def gate_up(cls, gate: np.ndarray, up: np.ndarray, gate_bias: Optional[np.ndarray] = None,
                up_bias: Optional[np.ndarray] = None) -> "Weight":
        """A gate/up pair for epilogue="swiglu": Y = silu(x.Wg^T + bg) * (x.Wu^T + bu).
        gate and up are [F x K] bf16 bits (FLUX2's fused [2F x K] linear_in splits as
        gate = rows [0, F), up = rows [F, 2F), src/quicknn_transformers.pas:595-597)."""
        init()
        g = np.ascontiguousarray(gate, dtype=np.uint16)
        u = np.ascontiguousarray(up, dtype=np.uint16)
        if g.ndim != 2 or g.shape != u.shape:
            raise ValueError("gate and up must be [F x K] of the same shape")
        F, K = (int(x) for x in g.shape)
        bg = None if gate_bias is None else np.ascontiguousarray(gate_bias, dtype=np.float32)
        bu = None if up_bias is None else np.ascontiguousarray(up_bias, dtype=np.float32)
        for b in (bg, bu):
            if b is not None and b.shape != (F,):
                raise ValueError("biases must have shape (F,)")
        h = ctypes.c_void_p()
        hip.call("inv_hip_weight_upload_gate_up", _ptr(g), _ptr(u), F, K, _ptr(bg) if bg is not None else None,
                 _ptr(bu) if bu is not None else None, ctypes.byref(h))
        self = cls.__new__(cls)
        self.handle, self.N, self.K = h.value, F, K
        self.has_bias = bg is not None or bu is not None
        self.gated = True
        return self

    @classmethod
    def from_safetensors(cls, path: str, name: str, bias_name: Optional[str] = None,
                         truncate: bool = False, gate_up: bool = False, cached: bool = False) -> "Weight":
        """Upload the [N x K] tensor `name` (and 1-D `bias_name`) of a .safetensors
        file: the reference's getTensorDataMemBlockBF16 (src/safetensor.pas:650-683)
        feeding the device once.  BF16 is copied as is; F32/F16 are rounded to bf16
        (ties to even, or truncated like the reference's SingleToBF16 with truncate).
        cached=True takes the handle from the library's weight cache: the first
        request uploads, later ones for the same file and tensor return the resident
        weight, and free() releases the reference instead of the memory."""
        init()
        h = ctypes.c_void_p()
        flags = (hip.INV_ST_TRUNCATE if truncate else 0) | (hip.INV_ST_GATE_UP if gate_up else 0)
        hip.call("inv_hip_weight_cache_get" if cached else "inv_hip_weight_load_safetensors", os.fsencode(path),
                 name.encode(), bias_name.encode() if bias_name else None, flags, ctypes.byref(h))
        self = cls.__new__(cls)
        self.handle = h.value
        n, k = ctypes.c_int64(), ctypes.c_int64()
        hip.call("inv_hip_weight_shape", self.handle, ctypes.byref(n), ctypes.byref(k))
        self.N, self.K = n.value, k.value
        self.has_bias = bool(bias_name)
        self.gated = gate_up
        return self

    def free(self) -> None:
        if self.handle:
            hip.call("inv_hip_weight_free", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


_EPI = {"none": hip.INV_EPI_NONE, "silu": hip.INV_EPI_SILU, "gelu": hip.INV_EPI_GELU_ERF,
        "swiglu": hip.INV_EPI_SWIGLU}


def linear_device(x: DeviceArray, W: Weight, y: DeviceArray, M: int, epilogue: str = "none",
                  bias: Optional[DeviceArray] = None, asynchronous: bool = False, precise: bool = False) -> None:
    """inv_hip_linear on device-resident activations: y = epi(x . W^T + bias)."""
    flags = hip.INV_FLAG_DEVICE_PTRS | (hip.INV_FLAG_ASYNC if asynchronous else 0)
    flags |= hip.INV_FLAG_PRECISE if precise else 0
    hip.call("inv_hip_linear", x.ptr, x.inv_dtype, W.handle, bias.ptr if bias is not None else None, y.ptr,
             y.inv_dtype, M, W.K, W.N, _EPI[epilogue], flags)


def linear(x: np.ndarray, W: Weight, bias: Optional[np.ndarray] = None, epilogue: str = "none",
           out_dtype: str = "f32", precise: bool = False) -> np.ndarray:
    """Host arrays in and out: Y[M x N] = epi(X[M x K] . W^T + bias)."""
    if x.dtype not in (np.float32, np.uint16):
        raise TypeError("x must be float32 or bf16 bits (uint16)")
    x = np.ascontiguousarray(x)
    M = x.shape[0]
    if x.ndim != 2 or x.shape[1] != W.K:
        raise ValueError(f"x must be [M x {W.K}]")
    xdt = hip.INV_DT_F32 if x.dtype == np.float32 else hip.INV_DT_BF16
    ydt, ynp = (hip.INV_DT_F32, np.float32) if out_dtype == "f32" else (hip.INV_DT_BF16, np.uint16)
    y = np.empty((M, W.N), dtype=ynp)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    hip.call("inv_hip_linear", _ptr(x), xdt, W.handle, _ptr(b) if b is not None else None, _ptr(y), ydt, M, W.K,
             W.N, _EPI[epilogue], hip.INV_FLAG_PRECISE if precise else 0)
    return y


def linear_gated_add_device(x: DeviceArray, W: Weight, y: DeviceArray, M: int, gate: Optional[DeviceArray] = None,
                            bias: Optional[DeviceArray] = None, asynchronous: bool = False,
                            precise: bool = False) -> None:
    """inv_hip_linear_gated_add on resident buffers: y += gate * (x . W^T + bias), y fp32 [M x N]."""
    if y.inv_dtype != hip.INV_DT_F32:
        raise TypeError("the residual stream y must be f32")
    flags = hip.INV_FLAG_DEVICE_PTRS | (hip.INV_FLAG_ASYNC if asynchronous else 0)
    flags |= hip.INV_FLAG_PRECISE if precise else 0
    hip.call("inv_hip_linear_gated_add", x.ptr, x.inv_dtype, W.handle, bias.ptr if bias is not None else None,
             gate.ptr if gate is not None else None, y.ptr, M, W.K, W.N, flags)


def linear_gated_add(y: np.ndarray, x: np.ndarray, W: Weight, gate: Optional[np.ndarray],
                     bias: Optional[np.ndarray] = None, precise: bool = False) -> np.ndarray:
    """Host arrays, y updated in place: y[M x N] += gate[N] * (x[M x K] . W^T + bias)."""
    if x.dtype not in (np.float32, np.uint16):
        raise TypeError("x must be float32 or bf16 bits (uint16)")
    _check_host(y, np.float32, "y")
    x = np.ascontiguousarray(x)
    M = x.shape[0]
    if x.ndim != 2 or x.shape[1] != W.K:
        raise ValueError(f"x must be [M x {W.K}]")
    if y.shape != (M, W.N):
        raise ValueError(f"y must be [{M} x {W.N}]")
    xdt = hip.INV_DT_F32 if x.dtype == np.float32 else hip.INV_DT_BF16
    g = np.ascontiguousarray(gate, dtype=np.float32) if gate is not None else None
    if g is not None and g.size != W.N:
        raise ValueError(f"gate must have {W.N} values")
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    hip.call("inv_hip_linear_gated_add", _ptr(x), xdt, W.handle, _ptr(b) if b is not None else None,
             _ptr(g) if g is not None else None, _ptr(y), M, W.K, W.N, hip.INV_FLAG_PRECISE if precise else 0)
    return y


_NORM = {"adaln": hip.INV_NORM_ADALN, "rms": hip.INV_NORM_RMS}
EPSILON = 1e-6  # the reference's normalisation epsilon (src/quicknn_common.pas:51)


def linear_norm(x: np.ndarray, norm: str, W: Weight, scale: Optional[np.ndarray], shift: Optional[np.ndarray] = None,
                bias: Optional[np.ndarray] = None, epilogue: str = "none", out_dtype: str = "f32",
                eps: float = EPSILON) -> np.ndarray:
    """Host arrays: Y = epi(norm(x) . W^T + bias), norm "adaln" ((1 + scale) * layernorm(x) + shift,
    QNNAdaLN) or "rms" (x * scale / rms(x), QNNRMSNorm), x fp32 [M x K]."""
    _check_host(x, np.float32, "x")
    if x.ndim != 2 or x.shape[1] != W.K:
        raise ValueError(f"x must be [M x {W.K}]")
    vecs = []
    for v, nm in ((scale, "scale"), (shift, "shift"), (bias, "bias")):
        if v is not None:
            v = np.ascontiguousarray(v, dtype=np.float32)
            if v.size != (W.N if nm == "bias" else W.K):
                raise ValueError(f"{nm} has {v.size} values")
        vecs.append(v)
    sc, sh, b = vecs
    ydt, ynp = (hip.INV_DT_F32, np.float32) if out_dtype == "f32" else (hip.INV_DT_BF16, np.uint16)
    y = np.empty((x.shape[0], W.N), dtype=ynp)
    hip.call("inv_hip_linear_norm", _ptr(x), _NORM[norm], _ptr(sc) if sc is not None else None,
             _ptr(sh) if sh is not None else None, float(eps), W.handle, _ptr(b) if b is not None else None, _ptr(y),
             ydt, x.shape[0], W.K, W.N, _EPI[epilogue], 0)
    return y


def QNNAdaLNLinear(dst: np.ndarray, x: np.ndarray, shift: np.ndarray, scale: np.ndarray, weight, weight_bf16,
                   seq: int, hidden: int, dstDim: int) -> None:
    """QNNAdaLN(norm, x, shift, scale, seq, hidden) then QNNLINEAR_BF16_OR_F32(dst, norm, ...)
    (src/quicknn_transformers.pas:1400-1404), as one normalising projection."""
    _bound(weight is not None or weight_bf16 is not None,
           "ERROR QNNLINEAR_BF16_OR_F32 : no weight or weight_16 assigned!")
    for a, nm in ((dst, "dst"), (x, "x"), (shift, "shift"), (scale, "scale")):
        _check_host(a, np.float32, nm)
    _bound(x.size >= seq * hidden and dst.size >= seq * dstDim, "ERROR : QNNAdaLN out of bound")
    _bound(shift.size >= hidden and scale.size >= hidden, "ERROR : QNNAdaLN out of bound [shift/scale]")
    W = weight_bf16 if weight_bf16 is not None else weight
    w = _linear_weight(W)
    try:
        _bound(w.N == dstDim and w.K == hidden, "ERROR : QNNLinear weight shape mismatch")
        _bound(not w.has_bias, "ERROR : QNNLINEAR_BF16_OR_F32 takes no bias")
        hip.call("inv_hip_linear_norm", _ptr(x), hip.INV_NORM_ADALN, _ptr(scale), _ptr(shift), EPSILON, w.handle, None,
                 _ptr(dst), hip.INV_DT_F32, seq, hidden, dstDim, hip.INV_EPI_NONE, 0)
    finally:
        if w is not W:
            w.free()


def _key_mask_host(key_mask, seq_k: int):
    if key_mask is None:
        return None
    m = np.ascontiguousarray(key_mask, dtype=np.int32)
    if m.shape != (seq_k,):
        raise ValueError(f"key_mask must have seq_k = {seq_k} entries")
    return m


def attention(Q: np.ndarray, K: np.ndarray, V: np.ndarray, heads: int, head_dim: int, kv_heads: Optional[int] = None,
              scale: Optional[float] = None, causal: bool = False, out_dtype: str = "f32",
              key_mask: Optional[np.ndarray] = None) -> np.ndarray:
    """Host arrays: O[seq_q x heads*head_dim] = softmax(scale * Q.K^T) V per head.

    Q [seq_q x heads*head_dim], K and V [seq_k x kv_heads*head_dim], float32 or bf16
    bits (uint16, all three alike); scale defaults to 1/sqrt(head_dim).  key_mask
    (seq_k ints): keys with 0 are hidden from every query (Qwen3's attention
    mask, src/quicknn_qwen3.pas:753)."""
    kv_heads = heads if kv_heads is None else kv_heads
    if Q.dtype not in (np.float32, np.uint16) or K.dtype != Q.dtype or V.dtype != Q.dtype:
        raise TypeError("Q, K and V must all be float32 or all bf16 bits (uint16)")
    Q, K, V = (np.ascontiguousarray(a) for a in (Q, K, V))
    if Q.ndim != 2 or Q.shape[1] != heads * head_dim:
        raise ValueError(f"Q must be [seq_q x {heads * head_dim}]")
    if K.ndim != 2 or K.shape[1] != kv_heads * head_dim or V.shape != K.shape:
        raise ValueError(f"K and V must be [seq_k x {kv_heads * head_dim}]")
    dt = hip.INV_DT_F32 if Q.dtype == np.float32 else hip.INV_DT_BF16
    odt, onp = (hip.INV_DT_F32, np.float32) if out_dtype == "f32" else (hip.INV_DT_BF16, np.uint16)
    O = np.empty((Q.shape[0], heads * head_dim), dtype=onp)
    sc = 1.0 / float(np.sqrt(head_dim)) if scale is None else float(scale)
    flags = hip.INV_ATTN_CAUSAL if causal else 0
    m = _key_mask_host(key_mask, K.shape[0])
    if m is None:
        hip.call("inv_hip_attention", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), dt, odt, heads, kv_heads, Q.shape[0],
                 K.shape[0], head_dim, sc, flags)
    else:
        hip.call("inv_hip_attention_masked", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), dt, odt, heads, kv_heads, Q.shape[0],
                 K.shape[0], head_dim, sc, _ptr(m), flags)
    return O


def attention_device(Q: DeviceArray, K: DeviceArray, V: DeviceArray, O: DeviceArray, heads: int, head_dim: int,
                     kv_heads: Optional[int] = None, scale: Optional[float] = None, causal: bool = False,
                     asynchronous: bool = False, key_mask: Optional[DeviceArray] = None) -> None:
    """inv_hip_attention on resident buffers (the shapes as for attention();
    key_mask an i32 DeviceArray of seq_k entries)."""
    kv_heads = heads if kv_heads is None else kv_heads
    if not (Q.dtype == K.dtype == V.dtype):
        raise TypeError("Q, K and V must share a dtype")
    sc = 1.0 / float(np.sqrt(head_dim)) if scale is None else float(scale)
    flags = hip.INV_FLAG_DEVICE_PTRS | (hip.INV_FLAG_ASYNC if asynchronous else 0)
    flags |= hip.INV_ATTN_CAUSAL if causal else 0
    if key_mask is None:
        hip.call("inv_hip_attention", Q.ptr, K.ptr, V.ptr, O.ptr, Q.inv_dtype, O.inv_dtype, heads, kv_heads,
                 Q.shape[0], K.shape[0], head_dim, sc, flags)
    else:
        if key_mask.dtype != "i32" or key_mask.shape != (K.shape[0],):
            raise ValueError("key_mask must be an i32 DeviceArray of seq_k entries")
        hip.call("inv_hip_attention_masked", Q.ptr, K.ptr, V.ptr, O.ptr, Q.inv_dtype, O.inv_dtype, heads, kv_heads,
                 Q.shape[0], K.shape[0], head_dim, sc, key_mask.ptr, flags)


def QNNFlashAttention(dst: np.ndarray, Q: np.ndarray, K: np.ndarray, V: np.ndarray, heads: int, seq_q: int,
                      seq_k: int, head_dim: int, scale: float) -> None:
    """TQNNSingleOPS.QNNFlashAttention (src/quicknncpu.pas:2763) on fp32 host arrays:
    dst[seq_q x heads*head_dim] = softmax(scale * Q.K^T) V for every head.  The
    argument order is the one its callers use (src/quicknn_transformers.pas:1203,
    1301-1302)."""
    for a, nm in ((dst, "dst"), (Q, "Q"), (K, "K"), (V, "V")):
        _check_host(a, np.float32, nm)
    hidden = heads * head_dim
    _bound(Q.size >= seq_q * hidden and dst.size >= seq_q * hidden, "ERROR : QNNFlashAttention out of bound [Q/dst]")
    _bound(K.size >= seq_k * hidden and V.size >= seq_k * hidden, "ERROR : QNNFlashAttention out of bound [K/V]")
    hip.call("inv_hip_attention", _ptr(Q), _ptr(K), _ptr(V), _ptr(dst), hip.INV_DT_F32, hip.INV_DT_F32, heads, heads,
             seq_q, seq_k, head_dim, float(scale), 0)


# ---------------------------------------------------------------------------
# Between the Q/K projections and attention
# ---------------------------------------------------------------------------

_ROPE = {None: hip.INV_ROPE_NONE, "interleaved": hip.INV_ROPE_INTERLEAVED, "half": hip.INV_ROPE_HALF}


def head_norm_rope(x: np.ndarray, heads: int, head_dim: int, norm_weight: Optional[np.ndarray] = None,
                   rope: Optional[str] = None, cos: Optional[np.ndarray] = None,
                   sin: Optional[np.ndarray] = None, seq: Optional[int] = None) -> None:
    """In place on the first seq rows of fp32 x [seq x heads*head_dim] (seq
    defaults to all of x): each head's RMSNorm (weight [head_dim], or none),
    then the rotary embedding ("interleaved": tables [seq x head_dim]; "half":
    [seq x head_dim/2]; None: none)."""
    _check_host(x, np.float32, "x")
    seq = x.size // (heads * head_dim) if seq is None else int(seq)
    if x.size < seq * heads * head_dim:
        raise ValueError("x must hold seq x heads*head_dim values")
    w = None if norm_weight is None else np.ascontiguousarray(norm_weight, dtype=np.float32)
    if w is not None and w.size != head_dim:
        raise ValueError("norm_weight must have head_dim entries")
    c = s_ = None
    if rope is not None:
        width = head_dim if rope == "interleaved" else head_dim // 2
        c, s_ = (np.ascontiguousarray(np.asarray(t, dtype=np.float32).reshape(-1)[:seq * width]) for t in (cos, sin))
        if c.size != seq * width or s_.size != seq * width:
            raise ValueError(f"rotary tables must hold seq x {width} values")
    hip.call("inv_hip_head_norm_rope", _ptr(x), seq, heads, head_dim, _ptr(w) if w is not None else None, _ROPE[rope],
             _ptr(c) if c is not None else None, _ptr(s_) if s_ is not None else None, 0)


def attention_qk_norm_rope(Q: np.ndarray, K: np.ndarray, V: np.ndarray, heads: int, head_dim: int,
                           kv_heads: Optional[int] = None, scale: Optional[float] = None, causal: bool = False,
                           q_norm_weight: Optional[np.ndarray] = None, k_norm_weight: Optional[np.ndarray] = None,
                           rope: Optional[str] = None, q_cos=None, q_sin=None, k_cos=None, k_sin=None,
                           key_mask: Optional[np.ndarray] = None, out_dtype: str = "f32") -> np.ndarray:
    """Attention on fp32 host Q, K, V with each head's RMSNorm and the rotary
    embedding of Q and K fused into their staging (inv_hip_attention_qk_norm_rope):
    the same result as head_norm_rope on Q and K, then attention()."""
    kv_heads = heads if kv_heads is None else kv_heads
    Q, K, V = (np.ascontiguousarray(a, dtype=np.float32) for a in (Q, K, V))
    sq, sk = Q.shape[0], K.shape[0]
    if Q.shape[1] != heads * head_dim or K.shape[1] != kv_heads * head_dim or V.shape != K.shape:
        raise ValueError("Q [seq_q x heads*head_dim], K and V [seq_k x kv_heads*head_dim]")
    vec = lambda a, n: None if a is None else np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1)[:n])
    width = head_dim if rope == "interleaved" else head_dim // 2
    qw, kw = vec(q_norm_weight, head_dim), vec(k_norm_weight, head_dim)
    qc, qs = (vec(t, sq * width) for t in (q_cos, q_sin)) if rope else (None, None)
    kc, ks = (vec(t, sk * width) for t in (k_cos, k_sin)) if rope else (None, None)
    m = _key_mask_host(key_mask, sk)
    odt, onp = (hip.INV_DT_F32, np.float32) if out_dtype == "f32" else (hip.INV_DT_BF16, np.uint16)
    O = np.empty((sq, heads * head_dim), dtype=onp)
    sc = 1.0 / float(np.sqrt(head_dim)) if scale is None else float(scale)
    p = lambda a: _ptr(a) if a is not None else None
    hip.call("inv_hip_attention_qk_norm_rope", _ptr(Q), 0, _ptr(K), 0, _ptr(V), 0, _ptr(O), odt, heads, kv_heads, sq,
             sk, head_dim, sc, p(qw), p(kw), _ROPE[rope], p(qc), p(qs), p(kc), p(ks), p(m),
             hip.INV_ATTN_CAUSAL if causal else 0)
    return O


def QNNQKRMSNorm(Q: np.ndarray, K: np.ndarray, QWeights: np.ndarray, KWeights: np.ndarray, seq: int, heads: int,
                 headDim: int) -> None:
    """TQNNSingleOPS.QNNQKRMSNorm (src/quicknncpu.pas:2209-2246), in place."""
    _bound(Q.size >= seq * heads * headDim and K.size >= seq * heads * headDim, "ERROR : QNNQKRMSNorm out of bound")
    head_norm_rope(Q, heads, headDim, QWeights, seq=seq)
    head_norm_rope(K, heads, headDim, KWeights, seq=seq)


def QNNApplyRoPE2D(dst: np.ndarray, cos_freq: np.ndarray, sin_freq: np.ndarray, seq: int, heads: int, head_dim: int,
                   dim: int) -> None:
    """TQNNSingleOPS.QNNApplyRoPE2D (src/quicknncpu.pas:2968-2992), in place: pairs
    (2k, 2k+1) with cos/sin[s*head_dim + 2k] (dim, the axis size, is unused there too)."""
    _bound(dst.size >= seq * heads * head_dim, "ERROR : QNNApplyRoPE2D out of bound")
    head_norm_rope(dst, heads, head_dim, None, "interleaved", cos_freq, sin_freq, seq=seq)


def QNNApplyRoPE3(dst: np.ndarray, cosIn: np.ndarray, sinIn: np.ndarray, seqLen: int, numHeads: int,
                  headDim: int) -> None:
    """TQNNSingleOPS.QNNApplyRoPE3 (src/quicknncpu.pas:2910-2917), in place: pairs
    (i, i + headDim/2) with cos/sin[s*headDim/2 + i]."""
    _bound(dst.size >= seqLen * numHeads * headDim, "ERROR : QNNApplyRoPE3 out of bound")
    head_norm_rope(dst, numHeads, headDim, None, "half", cosIn, sinIn, seq=seqLen)


def QNNHeadRSMNorm(dst: np.ndarray, src: np.ndarray, weight: np.ndarray, seqLen: int, numHeads: int,
                   headDim: int) -> None:
    """QNNHeadRSMNorm (src/quicknn_qwen3.pas:223-230): dst = per-head RMSNorm(src)."""
    _bound(src.size >= seqLen * numHeads * headDim and dst.size >= seqLen * numHeads * headDim,
           "ERROR : QNNHeadRSMNorm out of bound")
    if dst is not src:
        np.copyto(dst.reshape(-1)[:seqLen * numHeads * headDim], src.reshape(-1)[:seqLen * numHeads * headDim])
    head_norm_rope(dst, numHeads, headDim, weight, seq=seqLen)


# ---------------------------------------------------------------------------
# Convolution (TQNNSingleOPS.QNNConv2d, src/quicknncpu.pas:1958-2124)
# ---------------------------------------------------------------------------

def QNNConv2DShape(batch: int, filters: int, srcH: int, srcW: int, kH: int, kW: int, padding: int,
                   stride: int) -> list:
    """Output dims [batch, filters, outH, outW] (src/quicknn_kernels.pas:984-987)."""
    return [batch, filters, (srcH + 2 * padding - kH) // stride + 1, (srcW + 2 * padding - kW) // stride + 1]


def _conv_weight(weights, out_ch: int, K: int, bias: Optional[np.ndarray] = None) -> Weight:
    if isinstance(weights, Weight):
        return weights
    w = np.ascontiguousarray(weights, dtype=np.float32).reshape(-1)
    _bound(w.size >= out_ch * K, "ERROR [Conv2D] : weights out of bound")
    return Weight(w[:out_ch * K].reshape(out_ch, K))


def conv2d_device(src: DeviceArray, weight: Weight, dst: DeviceArray, in_ch: int, out_ch: int, H: int, W: int,
                  kH: int, kW: int, stride: int, padding: int, batch: int = 1, bias: Optional[DeviceArray] = None,
                  asynchronous: bool = False) -> None:
    """inv_hip_conv2d on device-resident NCHW fp32 images."""
    flags = hip.INV_FLAG_DEVICE_PTRS | (hip.INV_FLAG_ASYNC if asynchronous else 0)
    hip.call("inv_hip_conv2d", src.ptr, weight.handle, bias.ptr if bias is not None else None, dst.ptr, in_ch, out_ch,
             H, W, kH, kW, stride, padding, batch, flags)


def conv2d(src: np.ndarray, weights, bias: Optional[np.ndarray], in_ch: int, out_ch: int, H: int, W: int, kH: int,
           kW: int, stride: int, padding: int, batch: int = 1) -> np.ndarray:
    """Host arrays in and out: dst [batch x out_ch x outH x outW] = conv(src) + bias.

    weights: a resident Weight of [out_ch x in_ch*kH*kW] or the host fp32
    filter (uploaded for this call only)."""
    dims = QNNConv2DShape(batch, out_ch, H, W, kH, kW, padding, stride)
    dst = np.empty(dims, dtype=np.float32)
    QNNConv2d(dst, src, weights, bias, in_ch, out_ch, H, W, kH, kW, stride, padding, batch)
    return dst


def QNNConv2d(dst: np.ndarray, src: np.ndarray, weights, bias: Optional[np.ndarray], in_ch: int, out_ch: int,
              H: int, W: int, kH: int, kW: int, stride: int, padding: int, batch: int = 1) -> None:
    """QNNConv2d (src/quicknn_kernels.pas:990-1006 -> src/quicknncpu.pas:1958-2124): NCHW fp32
    dst = conv(src, weights [out_ch x in_ch*kH*kW]) + bias[out_ch] (bias may be None)."""
    _check_host(dst, np.float32, "dst")
    _check_host(src, np.float32, "src")
    dims = QNNConv2DShape(batch, out_ch, H, W, kH, kW, padding, stride)
    _bound(all(d > 0 for d in dims[1:]), "ERROR [Conv2D] : empty output")
    _bound(dst.size >= int(np.prod(dims)), "ERROR [Conv2D] : Incorrect destination size")
    _bound(src.size >= batch * in_ch * H * W, "ERROR [Conv2D] : source out of bound")
    b = None
    if bias is not None:
        _check_host(bias, np.float32, "bias")
        _bound(bias.size >= out_ch, "ERROR [Conv2D] : bias out of bound")
        b = bias
    w = _conv_weight(weights, out_ch, in_ch * kH * kW)
    try:
        hip.call("inv_hip_conv2d", _ptr(src), w.handle, _ptr(b) if b is not None else None, _ptr(dst), in_ch,
                 out_ch, H, W, kH, kW, stride, padding, batch, 0)
    finally:
        if w is not weights:
            w.free()


def set_sgemm_precision(mode: int) -> None:
    """INV_PREC_BF16 / INV_PREC_SPLIT_A / INV_PREC_SPLIT_AB for cblas_gemm."""
    init()
    hip.call("inv_hip_set_sgemm_precision", mode)


# ---------------------------------------------------------------------------
# The reference's operator surface
# ---------------------------------------------------------------------------

def _bound(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def cblas_gemm(Order: int, TransA: int, TransB: int, M: int, N: int, K: int, alpha: float, A: np.ndarray, lda: int,
               B: np.ndarray, ldb: int, beta: float, C: np.ndarray, ldc: int) -> None:
    """TQNNSingleOPS.cblas_gemm -> cblas_sgemm slot (src/quicknncpu.pas:335-350), fp32 host arrays."""
    _check_host(A, np.float32, "A")
    _check_host(B, np.float32, "B")
    _check_host(C, np.float32, "C")
    hip.call("inv_hip_sgemm", Order, TransA, TransB, M, N, K, float(alpha), _ptr(A), lda, _ptr(B), ldb,
             float(beta), _ptr(C), ldc)


def cblas_sbgemm(Order: int, TransA: int, TransB: int, M: int, N: int, K: int, alpha: float, A: np.ndarray,
                 lda: int, B: np.ndarray, ldb: int, beta: float, C: np.ndarray, ldc: int) -> None:
    """The cblas_sbgemm slot (src/quicknncpu.pas:110-111): bf16 A and B, fp32 C."""
    _check_host(A, np.uint16, "A")
    _check_host(B, np.uint16, "B")
    _check_host(C, np.float32, "C")
    hip.call("inv_hip_sbgemm", Order, TransA, TransB, M, N, K, float(alpha), _ptr(A), lda, _ptr(B), ldb,
             float(beta), _ptr(C), ldc)


def QNNMatMulNT(C: np.ndarray, A: np.ndarray, B: np.ndarray, M: int, K: int, N: int) -> None:
    """C[M x N] = A[M x K] . B[N x K]^T  (src/quicknncpu.pas:1773-1784)."""
    _bound(A.size >= M * K, "ERROR : QNNMatMul out of bound [A]")
    _bound(B.size >= N * K, "ERROR : QNNMatMul out of bound [B]")
    _bound(C.size >= M * N, "ERROR : QNNMatMul out of bound [C]")
    cblas_gemm(hip.CblasRowMajor, hip.CblasNoTrans, hip.CblasTrans, M, N, K, 1.0, A, K, B, K, 0.0, C, N)


def QNNMatMulNN(C: np.ndarray, A: np.ndarray, B: np.ndarray, M: int, K: int, N: int) -> None:
    """C[M x N] = A[M x K] . B[K x N]  (src/quicknncpu.pas:1760-1771)."""
    _bound(A.size >= M * K, "ERROR : QNNMatMul out of bound [A]")
    _bound(B.size >= K * N, "ERROR : QNNMatMul out of bound [B]")
    _bound(C.size >= M * N, "ERROR : QNNMatMul out of bound [C]")
    cblas_gemm(hip.CblasRowMajor, hip.CblasNoTrans, hip.CblasNoTrans, M, N, K, 1.0, A, K, B, N, 0.0, C, N)


def QNNMatMulTN(C: np.ndarray, A: np.ndarray, B: np.ndarray, M: int, K: int, N: int) -> None:
    """C[M x N] = A[K x M]^T . B[K x N] as the reference calls it (src/quicknncpu.pas:1786-1797)."""
    _bound(A.size >= K * M, "ERROR : QNNMatMul out of bound [A]")
    _bound(B.size >= N * K, "ERROR : QNNMatMul out of bound [B]")
    _bound(C.size >= M * N, "ERROR : QNNMatMul out of bound [C]")
    cblas_gemm(hip.CblasRowMajor, hip.CblasTrans, hip.CblasNoTrans, M, N, K, 1.0, A, K, B, K, 0.0, C, N)


def _linear_weight(W) -> Weight:
    if isinstance(W, Weight):
        return W
    return Weight(W)


def _run_linear(dst: np.ndarray, x: np.ndarray, W, B: Optional[np.ndarray], seqLen: int, inDIM: int,
                outDIM: int) -> None:
    _check_host(dst, np.float32, "dst")
    _check_host(x, np.float32, "x")
    _bound(x.size >= seqLen * inDIM, "ERROR : QNNLinear out of bound [x]")
    _bound(dst.size >= seqLen * outDIM, "ERROR : QNNLinear out of bound [dst]")
    w = _linear_weight(W)
    try:
        _bound(w.N == outDIM and w.K == inDIM, "ERROR : QNNLinear weight shape mismatch")
        b = None
        if B is not None:
            _check_host(B, np.float32, "B")
            _bound(B.size >= outDIM, "ERROR : QNNLinear out of bound [B]")
            b = B
        hip.call("inv_hip_linear", _ptr(x), hip.INV_DT_F32, w.handle, _ptr(b) if b is not None else None, _ptr(dst),
                 hip.INV_DT_F32, seqLen, inDIM, outDIM, hip.INV_EPI_NONE, 0)
    finally:
        if w is not W:
            w.free()


def QNNLinear(dst: np.ndarray, x: np.ndarray, W, B: Optional[np.ndarray], seqLen: int, inDIM: int,
              outDIM: int) -> None:
    """dst = x . W^T (+ B per row)  (src/quicknncpu.pas:1807-1820).

    W may be a resident Weight (uploaded once) or a host array (float32 or bf16
    bits), which is uploaded for this call only."""
    _run_linear(dst, x, W, B, seqLen, inDIM, outDIM)


def QNNLinearNoBias(dst: np.ndarray, x: np.ndarray, W, seqLen: int, inDIM: int, outDIM: int) -> None:
    """dst = x . W^T  (src/quicknncpu.pas:1822-1828)."""
    if isinstance(W, Weight):
        # A resident weight may carry a bias; QNNLinearNoBias must not add it.
        _bound(not _weight_has_bias(W), "ERROR : QNNLinearNoBias called with a biased Weight")
    _run_linear(dst, x, W, None, seqLen, inDIM, outDIM)


def QNNLinearNoBias_BF16(dst: np.ndarray, x: np.ndarray, W: np.ndarray, seqLen: int, inDIM: int,
                         outDIM: int) -> None:
    """dst = x . bf16(W)^T  (src/quicknncpu.pas:1830-1847); W is bf16 bits or a Weight."""
    if not isinstance(W, Weight):
        _check_host(W, np.uint16, "W")
    _run_linear(dst, x, W, None, seqLen, inDIM, outDIM)


def QNNLINEAR_BF16_OR_F32(dst: np.ndarray, src: np.ndarray, weight, weight_bf16, seq: int, srcDim: int,
                          dstDim: int) -> None:
    """bf16 weight if assigned, else fp32 (src/quicknncpu.pas:3062-3071)."""
    _bound(weight is not None or weight_bf16 is not None,
           "ERROR QNNLINEAR_BF16_OR_F32 : no weight or weight_16 assigned!")
    if weight_bf16 is not None:
        QNNLinearNoBias_BF16(dst, src, weight_bf16, seq, srcDim, dstDim)
    else:
        QNNLinearNoBias(dst, src, weight, seq, srcDim, dstDim)


def QNNLinearGatedAdd(dst: np.ndarray, src: np.ndarray, weight, weight_bf16, gate: np.ndarray, seq: int,
                      srcDim: int, dstDim: int) -> None:
    """QNNLINEAR_BF16_OR_F32 into a scratch projection followed by QNNGatedAdd
    (src/quicknn_transformers.pas:1432-1438), as one GEMM: dst += gate * src . W^T."""
    _bound(weight is not None or weight_bf16 is not None,
           "ERROR QNNLINEAR_BF16_OR_F32 : no weight or weight_16 assigned!")
    _check_host(dst, np.float32, "dst")
    _check_host(src, np.float32, "src")
    _bound(src.size >= seq * srcDim, "ERROR : QNNLinear out of bound [x]")
    _bound(dst.size >= seq * dstDim, "ERROR : QNNLinear out of bound [dst]")
    W = weight_bf16 if weight_bf16 is not None else weight
    if not isinstance(W, Weight) and weight_bf16 is not None:
        _check_host(W, np.uint16, "W")
    w = _linear_weight(W)
    try:
        _bound(w.N == dstDim and w.K == srcDim, "ERROR : QNNLinear weight shape mismatch")
        _bound(not w.has_bias, "ERROR : QNNLINEAR_BF16_OR_F32 takes no bias")
        g = None
        if gate is not None:
            _check_host(gate, np.float32, "gate")
            _bound(gate.size >= dstDim, "ERROR : QNNGatedAdd out of bound [gate]")
            g = gate
        hip.call("inv_hip_linear_gated_add", _ptr(src), hip.INV_DT_F32, w.handle, None,
                 _ptr(g) if g is not None else None, _ptr(dst), seq, srcDim, dstDim, 0)
    finally:
        if w is not W:
            w.free()


def _weight_has_bias(W: Weight) -> bool:
    return W.has_bias


def stats() -> dict:
    calls, ms, flops = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()
    hip.call("inv_hip_stats", ctypes.byref(calls), ctypes.byref(ms), ctypes.byref(flops))
    return {"calls": calls.value, "gemm_ms": ms.value, "flops": flops.value}


def as_weight(w: np.ndarray, bias: Optional[np.ndarray] = None) -> Weight:
    """Upload a host weight (bf16 bits, or float32 rounded to bf16)."""
    if w.dtype not in (np.uint16, np.float32):
        w = as_bf16_bits(w)
    return Weight(w, bias)


_ST_DTYPES = {hip.INV_DT_F16: "F16", hip.INV_DT_BF16: "BF16", hip.INV_DT_F32: "F32"}


def safetensors_info(path: str, name: str) -> dict:
    """dtype ("F32"/"BF16"/"F16", or None for other dtypes), shape and data byte
    offset of tensor `name` (TSafeTensorFile.find, src/safetensor.pas:491-507).
    Parses the header only: no device needed."""
    dt, nd, off = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    shape = (ctypes.c_int64 * hip.INV_ST_MAX_DIMS)()
    hip.call("inv_hip_safetensors_info", os.fsencode(path), name.encode(), ctypes.byref(dt), ctypes.byref(nd),
             shape, ctypes.byref(off))
    return {"dtype": _ST_DTYPES.get(dt.value), "shape": tuple(shape[i] for i in range(nd.value)),
            "data_offset": off.value}


class SafeTensorFiles:
    """The reference's TSafeTensorFilesHelper (src/safetensor.pas:584-683): a set
    of .safetensors shards searched by tensor name.  Built from file paths, or
    from a directory holding `model.safetensors.index.json` (its "weight_map",
    as src/quicknn_transformers.pas:536-556 reads it) or *.safetensors files."""

    def __init__(self, paths):
        import glob
        import json
        if isinstance(paths, (str, os.PathLike)) and os.path.isdir(paths):
            idx = os.path.join(paths, "model.safetensors.index.json")
            if os.path.exists(idx):
                wm = json.load(open(idx))["weight_map"]
                self._where = {n: os.path.join(paths, f) for n, f in wm.items()}
                self.paths = sorted(set(self._where.values()))
                return
            paths = sorted(glob.glob(os.path.join(paths, "*.safetensors")))
        elif isinstance(paths, (str, os.PathLike)):
            paths = [paths]
        self.paths = [os.fspath(p) for p in paths]
        self._where = None

    def find(self, name: str) -> str:
        """The shard that holds `name` (assert-style error if none does)."""
        if self._where is not None:
            if name not in self._where:
                raise KeyError(f"cannot find tensor \"{name}\" in the index")
            return self._where[name]
        for p in self.paths:
            try:
                safetensors_info(p, name)
                return p
            except hip.HipError:
                continue
        raise KeyError(f"cannot find tensor \"{name}\" in {len(self.paths)} file(s)")

    def linear_weight(self, name: str, bias_name: Optional[str] = None, truncate: bool = False,
                      cached: bool = True) -> Weight:
        """A device weight for a Linear layer (bias from the same shard).  By default from the
        library's weight cache: the reference loads every block's weights again on every
        sampler step and frees them (src/quicknn_transformers.pas:1581-1602); here the first
        request uploads and the rest reuse the resident copy (free() releases the reference)."""
        return Weight.from_safetensors(self.find(name), name, bias_name, truncate, cached=cached)


def weight_cache_stats() -> dict:
    """Entries, resident bytes, hits, misses and bytes uploaded by the weight cache."""
    v = [ctypes.c_int64() for _ in range(5)]
    hip.call("inv_hip_weight_cache_stats", *(ctypes.byref(x) for x in v))
    return dict(zip(("entries", "bytes", "hits", "misses", "uploaded_bytes"), (x.value for x in v)))


def weight_cache_set_budget(nbytes: int) -> None:
    """Evict least recently used, unreferenced cached weights above nbytes (0: no limit)."""
    hip.call("inv_hip_weight_cache_set_budget", int(nbytes))


def weight_cache_clear() -> None:
    hip.call("inv_hip_weight_cache_clear")
