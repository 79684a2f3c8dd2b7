"""ctypes binding of libinvision_hip.so (declarations in include/inv_hip.h).

This module only loads the in-tree native library; there is no CPU fallback.
If the library is missing or fails to load, every entry point raises
HipLibraryError, so a caller can never silently run without the GPU kernels.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint16, c_void_p

from .build import LIB_PATH

# Status codes (include/inv_hip.h)
INV_OK = 0
INV_ERR_ARG = 1
INV_ERR_UNSUPPORTED = 2
INV_ERR_NO_DEVICE = 3
INV_ERR_OOM = 4
INV_ERR_HIP = 5
INV_ERR_NOT_INIT = 6

# TQNNDataType values (src/quicknn_common.pas:77-98)
INV_DT_F16 = 1
INV_DT_BF16 = 2
INV_DT_F32 = 3

# CBLAS enums (src/quicknn_common.pas:55-58)
CblasRowMajor = 101
CblasColMajor = 102
CblasNoTrans = 111
CblasTrans = 112

INV_EPI_NONE = 0
INV_EPI_SILU = 1
INV_EPI_GELU_ERF = 2
INV_EPI_SWIGLU = 3

INV_FLAG_DEVICE_PTRS = 0x1
INV_FLAG_ASYNC = 0x2
INV_FLAG_PRECISE = 0x4
INV_ATTN_CAUSAL = 0x100
INV_NORM_ADALN = 1
INV_NORM_RMS = 2
INV_ROPE_NONE = 0
INV_ROPE_INTERLEAVED = 1
INV_ROPE_HALF = 2

INV_ST_MAX_DIMS = 8
INV_ST_TRUNCATE = 0x1
INV_ST_GATE_UP = 0x2

INV_PREC_BF16 = 0
INV_PREC_SPLIT_A = 1
INV_PREC_SPLIT_AB = 2

# Every symbol include/inv_hip.h declares, with (restype, argtypes).
_PROTOS = {
    "inv_hip_abi_version": (c_int, []),
    "inv_hip_last_error": (c_char_p, []),
    "inv_hip_init": (c_int, [c_int]),
    "inv_hip_shutdown": (c_int, []),
    "inv_hip_device_info": (c_int, [c_char_p, c_size_t, POINTER(c_int), POINTER(c_int)]),
    "inv_hip_weight_upload": (c_int, [c_void_p, c_int64, c_int64, c_void_p, POINTER(c_void_p)]),
    "inv_hip_weight_upload_f32": (c_int, [c_void_p, c_int64, c_int64, c_void_p, POINTER(c_void_p)]),
    "inv_hip_weight_upload_gate_up": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                              POINTER(c_void_p)]),
    "inv_hip_weight_free": (c_int, [c_void_p]),
    "inv_hip_weight_shape": (c_int, [c_void_p, POINTER(c_int64), POINTER(c_int64)]),
    "inv_hip_weight_cache_get": (c_int, [c_char_p, c_char_p, c_char_p, c_int, POINTER(c_void_p)]),
    "inv_hip_weight_cache_set_budget": (c_int, [c_int64]),
    "inv_hip_weight_cache_clear": (c_int, []),
    "inv_hip_weight_cache_stats": (c_int, [POINTER(c_int64), POINTER(c_int64), POINTER(c_int64),
                                           POINTER(c_int64), POINTER(c_int64)]),
    "inv_hip_safetensors_info": (c_int, [c_char_p, c_char_p, POINTER(c_int), POINTER(c_int), POINTER(c_int64),
                                         POINTER(c_int64)]),
    "inv_hip_weight_load_safetensors": (c_int, [c_char_p, c_char_p, c_char_p, c_int, POINTER(c_void_p)]),
    "inv_hip_linear": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                               c_int, c_int]),
    "inv_hip_linear_noalloc": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64,
                                       c_int64, c_int, c_int]),
    "inv_hip_linear_gated_add": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                         c_int64, c_int]),
    "inv_hip_linear_norm": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_int,
                                    c_int64, c_int64, c_int64, c_int, c_int]),
    "inv_hip_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64, c_int64, c_int64,
                                  c_int64, c_int64, c_float, c_int]),
    "inv_hip_attention_masked": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64, c_int64,
                                         c_int64, c_int64, c_int64, c_float, c_void_p, c_int]),
    "inv_hip_head_norm_rope": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p, c_void_p,
                                       c_int]),
    "inv_hip_attention_qk_norm_rope": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                               c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_void_p,
                                               c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_int]),
    "inv_hip_conv2d": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                               c_int64, c_int64, c_int64, c_int64, c_int]),
    "inv_hip_sgemm": (c_int, [c_int, c_int, c_int, c_int64, c_int64, c_int64, c_float, c_void_p, c_int64, c_void_p,
                              c_int64, c_float, c_void_p, c_int64]),
    "inv_hip_sbgemm": (c_int, [c_int, c_int, c_int, c_int64, c_int64, c_int64, c_float, c_void_p, c_int64, c_void_p,
                               c_int64, c_float, c_void_p, c_int64]),
    "inv_hip_set_sgemm_precision": (c_int, [c_int]),
    "inv_hip_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "inv_hip_free": (c_int, [c_void_p]),
    "inv_hip_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "inv_hip_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t]),
    "inv_hip_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "inv_hip_memset": (c_int, [c_void_p, c_int, c_size_t]),
    "inv_hip_synchronize": (c_int, []),
    "inv_hip_timer_start": (c_int, []),
    "inv_hip_timer_stop": (c_int, [POINTER(c_float)]),
    "inv_hip_stats_enable": (c_int, [c_int]),
    "inv_hip_stats": (c_int, [POINTER(c_int64), POINTER(c_double), POINTER(c_double)]),
    "inv_hip_stats_reset": (c_int, []),
    "inv_hip_sample_seed": (c_int, [ctypes.c_uint64]),
    "inv_hip_sample_randn": (c_int, [c_void_p, c_int64, c_float, c_int]),
}


class HipLibraryError(RuntimeError):
    """libinvision_hip.so is missing or could not be loaded."""


class HipError(RuntimeError):
    """A library call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code
        self.fn = fn


_lib = None


def lib_path() -> str:
    return os.environ.get("INVISION_HIP_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load the native library once; raise HipLibraryError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise HipLibraryError(
            f"{path} not found: build it with `python -m invision_amd.build` (hipcc, gfx950). "
            "There is no CPU fallback.")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the runtime
        raise HipLibraryError(f"cannot load {path}: {e}") from e
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().inv_hip_last_error()
    return msg.decode() if msg else ""


def check(fn: str, code: int) -> None:
    if code != INV_OK:
        raise HipError(fn, code, last_error())


def call(fn: str, *args) -> None:
    """Call an int-returning entry point and raise HipError on failure."""
    check(fn, getattr(load(), fn)(*args))


def exported_symbols() -> list[str]:
    return list(_PROTOS)
