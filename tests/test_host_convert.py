"""Host-side fp32 -> bf16 rounding (csrc/host_convert.cpp), on the CPU.

Host fp32 operands are rounded while they are copied into the pinned bounce
buffers, so the bits must be the device's bf16_rne: round to nearest, ties to
even, NaN kept quiet, overflow to infinity.  Both bodies (AVX2 and portable)
are compiled here with g++ and checked against the oracle's rounding on every
upper half-word with the lower half-words around the ties, on a strided sweep
of all 2^32 patterns, and on ragged rows with zero padding.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "invision_amd", "csrc", "host_convert.cpp")
SHIM = r"""
#include "host_convert.hpp"
extern "C" void cvt_rows(uint16_t *d, int64_t ldd, const float *s, int64_t lds, int64_t rows, int64_t cols,
                         int64_t cols_pad) {
    inv::host_f32_to_bf16_rows(d, ldd, s, lds, rows, cols, cols_pad);
}
"""


@pytest.fixture(scope="module", params=["avx2", "generic"])
def cvt(request, tmp_path_factory):
    d = tmp_path_factory.mktemp(f"hcvt_{request.param}")
    shim = d / "shim.cpp"
    shim.write_text(SHIM)
    so = d / "libhcvt.so"
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-I", os.path.dirname(SRC), str(shim), SRC, "-o", str(so)]
    if request.param == "generic":
        cmd.insert(1, "-DINV_HOST_CONVERT_GENERIC")
    subprocess.run(cmd, check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.cvt_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                             ctypes.c_int64, ctypes.c_int64]
    lib.cvt_rows.restype = None

    def run(x, cols=None, cols_pad=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, lds = x.shape
        cols = lds if cols is None else cols
        cols_pad = cols if cols_pad is None else cols_pad
        out = np.full((rows, cols_pad), 0xABCD, dtype=np.uint16)
        lib.cvt_rows(out.ctypes.data, cols_pad, x.ctypes.data, lds, rows, cols, cols_pad)
        return out

    return run


def test_ties_and_neighbours_every_exponent(cvt):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    for low in (0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF):
        u = (hi | low).view(np.float32).reshape(256, 256)
        np.testing.assert_array_equal(cvt(u), oracle.f32_to_bf16_rne(u))


def test_strided_sweep_of_all_patterns(cvt):
    u = (np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)).view(np.float32)
    u = u[: (u.size // 1024) * 1024].reshape(-1, 1024)
    np.testing.assert_array_equal(cvt(u), oracle.f32_to_bf16_rne(u))


def test_special_values(cvt):
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 3.4028235e38, -3.4028235e38, 1e-45, -1e-45,
                     1.1754942e-38, 1.0, -1.0, 1.00390625, 1.01171875], dtype=np.float32)
    sig_nan = np.array([0x7F800001, 0xFF800001, 0x7FBFFFFF], dtype=np.uint32).view(np.float32)
    x = np.concatenate([vals, sig_nan])
    x = np.concatenate([x, np.zeros(32 - x.size, np.float32)]).reshape(1, 32)
    got = cvt(x)
    np.testing.assert_array_equal(got, oracle.f32_to_bf16_rne(x))
    assert np.all(got[0, 15:18] & 0x40)  # signalling NaNs come out quiet


@pytest.mark.parametrize("rows,lds,cols,cols_pad", [(5, 37, 35, 40), (3, 1001, 1001, 1008), (7, 16, 16, 16),
                                                    (2, 9, 1, 8), (4, 100, 33, 40)])
def test_ragged_rows_with_padding(cvt, rows, lds, cols, cols_pad):
    x = np.random.default_rng(rows * lds).standard_normal((rows, lds)).astype(np.float32)
    got = cvt(x, cols, cols_pad)
    np.testing.assert_array_equal(got[:, :cols], oracle.f32_to_bf16_rne(x[:, :cols]))
    assert np.all(got[:, cols:] == 0)
