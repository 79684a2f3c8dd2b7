"""The C-ABI library loads and exports every symbol include/inv_hip.h declares
(CPU only: no compute calls)."""
import ctypes
import os
import re

import pytest

from invision_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "inv_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(inv_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_surface():
    decl = declared_symbols()
    assert "inv_hip_linear" in decl and "inv_hip_sgemm" in decl and "inv_hip_weight_upload" in decl
    # The ctypes binding declares exactly what the header declares.
    assert sorted(hip.exported_symbols()) == decl


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(hip.lib_path())
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_versioned_name_loads_the_same_library():
    # A probe list may try libinvision_hip.so.0 (as the reference probes libopenblas.so.0):
    # the build links that name to the library, whose soname it is.
    so0 = hip.lib_path() + ".0"
    assert os.path.realpath(so0) == os.path.realpath(hip.lib_path())
    assert "libinvision_hip.so.0" in os.popen(f"readelf -d {hip.lib_path()}").read()
    lib = ctypes.CDLL(so0)
    assert all(hasattr(lib, s) for s in declared_symbols())


def test_only_c_symbols_are_exported_by_the_abi():
    # extern "C": the declared names are exported unmangled.
    out = os.popen(f"nm -D --defined-only {hip.lib_path()}").read()
    for s in declared_symbols():
        assert re.search(rf"\bT {s}$", out, re.M), s


def test_abi_version_and_error_channel():
    lib = hip.load()
    assert lib.inv_hip_abi_version() == 1
    assert isinstance(hip.last_error(), str)


def test_calls_before_init_fail_cleanly():
    lib = hip.load()
    if os.environ.get("HIP_VISIBLE_DEVICES", None) is None and _has_gpu():
        pytest.skip("a GPU is visible; covered by the GPU tests")
    # No device here: init reports NO_DEVICE, and every other call NOT_INIT.
    assert lib.inv_hip_init(0) == hip.INV_ERR_NO_DEVICE
    assert "device" in hip.last_error().lower()
    h = ctypes.c_void_p()
    assert lib.inv_hip_weight_upload(None, 4, 4, None, ctypes.byref(h)) == hip.INV_ERR_NOT_INIT
    assert lib.inv_hip_linear(None, 3, None, None, None, 3, 1, 1, 1, 0, 0) == hip.INV_ERR_NOT_INIT
    assert lib.inv_hip_sgemm(101, 111, 112, 1, 1, 1, 1.0, None, 1, None, 1, 0.0, None, 1) == hip.INV_ERR_NOT_INIT
    assert lib.inv_hip_shutdown() == hip.INV_OK


def _has_gpu():
    return os.path.exists("/dev/kfd") and any(os.path.exists(f"/dev/dri/renderD{128 + i}") for i in range(8))


def test_missing_library_raises_instead_of_falling_back(monkeypatch, tmp_path):
    import invision_amd.hip as h
    monkeypatch.setenv("INVISION_HIP_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(h, "_lib", None)
    with pytest.raises(h.HipLibraryError):
        h.load()


def test_mfma_ceiling_probe_library_loads():
    """The bench's measurement aid is a separate library, outside the linear-layer ABI."""
    from invision_amd import build as B
    lib = ctypes.CDLL(B.PROBE_PATH)
    assert hasattr(lib, "inv_probe_mfma_ceiling")
    assert not hasattr(hip.load(), "inv_probe_mfma_ceiling")


def test_library_sampler_matches_the_golden_draws_and_the_oracle():
    """inv_hip_sample_* (the reference's rng_seed / random_normal, src/quicknn_sample.pas:212-276)
    gives the committed seed-0 and seed-1234 normals bit for bit, and the oracle's stream over a long
    run (both seeded, X then W drawn in order, the second rounded to bf16 as the workloads do)."""
    import json

    import numpy as np

    import oracle
    from invision_amd import quicknn_hip as q

    with open(os.path.join(ROOT, "tests", "golden", "rng_seed0.json")) as f:
        gold = json.load(f)
    for seed, rec in gold.items():
        q.rng_seed(int(seed))
        got = [f"{int(v):08x}" for v in q.randn(8).view(np.uint32)]
        assert got == rec["random_normal_f32"], seed
    q.rng_seed(0)
    a1, a2 = q.randn((300, 70), 1.0), q.randn((50, 70), 0.02, round_bf16=True)
    oracle.rng_seed(0)
    b1, b2 = oracle.randn_scaled((300, 70), 1.0, False), oracle.randn_scaled((50, 70), 0.02, True)
    assert np.array_equal(a1.view(np.uint32), b1.view(np.uint32))
    assert np.array_equal(a2.view(np.uint32), b2.view(np.uint32))
    assert np.all(a2.view(np.uint32) & 0xFFFF == 0)  # bf16 values
