"""Build recipe for libinvision_hip.so (gfx950) and the CPU oracle.

    python -m invision_amd.build            # HIP library only
    python -m invision_amd.build --oracle   # also oracle/ (and oracle/_ref when the reference tree exists)

The library is compiled in-tree with hipcc, so the built .so travels with the
source tree.  Packed-FP32 instructions are disabled for all device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
import time

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libinvision_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The versioned name a library probe list may also try (the reference probes "libopenblas.so"
# then "libopenblas.so.0", src/quicknncpu.pas:3967-3978): a symlink beside the library.
SONAME = LIB_NAME + ".0"
PROBE_NAME = "libinv_probe.so"  # the MFMA-ceiling measurement aid (not the linear-layer ABI)
PROBE_PATH = os.path.join(PKG_DIR, PROBE_NAME)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# host-only sources: ROCm's clang as a plain C++ compiler (hipcc would compile them as HIP)
HOST_CXX = os.environ.get("INV_HOST_CXX", "/opt/rocm/llvm/bin/clang++")
ARCH = "gfx950"

BUILD_DIR = os.path.join(PKG_DIR, "_build")
NUM_GEMM_CONFIGS = 19  # INV_GEMM_NUM_CONFIGS in csrc/gemm_configs.hpp

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    # No packed-FP32 instructions anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def compile_jobs() -> list[tuple[list[str], str]]:
    """(hipcc command, object path) for every translation unit."""
    inc = ["-I", os.path.join(ROOT, "include")]
    jobs = []
    obj = os.path.join(BUILD_DIR, "inv_hip.o")
    jobs.append(([HIPCC] + COMMON_FLAGS + inc + ["-c", os.path.join(CSRC, "inv_hip.hip"), "-o", obj], obj))
    obj = os.path.join(BUILD_DIR, "attention.o")
    jobs.append(([HIPCC] + COMMON_FLAGS + inc + ["-c", os.path.join(CSRC, "attention.hip"), "-o", obj], obj))
    for host_src in ("safetensors.cpp", "sample.cpp", "host_convert.cpp"):  # host code only
        obj = os.path.join(BUILD_DIR, host_src.replace(".cpp", ".o"))
        jobs.append(([HOST_CXX, "-O2", "-std=c++17", "-fPIC", "-Wall"] + inc + ["-c", os.path.join(CSRC, host_src),
                                                                             "-o", obj], obj))
    for cfg in range(NUM_GEMM_CONFIGS):
        obj = os.path.join(BUILD_DIR, f"gemm_cfg{cfg}.o")
        jobs.append(([HIPCC] + COMMON_FLAGS + inc + [f"-DINV_CFG_ID={cfg}", "-c",
                                                     os.path.join(CSRC, "gemm_instance.hip"), "-o", obj], obj))
    return jobs


def probe_job() -> tuple[list[str], str]:
    """hipcc command building libinv_probe.so straight from its one source."""
    return ([HIPCC] + COMMON_FLAGS + ["-shared", os.path.join(CSRC, "mfma_ceiling.hip"), "-o", PROBE_PATH + ".tmp"],
            PROBE_PATH)


def _run(cmd: list[str]) -> tuple[int, str, list[str]]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless.
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    return res.returncode, err, cmd


def build_lib(verbose: bool = True, jobs: int = 0) -> str:
    """Compile libinvision_hip.so in place (always recompiles); translation units in parallel."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(BUILD_DIR, exist_ok=True)
    t0 = time.time()
    todo = compile_jobs()
    workers = jobs or min(len(todo), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        results = list(ex.map(lambda j: _run(j[0]), todo + [probe_job()]))
    results, probe_res = results[:-1], results[-1]
    if probe_res[0] != 0:
        raise RuntimeError(f"hipcc failed ({probe_res[0]}):\n{' '.join(probe_res[2])}\n{probe_res[1]}")
    os.replace(PROBE_PATH + ".tmp", PROBE_PATH)
    for rc, err, cmd in results:
        if rc != 0:
            raise RuntimeError(f"hipcc failed ({rc}):\n{' '.join(cmd)}\n{err}")
    tmp = LIB_PATH + ".tmp"
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{SONAME}", "-o", tmp] + [o for _, o in todo]
    rc, err, cmd = _run(link)
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{' '.join(cmd)}\n{err}")
    os.replace(tmp, LIB_PATH)
    link_soname()
    if verbose:
        print(f"[build] {LIB_NAME} ({len(todo)} translation units) in {time.time() - t0:.1f}s", flush=True)
        warn = "\n".join(e for rc, e, _ in results if e.strip())
        if warn.strip():
            print(warn, flush=True)
    return LIB_PATH


def link_soname() -> None:
    """libinvision_hip.so.0 -> libinvision_hip.so, in the package directory."""
    path = os.path.join(PKG_DIR, SONAME)
    if os.path.islink(path) or os.path.exists(path):
        os.remove(path)
    os.symlink(LIB_NAME, path)


def build_oracle(verbose: bool = True) -> None:
    """Compile oracle/liboracle.so and, when the reference source exists, oracle/_ref."""
    res = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "all"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print(res.stdout.strip().splitlines()[-1] if res.stdout.strip() else "[build] oracle", flush=True)


def main(argv: list[str]) -> int:
    build_lib()
    if "--oracle" in argv:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
