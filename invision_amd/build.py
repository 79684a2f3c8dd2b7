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
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["inv_hip.hip"]
HEADERS = ["gemm_kernel.hpp", "convert_kernels.hpp"]


def hipcc_cmd(out: str = LIB_PATH) -> list[str]:
    return [
        HIPCC,
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-command-line-argument",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
        "-o", out,
    ] + [os.path.join(CSRC, s) for s in SOURCES]


def build_lib(verbose: bool = True) -> str:
    """Compile libinvision_hip.so in place (always recompiles)."""
    tmp = LIB_PATH + ".tmp"
    cmd = hipcc_cmd(tmp)
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless.
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[build] {LIB_NAME} in {time.time() - t0:.1f}s", flush=True)
        if err.strip():
            print(err, flush=True)
    return LIB_PATH


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
