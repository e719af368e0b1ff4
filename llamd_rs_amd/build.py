"""Build the gfx950 HIP library and the CPU oracle, in-tree.

    python -m llamd_rs_amd.build        # or: python llamd_rs_amd/build.py

Produces llamd_rs_amd/libllamd_hip.so (kernels + C ABI, include/llamd_hip.h)
and oracle/libllamd_oracle.so (the CPU restatement used only by tests and the
benchmark's CPU baseline). hipcc cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libllamd_hip.so"
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libllamd_oracle.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: the bit-exact paths replay the reference's (Rust, never
# fused) float operations one for one. The packed-FP32 target feature is
# disabled for the device code: plain float code only.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: no accumulator-register reads after every MFMA
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # leading scalar kernel arguments arrive preloaded in SGPRs (gfx950's
    # kernarg preload): a latency-bound launch starts its first loads without
    # waiting for the kernarg segment
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", f"-I{ROOT / 'include'}",
              f"-I{CSRC}"]

HIP_SOURCES = ["q6k_mv.hip", "q8k.hip", "moe.hip", "moe_decode.hip", "group.hip", "norm.hip",
               "decode.hip", "noalloc.hip", "compat.hip"]
HOST_HIP_SOURCES = ["capi.cpp", "model.cpp", "compat_abi.cpp"]  # host code that calls the HIP runtime
HOST_SOURCES = ["host/layout.cpp", "host/synth.cpp", "host/gguf.cpp"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ORACLE_DIR)])
    return ORACLE_LIB


def build_hip(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    steps = []
    objs = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        steps.append([HIPCC, *DEVICE_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    for src in HOST_HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        steps.append([HIPCC, "-x", "hip", "--offload-arch=" + ARCH, "-O2", "-std=c++17", "-fPIC",
                      "-ffp-contract=off", "-fno-fast-math", "-Wall", f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(CSRC / src), "-o",
                      str(obj)])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        steps.append(["g++", *HOST_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, steps))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build(jobs: int = 8) -> None:
    build_oracle()
    build_hip(jobs)


if __name__ == "__main__":
    build()
    print(LIB)
    print(ORACLE_LIB)
