"""Builds the native libraries in-tree.

- librusty_hip.so: the HIP kernels and the C ABI of include/rusty_hip.h,
  compiled for gfx950 only.  -ffp-contract=off keeps a*b+c unfused wherever the
  kernels reproduce a reference rounding point (explicit fmaf is used where an
  FMA is intended); packed-fp32 instructions are disabled.
- libsynth.so: host-only seeded weight generator and block quantizers.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HIP_LIB = os.path.join(HERE, "librusty_hip.so")
SYNTH_LIB = os.path.join(HERE, "libsynth.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in architectural VGPRs: the batched products feed every C
    # element to VALU integer multiply-adds, which AGPR results would first
    # have to copy out one register at a time
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build_hip() -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = HIP_LIB + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "-o", tmp, os.path.join(CSRC, "rusty_hip.hip")])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_synth() -> str:
    tmp = SYNTH_LIB + ".tmp"
    _run(["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-mf16c", "-ffp-contract=off", "-o", tmp,
          os.path.join(CSRC, "synth.cpp")])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


def build_all() -> None:
    build_synth()
    build_hip()


if __name__ == "__main__":
    build_all()
    print("built", HIP_LIB, SYNTH_LIB)
