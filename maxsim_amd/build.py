"""Build the HIP/C-ABI library ``maxsim_amd/libmaxsim_hip.so`` for gfx950.

Usage: ``python -m maxsim_amd.build`` (also called by ``__graft_entry__.build``).
Compiles every source under ``maxsim_amd/csrc`` with hipcc in one link step.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmaxsim_hip.so")
ARCH = os.environ.get("MAXSIM_GPU_ARCH", "gfx950")

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    # Packed FP32 VALU forms are disabled: the kernels rely on plain VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Every float operation is the single rounding it reads as.
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    # MFMA results in VGPRs: the epilogue reads them directly (no accvgpr moves).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # Device code never produces or tests NaNs: fmaxf needs no operand
    # canonicalisation (host code keeps IEEE NaN semantics for validation).
    "-Xarch_device", "-fno-honor-nans",
    "-Wall",
    "-Wno-unused-result",
]


def sources() -> list[str]:
    names = sorted(os.listdir(CSRC))
    return [os.path.join(CSRC, n) for n in names if n.endswith((".hip", ".cpp"))]


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    cmd = [hipcc, *FLAGS, *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    lines = [
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line
    ]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
