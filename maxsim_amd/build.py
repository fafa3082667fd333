"""Build the HIP/C-ABI library ``maxsim_amd/libmaxsim_hip.so`` for gfx950.

Usage: ``python -m maxsim_amd.build`` (also called by ``__graft_entry__.build``).
Compiles every source under ``maxsim_amd/csrc`` with hipcc (one process per
source, in parallel), then links them into the library.
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmaxsim_hip.so")
# Instruction-rate tests behind the scan's design (bench.py --rates): a
# library of their own, not linked into the product.
RATES_SRC = os.path.join(HERE, "microbench", "rates.hip")
RATES_LIB = os.path.join(HERE, "libmaxsim_rates.so")
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


def _run(cmd: list[str]) -> tuple[int, list[str]]:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    lines = [line for line in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in line and "unused-command-line-argument" not in line]
    return proc.returncode, lines


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    srcs = sources()
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with tempfile.TemporaryDirectory(prefix="msim_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.basename(s) + ".o") for s in srcs]
        compile_flags = [f for f in FLAGS if f != "-shared"]
        cmds = [[hipcc, *compile_flags, "-c", s, "-o", o] for s, o in zip(srcs, objs)]
        if verbose:
            print(f"compiling {len(srcs)} sources with {jobs} jobs: " + " ".join(cmds[0][:-4]), flush=True)
        rates_tmp = RATES_LIB + ".tmp"
        cmds.append([hipcc, *FLAGS, RATES_SRC, "-o", rates_tmp])
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            results = list(pool.map(_run, cmds))
        messages: list[str] = []
        for src, (rc, lines) in zip(srcs + [RATES_SRC], results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n" + "\n".join(lines))
            messages.extend(lines)
        tmp = LIB + ".tmp"
        rc, lines = _run([hipcc, *FLAGS, *objs, "-o", tmp])
        if rc != 0:
            raise RuntimeError("hipcc link failed:\n" + "\n".join(lines))
        messages.extend(lines)
    if verbose and messages:
        print("\n".join(messages))
    os.replace(tmp, LIB)
    os.replace(rates_tmp, RATES_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
