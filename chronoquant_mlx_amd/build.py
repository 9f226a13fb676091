"""Build recipe for libchronoquant.so (the gfx950 HIP kernels + C ABI).

    python -m chronoquant_mlx_amd.build

compiles chronoquant_mlx_amd/csrc/*.hip with hipcc for gfx950 into
chronoquant_mlx_amd/libchronoquant.so (in-tree, so it travels with the tree).
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "libchronoquant.so")
ARCH = os.environ.get("CQ_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    # IEEE-correct fp32 divide/sqrt: the codec's quotients must round like
    # the reference's fp16 division.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-ffp-contract=off",
    # no packed-FP32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


PHASES_OUT = os.path.join(PKG, "libchronoquant_phases.so")


def build(verbose: bool = False, phases: bool = False) -> str:
    """Build libchronoquant.so; phases=True builds the diagnostic
    libchronoquant_phases.so instead (the decode kernels record per-workgroup
    phase times, read by phase_times.py)."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    out = PHASES_OUT if phases else OUT
    tmp = out + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, *(["-DCQ_PHASE_TIMES"] if phases else []), "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libchronoquant.so")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, phases="--phases" in sys.argv[1:]))
