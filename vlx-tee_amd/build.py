"""Build the HIP C-ABI library ``libztcp_hip.so`` in-tree for gfx950.

``python vlx-tee_amd/build.py`` compiles every ``csrc/*.hip`` (device code)
and ``csrc/*.cpp`` (host code: the session key ring) with hipcc into
``vlx-tee_amd/libztcp_hip.so`` (exported symbols: include/ztcp.h and
include/ztcp_keyring.h).

Flags: ``-ffp-contract=off`` and no fast-math (the quantizer's fp32 rounding
order must match the reference's), packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "libztcp_hip.so"
ARCH = os.environ.get("ZTCP_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def sources() -> list[Path]:
    return sorted((HERE / "csrc").glob("*.hip")) + sorted((HERE / "csrc").glob("*.cpp"))


def build(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, *HIPCC_FLAGS, *map(str, sources()), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
