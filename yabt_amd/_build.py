"""Compile the gfx950 HIP library in-tree (yabt_amd/_lib/libyabt_hip.so).

The library is plain C-ABI (include/yabt_hip.h); it links only the HIP runtime.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "libyabt_hip.so")
SOURCES = ["grow.hip", "grow_batch.hip", "grow_level.hip", "grow_ref.hip", "ops.hip", "leaf.hip", "slots.hip", "boost.hip", "binner.hip"]
ARCH = "gfx950"

# -ffp-contract=off: no fused multiply-add may change a rounding that the
#   fixed-point contract shares with the CPU oracle.
# -packed-fp32-ops off: packed fp32 VALU forms are avoided on this target.
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    return "hipcc"


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, "-I", CSRC, "-I", INCLUDE, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
