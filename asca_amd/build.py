"""Build libasca_hip.so in-tree with hipcc for gfx950 only.

Usage: python -m asca_amd.build   (or __graft_entry__.build())

The library is written next to this file (asca_amd/libasca_hip.so) so that it
travels with the source tree; nothing is installed.  This is the counterpart of
the reference's rust/build.rs, which ran `nvcc -ptx -arch=sm_89` on
rust/kernels/asca.cu (rust/build.rs:12-59).
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libasca_hip.so"
ARCH = "gfx950"

# Packed FP32 (v_pk_*_f32) is disabled for all device code on this pool.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> Path:
    """Compile every .hip source into asca_amd/libasca_hip.so (always rebuilds)."""
    srcs = [str(s) for s in sources()]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, "-I", str(HERE.parent / "include"), "-o", str(tmp), *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with status {res.returncode}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
