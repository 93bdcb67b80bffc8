"""Builds libnie_hip.so (gfx950) in-tree with hipcc.

    python nano-infer-engine_amd/build_native.py

The library lands next to the Python package
(``nano_infer_engine/libnie_hip.so``), where ``nano_infer_engine._native``
loads it from.  It is written to a temporary name and renamed, so a reader
never sees a half-written file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "nie_paged.hip")]
INCLUDE = os.path.join(REPO, "include")
OUTPUT = os.path.join(HERE, "nano_infer_engine", "libnie_hip.so")
ARCH = "gfx950"


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")


def build_library(verbose: bool = True) -> str:
    tmp = OUTPUT + ".tmp"
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-fvisibility=hidden",
        # no packed-fp32 VALU forms in generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # occupancy hints (amdgpu_waves_per_eu) that a head_dim-128 or fp32
        # instantiation cannot meet are advisory
        "-Wno-pass-failed",
        f"-I{INCLUDE}",
        *SOURCES,
        "-o", tmp,
    ]
    if verbose:
        print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    stderr = "\n".join(
        line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library())
