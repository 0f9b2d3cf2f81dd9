"""Builds libsynapse_kv.so (HIP for gfx950) in-tree, and the oracle restatement used by the tests.

Run as ``python -m synapse_amd.build`` or through ``__graft_entry__.build()``. The library lands in
``synapse_amd/_lib/libsynapse_kv.so``; nothing is installed outside the repository.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = sorted((PACKAGE / "csrc").glob("*.hip"))
OUTPUT = PACKAGE / "_lib" / "libsynapse_kv.so"
ARCH = "gfx950"

# Packed FP32 instructions are switched off for every device compile: some of their forms have given wrong
# results on the target machines, and the kernels do not need them. The kernels produce no NaN from finite inputs
# (empty columns are guarded explicitly), so fmaxf needs no NaN canonicalization.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-fno-honor-nans"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def build_library(verbose: bool = False) -> Path:
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    temporary = OUTPUT.with_suffix(".so.tmp")
    command = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-result",
        *DEVICE_FLAGS,
        "-o",
        str(temporary),
        *map(str, SOURCES),
    ]
    result = subprocess.run(command, cwd=PACKAGE, capture_output=True, text=True)
    output = "\n".join(
        line
        for line in (result.stdout + result.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the device feature
    )
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{output}")
    if verbose and output.strip():
        print(output, file=sys.stderr)
    temporary.replace(OUTPUT)
    return OUTPUT


def build_oracle() -> Path:
    """Compiles the CPU restatement (test infrastructure; see oracle/Makefile)."""
    result = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{result.stdout}{result.stderr}")
    return ROOT / "oracle" / "build" / "liboracle.so"


def main() -> None:
    path = build_library(verbose=True)
    print(path)
    print(build_oracle())


if __name__ == "__main__":
    main()
