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


def _filter(text: str) -> str:
    # the host pass does not know the device feature
    return "\n".join(line for line in text.splitlines() if "packed-fp32-ops" not in line)


def build_library(verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip to an object in parallel, then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    objects_dir = OUTPUT.parent / "obj"
    objects_dir.mkdir(exist_ok=True)
    flags = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", *DEVICE_FLAGS]

    def compile_one(source: Path) -> tuple[Path, subprocess.CompletedProcess]:
        target = objects_dir / (source.stem + ".o")
        command = [hipcc(), *flags, "-c", "-o", str(target), str(source)]
        return target, subprocess.run(command, cwd=PACKAGE, capture_output=True, text=True)

    workers = max(1, min(len(SOURCES), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(compile_one, SOURCES))
    messages = []
    for (target, result), source in zip(results, SOURCES):
        output = _filter(result.stdout + result.stderr)
        if result.returncode != 0:
            raise RuntimeError(f"hipcc failed on {source.name} ({result.returncode}):\n{output}")
        if output.strip():
            messages.append(output)
    temporary = OUTPUT.with_suffix(".so.tmp")
    # Every symbol resolved at link time: a kernel whose host launch stub the compiler did not emit fails the build
    # here instead of the library's first load.
    command = [hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", "-Wl,--no-undefined", "-o", str(temporary),
               *(str(target) for target, _ in results)]
    result = subprocess.run(command, cwd=PACKAGE, capture_output=True, text=True)
    output = _filter(result.stdout + result.stderr)
    if result.returncode != 0:
        raise RuntimeError(f"link failed ({result.returncode}):\n{output}")
    if output.strip():
        messages.append(output)
    if verbose and messages:
        print("\n".join(messages), file=sys.stderr)
    temporary.replace(OUTPUT)
    return OUTPUT


def build_calibration(verbose: bool = False) -> Path:
    """Compiles the benchmark's calibration kernels (bench_support/calibrate.hip, not part of the library)."""
    source = ROOT / "bench_support" / "calibrate.hip"
    output = ROOT / "bench_support" / "_lib" / "libcalibrate.so"
    output.parent.mkdir(parents=True, exist_ok=True)
    command = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", *DEVICE_FLAGS, "-o",
               str(output), str(source)]
    result = subprocess.run(command, capture_output=True, text=True)
    output_text = "\n".join(line for line in (result.stdout + result.stderr).splitlines()
                            if "packed-fp32-ops" not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{output_text}")
    if verbose and output_text.strip():
        print(output_text, file=sys.stderr)
    return output


def build_oracle() -> Path:
    """Compiles the CPU restatement (test infrastructure; see oracle/Makefile)."""
    result = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{result.stdout}{result.stderr}")
    return ROOT / "oracle" / "build" / "liboracle.so"


def main() -> None:
    path = build_library(verbose=True)
    print(path)
    print(build_calibration(verbose=True))
    print(build_oracle())


if __name__ == "__main__":
    main()
