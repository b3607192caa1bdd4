"""Build ``hffn_amd/libhffn_amd.so`` from ``hffn_amd/csrc/*.hip`` with hipcc for gfx950 (in-tree, no cache).

    python -m hffn_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIBRARY = HERE / "libhffn_amd.so"
ARCH = "gfx950"

# Packed FP32 instructions (v_pk_fma_f32 and friends) are switched off for every device pass.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build the HFFN kernels)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every source into the library (always recompiles) and return its path."""
    partial = LIBRARY.with_name(f"{LIBRARY.name}.tmp{os.getpid()}")
    command = [hipcc(), *FLAGS, "-o", str(partial), *map(str, sources())]
    result = subprocess.run(command, cwd=CSRC, capture_output=True, text=True)
    if result.returncode != 0:
        partial.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{' '.join(command)}\n{result.stdout}\n{result.stderr}")
    if verbose:
        print(" ".join(command))
    partial.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
