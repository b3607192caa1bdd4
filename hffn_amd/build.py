"""Build ``hffn_amd/libhffn_amd.so`` from ``hffn_amd/csrc/*.hip`` with hipcc for gfx950 (in-tree, no cache).

Every source is compiled to an object in ``hffn_amd/_build`` (one hipcc per source, in parallel), then the objects
are linked into the library. Every call recompiles everything.

    python -m hffn_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJECTS = HERE / "_build"
LIBRARY = HERE / "libhffn_amd.so"
ARCH = "gfx950"

# Packed FP32 instructions (v_pk_fma_f32 and friends) are switched off for every device pass.
COMPILE = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]
LINK = ["-shared", "-fPIC", f"--offload-arch={ARCH}"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build the HFFN kernels)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(command: list[str]) -> None:
    result = subprocess.run(command, cwd=CSRC, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{' '.join(command)}\n{result.stdout}\n{result.stderr}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source, link the library (replaced atomically) and return its path."""
    compiler = hipcc()
    OBJECTS.mkdir(exist_ok=True)
    tag = os.getpid()
    commands = {source: [compiler, *COMPILE, "-c", "-o", str(OBJECTS / f"{source.stem}.{tag}.o"), str(source)]
                for source in sources()}
    workers = jobs or min(len(commands), max(1, min(os.cpu_count() or 1, 16)))
    objects = [command[command.index("-o") + 1] for command in commands.values()]
    try:
        with ThreadPoolExecutor(workers) as pool:
            for _ in pool.map(_run, commands.values()):
                pass
        partial = LIBRARY.with_name(f"{LIBRARY.name}.tmp{tag}")
        _run([compiler, *LINK, "-o", str(partial), *objects])
        partial.replace(LIBRARY)
    finally:
        for path in objects:
            Path(path).unlink(missing_ok=True)
    if verbose:
        for command in commands.values():
            print(" ".join(command))
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
