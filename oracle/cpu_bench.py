"""CPU baseline of ``bench.py``: the reference x86 AVX2 kernel (``oracle/_ref``) timed on this host's cores, pinned, as
the reference's own CPU protocol does (``runtime/cpu/x86/ffn/inference/bench/threads.py:29-100``, pinning
``bench/common.py:45-53``). Test infrastructure: it times the reference kernel, never this repository's kernels.

One invocation = one pinned process: ``--cpus`` sets the affinity before the kernel's thread pool exists, so its T
threads run on those CPUs. For each (workload, N) it checks the kernel against the float64 oracle on a token sample,
then alternates blocks of whole calls until ``--seconds`` of wall time are spent: each block first warms up for at least
5 ms (a core leaving idle runs slower for a while), then times ``--repeat`` calls. Reported: the median in-kernel time
(the kernel's own four phase timers), the median wall time per call, tokens/s from each. The process prints one JSON
line.

    python -m oracle.cpu_bench --cpus 0-7 --threads 8 --workload pythia410m_d50 --tokens 2048 --seconds 6
    python -m oracle.cpu_bench --machine            (the host record only)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

WARMUP_S, WARMUP_CALLS = 0.005, 3


def parse_cpus(text: str) -> list[int]:
    cpus: list[int] = []
    for part in text.split(","):
        first, _, last = part.partition("-")
        cpus += range(int(first), int(last or first) + 1)
    return cpus


def _read(path: str) -> str | None:
    try:
        return Path(path).read_text().strip()
    except OSError:
        return None


def machine() -> dict:
    """Model, logical CPUs, the CPUs this process may use, NUMA nodes with their CPU lists, physical cores per node
    (distinct (package, core) pairs), and the frequency governor where the kernel exposes it."""
    model = None
    for line in (_read("/proc/cpuinfo") or "").splitlines():
        if line.startswith("model name"):
            model = line.split(":", 1)[1].strip()
            break
    nodes = {}
    for node in sorted(Path("/sys/devices/system/node").glob("node[0-9]*")):
        cpus = parse_cpus(_read(str(node / "cpulist")) or "")
        cores = {(_read(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id"),
                  _read(f"/sys/devices/system/cpu/cpu{c}/topology/core_id")) for c in cpus}
        nodes[node.name] = {"cpus": cpus, "physical_cores": len(cores)}
    governors = {_read(f"/sys/devices/system/cpu/cpu{c}/cpufreq/scaling_governor") for c in range(os.cpu_count() or 1)}
    return {"model": model, "logical_cpus": os.cpu_count(), "affinity": sorted(os.sched_getaffinity(0)), "numa": nodes,
            "governor": sorted(g for g in governors if g) or "not exposed"}


def one_core_per_node_cpu(node_cpus: list[int], allowed: set[int]) -> list[int]:
    """The allowed CPUs of a NUMA node, one logical CPU per physical core (the first sibling of each)."""
    chosen, seen = [], set()
    for cpu in node_cpus:
        if cpu not in allowed:
            continue
        core = (_read(f"/sys/devices/system/cpu/cpu{cpu}/topology/physical_package_id"),
                _read(f"/sys/devices/system/cpu/cpu{cpu}/topology/core_id"))
        if core not in seen:
            seen.add(core)
            chosen.append(cpu)
    return chosen


def measure(workload: str, n: int, threads: int, seconds: float, repeat: int) -> dict:
    import numpy as np

    from hffn_amd import synth
    from oracle import reference, x86_ref

    compact = synth.make_workload_layer(workload)
    kernel = x86_ref.ReferenceKernel(compact, threads=threads)
    x = synth.make_input(synth.WORKLOADS[workload], n)
    sample = x[: min(n, 96)]
    error = float(np.max(np.abs(kernel.forward(sample) - reference.forward(compact, sample))))
    scale = float(np.max(np.abs(reference.forward(compact, sample)))) or 1.0
    if error > 2e-5 * max(1.0, scale):
        raise RuntimeError(f"reference x86 kernel differs from the float64 oracle by {error:.3e} on {workload}")
    inside, wall, blocks = [], [], 0
    began = time.perf_counter()
    while blocks < 2 or time.perf_counter() - began < seconds:
        warm, count = time.perf_counter(), 0
        while count < WARMUP_CALLS or time.perf_counter() - warm < WARMUP_S:
            kernel.forward(x)
            count += 1
        for _ in range(repeat):
            start = time.perf_counter_ns()
            kernel.forward(x)
            wall.append((time.perf_counter_ns() - start) / 1e3)
            inside.append(float(kernel.timing.sum()) / 1e3)
        blocks += 1
    kernel_us, wall_us = statistics.median(inside), statistics.median(wall)
    return {"workload": workload, "tokens": n, "threads": threads, "calls": len(wall), "blocks": blocks,
            "kernel_us_median": round(kernel_us, 2), "wall_us_median": round(wall_us, 2),
            "tokens_per_s_kernel": round(n / kernel_us * 1e6, 1), "tokens_per_s_wall": round(n / wall_us * 1e6, 1),
            "max_abs_error_vs_float64": error, "checked_tokens": int(sample.shape[0])}


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--cpus", help="pin this process to these CPUs first, e.g. 0-7")
    parser.add_argument("--threads", type=int, default=8)
    parser.add_argument("--workload", default="pythia410m_d50")
    parser.add_argument("--tokens", type=int, default=2048)
    parser.add_argument("--seconds", type=float, default=5.0)
    parser.add_argument("--repeat", type=int, default=5, help="timed calls per block")
    parser.add_argument("--machine", action="store_true")
    args = parser.parse_args(argv)
    if args.cpus:
        os.sched_setaffinity(0, parse_cpus(args.cpus))
    if args.machine:
        print(json.dumps(machine()), flush=True)
        return 0
    root = Path(__file__).resolve().parents[1]
    if str(root) not in sys.path:
        sys.path.insert(0, str(root))
    row = measure(args.workload, args.tokens, args.threads, args.seconds, args.repeat)
    row["cpus"] = sorted(os.sched_getaffinity(0))
    print(json.dumps(row), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
