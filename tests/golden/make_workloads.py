"""Writes tests/golden/workloads.json: the SHA-256 pins of this repository's workload layers (hffn_amd.synth.WORKLOADS)
and of their inputs, so that a change of the generator or of numpy's streams is caught.

    python tests/golden/make_workloads.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from hffn_amd import synth  # noqa: E402


def input_digest(workload, tokens) -> str:
    digest = hashlib.sha256()
    for n in tokens:
        digest.update(synth.make_input(workload, n).tobytes())
    return digest.hexdigest()


def main() -> None:
    pins = {}
    for name, workload in synth.WORKLOADS.items():
        layer = synth.make_workload_layer(workload)
        pins[name] = {"layer": synth.layer_digest(layer), "inputs": input_digest(workload, workload.tokens),
                      "tokens": list(workload.tokens), "nnz_up": int(layer.up_idx.size), "nnz_down": int(layer.down_idx.size)}
        print(name, pins[name])
    (HERE / "workloads.json").write_text(json.dumps(pins, indent=2) + "\n")


if __name__ == "__main__":
    main()
