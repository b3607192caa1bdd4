"""A decode step's FFN calls replayed from a HIP graph: the C-ABI launches of every path the policy takes at decode
sizes (the lane-per-slot kernels and the tiles path with its reduce pass) carry no allocation, copy, memset or
synchronisation, so PyTorch's graph capture records them; every replay equals the eager step bit for bit, with eager
work and synchronisations between the replays."""
from __future__ import annotations

import pytest
import torch

from hffn_amd import synth
from hffn_amd.bench_decode import step
from hffn_amd.ffn import hip_layer
from hffn_amd.prepared_runtime import PreparedRuntime

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 8, 24])
def test_graph_replays_equal_the_eager_step(batch, device):
    case = synth.CASES["irreg_512_2048"]
    compacts = [synth.make_layer(case)] + [synth.make_workload_layer(synth.Workload(f"stack{i}", 512, 2048, 51, 900 + i))
                                           for i in range(3)]
    runtime = PreparedRuntime([hip_layer(c) for c in compacts], device)
    xs = [torch.from_numpy(synth.make_input(case, batch)).to(device) * (1 + 0.1 * i) for i in range(len(compacts))]
    eager = [torch.empty(batch, 512, device=device) for _ in compacts]
    replayed = [torch.empty_like(t) for t in eager]
    step(runtime, xs, eager)
    torch.cuda.synchronize()
    modes = runtime.modes(batch)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(runtime, xs, replayed)
    for _ in range(4):
        for t in replayed:
            t.fill_(float("nan"))
        graph.replay()
        step(runtime, xs, eager)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(eager, replayed)), modes
    assert modes in (("edges", "edges"), ("tiles", "tiles"))
