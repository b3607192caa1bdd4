"""The allocation-free decode-GEMV entry point (``hffn_forward_gemv_static``) through the C ABI: on the same layers
and inputs its activations and outputs are bitwise those of ``hffn_forward_gemv`` with a caller workspace, over two
calls in a row on one layer, the second with fewer tokens (the static partials keep the first call's contents), and
on a layer whose sides take no k split. Shapes beyond the static scratch are refused before any launch."""
from __future__ import annotations

import pytest
import torch

from hffn_amd import _lib, synth
from hffn_amd.ffn import hip_layer
from hffn_amd.runtime import HFFNRuntime

pytestmark = pytest.mark.gpu


def _planes_call(runtime: HFFNRuntime, x: torch.Tensor, static: bool) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    n = x.shape[0]
    planes, tensors = runtime._planes[0], runtime._tensors[0]
    value_type = runtime._args[0][0]
    act = torch.full((n, runtime.d_ff), float("nan"), device=x.device)
    y = torch.full((n, runtime.d_model), float("nan"), device=x.device)
    common = (value_type, x.data_ptr(), planes["up"].data_ptr(), planes["up_binades"].data_ptr(), tensors["b_up"].data_ptr(),
              planes["down"].data_ptr(), planes["down_binades"].data_ptr(), tensors["b_down"].data_ptr(), act.data_ptr())
    stream = torch.cuda.current_stream(x.device).cuda_stream
    if static:
        status = lib.hffn_forward_gemv_static(*common, y.data_ptr(), runtime.d_model, runtime.d_ff, n, stream)
    else:
        work = torch.full((_lib.query_bytes(lib.hffn_gemv_workspace, runtime.d_model, runtime.d_ff) // 4,), float("nan"),
                          device=x.device)
        status = lib.hffn_forward_gemv(*common, work.data_ptr(), 4 * work.numel(), y.data_ptr(), runtime.d_model, runtime.d_ff, n,
                                       stream)
    _lib.check(status, "gemv static" if static else "gemv")
    torch.cuda.synchronize()
    return act, y


@pytest.mark.parametrize("name,calls", [("pythia410m_d50", (48, 5)), ("pythia1p4b_d20_bf16", (64, 17))])
def test_static_scratch_matches_the_workspace_entry(name, calls, device):
    workload = synth.WORKLOADS[name]
    runtime = HFFNRuntime([hip_layer(synth.make_workload_layer(workload))], device, dense=True)
    for n in calls:
        x = torch.from_numpy(synth.make_input(workload, n)).to(device)
        act, y = _planes_call(runtime, x, static=False)
        act_static, y_static = _planes_call(runtime, x, static=True)
        assert torch.equal(act_static, act), (name, n)
        assert torch.equal(y_static, y), (name, n)
        assert not bool(torch.isnan(y_static).any())


def test_static_scratch_without_splits(device):
    case = synth.CASES["irreg_512_2048"]
    runtime = HFFNRuntime([hip_layer(synth.make_layer(case))], device, dense=True)
    for n in (33, 2):
        x = torch.from_numpy(synth.make_input(case, n)).to(device)
        assert all(torch.equal(a, b) for a, b in zip(_planes_call(runtime, x, True), _planes_call(runtime, x, False)))


def test_static_scratch_refusals(device):
    lib = _lib.load()
    fake = 256  # aligned, never dereferenced: the call is refused before any launch
    stream = torch.cuda.current_stream(device).cuda_stream
    status = lib.hffn_forward_gemv_static(_lib.VALUE_F32, *([fake] * 9), 1024, 4096, 65, stream)
    assert status == _lib.OK - 1 and "above 64" in lib.hffn_last_error().decode()
    status = lib.hffn_forward_gemv_static(_lib.VALUE_F32, *([fake] * 9), 1000, 4096, 1, stream)
    assert status == _lib.OK - 1
