"""Host-side checks without a GPU: the C-ABI library loads and exports what include/hffn_amd.h declares, its argument
validation refuses bad shapes before any launch, and the Python boundary keeps the reference's policy and errors."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from hffn_amd import _lib, runtime, synth

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "hffn_amd.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(hffn_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} is declared but not bound"
    assert lib.hffn_abi_version() == _lib.ABI_VERSION


def test_library_is_not_loaded_from_elsewhere():
    assert _lib.LIBRARY.parent == ROOT / "hffn_amd"


def _expect_argument_error(status: int, fragment: str) -> None:
    assert status == _lib.OK - 1
    assert fragment in _lib.load().hffn_last_error().decode()


@pytest.mark.skipif(torch.cuda.is_available(), reason="uses placeholder pointers: never run where a launch could reach a GPU")
def test_abi_refuses_bad_shapes_before_launching():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 17, 64, 64, 1, 4, None), "d_model=17")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 64, 0, 64, 1, 4, None), "d_ff=0")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 64, 64, 64, 0, 4, None), "n=0")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 64, 64, 64, (1 << 18) + 1, 1 << 19, None), "unsupported token count")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 64, 64, 64, 5, 6, None), "ld=6")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 64, 64, 64, 5, 12, None), "multiple of 8")
    _expect_argument_error(lib.hffn_up(9, 0, p, p, p, p, p, p, 64, 64, 64, 1, 4, None), "unknown up mode")
    _expect_argument_error(lib.hffn_up(1, 7, p, p, p, p, p, p, 64, 64, 64, 1, 4, None), "unknown value type")
    _expect_argument_error(lib.hffn_up(1, 0, None, p, p, p, p, p, 64, 64, 64, 1, 4, None), "null pointer")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 4096, 64, 64, 8, 8, None), "LDS")
    _expect_argument_error(lib.hffn_up(1, 0, p, p, p, p, p, p, 8192, 64, 64, 4, 4, None), "LDS")
    _expect_argument_error(lib.hffn_down(3, 0, p, p, p, p, p, p, 64, 64, 64, 1, 4, None), "unknown down mode")
    odd = ctypes.c_void_p(18)
    _expect_argument_error(lib.hffn_up(1, 0, p, p, odd, p, p, p, 64, 64, 64, 1, 4, None), "aligned")
    _expect_argument_error(lib.hffn_down(1, 0, p, p, p, ctypes.c_void_p(24), p, p, 64, 64, 64, 1, 4, None), "aligned")
    _expect_argument_error(lib.hffn_forward(2, 2, 0, p, p, p, p, p, p, p, p, p, None, p, p, p, 64, 64, 64, 64, 1, 4, None), "x_t")
    mfma_needed = ctypes.c_uint64(0)
    assert lib.hffn_mfma_workspace(2048, 1024, 4096, ctypes.byref(mfma_needed)) == _lib.OK
    small = mfma_needed.value - 1
    _expect_argument_error(lib.hffn_mfma_up(0, p, p, p, p, p, small, 1024, 4096, 2048, None), "workspace")
    _expect_argument_error(lib.hffn_mfma_down(0, p, p, p, p, p, small, 1024, 4096, 2048, None), "workspace")
    _expect_argument_error(lib.hffn_forward_mfma(0, p, p, p, p, p, p, p, p, small, p, 1024, 4096, 2048, None), "workspace")
    _expect_argument_error(lib.hffn_mfma_up(0, p, p, p, p, p, 1 << 40, 1024, 4000, 2048, None), "multiples")
    _expect_argument_error(lib.hffn_mfma_up(0, ctypes.c_void_p(20), p, p, p, p, 1 << 40, 1024, 4096, 2048, None), "aligned")
    gemv_needed = ctypes.c_uint64(0)
    assert lib.hffn_gemv_workspace(1024, 4096, ctypes.byref(gemv_needed)) == _lib.OK
    big = gemv_needed.value
    _expect_argument_error(lib.hffn_forward_gemv(0, p, p, p, p, p, p, p, p, p, big, p, 1024, 4096, 65, None), "above 64")
    _expect_argument_error(lib.hffn_forward_gemv(0, p, p, p, p, p, p, p, p, p, big, p, 1024, 4000, 8, None), "multiples")
    _expect_argument_error(lib.hffn_forward_gemv(0, ctypes.c_void_p(20), p, p, p, p, p, p, p, p, big, p, 1024, 4096, 8, None), "aligned")
    _expect_argument_error(lib.hffn_forward_gemv(0, p, p, p, p, p, p, p, None, p, big, p, 1024, 4096, 8, None), "null")
    _expect_argument_error(lib.hffn_forward_gemv(0, p, p, p, p, p, p, p, p, p, big - 1, p, 1024, 4096, 8, None), "workspace")
    dense = ctypes.c_uint64(0)
    _expect_argument_error(lib.hffn_grad_dense_workspace(256, 1024, 64, ctypes.byref(dense)), "streamed GEMM")
    assert lib.hffn_grad_dense_workspace(1024, 4096, 64, ctypes.byref(dense)) == _lib.OK and dense.value > 0
    work = ctypes.c_void_p(256)
    _expect_argument_error(lib.hffn_grad_dense(p, p, p, p, p, p, 1024, 4096, 64, 62, work, dense.value, None), "ld=62")
    _expect_argument_error(lib.hffn_grad_dense(ctypes.c_void_p(20), p, p, p, p, p, 1024, 4096, 64, 64, work, dense.value, None),
                           "aligned")
    _expect_argument_error(lib.hffn_grad_dense(p, p, None, p, p, p, 1024, 4096, 64, 64, work, dense.value, None), "null")
    _expect_argument_error(lib.hffn_grad_dense(p, p, p, p, p, p, 1024, 4096, 64, 64, work, dense.value - 1, None), "workspace")
    handle = ctypes.c_uint64(0)
    _expect_argument_error(lib.hffn_plan_gemv(0, p, p, p, p, p, p, p, p, big, p, 1024, 4096, 65, ctypes.byref(handle)), "above 64")
    _expect_argument_error(lib.hffn_plan_gemv(0, p, p, p, p, p, p, ctypes.c_void_p(20), p, big, p, 1024, 4096, 8,
                                              ctypes.byref(handle)), "aligned")
    _expect_argument_error(lib.hffn_plan_gemv(0, p, p, p, p, p, p, p, p, big, p, 1024, 4096, 8, None), "null result")
    needed = ctypes.c_uint64(0)
    assert lib.hffn_output_major_workspace(2_097_152, 1024, ctypes.byref(needed)) == _lib.OK
    assert needed.value == 1024 * 1024 * 4
    _expect_argument_error(lib.hffn_output_major(0, p, p, p, 1024, 4096, 2_097_152, p, p, p, p, needed.value - 1, None), "workspace")
    _expect_argument_error(lib.hffn_output_major(0, p, p, p, 20000, 4096, 16, p, p, p, p, 1 << 30, None), "d_model=20000")


def test_edges_stage_limit():
    lib = _lib.load()
    assert lib.hffn_edges_supported(1024, 8) == 1
    assert lib.hffn_edges_supported(2048, 8) == 1
    assert lib.hffn_edges_supported(2560, 8) == 1
    assert lib.hffn_edges_supported(4080, 8) == 1
    assert lib.hffn_edges_supported(4096, 4) == 1
    assert lib.hffn_edges_supported(4096, 8) == 0
    assert lib.hffn_edges_supported(4096, 4) == 1


def test_policy():
    assert [runtime.up_mode(n) for n in (1, 4, 8, 9, 32, 33, 64, 2048)] == ["edges"] * 5 + ["rows"] * 3
    assert runtime.up_mode(8, 4096) == "rows" and runtime.up_mode(4, 4096) == "edges" and runtime.up_mode(8, 2560) == "edges"
    assert [runtime.down_mode(n, 4096) for n in (1, 8, 32, 33, 2048)] == ["edges"] * 3 + ["rows"] * 2
    assert [runtime.leading_dim(n) for n in (1, 2, 3, 4, 5, 8, 9, 2048, 2049)] == [4, 4, 4, 4, 8, 8, 16, 2048, 2056]


def test_mfma_policy_crossovers():
    """The estimated crossovers land where the forced-pair timings put them: the 410M/50 % layer takes the MFMA path
    from 9 tokens (a second lane-per-slot pass), the 1.4B/20 % layer from 13, the narrow 70M/20 % layer from 29;
    above 32 tokens always."""
    def first(d, h, slots):
        return next(n for n in range(1, 40) if runtime.mfma_preferred(n, d, h, slots))
    assert first(1024, 4096, 2 * 4096 * 512) == 9
    assert first(2048, 8192, 2 * 8192 * 410) == 13
    assert first(512, 2048, 2 * 2048 * 102) == 29
    assert runtime.mfma_preferred(33, 512, 2048, 1) and not runtime.mfma_preferred(32, 512, 2048, 1)


def test_planes_policy():
    """Estimates up to 64 tokens: on the Pythia-410M layer at 50 % the lane-per-slot kernels at 1-4 tokens, the decode
    GEMVs from 8 to 40, the MFMA path at 64 and always above (when its GEMMs are streamed); on the dense 2.8B-shape
    layer the GEMVs up to 16 tokens and the MFMA path at 32; on the 1.4B layer at 20 % the gather kernels at 1-4
    tokens and the GEMVs at 16."""
    slots = 2 * 4096 * 512
    assert runtime.planes_mode(1, 1024, 4096, slots, True) is None
    assert runtime.planes_mode(2, 1024, 4096, slots, True) is None and runtime.planes_mode(4, 1024, 4096, slots, True) is None
    assert all(runtime.planes_mode(n, 1024, 4096, slots, True) == "gemv" for n in (8, 16, 24, 32, 33, 40))
    assert runtime.planes_mode(64, 1024, 4096, slots, True) == "mfma"
    assert runtime.planes_mode(65, 1024, 4096, slots, True) == "mfma"
    assert runtime.planes_mode(65, 1024, 4096, slots, False) is None
    assert runtime.planes_mode(48, 512, 2048, 2 * 2048 * 102, True) == "gemv"
    dense = 2 * 10240 * 2048
    assert all(runtime.planes_mode(n, 2560, 10240, dense, True) == "gemv" for n in (1, 4, 16))
    assert runtime.planes_mode(32, 2560, 10240, dense, True) == "mfma"
    sparse = 2 * 8192 * 410
    assert all(runtime.planes_mode(n, 2048, 8192, sparse, True) is None for n in (1, 4))
    assert runtime.planes_mode(16, 2048, 8192, sparse, True) == "gemv"


def test_mfma_streamed_query():
    """Both projections stream for the model shapes at every token count; a 256 x 1024 layer's up projection has too
    few 128-column tiles below 512 tokens and falls back to the register-staged GEMM."""
    for d, h in ((512, 2048), (1024, 4096), (2048, 8192), (2560, 10240)):
        assert all(runtime.mfma_streamed(n, d, h) for n in (1, 64, 65, 128, 129, 256, 257, 2048, 4096))
    assert not runtime.mfma_streamed(1, 256, 1024) and runtime.mfma_streamed(2048, 256, 1024)
    with pytest.raises(ValueError, match="multiples of 256"):
        runtime.mfma_streamed(1, 320, 1024)


def test_runtime_refuses_other_devices():
    with pytest.raises(ValueError, match="cuda:0"):
        runtime.HFFNRuntime([], "cuda:1")
    with pytest.raises(ValueError, match="cuda:0"):
        runtime.HFFNRuntime([], "cpu")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error")
def test_runtime_needs_a_gpu():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        runtime.HFFNRuntime([], "cuda")


def test_layer_validation_on_host():
    """Malformed stores are refused before anything reaches a kernel."""
    layer = synth.make_layer(synth.CASES["homog_256_1024"])
    t = torch.from_numpy
    good = (t(layer.up_offsets), t(layer.up_idx), t(layer.up_val))
    runtime._check_side("up", *good, layer.d_ff, layer.d_model)
    bad_index = t(layer.up_idx).clone()
    bad_index[3] = layer.d_model
    with pytest.raises(ValueError, match="index out of"):
        runtime._check_side("up", good[0], bad_index, good[2], layer.d_ff, layer.d_model)
    bad_offsets = t(layer.up_offsets).clone()
    bad_offsets[5] = bad_offsets[6] + 1
    with pytest.raises(ValueError, match="without decreasing"):
        runtime._check_side("up", bad_offsets, good[1], good[2], layer.d_ff, layer.d_model)
    with pytest.raises(ValueError, match="int32"):
        runtime._check_side("up", good[0].long(), good[1], good[2], layer.d_ff, layer.d_model)


def test_workload_generator_properties():
    layer = synth.make_workload_layer("pythia70m_d20")
    assert layer.up_idx.size == layer.d_ff * 102 and layer.down_idx.size == layer.d_ff * 102
    for offsets, idx in ((layer.up_offsets, layer.up_idx), (layer.down_offsets, layer.down_idx)):
        for r in range(0, layer.d_ff, 97):
            row = idx[offsets[r]:offsets[r + 1]].astype(int)
            assert (row >= 0).all() and (row < layer.d_model).all() and (row[1:] > row[:-1]).all()
    assert not layer.b_up.any() and not layer.b_down.any()
    assert abs(float(layer.up_val.std()) - 0.02) < 0.001


def test_bf16_rounding():
    values = torch.randn(10000).numpy().astype("float32")
    rounded = synth.round_bf16(values)
    assert torch.equal(torch.from_numpy(rounded), torch.from_numpy(values).to(torch.bfloat16).float())


@pytest.mark.skipif(torch.cuda.is_available(), reason="uses placeholder pointers: never run where a launch could reach a GPU")
def test_plans_are_checked_once_and_released():
    """hffn_plan_forward runs the checks of hffn_forward (without x); plans are kept under distinct handles until
    released; an unknown handle is refused before any launch."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    handle = ctypes.c_uint64(0)
    model = [p] * 8
    work = [p] * 4
    _expect_argument_error(lib.hffn_plan_forward(1, 1, 0, *model, *work, 17, 64, 64, 64, 1, 4, ctypes.byref(handle)), "d_model=17")
    _expect_argument_error(lib.hffn_plan_forward(9, 1, 0, *model, *work, 64, 64, 64, 64, 1, 4, ctypes.byref(handle)), "unknown up mode")
    _expect_argument_error(lib.hffn_plan_forward(1, 1, 0, *model, *work, 4096, 64, 64, 64, 8, 8, ctypes.byref(handle)), "LDS")
    _expect_argument_error(lib.hffn_plan_forward(2, 1, 0, *model, None, p, p, p, 64, 64, 64, 64, 1, 4, ctypes.byref(handle)), "x_t")
    _expect_argument_error(lib.hffn_plan_forward(1, 1, 0, *model, *work, 64, 64, 64, 64, 1, 4, None), "null result")
    assert lib.hffn_plan_forward(1, 1, 0, *model, *work, 64, 64, 64, 64, 1, 4, ctypes.byref(handle)) == _lib.OK
    first = handle.value
    assert lib.hffn_plan_forward(2, 2, 0, *model, *work, 64, 64, 64, 64, 5, 8, ctypes.byref(handle)) == _lib.OK
    assert first != 0 and handle.value not in (0, first)
    assert lib.hffn_plan_release(first) == _lib.OK
    assert lib.hffn_plan_release(handle.value) == _lib.OK
    _expect_argument_error(lib.hffn_plan_release(first), "unknown plan")
    _expect_argument_error(lib.hffn_plan_launch(first, p, None), "unknown plan")
    # a decode-GEMV plan: same table and handles; its launch still checks x's alignment before launching
    gemv_bytes = ctypes.c_uint64(0)
    assert lib.hffn_gemv_workspace(1024, 4096, ctypes.byref(gemv_bytes)) == _lib.OK
    assert lib.hffn_plan_gemv(0, p, p, p, p, p, p, p, p, gemv_bytes.value, p, 1024, 4096, 8, ctypes.byref(handle)) == _lib.OK
    assert handle.value not in (0, first)
    _expect_argument_error(lib.hffn_plan_launch(handle.value, ctypes.c_void_p(20), None), "aligned")
    assert lib.hffn_plan_release(handle.value) == _lib.OK
    _expect_argument_error(lib.hffn_plan_release(handle.value), "unknown plan")
