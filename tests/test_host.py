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
    # the tiles path: store sizes (an 8-slot group per 8 slots, one padding group per item at most, one spare group)
    size, entries = ctypes.c_uint64(0), ctypes.c_uint64(0)
    assert lib.hffn_tiles_store_size(0, 4096, 1024, 2_097_152, ctypes.byref(size), ctypes.byref(entries)) == _lib.OK
    items = 256 * 2
    assert (size.value, entries.value) == ((2_097_152 // 8 + items + 1) * 48, items + 1 + 4096)
    bf16_size, bf16_entries = ctypes.c_uint64(0), ctypes.c_uint64(0)
    assert lib.hffn_tiles_store_size(1, 2048, 8192, 3_358_720, ctypes.byref(bf16_size), ctypes.byref(bf16_entries)) == _lib.OK
    assert (bf16_size.value, bf16_entries.value) == ((3_358_720 // 8 + 128 * 16 + 1) * 32, 128 * 16 + 1)
    _expect_argument_error(lib.hffn_tiles_store_size(0, 0, 1024, 0, ctypes.byref(size), ctypes.byref(entries)), "rows=0")
    _expect_argument_error(lib.hffn_tiles_store_size(0, 16, 16, 257, ctypes.byref(size), ctypes.byref(entries)), "nnz=257")
    _expect_argument_error(lib.hffn_tiles_store_size(5, 16, 16, 1, ctypes.byref(size), ctypes.byref(entries)), "value type")
    assert lib.hffn_tiles_store_size(0, 4096, 1024, 2_097_152, ctypes.byref(size), ctypes.byref(entries)) == _lib.OK
    _expect_argument_error(lib.hffn_tiles_build(0, p, p, p, 4096, 1024, 2_097_152, p, size.value - 1, p, None), "store of")
    _expect_argument_error(lib.hffn_tiles_build(0, p, p, p, 4096, 1024, 2_097_152, ctypes.c_void_p(24), size.value, p, None),
                           "aligned")
    _expect_argument_error(lib.hffn_tiles_build(0, None, p, p, 4096, 1024, 2_097_152, p, size.value, p, None), "null")
    tiles_bytes = ctypes.c_uint64(0)
    # 410M shape, 16 tokens: the up side in one chunk, the down side's 64 row tiles over 4 chunks of K
    assert lib.hffn_tiles_workspace(0, 16, 1024, 4096, 2_097_152, 2_097_152, ctypes.byref(tiles_bytes)) == _lib.OK
    assert tiles_bytes.value == 4 * 16 * 1024 * 4
    # 1.4B shape, bf16, 20 %, 16 tokens: the up side in 256 blocks of 32 rows x 2048 k, the down side in 64 blocks of
    # 32 rows per chunk of 2048 (4 chunks: the shape model prices the 32 row runs a block reads, against 64 runs of
    # 4 x 1024 in 8 chunks)
    assert lib.hffn_tiles_workspace(1, 16, 2048, 8192, 3_358_720, 3_358_720, ctypes.byref(tiles_bytes)) == _lib.OK
    assert tiles_bytes.value == 4 * 16 * 2048 * 4
    _expect_argument_error(lib.hffn_tiles_workspace(1, 16, 2048, 8192, 1 << 40, 0, ctypes.byref(tiles_bytes)), "nnz_up")
    _expect_argument_error(lib.hffn_tiles_workspace(0, 65, 1024, 4096, 0, 0, ctypes.byref(tiles_bytes)), "n=65")
    _expect_argument_error(lib.hffn_tiles_workspace(0, 16, 1000, 4096, 0, 0, ctypes.byref(tiles_bytes)), "multiple of 16")
    assert lib.hffn_tiles_workspace(0, 16, 1024, 4096, 2_097_152, 2_097_152, ctypes.byref(tiles_bytes)) == _lib.OK
    ws = tiles_bytes.value
    _expect_argument_error(lib.hffn_forward_tiles(0, p, p, p, p, p, p, p, p, p, ws - 1, p, 1024, 4096, 2_097_152, 2_097_152, 16, None), "workspace")
    _expect_argument_error(lib.hffn_forward_tiles(0, ctypes.c_void_p(20), p, p, p, p, p, p, p, p, ws, p, 1024, 4096, 2_097_152, 2_097_152, 16,
                                                  None),
                           "aligned")
    _expect_argument_error(lib.hffn_forward_tiles(0, p, ctypes.c_void_p(24), p, p, p, p, p, p, p, ws, p, 1024, 4096, 2_097_152, 2_097_152, 16,
                                                  None),
                           "tiled stores")
    _expect_argument_error(lib.hffn_forward_tiles(0, p, p, None, p, p, p, p, p, p, ws, p, 1024, 4096, 2_097_152, 2_097_152, 16, None), "null")
    _expect_argument_error(lib.hffn_forward_tiles(0, p, p, p, p, p, p, p, p, p, ws, p, 1024, 4096, 2_097_152, 2_097_152, 65, None), "n=65")
    handle = ctypes.c_uint64(0)
    _expect_argument_error(lib.hffn_plan_tiles(0, p, p, p, p, p, p, p, p, ws - 1, p, 1024, 4096, 2_097_152, 2_097_152, 16, ctypes.byref(handle)),
                           "workspace")
    _expect_argument_error(lib.hffn_plan_tiles(0, p, p, p, p, p, p, p, p, ws, p, 1024, 4096, 2_097_152, 2_097_152, 16, None), "null result")
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


# Stored slots (both sides) and bytes of the layers the policy's estimates were fitted to: int16 indices and float32
# (6 bytes a slot) or bfloat16 (4 bytes) values.
S410 = runtime.StoreShape(2 * 4096 * 512, 6 * 2 * 4096 * 512, 4096)
S410_D10 = runtime.StoreShape(2 * 4096 * 102, 6 * 2 * 4096 * 102, 4096)
S1P4 = runtime.StoreShape(2 * 8192 * 410, 4 * 2 * 8192 * 410, 8192)
S70 = runtime.StoreShape(2 * 2048 * 102, 6 * 2 * 2048 * 102, 2048)
S2P8 = runtime.StoreShape(41_836_593, 4 * 41_836_593, 10240)


def test_decode_policy():
    """Up to 64 tokens the policy reads the compact store; the estimated crossovers land where the forced-pair timings
    put them (MI355X, 12 rotating copies, µs per call, lane-per-slot against tiles): the 410M/50 % layer on the
    lane-per-slot kernels at 1-4 tokens (14.3 against 17.5 at 4) and on the tiles path from 6 (20.5 against 17.0); the
    410M/10 % and 70M/20 % layers on the lane-per-slot kernels up to 8 tokens (15.0 against 17.3; 13.4 against 13.9)
    and on the tiles path from 12; the 1.4B/20 % bf16 layer on the lane-per-slot kernels at 1-4 tokens (17.9 against
    19.3 at 4) and on the tiles path from 6, where its activations no longer fit the down kernel's LDS stage (34.1
    against 19.7); the 2.8B/80 % bf16 layer on the lane-per-slot kernels at 1-2 tokens (52.6 against 67.9 at 1) and
    on the tiles path from 3 (124.8 against 69.0); above 32 tokens only the tiles path remains; without tiled stores
    the lane-per-slot kernels or nothing."""
    mode = lambda shape, ns: [runtime.decode_mode(n, shape, True, True) for n in ns]  # noqa: E731
    assert mode(S410, (1, 2, 3, 4, 6, 8, 16, 32, 64)) == ["edges"] * 4 + ["tiles"] * 5
    assert mode(S410_D10, (1, 4, 6, 8, 12, 16, 32)) == ["edges"] * 4 + ["tiles"] * 3
    assert mode(S1P4, (1, 2, 3, 4, 6, 8, 16, 32, 64)) == ["edges"] * 4 + ["tiles"] * 5
    assert mode(S70, (1, 4, 6, 8, 12, 16, 32)) == ["edges"] * 4 + ["tiles"] * 3
    assert mode(S2P8, (1, 2, 3, 4, 16, 64)) == ["edges"] * 2 + ["tiles"] * 4
    assert runtime.decode_mode(33, S410, True, False) is None and runtime.decode_mode(32, S410, True, False) == "edges"
    assert runtime.decode_mode(65, S410, True, True) is None
    assert runtime.decode_mode(4, S410, False, True) == "tiles"


def test_path_estimates():
    """The estimates against the forced-pair timings they were fitted to (µs per call, within 20 %): the tiles path
    at 1, 16 and 32 tokens, the lane-per-slot kernels where their activations fit the down kernel's stage."""
    tiles = {(S410, 1): 17.8, (S410, 16): 17.8, (S410, 32): 21.5, (S1P4, 1): 19.0, (S1P4, 16): 23.0, (S1P4, 32): 31.5,
             (S70, 16): 15.7, (S2P8, 1): 67.9, (S2P8, 32): 87.6, (S410_D10, 1): 17.2}
    for (shape, n), us in tiles.items():
        assert abs(runtime.tiles_us(n, shape) / us - 1) < 0.2, (shape, n)
    edges = {(S410, 1): 12.9, (S410, 4): 14.3, (S410, 8): 20.5, (S410, 16): 39.0, (S1P4, 1): 13.0, (S1P4, 2): 14.4,
             (S1P4, 4): 17.9, (S70, 8): 13.4, (S410_D10, 8): 15.0, (S2P8, 1): 52.6, (S2P8, 2): 55.8, (S2P8, 4): 125.1}
    for (shape, n), us in edges.items():
        assert abs(runtime.edges_us(n, shape) / us - 1) < 0.2, (shape, n)


def test_large_n_estimates():
    """Above 64 tokens, without planes, the tiles path in pieces of 64 against the lane-per-token kernels: the estimates
    pick the faster of the forced-pair timings they were fitted to (MI355X, µs per call): the 1.4B/20 % bf16 layer on
    the tiles path at every count (65: 59 against 213; 512: 332 against 500; 2048: 1321 against 1998), the 410M/50 %
    layer too (128: 57 against 165), the 70M/20 % layer on the lane-per-token kernels from 65 tokens (38.9 against 44.0;
    128: 37.9 against 63.1; 2048: 145 against 998); the rows estimate within 30 % of those timings from 128 tokens on."""
    faster = lambda n, shape: "tiles" if runtime.pieces_us(n, shape) < runtime.rows_us(n, shape) else "rows"  # noqa: E731
    assert [faster(n, S1P4) for n in (65, 128, 512, 2048)] == ["tiles"] * 4
    assert [faster(n, S410) for n in (65, 128, 2048)] == ["tiles"] * 3
    assert [faster(n, S70) for n in (65, 128, 256, 2048)] == ["rows"] * 4
    assert runtime.pieces_us(128, S70) == 2 * runtime.tiles_us(64, S70)
    assert runtime.pieces_us(65, S70) == runtime.tiles_us(64, S70) + runtime.tiles_us(1, S70)
    rows_measured = {(S70, 128): 37.9, (S70, 512): 69.1, (S70, 2048): 145.2, (S1P4, 512): 499.8, (S1P4, 2048): 1997.7,
                     (S410, 512): 313.4, (S410, 2048): 1085.7, (S1P4, 128): 222.6}
    for (shape, n), us in rows_measured.items():
        assert abs(runtime.rows_us(n, shape) / us - 1) < 0.3, (shape, n)


@pytest.mark.skipif(torch.cuda.is_available(), reason="uses placeholder pointers: never run where a launch could reach a GPU")
def test_read_probe_refuses_bad_arguments():
    """The plain-read probe of the decode measurements refuses null or misaligned data, a size that is not a nonzero
    multiple of 16 bytes, a grid outside 1-65535 blocks and a sink smaller than 4 words per block, before any launch."""
    lib = _lib.load()
    p, odd, sink = ctypes.c_void_p(256), ctypes.c_void_p(264), ctypes.c_void_p(4096)
    _expect_argument_error(lib.hffn_read_probe(None, 1024, sink, 16, 4, None), "null pointer")
    _expect_argument_error(lib.hffn_read_probe(p, 1024, None, 16, 4, None), "null pointer")
    _expect_argument_error(lib.hffn_read_probe(odd, 1024, sink, 16, 4, None), "multiple of 16")
    _expect_argument_error(lib.hffn_read_probe(p, 1000, sink, 16, 4, None), "multiple of 16")
    _expect_argument_error(lib.hffn_read_probe(p, 0, sink, 16, 4, None), "multiple of 16")
    _expect_argument_error(lib.hffn_read_probe(p, 1024, sink, 16, 0, None), "blocks")
    _expect_argument_error(lib.hffn_read_probe(p, 1024, sink, 15, 4, None), "blocks")
    _expect_argument_error(lib.hffn_read_probe(p, 1024, sink, 1 << 20, 65536, None), "blocks")


@pytest.mark.skipif(torch.cuda.is_available(), reason="uses placeholder pointers: never run where a launch could reach a GPU")
def test_training_planes_entries_refuse_bad_arguments():
    """The planes training products: sized only where the streamed GEMM takes N; the forward with z and the backward
    refuse a small or misaligned workspace, a bad ld and misaligned or null buffers before any launch."""
    lib = _lib.load()
    p, odd = ctypes.c_void_p(256), ctypes.c_void_p(264)
    need = ctypes.c_uint64(0)
    assert lib.hffn_train_mfma_workspace(512, 1024, 4096, ctypes.byref(need)) == _lib.OK
    mfma = ctypes.c_uint64(0)
    assert lib.hffn_mfma_workspace(512, 1024, 4096, ctypes.byref(mfma)) == _lib.OK
    assert need.value >= mfma.value  # the same layout with partials at every split count
    _expect_argument_error(lib.hffn_train_mfma_workspace(1, 256, 1024, ctypes.byref(need)), "streamed GEMM")
    _expect_argument_error(lib.hffn_train_mfma_workspace(512, 1040, 4096, ctypes.byref(need)), "multiples of 256")
    assert lib.hffn_train_mfma_workspace(512, 1024, 4096, ctypes.byref(need)) == _lib.OK
    ws = need.value
    fwd = lambda x, work, size, ld: lib.hffn_forward_mfma_z(x, p, p, p, p, p, p, work, size, p, p, p, p,  # noqa: E731
                                                            1024, 4096, 512, ld, None)
    _expect_argument_error(fwd(p, p, ws - 1, 512), "workspace")
    _expect_argument_error(fwd(p, odd, ws, 512), "256-byte aligned")
    _expect_argument_error(fwd(odd, p, ws, 512), "16-byte aligned")
    _expect_argument_error(fwd(None, p, ws, 512), "16-byte aligned")
    _expect_argument_error(fwd(p, p, ws, 510), "ld=510")
    _expect_argument_error(fwd(p, p, ws, 514), "ld=514")
    bwd = lambda gy, binades, size: lib.hffn_backward_mfma(gy, p, p, binades, p, p, p, size, p, p, 1024, 4096, 512, 512,  # noqa: E731
                                                           None)
    _expect_argument_error(bwd(p, p, ws - 1), "workspace")
    _expect_argument_error(bwd(odd, p, ws), "16-byte aligned")
    _expect_argument_error(bwd(p, None, ws), "null pointer")


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


class _StubRuntime:
    """The runtime interface parity.check uses, on the CPU: each pair adds a fixed offset to x (rows, rows: none),
    and the (edges, edges) pair changes its bits between calls."""
    mfma_available = tiles_available = True

    def __init__(self):
        self.pair, self.calls = (None, None), 0

    def force(self, up, down):
        self.pair = (up, down)

    def forward(self, index, x):
        self.calls += 1
        offset = {("rows", "rows"): 0.0, ("edges", "edges"): 1e-3 * (self.calls % 2)}.get(self.pair, 1e-4)
        return x + offset


def test_parity_result_reads_as_the_reference_callers_read_it():
    """runtime/gpu/nvidia/llm/inference/checks/parity_layers.py:51-53 and ffn/inference/checks/parity.py:49-51 read
    ``repeatable``, ``sequential_bits``, ``relative`` and ``error`` of each result; the reference runtime's module
    constants exist."""
    from hffn_amd import parity
    x = torch.linspace(-2, 2, 12, dtype=torch.float32).reshape(3, 4)
    result = parity.check(_StubRuntime(), 0, x, x.double())
    assert result.repeatable is False  # (edges, edges) changed its bits
    assert result.sequential_bits is True  # (rows, rows): same bits whole and in halves
    assert 1e-4 <= result.relative <= 2e-3 and result.error == pytest.approx(1e-3, rel=1e-3)
    assert result.pairs[("rows", "rows")] == 0.0
    steady = parity.check(_StubRuntime(), 0, x, x.double(), pairs=[("rows", "rows")])
    assert steady.repeatable and steady.sequential_bits and steady.error == 0.0
    assert runtime.COOP_MAX_TOKENS == runtime.EDGES_MAX_TOKENS
    assert runtime.BLOCK_MAX_WIDTH == 32768 and runtime.MAX_TOKENS == 1 << 18

