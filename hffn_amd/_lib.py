"""ctypes binding of ``libhffn_amd.so``, the HIP library built from ``hffn_amd/csrc`` (C ABI: ``include/hffn_amd.h``).

The library is built in-tree by ``hffn_amd.build`` (``python -c "import __graft_entry__ as g; g.build()"``). Loading
never builds and never falls back to anything: a missing library is an error, so no forward call can run on
anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().with_name("libhffn_amd.so")
ABI_VERSION = 18

OK = 0
VALUE_F32, VALUE_BF16 = 0, 1
UP_MODES = {"edges": 1, "rows": 2, "mfma": 3}
DOWN_MODES = {"edges": 1, "rows": 2, "mfma": 3}

_P, _I, _U32, _U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64

# name -> argument types (return type int for every entry but hffn_last_error)
SIGNATURES = {
    "hffn_abi_version": [],
    "hffn_last_error": [],
    "hffn_edges_supported": [_U32, _U32],
    "hffn_transpose": [_P, _P, _U32, _U32, _U32, _U32, _P],
    "hffn_up": [_I, _I, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P],
    "hffn_down": [_I, _I, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P],
    "hffn_forward": [_I, _I, _I] + [_P] * 13 + [_U32] * 6 + [_P],
    "hffn_plan_forward": [_I, _I, _I] + [_P] * 12 + [_U32] * 6 + [ctypes.POINTER(_U64)],
    "hffn_plan_launch": [_U64, _P, _P],
    "hffn_plan_release": [_U64],
    "hffn_forward_z": [_I, _I] + [_P] * 14 + [_U32] * 6 + [_P],
    "hffn_grad_dense_workspace": [_U32, _U32, _U32, _P],
    "hffn_grad_dense": [_P] * 6 + [_U32] * 4 + [_P, _U64, _P],
    "hffn_train_mfma_workspace": [_U32, _U32, _U32, ctypes.POINTER(_U64)],
    "hffn_forward_mfma_z": [_P] * 7 + [_P, _U64] + [_P] * 4 + [_U32] * 4 + [_P],
    "hffn_backward_mfma": [_P] * 7 + [_U64, _P, _P] + [_U32] * 4 + [_P],
    "hffn_grad_sddmm": [_P] * 6 + [_U32] * 4 + [_P],
    "hffn_grad_hidden": [_P] * 7 + [_U32] * 5 + [_P],
    "hffn_grad_x": [_P] * 6 + [_U32] * 5 + [_P],
    "hffn_reduce_tiles": [_P, _U32, _U32, _U32, _U32, _U32, _P, _P, _P, _P, _P],
    "hffn_adamw": [_P] * 4 + [_U32] + [ctypes.c_float] * 8 + [_P],
    "hffn_gather_values": [_P, _P, _P, _U32, _P],
    "hffn_read_probe": [_P, _U64, _P, _U32, _U32, _P],
    "hffn_output_major_workspace": [_U32, _U32, ctypes.POINTER(_U64)],
    "hffn_output_major": [_I, _P, _P, _P, _U32, _U32, _U32, _P, _P, _P, _P, _U64, _P],
    "hffn_mfma_supported": [_U32, _U32],
    "hffn_dense_planes_bytes": [_U32, _U32, ctypes.POINTER(_U64)],
    "hffn_densify": [_I, _P, _P, _P, _U32, _U32, _P, _P, _P],
    "hffn_mfma_workspace": [_U32, _U32, _U32, ctypes.POINTER(_U64)],
    "hffn_mfma_streamed": [_U32, _U32, _U32],
    "hffn_mfma_up": [_I, _P, _P, _P, _P, _P, _U64, _U32, _U32, _U32, _P],
    "hffn_mfma_split": [_P, _P, _U64, _U32, _U32, _U32, _P],
    "hffn_tiles_table_size": [_I, _U32, _U32, ctypes.POINTER(_U64)],
    "hffn_tiles_table_build": [_I, _P, _P, _P, _U32, _U32, _P, _P],
    "hffn_forward_tiles_compact": [_I] + [_P] * 11 + [_U64, _P, _U32, _U32, _U64, _U64, _U32, _P],
    "hffn_plan_tiles_compact": [_I] + [_P] * 10 + [_U64, _P, _U32, _U32, _U64, _U64, _U32, ctypes.POINTER(_U64)],
    "hffn_mfma_up_planes": [_I, _P, _P, _P, _P, _U64, _U32, _U32, _U32, _P],
    "hffn_mfma_down": [_I, _P, _P, _P, _P, _P, _U64, _U32, _U32, _U32, _P],
    "hffn_forward_mfma": [_I] + [_P] * 8 + [_U64, _P] + [_U32] * 3 + [_P],
    "hffn_gemv_workspace": [_U32, _U32, _P],
    "hffn_forward_gemv": [_I] + [_P] * 9 + [_U64, _P] + [_U32] * 3 + [_P],
    "hffn_plan_gemv": [_I] + [_P] * 8 + [_U64, _P] + [_U32] * 3 + [_P],
    "hffn_forward_gemv_static": [_I] + [_P] * 9 + [_U32] * 3 + [_P],
    "hffn_tiles_store_size": [_I, _U32, _U32, _U64, ctypes.POINTER(_U64), ctypes.POINTER(_U64)],
    "hffn_tiles_build": [_I, _P, _P, _P, _U32, _U32, _U64, _P, _U64, _P, _P],
    "hffn_tiles_workspace": [_I, _U32, _U32, _U32, _U64, _U64, ctypes.POINTER(_U64)],
    "hffn_forward_tiles": [_I] + [_P] * 9 + [_U64, _P, _U32, _U32, _U64, _U64, _U32, _P],
    "hffn_plan_tiles": [_I] + [_P] * 8 + [_U64, _P, _U32, _U32, _U64, _U64, _U32, ctypes.POINTER(_U64)],
}


class HIPError(RuntimeError):
    """A failure reported by the HIP library (invalid arguments or a refused launch)."""


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The bound library (loaded once per process). Raises ``RuntimeError`` when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise RuntimeError(f"{LIBRARY} is not built: run hffn_amd.build.build() (or __graft_entry__.build()) first; "
                           "the HFFN forward has no other implementation")
    lib = ctypes.CDLL(str(LIBRARY))
    for name, argtypes in SIGNATURES.items():
        function = getattr(lib, name)
        function.argtypes = argtypes
        function.restype = ctypes.c_char_p if name == "hffn_last_error" else ctypes.c_int
    if lib.hffn_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIBRARY}: ABI version {lib.hffn_abi_version()}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != OK:
        message = load().hffn_last_error().decode(errors="replace")
        if status == -1:
            raise ValueError(f"{what}: {message}")
        raise HIPError(f"{what}: {message}")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def query_bytes(function, *args) -> int:
    """Call a host-only size query of the library and return its uint64 result."""
    result = ctypes.c_uint64(0)
    check(function(*args, ctypes.byref(result)), function.__name__)
    return result.value
