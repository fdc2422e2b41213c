"""ctypes binding of ``libdflash_hip.so`` (the C ABI in ``include/dflash_hip.h``).

The library is built in-tree by ``build.py`` (``hipcc --offload-arch=gfx950``).
There is no fallback: if the library is missing or a call fails, an exception
is raised with the library's own message.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libdflash_hip.so"

ABI_VERSION = 6
DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_F16 = 2
LAYOUT_PORTABLE = 0
LAYOUT_TILED = 1

STATUS_NAMES = {
    1: "DFLASH_ERR_INVALID_ARGUMENT",
    2: "DFLASH_ERR_UNSUPPORTED",
    3: "DFLASH_ERR_WORKSPACE",
    4: "DFLASH_ERR_HIP",
}

# Every symbol the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


class W4Desc(ctypes.Structure):
    """``struct dflash_w4``."""

    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("experts", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("group_size", ctypes.c_int64),
        ("scale_dtype", ctypes.c_int32),
        ("layout", ctypes.c_int32),
    ]


_W4P = ctypes.POINTER(W4Desc)

SIGNATURES = {
    "dflash_abi_version": (ctypes.c_int, []),
    "dflash_w4_to_tiled": (ctypes.c_int, [_W4P, _P, _P, _P]),
    "dflash_w4_from_int8": (ctypes.c_int, [_P, _P, ctypes.c_int32, _I64, _I64, _I64, _I64, ctypes.c_int32, _P, _P,
                                           _P, _P]),
    "dflash_last_error": (ctypes.c_char_p, []),
    "dflash_qlinear_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "dflash_qlinear_w4a16": (ctypes.c_int, [_P, _I64, _W4P, _P, _P, _SZ, _P]),
    "dflash_qlinear_w4a16_f32": (ctypes.c_int, [_P, _I64, _W4P, _P, _P, _SZ, _P]),
    "dflash_router_logits": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _P, _P]),
    "dflash_moe_route_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "dflash_moe_route": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "dflash_moe_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_int]),
    "dflash_moe_experts_w4a16": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _W4P, _W4P, _W4P, _W4P,
                                                _P, _P, _P, _SZ, _P]),
    "dflash_moe_w4a16": (ctypes.c_int, [_P, _I64, _I64, _P, _P, _I64, _W4P, _W4P, _W4P, _W4P, _P, _P, _P, _P, _P,
                                        _P, _P, _P, _P, _SZ, _P]),
    "dflash_moe_w4a16_noalloc": (ctypes.c_int, [_P, _I64, _I64, _P, _P, _I64, _W4P, _W4P, _W4P, _W4P, _P, _P, _P, _P,
                                                _P, _P, _P, _P, _P]),
    "dflash_set_split_down": (ctypes.c_int, [ctypes.c_int]),
    "dflash_set_tile_pieces": (ctypes.c_int, [ctypes.c_int]),
    "dflash_moe_split_down": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int32,
                                             ctypes.c_int32]),
    "dflash_set_measure_stage": (ctypes.c_int, [ctypes.c_int]),
}

STAGE_NONE = 0
STAGE_GATE_UP = 1
STAGE_DOWN = 2
STAGE_EXPERTS = 3


class DflashError(RuntimeError):
    """A nonzero status from the C ABI."""

    def __init__(self, function: str, status: int, message: str):
        self.status = status
        super().__init__(f"{function} failed with {STATUS_NAMES.get(status, status)}: {message}")


_LIB = None


def load(path: Path = LIBRARY_PATH) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it was not built.

    ``path`` selects another build of the same ABI before the first call (the
    profiling build of ``timeline.py``); once loaded, the library stays.
    """
    global _LIB
    if _LIB is not None:
        if path != LIBRARY_PATH and Path(_LIB._name) != path:
            raise RuntimeError(f"{Path(_LIB._name).name} is already loaded; {path.name} must be loaded first")
        return _LIB
    if not path.is_file():
        raise RuntimeError(f"{path.name} not found at {path}; build it with build.py (hipcc, gfx950)")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.dflash_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libdflash_hip.so ABI {version} != expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(function: str, status: int) -> None:
    if status:
        message = load().dflash_last_error().decode(errors="replace")
        raise DflashError(function, status, message)


def call(function: str, *args) -> None:
    check(function, getattr(load(), function)(*args))
