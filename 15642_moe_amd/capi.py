"""ctypes binding of the C ABI in include/moe_fp8.h (and the test and
measurement instrumentation of include/moe_fp8_testing.h, same library).

The shared library is built in-tree by ``build.py``.  Loading it never falls
back to anything: a missing or stale library raises RuntimeError.  torch is
imported first so the library binds to the HIP runtime torch already loaded
(one runtime per process, so torch streams and pointers are valid here).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("lib15642_moe_fp8.so")
ABI_VERSION = 2

MOE_OK = 0
MOE_ERR_INVALID_ARG = 1
MOE_ERR_HIP = 2
MOE_ERR_WORKSPACE = 3
MAX_T = 262143  # include/moe_fp8.h MOE_MAX_T: 32-bit activation offsets in the grouped GEMMs

# Workspace buffer ids (enum moe_ws_buffer).
(WS_TOPK_IDS, WS_TOPK_W, WS_COUNTS, WS_OFFSETS, WS_ROUTE_TOKEN, WS_ROUTE_WEIGHT, WS_TOKEN_ROUTE, WS_CQ, WS_CS, WS_Y,
 WS_QUEUE) = range(11)
WS_NBUF = 11
FORWARD_EVENTS = 6

_c_int, _c_size, _c_float, _c_vp, _c_u64 = ctypes.c_int, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p, ctypes.c_uint64

# name -> (restype, argtypes); exactly the functions include/moe_fp8.h and
# include/moe_fp8_testing.h declare.
SIGNATURES = {
    "moe_abi_version": (_c_int, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_packed_w13_bytes": (_c_size, [_c_int]),
    "moe_packed_w2_bytes": (_c_size, [_c_int]),
    "moe_pack_w13": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "moe_pack_w2": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "moe_unpack_w13": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "moe_unpack_w2": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp]),
    "moe_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "moe_workspace_offsets": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_size), _c_int]),
    "moe_forward": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_float, _c_int, _c_int, _c_int, _c_vp, _c_size,
         _c_vp, _c_vp],
    ),
    "moe_forward_timed": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_float, _c_int, _c_int, _c_int, _c_vp, _c_size,
         _c_vp, _c_vp, ctypes.POINTER(_c_vp), _c_int],
    ),
    "moe_noalloc_scratch_bytes": (_c_size, []),
    "moe_forward_noalloc": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_float, _c_int, _c_int, _c_int, _c_vp, _c_vp],
    ),
    "moe_route": (_c_int, [_c_vp, _c_vp, _c_float, _c_int, _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "moe_packed_router_bytes": (_c_size, []),
    "moe_pack_router": (_c_int, [_c_vp, _c_vp, _c_vp]),
    "moe_unpack_router": (_c_int, [_c_vp, _c_vp, _c_vp]),
    "moe_router_workspace_bytes": (_c_size, [_c_int]),
    "moe_router_quant": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp, _c_size, _c_vp, _c_vp, _c_vp, _c_vp]),
    "moe_fill_normal_e4m3": (_c_int, [_c_vp, _c_size, _c_u64, _c_u64, _c_vp]),
    "moe_mfma_tiles": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_vp]),
    "moe_mfma_ceiling": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_vp]),
    "moe_host_fill_normal_e4m3": (_c_int, [_c_vp, _c_size, _c_u64, _c_u64, _c_u64, _c_int]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the library once and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"HIP library {LIB_PATH.name} is not built; run __graft_entry__.build() "
            "(or python <package>/build.py) first"
        )
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)

    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.moe_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH.name} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status, with the library's message."""
    if rc != MOE_OK:
        msg = load().moe_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def workspace_offsets(T: int, e_local: int) -> list[int]:
    arr = (_c_size * WS_NBUF)()
    check(load().moe_workspace_offsets(T, e_local, arr, WS_NBUF), "moe_workspace_offsets")
    return list(arr)
