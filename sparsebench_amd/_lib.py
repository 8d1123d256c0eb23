"""Loads libsparsebench_hip.so (the C ABI in include/sparsebench_hip.h) via ctypes.

There is no fallback: if the library is missing or does not load, every op
raises. torch is imported first so the library's libamdhip64.so.7 resolves to
the HIP runtime torch already loaded (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os
import pathlib

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libsparsebench_hip.so"

_c_int = ctypes.c_int
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/sparsebench_hip.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "sb_last_error": (ctypes.c_char_p, []),
    "sb_version": (_i32, []),
    "sb_set_test_hook": (_c_int, [_i32, _i32]),
    "sb_arch_probe": (_c_int, [_ptr, _i64, _ptr]),
    "sb_routing_sizes": (
        _c_int,
        [_i64, _i32, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    ),
    "sb_routing": (
        _c_int,
        [_ptr, _i32, _i64, _i32, _i32, _i32, _i32, _ptr, _ptr,
         _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    ),
    "sb_routing_noalloc": (
        _c_int,
        [_ptr, _i32, _i64, _i32, _i32, _i32, _i32, _ptr,
         _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    ),
    "sb_sdd": (_c_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i32, _ptr]),
    "sb_dsd": (_c_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i32, _ptr]),
    "sb_sdd_experts": (
        _c_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i32, _ptr]
    ),
    "sb_dsd_experts": (_c_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr]),
    "sb_combine": (_c_int, [_ptr, _ptr, _ptr, _i32, _ptr, _i64, _i32, _i64, _i64, _ptr, _ptr]),
    "sb_routing_assigned": (
        _c_int,
        [_ptr, _i32, _ptr, _i32, _i64, _i64, _i32, _i32, _i32, _ptr, _ptr,
         _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    ),
    "sb_token_csr": (_c_int, [_ptr, _i32, _ptr, _i64, _i64, _ptr, _ptr, _ptr]),
    "sb_combine_assigned": (_c_int, [_ptr, _ptr, _ptr, _i32, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr]),
    "sb_router_sizes": (
        _c_int,
        [_i64, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
         ctypes.POINTER(_i64)],
    ),
    "sb_router_topk": (_c_int, [_ptr, _i64, _i32, _i32, _ptr, _ptr, _ptr]),
    "sb_token_rounding": (
        _c_int,
        [_ptr, _i64, _i32, _i32, _i32, _i32, _i32, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
         _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    ),
}

SB_OK = 0

_lib: ctypes.CDLL | None = None


class LibraryNotBuilt(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LibraryNotBuilt(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -m sparsebench_amd.build, or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(rc: int) -> None:
    """Turns a non-zero status into RuntimeError with the library's message."""
    if rc != SB_OK:
        msg = lib().sb_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"sparsebench HIP call failed with status {rc}")


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on `device` (what every op launches on)."""
    return torch.cuda.current_stream(device).cuda_stream
