"""ctypes binding of libfusionmoe.so (declarations in include/fusionmoe.h).

The library is built in-tree by ``fusionllm_amd.build`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing or its ABI version differs, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfusionmoe.so"
ABI_VERSION = 13
MAX_EXPERTS = 64
MAX_TOPK = 8

BF16 = 0
F32 = 1

_P = c_void_p
_I32P = c_void_p  # int32_t* passed as raw addresses
_PP = POINTER(c_void_p)  # const void* const* (host array of device pointers)

# name -> (restype, argtypes); mirrors include/fusionmoe.h
SIGNATURES = {
    "fmoe_abi_version": (c_int, []),
    "fmoe_status_string": (c_char_p, [c_int]),
    "fmoe_router_fwd": (c_int, [_P, _P, _P, c_int64, c_int64, c_int, c_int, c_float,
                                _P, _P, _P, _P, _P]),
    "fmoe_dispatch_workspace_bytes": (c_size_t, [c_int64, c_int, c_int]),
    "fmoe_dispatch": (c_int, [_P, _P, c_int64, c_int64, c_int, c_int,
                              _P, _P, _P, _P, _P, _P, c_size_t, _P]),
    "fmoe_dispatch_noalloc": (c_int, [_P, _P, c_int64, c_int64, c_int, c_int, _P, _P, _P, _P, _P, _P]),
    "fmoe_route_and_dispatch_workspace_bytes": (c_size_t, [c_int64, c_int, c_int]),
    "fmoe_route_and_dispatch": (c_int, [_P, _P, _P, c_int64, c_int64, c_int, c_int, c_float,
                                        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P]),
    "fmoe_gateup_fwd": (c_int, [_P, _P, c_int, c_int64, _P, _P, c_int, c_int64, c_int64, c_int64, c_int64,
                                _PP, _PP, _P, _P, _P, c_size_t, _P]),
    "fmoe_split_workspace_bytes": (c_size_t, []),
    "fmoe_down_fwd": (c_int, [_P, _P, c_int, c_int64, c_int64, c_int64, c_int64,
                              _PP, _P, _P, c_size_t, _P]),
    "fmoe_combine_fwd": (c_int, [_P, _P, _P, _P, c_int64, c_int64, c_int, c_int64,
                                 c_int, c_int, _P, _P, _P]),
    "fmoe_combine_bwd": (c_int, [_P, c_int, _P, _P, _P, c_int64, c_int64, c_int,
                                 _P, _P, _P]),
    "fmoe_down_bwd_dx": (c_int, [_P, _P, _P, c_int, c_int64, c_int64, c_int64, c_int64,
                                 _PP, _P, _P, _P, c_size_t, _P]),
    "fmoe_gateup_bwd_dx": (c_int, [_P, _P, c_int, c_int64, c_int64, c_int64, c_int64,
                                   _PP, _PP, _P, _P, c_size_t, _P]),
    "fmoe_weight_grad_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int, c_int64, c_int64]),
    "fmoe_weight_grad": (c_int, [_P, _P, c_int64, _P, _P, c_int64, _P, c_int, c_int64, _P, c_int,
                                 c_int64, c_int64, c_int64, c_int64, c_int64,
                                 _PP, _PP, c_int, _P, c_size_t, _P]),
    "fmoe_router_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int, c_int]),
    "fmoe_router_bwd": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int, c_int, c_float,
                                _P, _P, _P, c_int, _P, c_size_t, _P]),
    "fmoe_dx_reduce": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int, c_int64,
                               c_int, c_int, _P, _P]),
    "fmoe_rmsnorm_fwd": (c_int, [_P, c_int, _P, c_int, c_int64, c_int64, c_float, _P, _P, _P]),
    "fmoe_norm_bwd_workspace_bytes": (c_size_t, [c_int64]),
    "fmoe_dx_reduce_norm": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int, c_int64, c_int,
                                    _P, _P, _P, c_int, _P, c_int, _P, _P, _P, c_size_t, _P]),
    "fmoe_normuon_step": (c_int, [_PP, _PP, _PP, _PP, POINTER(c_int64), POINTER(c_int64), POINTER(c_int),
                                  c_int, c_int, c_double, c_double, c_double, c_double, c_double, c_int,
                                  c_double, c_double, _P]),
    "fmoe_cast_bf16": (c_int, [_PP, _PP, POINTER(c_int64), c_int, _P]),
    "fmoe_route_dispatch": (c_int, [_P, _P, _P, c_int64, c_int64, c_int, c_int, c_float, _P, _P, _P, _P,
                                    _P, _P, _P, _P, _P, _P]),
}

_lock = threading.Lock()
_lib = None


class FusionMoEError(RuntimeError):
    """A libfusionmoe entry point returned a nonzero status."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points.

    Raises FileNotFoundError when the library has not been built, and
    FusionMoEError when its ABI version differs from this binding's.
    """
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise FileNotFoundError(
                f"{p} is missing: build the HIP extension first "
                "(python -m fusionllm_amd.build or __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.fmoe_abi_version()
        if ver != ABI_VERSION:
            raise FusionMoEError(f"libfusionmoe ABI {ver} != binding ABI {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().fmoe_status_string(rc).decode()
        raise FusionMoEError(f"{what} failed: {msg} (status {rc})")


_PTR_CACHE: dict = {}


def ptr_array(ptrs) -> ctypes.Array:
    """Host array of device pointers for the per-expert weight arguments.

    The arrays are read-only inputs of the C entry points, so one array per
    distinct pointer tuple is kept and reused (the weights of a module keep
    their storage from step to step)."""
    key = tuple(ptrs)
    arr = _PTR_CACHE.get(key)
    if arr is None:
        if len(_PTR_CACHE) > 4096:
            _PTR_CACHE.clear()
        arr = (c_void_p * len(key))(*key)
        _PTR_CACHE[key] = arr
    return arr
