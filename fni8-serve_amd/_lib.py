"""ctypes binding of libfni8amd.so (the C ABI declared in include/fni8amd.h).

The library is built in-tree next to this file (csrc/Makefile).  It is loaded
on first use; if it is missing, every GPU entry point raises RuntimeError --
there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libfni8amd.so")

# FNI8_ERR_* codes (include/fni8amd.h)
OK, ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_STRIDE, ERR_LAUNCH, ERR_DEVICE = 0, -1, -2, -3, -4, -5, -6
_ARG_ERRORS = (ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_STRIDE)

_P = ctypes.c_void_p
_I = ctypes.c_int64
_C = ctypes.c_int
_F = ctypes.c_float

# name -> argument types; every entry point returns int
SIGNATURES = {
    "fni8_init": [],
    "fni8_quantize_rowwise_f16": [_P, _I, _I, _I, _P, _I, _P, _P],
    "fni8_gemm_w8a8": [_P, _I, _P, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P],
    "fni8_gemm_w8a8_ws": [_P, _I, _P, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _P],
    "fni8_linear_w8a8_f16": [_P, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P],
    "fni8_linear_w8a8_f16_ws": [_P, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P, _I, _P],
    "fni8_linear_w8a8_f16_noalloc": [_P, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P],
    "fni8_moe_sort": [_P, _I, _I, _I, _P, _P, _P, _P],
    "fni8_gemm_w8a8_grouped": [_P, _P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _P, _P, _P],
    "fni8_moe_combine_f16": [_P, _I, _P, _P, _P, _I, _I, _P, _P],
    "fni8_gemm_w4a8": [_P, _I, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P],
    "fni8_gemm_w4a8_grouped": [_P, _P, _P, _I, _I, _P, _P, _I, _I, _I, _P, _P, _P, _P],
    "fni8_linear_w4a8_f16": [_P, _I, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P, _P, _P],
    "fni8_moe_route": [_P, _I, _I, _I, _C, _P, _I, _I, _I, _C, _F, _P, _P, _P],
    "fni8_act_and_mul_f16": [_P, _I, _I, _I, _C, _P, _I, _P],
    "fni8_act_and_mul_quant_f16": [_P, _I, _I, _I, _C, _P, _I, _P, _P],
    "fni8_act_and_mul_quant_f16_ws": [_P, _I, _I, _I, _C, _P, _I, _P, _P, _I, _P],
    "fni8_rmsnorm_f16": [_P, _I, _P, _I, _P, _F, _C, _I, _I, _P, _I, _P, _I, _P],
    "fni8_rmsnorm_quant_f16": [_P, _I, _P, _I, _P, _F, _C, _I, _I, _P, _I, _P, _P, _I, _P],
}
STRING_FUNCS = ("fni8_strerror", "fni8_last_error", "fni8_version")
INT64_FUNCS = {"fni8_linear_workspace_bytes": [_I, _I, _I],
               "fni8_act_and_mul_quant_workspace_bytes": [_I, _I]}
VOID_FUNCS = {"fni8_debug_coop_wait_ticks": [_I], "fni8_debug_gemm_plan": [_I, _I, _I]}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {os.path.join(_PKG_DIR, 'csrc')}`"
                " (or __graft_entry__.build()); the W8A8 path has no fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.fni8_strerror.argtypes = [ctypes.c_int]
        lib.fni8_strerror.restype = ctypes.c_char_p
        lib.fni8_last_error.argtypes = []
        lib.fni8_last_error.restype = ctypes.c_char_p
        lib.fni8_version.argtypes = []
        lib.fni8_version.restype = ctypes.c_char_p
        for name, argtypes in VOID_FUNCS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = None
        for name, argtypes in INT64_FUNCS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int64
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Call an entry point; map its error code to ValueError / RuntimeError."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != OK:
        msg = f"{name}: {lib.fni8_strerror(rc).decode()}: {lib.fni8_last_error().decode()}"
        raise (ValueError if rc in _ARG_ERRORS else RuntimeError)(msg)


def workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes fni8_linear_w8a8_f16_ws / fni8_gemm_w8a8_ws use for an [M, K] x [N, K]
    product (0: none)."""
    return int(load().fni8_linear_workspace_bytes(M, N, K))


def version() -> str:
    return load().fni8_version().decode()
