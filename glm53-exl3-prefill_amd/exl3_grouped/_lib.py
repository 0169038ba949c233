"""ctypes binding of libexl3_grouped.so (the C ABI declared in include/exl3_grouped.h).

The library is built in-tree by `make -C glm53-exl3-prefill_amd/csrc` (or __graft_entry__.build()).
EXL3_GROUPED_LIB overrides its path. There is no fallback: every op raises if the library is missing.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_PATH = os.path.join(_HERE, "libexl3_grouped.so")

EXL3_OK = 0
EXL3_ERR_ARG = 1
EXL3_ERR_HIP = 2

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I32, DTYPE_I64 = 0, 1, 2, 3, 4
LAYOUT_ROWS, LAYOUT_T16 = 0, 1

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# name -> (restype, argtypes); every name here is declared in include/exl3_grouped.h
SIGNATURES = {
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_abi_version": (I32, []),
    "exl3_sort_routes_workspace_bytes": (SZ, [I64, I32, I32]),
    "exl3_sort_routes": (I32, [P, I32, P, I32, I64, I32, I32, P, P, P, P, P, P, P, SZ, P]),
    "exl3_build_blocks": (I32, [P, I32, I32, P, P, P, P]),
    "exl3_build_tiles": (I32, [P, I32, I32, I32, P, P, P, P]),
    "exl3_build_tiles_split": (I32, [P, I32, I32, I32, I32, I32, P, P, P, P, P, P, I64, P]),
    "exl3_sort_routes_split_tiles": (I32, [P, I32, P, I32, I64, I32, I32, P, P, P, P, P, P, P, SZ, I32, I32, I32, I32,
                                           P, P, P, P, P, P, I64, P]),
    "exl3_row_had": (I32, [P, P, P, P, P, I64, I64, I64, I32, I32, P]),
    "exl3_row_had_ex": (I32, [P, P, P, P, P, I64, I64, I64, I32, I32, I32, P]),
    "exl3_act_had": (I32, [P, I64, P, P, P, I64, I64, I32, F32, P]),
    "exl3_act_had_ex": (I32, [P, I64, P, P, P, I64, I64, I32, F32, I32, P]),
    "exl3_act_had_f32": (I32, [P, I64, P, P, P, I64, I64, I32, F32, P]),
    "exl3_act_had_t16": (I32, [P, I64, P, P, P, I64, I64, I32, F32, P]),
    "exl3_grouped_gemm": (I32, [P, I64, I32, P, P, I64, I32, I32, I32, P, P, I64, P, P, I32, P, P, I32, P, P,
                                P, P, I64, I32, P]),
    "exl3_grouped_gemm_ex": (I32, [P, I64, I32, I32, P, P, I64, I32, I32, I32, P, P, I64, P, P, I32, I32, P, P,
                                   I32, P, P, P, P, I64, I32, P]),
    "exl3_grouped_gemm_split": (I32, [P, I64, I32, I32, P, P, I64, I32, I32, I32, P, P, I64, P, P, I32, I32, P, P,
                                      I32, P, P, P, P, I64, I32, I32, P]),
    "exl3_grouped_gemm_clear": (I32, [P, I64, I32, I32, P, P, I64, I32, I32, I32, P, P, I64, P, P, I32, I32, P, P,
                                      I32, P, P, P, P, I64, I32, I32, P, I64, P]),
    "exl3_combine_routes": (I32, [P, P, P, I32, I32, I64, I32, I64, P]),
    "exl3_combine_routes_dt": (I32, [P, P, I32, P, I32, I32, I64, I32, I64, P]),
    "exl3_fat_gemm": (I32, [P, I64, I32, P, I32, I32, I32, P, I64, P, I64, I32, I32, I32, I32, P]),
    "exl3_fat_gemm_scatter": (I32, [P, I64, I32, P, I32, I32, I32, P, I64, P, I64, P, P, I32, I32, I32, I32, P]),
    "exl3_smem_bytes": (I64, [I64]),
    "exl3_linear_workspace_bytes": (I64, [I64, I32]),
    "exl3_route_topk": (I32, [P, I32, I64, P, I64, I32, I32, I32, F32, P, I32, P, P]),
    "exl3_linear": (I32, [P, I64, I32, P, I32, I32, I32, P, P, P, P, I32, P]),
    "exl3_reconstruct": (I32, [P, P, I32, I32, I32, I32, I32, P]),
    "exl3_decode_states": (I32, [P, P, I64, P]),
    "exl3_route_prep_small": (I32, [P, I32, P, I32, I64, I32, I32, I32, I32, P, P, P, P, P, P, P, P, P, I64, P, I64,
                                    P]),
    "exl3_moe_decode_workspace_bytes": (I64, [I64, I32, I32, I32, I32]),
    "exl3_moe_decode": (I32, [P, I64, I32, P, I32, P, I32, I32, I32, I32, I32, P, P, I64, P, I64, P, P, I64, P, I64,
                              P, I64, P, I64, F32, P, P, I64, P]),
    "exl3_moe_decode_noalloc": (I32, [P, I64, I32, P, I32, P, I32, I32, I32, I32, I32, P, P, I64, P, I64, P, P, I64,
                                      P, I64, P, I64, P, I64, F32, P, P]),
}

ABI_VERSION = 10

_lib = None
_path = None


def path() -> str:
    return os.environ.get("EXL3_GROUPED_LIB", DEFAULT_PATH)


def load():
    """Load (once) and return the ctypes library; raises RuntimeError if it is missing or mismatched."""
    global _lib, _path
    if _lib is not None:
        return _lib
    p = path()
    if not os.path.exists(p):
        raise RuntimeError(f"EXL3 grouped prefill library not found at {p}; build it with "
                           "`make -C glm53-exl3-prefill_amd/csrc` (there is no CPU fallback)")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.exl3_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {v}, expected {ABI_VERSION}")
    _lib, _path = lib, p
    return lib


def last_error() -> str:
    return load().exl3_last_error().decode()


def check(rc: int) -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK failure type) for a non-zero status."""
    if rc != EXL3_OK:
        kind = "invalid argument" if rc == EXL3_ERR_ARG else "HIP error"
        raise RuntimeError(f"{last_error()} ({kind})")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
