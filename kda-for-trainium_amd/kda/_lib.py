"""ctypes binding of libkda.so, the gfx950 operator library (C ABI: include/kda.h).

The shared object is built in-tree by ``make -C kda-for-trainium_amd/csrc`` (or
``__graft_entry__.build()``) and loaded from this directory.  There is no
fallback: if the library is missing or a symbol is absent, loading raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkda.so"

KDA_OK = 0
KDA_ERR_INVALID_ARG = 1
KDA_ERR_UNSUPPORTED = 2
KDA_ERR_HIP = 3

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> argtypes, mirroring include/kda.h one-to-one.  Every entry returns int
# (a KDA_* status) except those listed in RESTYPES.
SIGNATURES = {
    "kda_silu_f32": [_p, _p, _i64, _p],
    "kda_adamw_f32": [_p, _p, _p, _p, _p, _p, _p, _i64, _f32, _f32, _f32, _f32, _f32, _i64, _p],
    "kda_rope_f32": [_p, _p, _p, _p, _i64, _i64, _p],
    "kda_matmul_bf16": [_p, _p, _p, _i64, _i64, _i64, _p],
    "kda_rmsnorm_matmul_bf16": [_p, _p, _p, _p, _i64, _i64, _i64, _f32, _p, _i64, _p],
    "kda_rmsnorm_matmul_bf16_noalloc": [_p, _p, _p, _p, _i64, _i64, _i64, _f32, _p],
    "kda_workspace_size": [_int, _i64, _i64, _i64, _i64, _i64],
    "kda_matmul_f32": [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_transpose_matmul_f32": [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_bmm_f32": [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "kda_lora_f32": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "kda_rmsnorm_matmul_f32": [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_add_rmsnorm_matmul_f32": [_p, _p, _f32, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_matmul_add_rmsnorm_f32": [_p, _p, _f32, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_add_rmsnorm_matmul_bf16": [_p, _p, _f32, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_matmul_add_rmsnorm_bf16": [_p, _p, _f32, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_swiglu_f32": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_bmm_softmax_f32": [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "kda_mamba_f32": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "kda_swiglu_bf16": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "kda_gqa_fwd_bf16": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _int,
                         _i64, _i64, _i64, _p],
    "kda_gqa_fwd_f32": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _int,
                        _i64, _i64, _i64, _p, _i64, _p],
}


# Entry points that return something other than an int status.
RESTYPES = {
    "kda_workspace_size": _i64,
}

# Operator ids of kda_workspace_size (include/kda.h).
OP_MATMUL_F32 = 1
OP_TRANSPOSE_MATMUL_F32 = 2
OP_BMM_F32 = 3
OP_LORA_F32 = 4
OP_RMSNORM_MATMUL_F32 = 5
OP_ADD_RMSNORM_MATMUL_F32 = 6
OP_MATMUL_ADD_RMSNORM_F32 = 7
OP_SWIGLU_F32 = 8
OP_RMSNORM_MATMUL_BF16 = 9
OP_BMM_SOFTMAX_F32 = 10
OP_GQA_F32 = 11
OP_SWIGLU_BF16 = 12
OP_ADD_RMSNORM_MATMUL_BF16 = 13
OP_MATMUL_ADD_RMSNORM_BF16 = 14


class KdaError(RuntimeError):
    """A libkda entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


_LIB = None


def lib() -> ctypes.CDLL:
    """Loads libkda.so once; raises OSError with a build hint if it is missing."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise OSError(
                f"{LIB_PATH} is not built; run `make -C {LIB_PATH.parent.parent / 'csrc'}` "
                "or __graft_entry__.build()")
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        handle.kda_version.restype = _int
        handle.kda_version.argtypes = []
        handle.kda_last_error.restype = ctypes.c_char_p
        handle.kda_last_error.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)  # AttributeError if the symbol is missing
            fn.restype = RESTYPES.get(name, _int)
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    """Calls entry point `name`; raises ValueError / KdaError on a non-zero status."""
    handle = lib()
    status = getattr(handle, name)(*args)
    if status != KDA_OK:
        msg = handle.kda_last_error().decode(errors="replace")
        if status in (KDA_ERR_INVALID_ARG, KDA_ERR_UNSUPPORTED):
            raise ValueError(f"{name}: {msg}")
        raise KdaError(name, status, msg)


def query(name: str, *args) -> int:
    """Calls a non-status entry point (a size query) and returns its value."""
    return int(getattr(lib(), name)(*args))


def version() -> int:
    return int(lib().kda_version())
