"""ctypes binding of libmi355x_fp8.so.  Fails loudly when the library is missing.

torch is imported first on purpose: torch's bundled HIP runtime then owns the
``libamdhip64.so.7`` soname, and the library binds to that same runtime, so torch's
streams and device pointers are valid arguments.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must load the HIP runtime before the library)

from .build import LIB_PATH

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_size = ctypes.c_size_t

# Mirrors include/mi355x_fp8.h.
ABI_VERSION = 2
DTYPE_BF16 = 0
DTYPE_F16 = 1
CONFIG_AUTO = 0
CONFIG_STREAM = 1
CONFIG_TILE128 = 2
CONFIG_TILE256 = 3
CONFIG_DMA128_64, CONFIG_DMA128_128, CONFIG_DMA128_160 = 4, 5, 6
CONFIG_T256_128, CONFIG_T256_160, CONFIG_T256_192, CONFIG_T256_224, CONFIG_T256_256 = 7, 8, 9, 10, 11
CONFIG_T192_128, CONFIG_T192_160, CONFIG_T192_192, CONFIG_T192_224, CONFIG_T192_256 = 12, 13, 14, 15, 16
CONFIG_DMA64_64, CONFIG_DMA64_128 = 17, 18
OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_LAUNCH = 4
ERR_SCRATCH = 5
NOALLOC_SCRATCH_BYTES = 24 << 20

EXPORTS = {
    "mi355x_fp8_abi_version": ([], _int),
    "mi355x_fp8_status_string": ([_int], ctypes.c_char_p),
    "mi355x_fp8_act_quant": ([_ptr, _int, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr], _int),
    "mi355x_fp8_block_gemm_workspace_bytes": ([_i64, _i64, _i64, _int], _size),
    "mi355x_fp8_block_gemm": ([_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _int, _i64,
                               _i64, _i64, _i64, _ptr, _size, _int, _ptr], _int),
    "mi355x_fp8_silu_mul_quant": ([_ptr, _ptr, _int, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64,
                                   _ptr], _int),
    "mi355x_fp8_rmsnorm_quant": ([_ptr, _int, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, ctypes.c_float, _ptr,
                                  _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr], _int),
    "mi355x_fp8_rmsnorm_linear": ([_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, ctypes.c_float, _ptr, _i64,
                                   _ptr, _i64, _i64, _i64, _ptr, _i64, _ptr], _int),
    "mi355x_fp8_rmsnorm_gate_up_silu": ([_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, ctypes.c_float, _ptr,
                                         _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _ptr], _int),
    "mi355x_fp8_linear_workspace_bytes": ([_i64, _i64, _i64, _int], _size),
    "mi355x_fp8_linear_noalloc": ([_ptr, _int, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _ptr,
                                   _int, _i64, _int, _ptr], _int),
    "mi355x_fp8_linear_noalloc_scratch_bytes": ([], _size),
    "mi355x_fp8_read_probe": ([_ptr, _size, _ptr, _size, _ptr], _int),
    "mi355x_fp8_prefill_choice": ([_i64, _i64, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int)], _int),
    "mi355x_fp8_dispatch_choice": ([_i64, _i64, _i64, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int),
                                    ctypes.POINTER(_int)], _int),
    "mi355x_fp8_linear": ([_ptr, _int, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _ptr, _int,
                           _i64, _ptr, _size, _int, _ptr], _int),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""

    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m minillm_amd.build` "
                "(there is no fallback implementation)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.mi355x_fp8_abi_version() != ABI_VERSION:
            raise RuntimeError("libmi355x_fp8.so ABI version mismatch; rebuild it")
        _lib = lib
    return _lib


def check(status: int) -> None:
    """Map a C status code to the reference's exception types."""

    if status == OK:
        return
    text = load().mi355x_fp8_status_string(status).decode()
    if status in (ERR_INVALID, ERR_WORKSPACE, ERR_SCRATCH):
        raise ValueError(f"libmi355x_fp8: {text}")
    raise RuntimeError(f"libmi355x_fp8: {text} (status {status})")
