"""ctypes binding of the C ABI in include/consumer_int8_amd.h (libci8_amd.so).

This is the binding an FFI caller would write; the torch ops do not use it (they call
the same entry points from C++). Tests use it to reach the C ABI directly.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libci8_amd.so"

CI8_OK = 0
CI8_ERR_GEOMETRY = 1
CI8_ERR_ALIGNMENT = 2
CI8_ERR_OVERLAP = 3
CI8_ERR_SCHEDULE = 4
CI8_ERR_TOO_LARGE = 5
CI8_ERR_LAUNCH = 6

_p = ctypes.c_void_p
_i64 = ctypes.c_int64

SIGNATURES = {
    "ci8_last_error": ([], ctypes.c_char_p),
    "ci8_version": ([], ctypes.c_char_p),
    "ci8_quantize_rows": ([_p, _p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_quantize_grouped4096": ([_p, _p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_fused_channel_mm": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_cutlass_channel_mm": ([_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_cutlass_channel_mm_noalloc": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_channel_mm": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_channel_gemv": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_grouped_summed_mm": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_silu_mul": ([_p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_silu_mul_quantize": ([_p, _p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_unpack_allspark": ([_p, _p, _p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_quantize_block32": ([_p, _p, _p, _i64, _i64, _p], ctypes.c_int),
    "ci8_q8_block_mm": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_q8_block_int8": ([_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p], ctypes.c_int),
    "ci8_gguf_q8_packed_mm": ([_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p],
                              ctypes.c_int),
}

_lib = None


def load(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(path))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def last_error() -> str:
    return load().ci8_last_error().decode()


def check(status: int) -> None:
    if status != CI8_OK:
        raise RuntimeError(last_error())
