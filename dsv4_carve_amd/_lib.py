"""ctypes binding of libexl3_amd.so (the C ABI declared in include/exl3_amd.h).

The product path has no CPU fallback: if the library is missing, or no HIP
device is present, every op raises."""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libexl3_amd.so")

# Every symbol the header declares; tests check the library exports them all.
EXPORTS = (
    "exl3_last_error",
    "exl3_dequant",
    "exl3_dequant_nk",
    "exl3_had_rows",
    "exl3_gemm_scratch_bytes",
    "exl3_gemm",
    "exl3_gemm_group_scratch_bytes",
    "exl3_gemm_group",
    "exl3_moe_scratch_bytes",
    "exl3_moe_scratch_bytes_rows",
    "exl3_moe_max_rows",
    "exl3_moe_error_offset",
    "exl3_moe_decode",
    "exl3_moe_decode_routed",
    "exl3_moe_noalloc_scratch_bytes",
    "exl3_moe_decode_noalloc",
    "exl3_moe_noalloc_error",
    "exl3_moe_info",
    "exl3_moe_prefill_scratch_bytes",
    "exl3_moe_prefill",
    "exl3_moe_prefill_routed",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

_SIGS = {
    "exl3_last_error": ([], ctypes.c_char_p),
    "exl3_dequant": ([_P, _L, _L, _I, _I, _P, _P, _P, _P], _I),
    "exl3_dequant_nk": ([_P, _L, _L, _I, _I, _P, _P, _P, _P], _I),
    "exl3_had_rows": ([_P, _I, _P, _I, _L, _L, _P, _P, _F, _P], _I),
    "exl3_gemm_scratch_bytes": ([_L, _L, _L], _L),
    "exl3_gemm": ([_P, _L, _L, _P, _L, _I, _I, _P, _P, _P, _I, _P, _L, _P], _I),
    "exl3_gemm_group_scratch_bytes": ([_L, _L, _L, _P], _L),
    "exl3_gemm_group": ([_P, _L, _L, _L, _P, _P, _P, _P, _P, _I, _P, _I, _P, _L, _P], _I),
    "exl3_moe_scratch_bytes": ([_L, _L, _L], _L),
    "exl3_moe_scratch_bytes_rows": ([_L, _L, _L, _L], _L),
    "exl3_moe_max_rows": ([], _I),
    "exl3_moe_error_offset": ([], _L),
    "exl3_moe_decode": ([_P, _I, _P, _I, _L, _L, _L, _L, _L,
                         _P, _P, _P, _P, _P, _P, _P, _P, _P,
                         _P, _P, _P, _I, _I, _I, _F, _P, _L, _P], _I),
    "exl3_moe_decode_routed": ([_P, _I, _P, _I, _L, _L, _L, _L, _L,
                                _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                _P, _I, _P, _I, _P, _L,
                                _P, _I, _I, _I, _F, _P, _L, _P], _I),
    "exl3_moe_noalloc_scratch_bytes": ([], _L),
    "exl3_moe_decode_noalloc": ([_P, _I, _P, _I, _L, _L, _L, _L, _L,
                                 _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _P, _I, _P, _I, _P, _L,
                                 _P, _I, _I, _I, _F, _P], _I),
    "exl3_moe_noalloc_error": ([_I, _P], _I),
    "exl3_moe_info": ([ctypes.POINTER(ctypes.c_int64), _I], _I),
    "exl3_moe_prefill_scratch_bytes": ([_L, _L, _L, _L, _L], _L),
    "exl3_moe_prefill": ([_P, _I, _P, _I, _L, _L, _L, _L, _L,
                          _P, _P, _P, _P, _P, _P, _P, _P, _P,
                          _P, _P, _P, _I, _I, _I, _F, _P, _L, _P], _I),
    "exl3_moe_prefill_routed": ([_P, _I, _P, _I, _L, _L, _L, _L, _L,
                                 _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _P, _I, _P, _I, _P, _L,
                                 _P, _I, _I, _I, _F, _P, _L, _P], _I),
}


class Exl3Error(RuntimeError):
    """Argument or launch error reported by libexl3_amd.so."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load and type the library (no device work)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.isfile(path):
            raise ImportError(
                f"{path} is not built; run `python -m dsv4_carve_amd.build` (hipcc, gfx950)")
        lib = ctypes.CDLL(path)
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
        return lib


def load_twin(path: str) -> ctypes.CDLL:
    """A library with this C ABI built another way (the benchmark's timing-only
    null-decode build), typed from the same signature table; not cached, and
    never the library the ops call."""
    if not os.path.isfile(path):
        raise ImportError(f"{path} is not built; run `python -m dsv4_carve_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def check(rc: int) -> int:
    if rc < 0:
        msg = load().exl3_last_error()
        raise Exl3Error((msg or b"unknown error").decode())
    return rc
