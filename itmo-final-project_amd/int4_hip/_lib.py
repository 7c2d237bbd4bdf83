"""ctypes binding of libint4_hip.so (the C-ABI declared in include/int4_hip.h).

The library is loaded lazily on first use.  If it is missing or stale every
GPU entry point raises ``RuntimeError``: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("INT4_HIP_LIB", Path(__file__).resolve().parent / "libint4_hip.so"))
ABI_VERSION = 1

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_LAUNCH = 4
MAX_GROUPED = 8
WORKSPACE_COUNTER_BYTES = 65536
NOALLOC_SCRATCH_BYTES = WORKSPACE_COUNTER_BYTES + (32 << 20)

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_sz = ctypes.c_size_t


class Problem(ctypes.Structure):
    """Mirror of ``w4a16_problem`` (include/int4_hip.h)."""

    _fields_ = [
        ("x", _c_vp),
        ("qweight", _c_vp),
        ("scales", _c_vp),
        ("zeros", _c_vp),
        ("y", _c_vp),
        ("N", _c_i64),
        ("K", _c_i64),
        ("group_size", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class QuantProblem(ctypes.Structure):
    """Mirror of ``w4_quantize_problem`` (include/int4_hip.h)."""

    _fields_ = [
        ("w", _c_vp),
        ("qweight", _c_vp),
        ("scales", _c_vp),
        ("zeros", _c_vp),
        ("N", _c_i64),
        ("K", _c_i64),
        ("stride_wn", _c_i64),
        ("stride_wk", _c_i64),
        ("group_size", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


# symbol -> (restype, argtypes); exactly the functions include/int4_hip.h declares
SIGNATURES = {
    "w4_abi_version": (_c_int, []),
    "w4_last_error": (ctypes.c_char_p, []),
    "w4_quantize": (_c_int, [_c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_vp, _c_vp, _c_vp, _c_vp]),
    "w4_quantize_grouped": (_c_int, [ctypes.POINTER(QuantProblem), _c_int, _c_int, _c_vp]),
    "w4_dequantize": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_vp]),
    "w4a16_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_int]),
    "w4a16_gemm": (_c_int, [_c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_int,
                            _c_vp, _c_i64, _c_vp, _c_sz, _c_vp]),
    "w4a16_grouped_workspace_bytes": (_c_sz, [ctypes.POINTER(Problem), _c_int, _c_i64]),
    "w4a16_gemm_grouped": (_c_int, [ctypes.POINTER(Problem), _c_int, _c_int, _c_i64, _c_vp, _c_sz, _c_vp]),
    "w4a16_gemm_noalloc": (_c_int, [_c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                    _c_int, _c_vp, _c_i64, _c_vp]),
}

_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the library; raise RuntimeError if it is unusable."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"int4_hip: HIP library {p} is not built; run "
                "`python itmo-final-project_amd/build_lib.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.w4_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"int4_hip: {p} has ABI version {v}, bindings expect {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != OK:
        msg = load().w4_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")
