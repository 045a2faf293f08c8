"""CPU oracle for the FP8 path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package.
``fp8_oracle`` is the numpy/torch-CPU restatement; ``c_oracle()`` loads the C restatement of
the cast (``fp8_cast.c``) built by ``oracle/Makefile``.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
C_LIB = ORACLE_DIR / "_build" / "libfp8oracle.so"

_c = None


def build_c() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return C_LIB


def c_oracle() -> ctypes.CDLL:
    global _c
    if _c is None:
        if not C_LIB.exists():
            build_c()
        lib = ctypes.CDLL(str(C_LIB))
        lib.oracle_e4m3_rne.restype = ctypes.c_uint8
        lib.oracle_e4m3_rne.argtypes = [ctypes.c_float]
        lib.oracle_e4m3_rne_array.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_e4m3_rne_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        lib.oracle_scale_from_amax.restype = ctypes.c_float
        lib.oracle_scale_from_amax.argtypes = [ctypes.c_float]
        lib.oracle_cast.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p]
        lib.oracle_quantize.restype = ctypes.c_float
        lib.oracle_quantize.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_cast_digest.restype = ctypes.c_uint64
        lib.oracle_cast_digest.argtypes = [ctypes.c_float]
        lib.oracle_cast_digests.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int]
        _c = lib
    return _c
