"""ORACLE -- ctypes binding of oracle/liboracle.so (test infrastructure).

Functions mirror stream_oracle.c and parity_inputs.cpp. Buffers are numpy
arrays on the host; nothing here touches a GPU.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
import subprocess

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile liboracle.so with gcc/g++ (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "all"], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, u64, i64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int64
        lib.oracle_stream.restype = ctypes.c_int
        lib.oracle_stream.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp, u64, ctypes.c_double]
        for name in ("oracle_decode_bf16", "oracle_encode_bf16", "oracle_decode_f16", "oracle_encode_f16",
                     "oracle_decode_e4m3", "oracle_decode_e5m2"):
            fn = getattr(lib, name)
            fn.restype = None
            fn.argtypes = [vp, vp, u64]
        lib.oracle_gemm_f64.restype = None
        lib.oracle_gemm_f64.argtypes = [vp, vp, vp, i64, i64, i64]
        lib.oracle_fill_uniform_mt19937.restype = None
        lib.oracle_fill_uniform_mt19937.argtypes = [vp, u64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        _lib = lib
    return _lib


OPS = {"copy": 0, "scale": 1, "triad": 2}
DTYPES = {"float32": 0, "bfloat16": 1, "float16": 2, "float64": 3, "int8": 4}
NP_STORAGE = {"float32": np.float32, "bfloat16": np.uint16, "float16": np.uint16, "float64": np.float64,
              "int8": np.int8}


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def stream(mode: str, dtype: str, b: np.ndarray, c: np.ndarray | None, s: float) -> np.ndarray:
    """Oracle stream op on host arrays of the storage type (uint16 bits for bf16/f16)."""
    b = np.ascontiguousarray(b)
    dst = np.empty_like(b)
    cc = np.ascontiguousarray(c) if c is not None else None
    rc = load().oracle_stream(OPS[mode], DTYPES[dtype], _ptr(dst), _ptr(b), _ptr(cc) if cc is not None else None,
                              b.size, float(s))
    if rc != 0:
        raise ValueError(f"oracle_stream does not support {mode}/{dtype}")
    return dst


def decode_bf16(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    load().oracle_decode_bf16(_ptr(bits), _ptr(out), bits.size)
    return out


def encode_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().oracle_encode_bf16(_ptr(x), _ptr(out), x.size)
    return out


def decode_f16(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    load().oracle_decode_f16(_ptr(bits), _ptr(out), bits.size)
    return out


def encode_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().oracle_encode_f16(_ptr(x), _ptr(out), x.size)
    return out


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.shape, dtype=np.float32)
    load().oracle_decode_e4m3(_ptr(codes), _ptr(out), codes.size)
    return out


def decode_e5m2(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.shape, dtype=np.float32)
    load().oracle_decode_e5m2(_ptr(codes), _ptr(out), codes.size)
    return out


def gemm_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("inner dimensions differ")
    out = np.empty((m, n), dtype=np.float64)
    load().oracle_gemm_f64(_ptr(a), _ptr(b), _ptr(out), m, n, k)
    return out


def fill_uniform_mt19937(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().oracle_fill_uniform_mt19937(_ptr(out), n, seed, lo, hi)
    return out
