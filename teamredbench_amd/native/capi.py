"""ctypes binding of libmi355bench.so (C ABI in include/mi355bench.h).

This is the in-process replacement of the reference's executable contract
(argv in, one JSON line out; src/teamredbench/native/runtime.py:249-291).
Tensors are passed as raw device pointers (``tensor.data_ptr()``) together
with the HIP stream torch is using, so torch owns every allocation and the
library only enqueues kernels.

Loading never falls back to anything else: if the shared library is missing
or was built from other sources, :func:`load_library` raises
:class:`NativeLibraryError`, and callers surface that as the error of a
skipped record, the way the reference surfaces a failed hipcc build
(src/teamredbench/benchmarks/hbm.py:59-81).
"""
from __future__ import annotations

import contextlib
import ctypes
from dataclasses import dataclass
import json
import os
from pathlib import Path
import threading
from typing import Any, Iterator

from teamredbench_amd.native import build as _build

MB_OK = 0
MB_ERR_INVALID_ARG = -1
MB_ERR_UNSUPPORTED = -2
MB_ERR_SHAPE = -3
MB_ERR_WORKSPACE = -4
MB_ERR_DEVICE = -5

NOALLOC_SCRATCH_BYTES = 64 << 20   # MB_NOALLOC_SCRATCH_BYTES
CLOCK_BLOCKS = 1024                # MB_CLOCK_BLOCKS
CLOCK_REALTIME_HZ = 100_000_000    # MB_CLOCK_REALTIME_HZ
# MFMA ceiling instructions (MB_MFMA_*): name -> (code, FLOP per wave instruction, peak-table dtype)
MFMA_INSTRUCTIONS = {
    "v_mfma_f32_32x32x16_bf16": (0, 32768, "bfloat16"),
    "v_mfma_f32_16x16x32_bf16": (1, 16384, "bfloat16"),
    "v_mfma_scale_f32_32x32x64_f8f6f4": (2, 131072, "float8_e4m3fn"),
    "v_mfma_scale_f32_16x16x128_f8f6f4": (3, 65536, "float8_e4m3fn"),
    "v_mfma_f32_32x32x2_f32": (4, 4096, "float32"),
}
MFMA_CEILING_OPERAND_BYTES = 8192   # MB_MFMA_CEILING_OPERAND_BYTES
MFMA_CEILING_CHAINS = 8

OP_COPY, OP_SCALE, OP_TRIAD = 0, 1, 2
OPS = {"copy": OP_COPY, "scale": OP_SCALE, "triad": OP_TRIAD}

DT_FLOAT32, DT_BFLOAT16, DT_FLOAT16, DT_FLOAT64, DT_INT8, DT_FLOAT8_E4M3FN, DT_FLOAT8_E5M2 = 0, 1, 2, 3, 4, 5, 6
DTYPES = {
    "float32": DT_FLOAT32,
    "bfloat16": DT_BFLOAT16,
    "float16": DT_FLOAT16,
    "float64": DT_FLOAT64,
    "int8": DT_INT8,
    "float8_e4m3fn": DT_FLOAT8_E4M3FN,
    "float8_e5m2": DT_FLOAT8_E5M2,
}
STREAM_DTYPES = ("float32", "bfloat16", "float16", "float64", "int8")
GEMM_DTYPES = ("bfloat16", "float16", "float8_e4m3fn", "float8_e5m2", "float32", "float64")
FP8_DTYPES = ("float8_e4m3fn", "float8_e5m2")
# C's element type per GEMM input type: fp8 inputs produce bf16, the others their own type.
GEMM_OUTPUT_DTYPES = {"bfloat16": "bfloat16", "float16": "float16", "float8_e4m3fn": "bfloat16",
                      "float8_e5m2": "bfloat16", "float32": "float32", "float64": "float64"}

KIND_STREAM, KIND_GEMM = 0, 1

# Plan overrides (mb_set_tuning); names follow the "overrides" keys of mb_kernel_info.
TUNING_KNOBS = {
    "stream_unroll": 0,
    "stream_nontemporal": 1,
    "stream_threads": 2,
    "stream_schedule": 3,
    "gemm_force_generic": 4,
    "gemm_no_small_m": 5,
    "gemm_tiled_config": 6,
    "gemm_splits": 7,
    "gemm_fp8_mfma": 8,
    "gemm_highp_staged": 9,
}

# Every symbol include/mi355bench.h declares, with (restype, argtypes).
_u64, _i64, _vp, _cvp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "mb_abi_version": (ctypes.c_int, []),
    "mb_last_error": (ctypes.c_char_p, []),
    "mb_stream": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, _vp, _cvp, _cvp, _u64, ctypes.c_double, ctypes.c_int, _vp],
    ),
    "mb_time_stream": (
        ctypes.c_int,
        [
            ctypes.c_int, ctypes.c_int, _vp, _cvp, _cvp, _u64, ctypes.c_double, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_double),
        ],
    ),
    "mb_gemm": (
        ctypes.c_int,
        [
            ctypes.c_int, _cvp, _cvp, _vp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float, _vp,
            ctypes.c_size_t, _vp,
        ],
    ),
    "mb_gemm_workspace_size": (ctypes.c_size_t, [ctypes.c_int, _i64, _i64, _i64]),
    "mb_gemm_noalloc": (
        ctypes.c_int,
        [ctypes.c_int, _cvp, _cvp, _vp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float, _vp],
    ),
    "mb_time_gemm": (
        ctypes.c_int,
        [
            ctypes.c_int, _cvp, _cvp, _vp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float, _vp,
            ctypes.c_size_t, ctypes.c_int, ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_double),
        ],
    ),
    "mb_time_gemm_rotating": (
        ctypes.c_int,
        [
            ctypes.c_int, ctypes.POINTER(_cvp), ctypes.POINTER(_cvp), ctypes.POINTER(_vp), ctypes.c_int, _i64, _i64,
            _i64, ctypes.c_float, ctypes.c_float, _vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, _vp,
            ctypes.POINTER(ctypes.c_double),
        ],
    ),
    "mb_kernel_info": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64, _i64, _i64, ctypes.c_char_p, ctypes.c_size_t],
    ),
    "mb_set_tuning": (ctypes.c_int, [ctypes.c_int, _i64]),
    "mb_clock_stamp": (ctypes.c_int, [_vp, _vp]),
    "mb_mfma_ceiling": (
        ctypes.c_int,
        [ctypes.c_int, _cvp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp,
         ctypes.POINTER(ctypes.c_double)],
    ),
    "mb_get_tuning": (_i64, [ctypes.c_int]),
}

ABI_VERSION = 3


class NativeLibraryError(RuntimeError):
    """The shared library is missing, stale, or a call into it failed."""

    def __init__(self, message: str, status: int | None = None):
        super().__init__(message)
        self.status = status


@dataclass
class NativeLibrary:
    path: Path
    handle: ctypes.CDLL

    # ---- helpers -----------------------------------------------------------
    def _check(self, status: int, what: str) -> None:
        if status != MB_OK:
            detail = (self.handle.mb_last_error() or b"").decode("utf-8", "replace")
            raise NativeLibraryError(f"{what} failed with status {status}: {detail}", status)

    # ---- stream ------------------------------------------------------------
    def stream(self, op: int, dtype: int, dst: int, b: int, c: int | None, n: int, s: float,
               blocks_per_cu: int = 0, stream: int | None = None) -> None:
        status = self.handle.mb_stream(op, dtype, dst, b, c or None, n, float(s), int(blocks_per_cu), stream or None)
        self._check(status, "mb_stream")

    def time_stream(self, op: int, dtype: int, dst: int, b: int, c: int | None, n: int, s: float,
                    blocks_per_cu: int, warmup: int, iterations: int, stream: int | None = None) -> float:
        out = ctypes.c_double(0.0)
        status = self.handle.mb_time_stream(
            op, dtype, dst, b, c or None, n, float(s), int(blocks_per_cu), int(warmup), int(iterations),
            stream or None, ctypes.byref(out),
        )
        self._check(status, "mb_time_stream")
        return out.value

    # ---- gemm --------------------------------------------------------------
    def gemm_workspace_size(self, dtype: int, m: int, n: int, k: int) -> int:
        return int(self.handle.mb_gemm_workspace_size(dtype, m, n, k))

    def gemm(self, dtype: int, a: int, b: int, c: int, m: int, n: int, k: int, scale_a: float = 1.0,
             scale_b: float = 1.0, workspace: int | None = None, workspace_bytes: int = 0,
             stream: int | None = None) -> None:
        status = self.handle.mb_gemm(
            dtype, a, b, c, m, n, k, float(scale_a), float(scale_b), workspace or None, int(workspace_bytes),
            stream or None,
        )
        self._check(status, "mb_gemm")

    def gemm_noalloc(self, dtype: int, a: int, b: int, c: int, m: int, n: int, k: int, scale_a: float = 1.0,
                     scale_b: float = 1.0, stream: int | None = None) -> None:
        """mb_gemm with the library's own per-GPU scratch array instead of a workspace argument."""
        status = self.handle.mb_gemm_noalloc(dtype, a, b, c, m, n, k, float(scale_a), float(scale_b),
                                             stream or None)
        self._check(status, "mb_gemm_noalloc")

    def time_gemm(self, dtype: int, a: int, b: int, c: int, m: int, n: int, k: int, scale_a: float,
                  scale_b: float, workspace: int | None, workspace_bytes: int, warmup: int, iterations: int,
                  stream: int | None = None) -> float:
        out = ctypes.c_double(0.0)
        status = self.handle.mb_time_gemm(
            dtype, a, b, c, m, n, k, float(scale_a), float(scale_b), workspace or None, int(workspace_bytes),
            int(warmup), int(iterations), stream or None, ctypes.byref(out),
        )
        self._check(status, "mb_time_gemm")
        return out.value

    def time_gemm_rotating(self, dtype: int, a: list[int], b: list[int], c: list[int], m: int, n: int, k: int,
                           scale_a: float, scale_b: float, workspace: int | None, workspace_bytes: int, warmup: int,
                           iterations: int, stream: int | None = None) -> float:
        """mb_time_gemm cycling over len(a) operand sets (a[i], b[i] -> c[i])."""
        sets = len(a)
        if not sets or len(b) != sets or len(c) != sets:
            raise ValueError("operand lists must be non-empty and of equal length")
        arrays = [(ctypes.c_void_p * sets)(*ptrs) for ptrs in (a, b, c)]
        out = ctypes.c_double(0.0)
        status = self.handle.mb_time_gemm_rotating(
            dtype, *arrays[:3], sets, m, n, k, float(scale_a), float(scale_b), workspace or None,
            int(workspace_bytes), int(warmup), int(iterations), stream or None, ctypes.byref(out),
        )
        self._check(status, "mb_time_gemm_rotating")
        return out.value

    # ---- metadata ----------------------------------------------------------
    def kernel_info(self, kind: int, a: int, b: int, m: int, n: int, k: int) -> dict[str, Any]:
        buf = ctypes.create_string_buffer(4096)
        status = self.handle.mb_kernel_info(kind, a, b, m, n, k, buf, len(buf))
        self._check(status, "mb_kernel_info")
        return json.loads(buf.value.decode("utf-8"))

    def stream_info(self, op: int, dtype: int, n: int, blocks_per_cu: int = 0) -> dict[str, Any]:
        return self.kernel_info(KIND_STREAM, op, dtype, n, blocks_per_cu, 0)

    def gemm_info(self, dtype: int, m: int, n: int, k: int) -> dict[str, Any]:
        return self.kernel_info(KIND_GEMM, dtype, 0, m, n, k)

    # ---- clock stamps ------------------------------------------------------
    def clock_stamp(self, out: int, stream: int | None = None) -> None:
        """Enqueue one stamp (4 * CLOCK_BLOCKS uint64 at device address `out`): see mb_clock_stamp."""
        self._check(self.handle.mb_clock_stamp(out, stream or None), "mb_clock_stamp")

    def mfma_ceiling(self, instruction: int, operands: int, out: int, blocks: int, iterations: int, warmup: int,
                     launches: int, stream: int | None = None) -> float:
        """Seconds per launch of the MFMA-only kernel (see mb_mfma_ceiling)."""
        elapsed = ctypes.c_double(0.0)
        status = self.handle.mb_mfma_ceiling(int(instruction), operands, out, int(blocks), int(iterations), int(warmup),
                                             int(launches), stream or None, ctypes.byref(elapsed))
        self._check(status, "mb_mfma_ceiling")
        return elapsed.value

    # ---- plan overrides ----------------------------------------------------
    def set_tuning(self, knob: str, value: int | None) -> None:
        """Force a plan knob (see TUNING_KNOBS), or restore the library's choice with None."""
        status = self.handle.mb_set_tuning(TUNING_KNOBS[knob], -1 if value is None else int(value))
        self._check(status, f"mb_set_tuning({knob}={value})")

    def get_tuning(self, knob: str) -> int | None:
        value = int(self.handle.mb_get_tuning(TUNING_KNOBS[knob]))
        return None if value < 0 else value

    @contextlib.contextmanager
    def tuned(self, **knobs: int | None) -> Iterator[None]:
        """Hold the given knobs for the duration of a block, then restore what they held."""
        saved = {name: self.get_tuning(name) for name in knobs}
        try:
            for name, value in knobs.items():
                self.set_tuning(name, value)
            yield
        finally:
            for name, value in saved.items():
                self.set_tuning(name, value)


_lock = threading.Lock()
_cache: dict[Path, NativeLibrary] = {}


def library_path() -> Path:
    override = os.environ.get("MI355BENCH_LIBRARY")
    return Path(override).resolve() if override else _build.library_path()


def bind(handle: ctypes.CDLL) -> None:
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes


def load_library(path: str | Path | None = None, *, check_digest: bool = True) -> NativeLibrary:
    """Load (once per path) and bind libmi355bench.so.

    Raises NativeLibraryError when the file is absent, was built from sources
    other than the ones in this tree (BUILD_DIGEST mismatch), or exports a
    different ABI version.
    """
    lib_path = Path(path).resolve() if path else library_path()
    with _lock:
        if lib_path in _cache:
            return _cache[lib_path]
        if not lib_path.exists():
            raise NativeLibraryError(
                f"{lib_path} is not built; run `python -m teamredbench_amd.native.build` "
                "(or __graft_entry__.build())"
            )
        if check_digest and path is None and os.environ.get("MI355BENCH_LIBRARY") is None:
            stamp = lib_path.parent / "BUILD_DIGEST"
            recorded = stamp.read_text(encoding="utf-8").strip() if stamp.exists() else ""
            if recorded != _build.source_digest():
                raise NativeLibraryError(
                    f"{lib_path} was built from different sources than teamredbench_amd/csrc; rebuild it"
                )
        try:
            handle = ctypes.CDLL(str(lib_path))
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {lib_path}: {exc}") from exc
        bind(handle)
        version = handle.mb_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"{lib_path} has ABI version {version}, expected {ABI_VERSION}")
        lib = NativeLibrary(path=lib_path, handle=handle)
        _cache[lib_path] = lib
        return lib
