"""Shared driver for the external-executable contract of ``backend: native``.

One subprocess per case; its JSON line becomes a record. Failure handling is
the reference's (src/teamredbench/benchmarks/hbm.py:59-157, mfu.py:42-166):
a build failure skips every case with the compiler error; a non-zero exit,
invalid JSON, ``status != "ok"`` or a missing ``elapsed_s`` skips that case.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Any, Callable

from teamredbench_amd.benchmarks.base import Benchmark, BenchmarkRecord
from teamredbench_amd.native.runtime import (
    NativeKernelError,
    ResolvedNativeKernel,
    prepare_native_kernel_binary,
    run_native_kernel,
)


@dataclass
class ExecutableCase:
    case: str
    dtype: str
    metadata: dict[str, Any]
    argv: list[str] | None  # None: skip with `skip_error`
    defaults: Callable[[dict[str, Any]], None]  # fills moved_bytes / achieved_ops / peaks
    skip_error: str | None = None


def run_executable_cases(bench: Benchmark, kernel: ResolvedNativeKernel, cases: list[ExecutableCase]) -> list[BenchmarkRecord]:
    try:
        kernel = replace(kernel, binary_path=prepare_native_kernel_binary(kernel))
    except NativeKernelError as exc:
        return [bench.skip(case=c.case, dtype=c.dtype, error=str(exc), metadata=c.metadata) for c in cases]

    records: list[BenchmarkRecord] = []
    for c in cases:
        if c.argv is None:
            records.append(bench.skip(case=c.case, dtype=c.dtype, error=c.skip_error or "skipped", metadata=c.metadata))
            continue
        try:
            result = run_native_kernel(kernel, c.argv)
        except NativeKernelError as exc:
            records.append(bench.skip(case=c.case, dtype=c.dtype, error=str(exc), metadata=c.metadata))
            continue
        metadata = {**c.metadata, **result.metadata}
        if result.status != "ok":
            records.append(
                bench.skip(
                    case=c.case,
                    dtype=c.dtype,
                    error=result.error or "Native kernel did not report success.",
                    metadata=metadata,
                )
            )
            continue
        raw = dict(result.raw_metrics)
        raw.setdefault("elapsed_s", raw.get("elapsed_seconds"))
        if raw.get("elapsed_s") is None:
            records.append(
                bench.skip(case=c.case, dtype=c.dtype, error="Native kernel did not report elapsed_s.", metadata=metadata)
            )
            continue
        c.defaults(raw)
        records.append(
            bench.emit_record(
                BenchmarkRecord(benchmark=bench.name, case=c.case, dtype=c.dtype, raw_metrics=raw, metadata=metadata)
            )
        )
    return records
