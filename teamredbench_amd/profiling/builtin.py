"""Built-in profile engine: rocprofv3 with hardware-counter evidence.

Replaces the reference's rocprof (v1) flag builder
(src/teamredbench/profiling/builtin.py:37-150), which only recorded an
artifact directory. Here the suite runs once under
``rocprofv3 --kernel-trace [--stats]`` (records kept, per-kernel durations)
and then once per counter group under ``rocprofv3 --pmc ...`` (a pass holds
only counters that fit the hardware together: FETCH_SIZE and WRITE_SIZE go
in separate passes). :func:`collect` parses the CSV artifacts into a
per-kernel summary attached to the metadata sidecar:

  stream kernels: dram_fetch_bytes / dram_write_bytes per dispatch and the
                  counter-derived GB/s = (FETCH_SIZE + WRITE_SIZE) * 1024 / duration
  GEMM kernels:   mfma_busy_pct = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * CUs * 4)

Params (suite ``profiling.params``): binary (default rocprofv3), stats
(bool, default true), kernel_include_regex, counter_passes (list of counter
lists; default the three passes above; [] disables counters), hip_trace
(bool; only on the trace pass), extra_args, env.
The engine is registered as ``rocprofv3`` and, for suites written for the
reference, as ``rocprof``.
"""
from __future__ import annotations

import csv
import os
from pathlib import Path
import shutil
from statistics import mean
from typing import Any

from teamredbench_amd.profiling.registry import ProfilingLaunch, register_profile_engine

DEFAULT_COUNTER_PASSES = [["FETCH_SIZE"], ["WRITE_SIZE"], ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]]
SIMDS_PER_CU = 4


def _resolve(base: Path | None, value: str) -> Path:
    p = Path(value)
    if p.is_absolute():
        return p
    return (base / p).resolve() if base is not None else p.resolve()


def _profiler_binary(params: dict[str, Any]) -> str:
    value = str(params.get("binary", "rocprofv3"))
    if Path(value).is_absolute():
        return value
    return shutil.which(value) or value


def _common(params: dict[str, Any]) -> list[str]:
    args: list[str] = ["-f", "csv"]
    if params.get("kernel_include_regex"):
        args += ["--kernel-include-regex", str(params["kernel_include_regex"])]
    extra = params.get("extra_args") or []
    if not isinstance(extra, list):
        raise ValueError("profiling.params.extra_args must be a list of strings.")
    return args + [str(x) for x in extra]


def _build_rocprofv3_command(params: dict[str, Any], target_command: list[str], artifact_dir: Path,
                             base_dir: Path | None) -> ProfilingLaunch:
    binary = _profiler_binary(params)
    artifact_dir.mkdir(parents=True, exist_ok=True)
    trace = [binary, "--kernel-trace", "-d", str(artifact_dir / "trace"), "-o", "run"]
    if params.get("stats", True):
        trace.append("--stats")
    if params.get("hip_trace"):
        trace.append("--hip-trace")
    trace += _common(params) + ["--"]

    passes = params.get("counter_passes", DEFAULT_COUNTER_PASSES)
    if not isinstance(passes, list) or not all(isinstance(p, list) for p in passes):
        raise ValueError("profiling.params.counter_passes must be a list of counter lists.")
    extra = tuple(
        tuple([binary, "--pmc", *map(str, group), "-d", str(artifact_dir / f"pmc{i + 1}"), "-o", "run",
               *_common(params), "--"])
        for i, group in enumerate(passes)
    )
    env: dict[str, str] = {}
    rocm_bin = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin"
    env["PATH"] = os.pathsep.join([str(rocm_bin), os.environ.get("PATH", "")])
    for key, value in (params.get("env") or {}).items():
        env[str(key)] = str(value)
    return ProfilingLaunch(
        command=tuple(trace + list(target_command)),
        artifact_dir=artifact_dir,
        env=env,
        metadata={"binary": binary, "counter_passes": passes, "trace_dir": str(artifact_dir / "trace")},
        extra_passes=extra,
        collect=collect,
    )


# ---------------------------------------------------------------- parsing
def _rows(paths: list[Path]) -> list[dict[str, str]]:
    rows: list[dict[str, str]] = []
    for path in paths:
        with path.open(newline="", encoding="utf-8", errors="replace") as handle:
            rows.extend(csv.DictReader(handle))
    return rows


def _kernel_name(row: dict[str, str]) -> str:
    return row.get("Kernel_Name") or row.get("KernelName") or row.get("Name") or "?"


def parse_kernel_trace(trace_dir: Path) -> dict[str, dict[str, Any]]:
    """kernel name -> {dispatches, avg_duration_ns, total_duration_ns}."""
    durations: dict[str, list[int]] = {}
    for row in _rows(sorted(trace_dir.rglob("*kernel_trace.csv"))):
        try:
            start, end = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
        except (KeyError, ValueError):
            continue
        durations.setdefault(_kernel_name(row), []).append(end - start)
    return {
        name: {"dispatches": len(d), "avg_duration_ns": mean(d), "total_duration_ns": sum(d)}
        for name, d in durations.items()
    }


def parse_counters(pmc_dir: Path) -> dict[str, dict[str, float]]:
    """kernel name -> counter name -> mean value per dispatch (summed over the
    dimensions rocprofv3 reports a counter in, within one dispatch)."""
    per_dispatch: dict[tuple[str, str, str], float] = {}
    for row in _rows(sorted(pmc_dir.rglob("*counter_collection.csv"))):
        try:
            value = float(row["Counter_Value"])
        except (KeyError, ValueError):
            continue
        key = (_kernel_name(row), row.get("Counter_Name", "?"), row.get("Dispatch_Id", "?"))
        per_dispatch[key] = per_dispatch.get(key, 0.0) + value
    grouped: dict[str, dict[str, list[float]]] = {}
    for (kernel, counter, _), value in per_dispatch.items():
        grouped.setdefault(kernel, {}).setdefault(counter, []).append(value)
    return {k: {c: mean(v) for c, v in counters.items()} for k, counters in grouped.items()}


def collect(artifact_dir: Path, cu_count: int | None = None) -> dict[str, Any]:
    """Per-kernel summary from a rocprofv3 artifact directory (trace + pmc passes)."""
    kernels = parse_kernel_trace(artifact_dir / "trace") if (artifact_dir / "trace").exists() else {}
    counters: dict[str, dict[str, float]] = {}
    for pmc_dir in sorted(artifact_dir.glob("pmc*")):
        for kernel, values in parse_counters(pmc_dir).items():
            counters.setdefault(kernel, {}).update(values)
    cus = cu_count or int(os.environ.get("MB_CU_COUNT", "256"))
    summary: dict[str, Any] = {}
    for name in sorted(set(kernels) | set(counters)):
        entry: dict[str, Any] = dict(kernels.get(name, {}))
        values = counters.get(name, {})
        entry["counters"] = values
        duration = entry.get("avg_duration_ns")
        if "FETCH_SIZE" in values:
            entry["dram_fetch_bytes"] = values["FETCH_SIZE"] * 1024.0
        if "WRITE_SIZE" in values:
            entry["dram_write_bytes"] = values["WRITE_SIZE"] * 1024.0
        if duration and "FETCH_SIZE" in values and "WRITE_SIZE" in values:
            entry["dram_gbps"] = (values["FETCH_SIZE"] + values["WRITE_SIZE"]) * 1024.0 / duration
        if values.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in values:
            entry["mfma_busy_pct"] = (
                100.0 * values["SQ_VALU_MFMA_BUSY_CYCLES"] / (values["GRBM_GUI_ACTIVE"] * cus * SIMDS_PER_CU)
            )
        summary[name] = entry
    return summary


register_profile_engine(
    name="rocprofv3",
    description="Profile a run with rocprofv3: kernel trace plus FETCH/WRITE_SIZE and MFMA-busy counter passes.",
    build_command=_build_rocprofv3_command,
)
register_profile_engine(
    name="rocprof",
    description="Alias of rocprofv3 for suites written for the reference's rocprof engine.",
    build_command=_build_rocprofv3_command,
)
