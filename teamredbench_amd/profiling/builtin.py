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
                  counter-derived GB/s = (fetch + write bytes) / duration, with
                  FETCH_SIZE and WRITE_SIZE (KiB per dispatch) each scaled by a
                  calibration factor: every pass that collects one of them is
                  also run once over a plain copy kernel of known traffic
                  (teamredbench_amd.profiling.stream_probe --ops copy), and the
                  factor makes that copy's reading equal its known bytes (on
                  MI355X FETCH_SIZE reads half the bytes moved)
  GEMM kernels:   mfma_busy_pct = SQ_VALU_MFMA_BUSY_CYCLES /
                  (GRBM_GUI_ACTIVE / XCDs * CUs * 4 SIMDs); GRBM_GUI_ACTIVE is
                  summed over the XCDs

Params (suite ``profiling.params``): binary (default rocprofv3), stats
(bool, default true), kernel_include_regex, counter_passes (list of counter
lists; default the three passes above; [] disables counters), hip_trace,
hsa_trace, marker_trace, sys_trace (bools; only on the trace pass, never
beside counters), truncate_kernels (bool), calibrate (bool, default true),
extra_args, env.

The engine is registered as ``rocprofv3`` and, for suites written for the
reference, as ``rocprof``. The ``rocprof`` name takes the reference engine's
v1 parameters (src/teamredbench/profiling/builtin.py:37-143) and translates
each one that rocprofv3 can honour (:func:`translate_v1_params`); a suite
that sets one it cannot honour fails with an error naming every such
parameter, instead of running without what it asked for.
"""
from __future__ import annotations

import csv
import json
import os
from pathlib import Path
import shutil
from statistics import mean
import sys
from typing import Any

from teamredbench_amd.profiling.registry import ProfilingLaunch, register_profile_engine

DEFAULT_COUNTER_PASSES = [["FETCH_SIZE"], ["WRITE_SIZE"], ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]]
# API-trace domains: added to the kernel-trace pass only. No counter pass ever carries them (a counter
# collection combined with an API trace in one profiler run is not supported on this platform).
TRACE_ONLY_FLAGS = {"hip_trace": "--hip-trace", "hsa_trace": "--hsa-trace", "marker_trace": "--marker-trace",
                    "sys_trace": "--sys-trace"}
SIMDS_PER_CU = 4
CALIBRATION_ELEMENTS = 1 << 26          # fp32 copy: reads and writes 256 MiB
CALIBRATION_KERNEL = "stream_vec_kernel<0, "  # the library's copy kernel


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
    for key, flag in TRACE_ONLY_FLAGS.items():
        if params.get(key):
            trace.append(flag)
    if params.get("truncate_kernels"):
        trace.append("--truncate-kernels")
    trace += _common(params) + ["--"]

    passes = params.get("counter_passes", DEFAULT_COUNTER_PASSES)
    if not isinstance(passes, list) or not all(isinstance(p, list) for p in passes):
        raise ValueError("profiling.params.counter_passes must be a list of counter lists.")
    extra = tuple(
        tuple([binary, "--pmc", *map(str, group), "-d", str(artifact_dir / f"pmc{i + 1}"), "-o", "run",
               *_common(params), "--"])
        for i, group in enumerate(passes)
    )
    standalone: list[tuple[str, ...]] = []
    if params.get("calibrate", True):
        for i, group in enumerate(passes):
            if not {"FETCH_SIZE", "WRITE_SIZE"} & set(map(str, group)):
                continue
            standalone.append(tuple([
                binary, "--pmc", *map(str, group), "-d", str(artifact_dir / f"cal{i + 1}"), "-o", "run", "-f", "csv",
                "--", sys.executable, "-m", "teamredbench_amd.profiling.stream_probe", "--ops", "copy",
                "--elements", str(CALIBRATION_ELEMENTS), "--launches", "3",
            ]))
        (artifact_dir / "calibration.json").write_text(json.dumps({
            "kernel": CALIBRATION_KERNEL, "read_bytes": 4 * CALIBRATION_ELEMENTS,
            "write_bytes": 4 * CALIBRATION_ELEMENTS}), encoding="utf-8")
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
        standalone_passes=tuple(standalone),
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


def parse_counter_durations(pmc_dir: Path) -> dict[str, float]:
    """kernel name -> mean dispatch duration (ns) of a counter-collection run,
    from the Start/End timestamps rocprofv3 records with every counter row."""
    spans: dict[tuple[str, str], int] = {}
    for row in _rows(sorted(pmc_dir.rglob("*counter_collection.csv"))):
        try:
            span = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
        except (KeyError, ValueError):
            continue
        spans[(_kernel_name(row), row.get("Dispatch_Id", "?"))] = span
    grouped: dict[str, list[int]] = {}
    for (kernel, _), span in spans.items():
        grouped.setdefault(kernel, []).append(span)
    return {k: mean(v) for k, v in grouped.items()}


def calibration_factors(artifact_dir: Path) -> dict[str, float]:
    """FETCH_SIZE / WRITE_SIZE scale factors from the calibration passes:
    known bytes of the copy kernel / (counter KiB * 1024)."""
    spec_path = artifact_dir / "calibration.json"
    if not spec_path.exists():
        return {}
    spec = json.loads(spec_path.read_text(encoding="utf-8"))
    factors: dict[str, float] = {}
    for cal_dir in sorted(artifact_dir.glob("cal*")):
        for kernel, values in parse_counters(cal_dir).items():
            if spec["kernel"] not in kernel:
                continue
            if values.get("FETCH_SIZE"):
                factors["FETCH_SIZE"] = spec["read_bytes"] / (values["FETCH_SIZE"] * 1024.0)
            if values.get("WRITE_SIZE"):
                factors["WRITE_SIZE"] = spec["write_bytes"] / (values["WRITE_SIZE"] * 1024.0)
    return factors


def collect(artifact_dir: Path, cu_count: int | None = None, xcd_count: int | None = None) -> dict[str, Any]:
    """Per-kernel summary from a rocprofv3 artifact directory (trace + pmc passes)."""
    kernels = parse_kernel_trace(artifact_dir / "trace") if (artifact_dir / "trace").exists() else {}
    counters: dict[str, dict[str, float]] = {}
    gui_durations: dict[str, float] = {}   # durations of the runs that read GRBM_GUI_ACTIVE
    for pmc_dir in sorted(artifact_dir.glob("pmc*")):
        parsed = parse_counters(pmc_dir)
        durations = parse_counter_durations(pmc_dir)
        for kernel, values in parsed.items():
            counters.setdefault(kernel, {}).update(values)
            if "GRBM_GUI_ACTIVE" in values and kernel in durations:
                gui_durations[kernel] = durations[kernel]
    cus = cu_count or int(os.environ.get("MB_CU_COUNT", "256"))
    xcds = xcd_count or int(os.environ.get("MB_XCD_COUNT", "8"))
    factors = calibration_factors(artifact_dir)
    summary: dict[str, Any] = {"_calibration": factors} if factors else {}
    for name in sorted(set(kernels) | set(counters)):
        entry: dict[str, Any] = dict(kernels.get(name, {}))
        values = counters.get(name, {})
        entry["counters"] = values
        duration = entry.get("avg_duration_ns")
        fetch = write = None
        if "FETCH_SIZE" in values:
            fetch = values["FETCH_SIZE"] * 1024.0 * factors.get("FETCH_SIZE", 1.0)
            entry["dram_fetch_bytes"] = fetch
        if "WRITE_SIZE" in values:
            write = values["WRITE_SIZE"] * 1024.0 * factors.get("WRITE_SIZE", 1.0)
            entry["dram_write_bytes"] = write
        if factors:
            entry["calibrated"] = True
        if duration and fetch is not None and write is not None:
            entry["dram_gbps"] = (fetch + write) / duration
        if values.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in values:
            per_xcd = values["GRBM_GUI_ACTIVE"] / xcds
            entry["mfma_busy_pct"] = 100.0 * values["SQ_VALU_MFMA_BUSY_CYCLES"] / (per_xcd * cus * SIMDS_PER_CU)
            # the clock comes from the same run as the cycle count when that
            # run recorded timestamps, else from the trace run
            clock_span = gui_durations.get(name) or duration
            if clock_span:
                entry["clock_ghz"] = per_xcd / clock_span
        summary[name] = entry
    return summary


register_profile_engine(
    name="rocprofv3",
    description="Profile a run with rocprofv3: kernel trace plus FETCH/WRITE_SIZE and MFMA-busy counter passes.",
    build_command=_build_rocprofv3_command,
)
# ---------------------------------------------------------------- the reference's v1 parameters
# What the `rocprof` name does with each parameter of the reference's engine
# (src/teamredbench/profiling/builtin.py:37-143) that has no rocprofv3 counterpart here: the reason it is
# refused.
V1_REFUSED = {
    "tool_version": "selects between rocprof v1 and v2; this engine always drives rocprofv3",
    "metric_file": "names a v1 derived-metric XML file, which rocprofv3 does not read",
    "output": "names the v1 CSV file; rocprofv3 writes its CSVs under the run's artifact directory "
              "(outputs.profiling in the sidecar)",
    "data_dir": "names the v1 data directory; the artifact directory holds rocprofv3's data",
    "temporary_dir": "names the v1 temporary directory, which rocprofv3 does not use",
    "cmd_qts": "is a v1 toggle with no rocprofv3 option",
    "ctx_wait": "is a v1 toggle with no rocprofv3 option",
    "obj_tracking": "is a v1 toggle with no rocprofv3 option",
    "trace_start": "is a v1 toggle with no rocprofv3 option",
    "ctx_limit": "is a v1 option with no rocprofv3 counterpart",
    "heartbeat": "is a v1 option with no rocprofv3 counterpart",
    "trace_period": "is a v1 option with no rocprofv3 counterpart",
    "flush_rate": "is a v1 option with no rocprofv3 counterpart",
    "roctx_rename": "is a v1 flag with no rocprofv3 counterpart",
    "parallel_kernels": "is a v1 flag with no rocprofv3 counterpart",
}
V1_BINARIES = ("rocprof", "rocprofv2")


def read_v1_input(path: Path) -> tuple[list[list[str]], list[str], list[str]]:
    """A rocprof v1 counter input file: each ``pmc:`` line is one pass of counters (separated by spaces or
    commas), each ``kernel:`` line adds kernel names to profile; returns (passes, kernels, refused
    directives). ``#`` starts a comment."""
    passes: list[list[str]] = []
    kernels: list[str] = []
    refused: list[str] = []
    for raw in path.read_text(encoding="utf-8").splitlines():
        line = raw.split("#", 1)[0].strip()
        if not line:
            continue
        key, sep, rest = line.partition(":")
        names = [x for x in rest.replace(",", " ").split() if x]
        key = key.strip().lower()
        if sep and key == "pmc" and names:
            passes.append(names)
        elif sep and key == "kernel" and names:
            kernels += names
        else:
            refused.append(line)
    return passes, kernels, refused


def translate_v1_params(params: dict[str, Any], base_dir: Path | None) -> dict[str, Any]:
    """The rocprofv3 engine's params for a suite written for the reference's rocprof (v1) engine.

    Translated: stats, hip_trace, hsa_trace, sys_trace (same meaning, on the kernel-trace pass),
    roctx_trace (-> marker_trace), basenames on (-> truncate_kernels), timestamp on (rocprofv3 always
    records timestamps), input (a v1 counter file: its ``pmc:`` lines become the counter passes and its
    ``kernel:`` lines the kernel filter), binary (unless it names the v1/v2 tool), env, extra_args (handed
    to rocprofv3 as they are). Every other v1 parameter, and timestamp / basenames off, raises ValueError
    naming each one and why."""
    out: dict[str, Any] = {}
    errors: list[str] = []
    for key, value in params.items():
        if key in V1_REFUSED:
            errors.append(f"{key} {V1_REFUSED[key]}")
        elif key == "roctx_trace":
            out["marker_trace"] = bool(value)
        elif key == "basenames":
            if bool(value):
                out["truncate_kernels"] = True
        elif key == "timestamp":
            if not bool(value):
                errors.append("timestamp: off cannot be honoured; rocprofv3 always records kernel timestamps")
        elif key == "binary" and Path(str(value)).name in V1_BINARIES:
            errors.append(f"binary {value!r} is the v1/v2 profiler, whose flags differ; name rocprofv3 or leave "
                          "binary out")
        elif key == "input":
            path = _resolve(base_dir, str(value))
            try:
                passes, kernels, refused = read_v1_input(path)
            except OSError as exc:
                errors.append(f"input {str(path)!r} cannot be read: {exc}")
                continue
            for line in refused:
                errors.append(f"input {path.name}: {line!r} is not a pmc: or kernel: line")
            if passes:
                out["counter_passes"] = passes
            if kernels:
                out["kernel_include_regex"] = "|".join(kernels)
        else:
            out[key] = value
    if errors:
        raise ValueError("profiling.params for the rocprof engine: " + "; ".join(errors))
    return out


def _build_rocprof_v1_command(params: dict[str, Any], target_command: list[str], artifact_dir: Path,
                              base_dir: Path | None) -> ProfilingLaunch:
    return _build_rocprofv3_command(translate_v1_params(params, base_dir), target_command, artifact_dir, base_dir)


register_profile_engine(
    name="rocprof",
    description="rocprofv3, taking the reference rocprof engine's v1 parameters (translated, or refused by name).",
    build_command=_build_rocprof_v1_command,
)
