"""Profiled suite runs (behaviour of src/teamredbench/profiling/runtime.py:16-184).

The suite is re-executed as a child ``python -m teamredbench_amd run ...``
under the engine's profiler with ``TEAMREDBENCH_INTERNAL_RUN=1`` (so the
child does not recurse) and ``TEAMREDBENCH_FORCE_JSON_OUTPUT=1`` (so its
records can be reloaded). The parent reloads the child's records, then runs
the engine's extra counter passes (each writing results into its own
directory under the artifact dir), parses the artifacts with the engine's
``collect`` hook, and injects ``run.profiling`` -- including the parsed
counter summary -- into the child's metadata sidecar.
"""
from __future__ import annotations

from datetime import datetime, timezone
import json
import os
from pathlib import Path
import subprocess
import sys
from typing import Any

from teamredbench_amd.benchmarks.base import BenchmarkContext, BenchmarkRecord
from teamredbench_amd.config import ProfilingConfig, SuiteConfig
from teamredbench_amd.profiling.registry import get_profile_engine

INTERNAL_RUN_ENV = "TEAMREDBENCH_INTERNAL_RUN"
FORCE_JSON_OUTPUT_ENV = "TEAMREDBENCH_FORCE_JSON_OUTPUT"


class ProfilingError(RuntimeError):
    pass


def profiling_active() -> bool:
    return os.environ.get(INTERNAL_RUN_ENV) == "1"


def profiling_enabled(config: ProfilingConfig) -> bool:
    return bool(config.enabled and config.engine and not profiling_active())


def force_json_output_enabled() -> bool:
    return os.environ.get(FORCE_JSON_OUTPUT_ENV) == "1"


def effective_output_formats(formats: list[str]) -> list[str]:
    resolved = list(formats)
    if force_json_output_enabled() and "json" not in resolved:
        resolved.append("json")
    return resolved


def _artifact_dir(output_dir: Path, suite_name: str, engine_name: str) -> Path:
    stamp = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%SZ")
    return output_dir / "profiling" / f"{suite_name}-{engine_name}-{stamp}"


def _metadata_files(output_dir: Path, suite_name: str) -> set[Path]:
    return set(output_dir.glob(f"{suite_name}-*.metadata.json")) if output_dir.exists() else set()


def _record_from_dict(payload: dict[str, Any]) -> BenchmarkRecord:
    return BenchmarkRecord(
        benchmark=str(payload["benchmark"]),
        case=str(payload["case"]),
        dtype=str(payload["dtype"]),
        status=str(payload.get("status", "ok")),
        error=None if payload.get("error") is None else str(payload["error"]),
        metrics=dict(payload.get("metrics", {})),
        raw_metrics=dict(payload.get("raw_metrics", {})),
        metadata=dict(payload.get("metadata", {})),
    )


def child_command(suite_path: Path, device_id: int, output_dir: Path) -> list[str]:
    return [sys.executable, "-m", "teamredbench_amd", "run", str(suite_path), "--device-id", str(device_id),
            "--output-dir", str(output_dir), "--quiet-records"]


def _run(command: list[str], env: dict[str, str], what: str) -> None:
    proc = subprocess.run(command, check=False, capture_output=True, text=True, env=env)
    if proc.returncode != 0:
        detail = proc.stderr.strip() or proc.stdout.strip() or "unknown profiling failure"
        raise ProfilingError(f"{what} failed: {detail}")


def run_profiled_suite(*, suite: SuiteConfig, context: BenchmarkContext, output_dir: Path, device_id: int,
                       record_callback):
    from teamredbench_amd.runner import RunSummary

    if suite.path is None:
        raise ProfilingError("Suite path is required for profiled runs.")
    if not suite.profiling.engine:
        raise ProfilingError("Profiling is enabled but no engine is configured.")
    engine = get_profile_engine(suite.profiling.engine)
    artifact_dir = _artifact_dir(output_dir, suite.name, engine.name)
    launch = engine.build_command(dict(suite.profiling.params), child_command(suite.path, device_id, output_dir),
                                  artifact_dir, suite.path.parent)
    env = {**os.environ, INTERNAL_RUN_ENV: "1", FORCE_JSON_OUTPUT_ENV: "1", **launch.env}

    before = _metadata_files(output_dir, suite.name)
    _run(list(launch.command), env, f"Profile engine {engine.name}")
    created = sorted(_metadata_files(output_dir, suite.name) - before)
    if not created:
        raise ProfilingError("Profiled run completed but no metadata file was produced.")
    metadata_path = created[-1]
    payload = json.loads(metadata_path.read_text(encoding="utf-8"))
    json_path = payload.get("outputs", {}).get("json")
    if json_path is None or not Path(json_path).exists():
        raise ProfilingError("Profiled run did not produce a JSON results file.")
    records = [_record_from_dict(item) for item in json.loads(Path(json_path).read_text(encoding="utf-8"))]

    for index, prefix in enumerate(launch.extra_passes):
        pass_out = artifact_dir / f"pass{index + 1}-results"
        _run([*prefix, *child_command(suite.path, device_id, pass_out)], env, f"{engine.name} pass {index + 1}")
    for index, command in enumerate(launch.standalone_passes):
        _run(list(command), env, f"{engine.name} standalone pass {index + 1}")

    profiling: dict[str, Any] = {
        "enabled": True,
        "engine": engine.name,
        "artifact_dir": str(launch.artifact_dir),
        "command": list(launch.command),
        "extra_passes": [list(p) for p in launch.extra_passes],
        "standalone_passes": [list(p) for p in launch.standalone_passes],
        "engine_metadata": dict(launch.metadata),
    }
    if launch.collect is not None:
        try:
            profiling["counters"] = launch.collect(launch.artifact_dir)
        except Exception as exc:  # noqa: BLE001 -- a parse failure must not lose the records
            profiling["counters_error"] = f"{type(exc).__name__}: {exc}"
    payload.setdefault("outputs", {})["profiling"] = str(launch.artifact_dir)
    payload.setdefault("run", {})["profiling"] = profiling
    metadata_path.write_text(json.dumps(payload, indent=2), encoding="utf-8")

    outputs = {name: Path(p) for name, p in payload.get("outputs", {}).items()}
    run_metadata = dict(payload.get("run", {}))
    if record_callback is not None:
        for record in records:
            record_callback(record)
    return RunSummary(suite=suite, context=context, records=records, outputs=outputs, run_metadata=run_metadata,
                      profile_note=run_metadata.get("configs", {}).get("profile_note"))
