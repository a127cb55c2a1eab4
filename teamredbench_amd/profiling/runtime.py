"""Profiled suite runs.

A suite with ``profiling: {engine: <name>, params: {...}}`` is measured by
running the whole suite again in a child process under the engine's
profiler (the behaviour of src/teamredbench/profiling/runtime.py:93-184;
the two environment variables below are its names). :class:`ProfiledRun`
does it in steps:

  1. ``launch``   -- the engine wraps the child command
                     (``python -m teamredbench_amd run <suite> ...``); the
                     child gets ``TEAMREDBENCH_INTERNAL_RUN=1`` (so it does
                     not profile itself again), ``TEAMREDBENCH_FORCE_JSON_OUTPUT=1``
                     (so its records can be reloaded) and a run token;
  2. ``reload``   -- the child's sidecar is the one in the output directory
                     that carries that token (``run.run_token``), so runs
                     sharing a directory never pick up each other's files;
                     its JSON records become this run's records;
  3. ``passes``   -- further runs the engine asks for: the same child under
                     other counter groups (their records are discarded) and
                     standalone commands (a calibration workload);
  4. ``annotate`` -- the engine's ``collect`` hook parses the artifacts, and
                     ``run.profiling`` (engine, commands, artifacts and the
                     parsed counters) is written into the child's sidecar.
"""
from __future__ import annotations

from datetime import datetime, timezone
import json
import os
from pathlib import Path
import subprocess
import sys
import uuid
from typing import Any

from teamredbench_amd.benchmarks.base import BenchmarkContext
from teamredbench_amd.config import ProfilingConfig, SuiteConfig
from teamredbench_amd.io import read_results
from teamredbench_amd.profiling.registry import ProfilingLaunch, get_profile_engine

INTERNAL_RUN_ENV = "TEAMREDBENCH_INTERNAL_RUN"
FORCE_JSON_OUTPUT_ENV = "TEAMREDBENCH_FORCE_JSON_OUTPUT"
RUN_TOKEN_ENV = "TEAMREDBENCH_RUN_TOKEN"
# The hardware profile the parent resolved for a suite whose own profile has no peaks, and the note saying
# so: the child under the profiler measures against the same profile instead of detecting it again.
RESOLVED_PROFILE_ENV = "TEAMREDBENCH_RESOLVED_HARDWARE_PROFILE"
RESOLVED_NOTE_ENV = "TEAMREDBENCH_RESOLVED_PROFILE_NOTE"


class ProfilingError(RuntimeError):
    pass


def profiling_active() -> bool:
    """True inside the child run of a profiled suite."""
    return os.environ.get(INTERNAL_RUN_ENV) == "1"


def profiling_enabled(config: ProfilingConfig) -> bool:
    return bool(config.enabled and config.engine) and not profiling_active()


def effective_output_formats(formats: list[str]) -> list[str]:
    """The suite's formats, plus json when the parent of a profiled run needs to reload the records."""
    forced = os.environ.get(FORCE_JSON_OUTPUT_ENV) == "1"
    return list(formats) + (["json"] if forced and "json" not in formats else [])


def inherited_hardware_profile() -> tuple[Path, str] | None:
    """Inside the child of a profiled run: the (profile path, note) its parent resolved, if it did."""
    path = os.environ.get(RESOLVED_PROFILE_ENV) if profiling_active() else None
    return (Path(path), os.environ.get(RESOLVED_NOTE_ENV, "")) if path else None


def run_token() -> str | None:
    """The token a profiled run's parent gave this process (recorded in the sidecar)."""
    return os.environ.get(RUN_TOKEN_ENV)


def child_command(suite_path: Path, device_id: int, output_dir: Path) -> list[str]:
    return [sys.executable, "-m", "teamredbench_amd", "run", str(suite_path), "--device-id", str(device_id),
            "--output-dir", str(output_dir), "--quiet-records"]


class ProfiledRun:
    def __init__(self, suite: SuiteConfig, output_dir: Path, device_id: int, resolved_profile: Path | None = None,
                 profile_note: str | None = None):
        if suite.path is None:
            raise ProfilingError("Suite path is required for profiled runs.")
        if not suite.profiling.engine:
            raise ProfilingError("Profiling is enabled but no engine is configured.")
        self.suite, self.output_dir, self.device_id = suite, Path(output_dir), device_id
        self.engine = get_profile_engine(suite.profiling.engine)
        stamp = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%SZ")
        self.artifact_dir = self.output_dir / "profiling" / f"{suite.name}-{self.engine.name}-{stamp}"
        self.token = uuid.uuid4().hex
        self.env = {**os.environ, INTERNAL_RUN_ENV: "1", FORCE_JSON_OUTPUT_ENV: "1", RUN_TOKEN_ENV: self.token}
        if resolved_profile is not None and profile_note:
            self.env.update({RESOLVED_PROFILE_ENV: str(resolved_profile), RESOLVED_NOTE_ENV: profile_note})
        self.launch_spec: ProfilingLaunch | None = None
        self.teardown_crashes: list[dict[str, Any]] = []

    # A profiler can crash in its own teardown (SIGSEGV) after the program it ran
    # has finished and its results are written; such an exit is recorded, not
    # fatal, when the step's output is there (`produced` says whether it is).
    PROFILER_TEARDOWN_CRASH = (-11, 139)

    def _run(self, command: list[str], what: str, produced=None) -> None:
        proc = subprocess.run(command, capture_output=True, text=True, env=self.env, check=False)
        if proc.returncode == 0:
            return
        if proc.returncode in self.PROFILER_TEARDOWN_CRASH and produced is not None and produced():
            self.teardown_crashes.append({"step": what, "exit_status": proc.returncode})
            return
        detail = proc.stderr.strip() or proc.stdout.strip() or "unknown profiling failure"
        raise ProfilingError(f"{what} failed (exit status {proc.returncode}): {detail}")

    def _has_sidecar(self) -> bool:
        try:
            self.sidecar_path()
        except ProfilingError:
            return False
        return True

    def launch(self) -> None:
        self.launch_spec = self.engine.build_command(
            dict(self.suite.profiling.params), child_command(self.suite.path, self.device_id, self.output_dir),
            self.artifact_dir, self.suite.path.parent)
        self.env.update(self.launch_spec.env)
        self._run(list(self.launch_spec.command), f"Profile engine {self.engine.name}", produced=self._has_sidecar)

    def sidecar_path(self) -> Path:
        for path in sorted(self.output_dir.glob(f"{self.suite.name}-*.metadata.json"), reverse=True):
            try:
                sidecar = json.loads(path.read_text(encoding="utf-8"))
            except (OSError, json.JSONDecodeError):
                continue
            if sidecar.get("run", {}).get("run_token") == self.token:
                return path
        raise ProfilingError("Profiled run completed but no metadata file was produced.")

    def passes(self) -> None:
        spec = self.launch_spec
        for number, prefix in enumerate(spec.extra_passes, start=1):
            out = self.artifact_dir / f"pass{number}-results"
            self._run([*prefix, *child_command(self.suite.path, self.device_id, out)],
                      f"{self.engine.name} pass {number}",
                      produced=lambda out=out: any(out.glob(f"{self.suite.name}-*.metadata.json")))
        for number, command in enumerate(spec.standalone_passes, start=1):
            self._run(list(command), f"{self.engine.name} standalone pass {number}",
                      produced=lambda: any(self.artifact_dir.rglob("*counter_collection.csv")))

    def profiling_metadata(self) -> dict[str, Any]:
        spec = self.launch_spec
        block: dict[str, Any] = {
            "enabled": True,
            "engine": self.engine.name,
            "artifact_dir": str(spec.artifact_dir),
            "command": list(spec.command),
            "extra_passes": [list(p) for p in spec.extra_passes],
            "standalone_passes": [list(p) for p in spec.standalone_passes],
            "engine_metadata": dict(spec.metadata),
        }
        if self.teardown_crashes:
            block["profiler_teardown_crashes"] = list(self.teardown_crashes)
        if spec.collect is not None:
            try:
                block["counters"] = spec.collect(spec.artifact_dir)
            except Exception as exc:  # noqa: BLE001 -- a parse failure must not lose the measurements
                block["counters_error"] = f"{type(exc).__name__}: {exc}"
        return block


def run_profiled_suite(*, suite: SuiteConfig, context: BenchmarkContext, output_dir: Path, device_id: int,
                       record_callback, profile_note: str | None = None):
    from teamredbench_amd.runner import RunSummary

    # A profile the parent auto-selected goes to the child with its note.
    resolved = getattr(context.hardware_profile, "path", None) if profile_note else None
    run = ProfiledRun(suite, output_dir, device_id, resolved_profile=resolved, profile_note=profile_note)
    run.launch()
    sidecar_path = run.sidecar_path()
    try:
        sidecar, records = read_results(sidecar_path)
    except FileNotFoundError as exc:
        raise ProfilingError("Profiled run did not produce a JSON results file.") from exc
    run.passes()
    sidecar.setdefault("outputs", {})["profiling"] = str(run.launch_spec.artifact_dir)
    sidecar.setdefault("run", {})["profiling"] = run.profiling_metadata()
    sidecar_path.write_text(json.dumps(sidecar, indent=2), encoding="utf-8")
    if record_callback is not None:
        for record in records:
            record_callback(record)
    run_metadata = dict(sidecar["run"])
    return RunSummary(suite=suite, context=context, records=records,
                      outputs={name: Path(p) for name, p in sidecar["outputs"].items()},
                      run_metadata=run_metadata,
                      profile_note=run_metadata.get("configs", {}).get("profile_note") or profile_note)
