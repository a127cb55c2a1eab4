"""``python -m teamredbench_amd <command>``: the reference's command line
(src/teamredbench/cli.py:85-163) for this path, plus ``build-native``.

  run SUITE [--output-dir D] [--device-id N] [--print-records/--quiet-records]
  list-benchmarks | list-metrics | list-native-kernels [--benchmark B]
  list-profile-engines | list-dtypes | discover [--device-id N] [--json]
  clean-native-cache [--cache-dir D] | build-native

``run`` prints one line per record as it is produced --
``[OK] hbm case=triad_1024MiB dtype=float32 hbm_bandwidth_gbps=6268.2, ...``
(a skipped or failed record shows its error instead of metrics) -- then a
summary and the files written. It exits with status 1 when any record
failed its in-run correctness check, so a wrong kernel cannot pass for a
slow one in scripts.
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Any

import typer
import yaml

from teamredbench_amd import builtin as _builtin  # noqa: F401  (registers the built-ins)
from teamredbench_amd.benchmarks.base import STATUS_FAILED, BenchmarkRecord
from teamredbench_amd.device import discover_environment, load_torch
from teamredbench_amd.dtypes import discover_dtypes
from teamredbench_amd.native.registry import list_native_kernels
from teamredbench_amd.native.runtime import clear_native_cache, native_cache_dir
from teamredbench_amd.profiling.registry import list_profile_engines
from teamredbench_amd.profiling.runtime import profiling_active
from teamredbench_amd.registry import list_benchmarks, list_metrics
from teamredbench_amd.runner import run_suite

app = typer.Typer(no_args_is_help=True)


def _value_text(name: str, value: Any) -> str:
    if value is None:
        return "n/a"
    if not isinstance(value, float):
        return str(value)
    return f"{value:.6g}%" if name.endswith("_pct") else f"{value:.6g}"


def format_record(record: BenchmarkRecord) -> str:
    """One printed line per record: status, identity, then metrics (or raw metrics, or the error)."""
    parts = [f"[{record.status.upper()}]", record.benchmark, f"case={record.case}", f"dtype={record.dtype}"]
    if not record.ok:
        return " ".join(parts + [f"error={record.error}"])
    shown = record.metrics or record.raw_metrics
    if shown:
        parts.append(", ".join(f"{k}={_value_text(k, shown[k])}" for k in sorted(shown)))
    return " ".join(parts)


def _runtime_line(run_metadata: dict[str, Any]) -> str | None:
    torch_info = run_metadata.get("torch") or {}
    fields = [("python", (run_metadata.get("python") or {}).get("version")),
              ("torch", torch_info.get("version")), ("hip", torch_info.get("hip_version")),
              ("rocm_profile", (run_metadata.get("rocm") or {}).get("profile_version"))]
    shown = [f"{k}={v}" for k, v in fields if v]
    return f"Runtime: {' '.join(shown)}" if shown else None


@app.command()
def run(
    suite: Path = typer.Argument(..., help="Path to suite YAML."),
    output_dir: Path | None = typer.Option(None, help="Override result directory."),
    device_id: int = typer.Option(0, help="GPU index."),
    print_records: bool = typer.Option(True, "--print-records/--quiet-records", help="Print each result record."),
) -> None:
    printer = (lambda record: typer.echo(format_record(record))) if print_records else None
    summary = run_suite(suite_path=suite, output_dir=output_dir, device_id=device_id, record_callback=printer)
    failed = sum(1 for r in summary.records if r.status == STATUS_FAILED)
    if not (profiling_active() or os.environ.get("TEAMREDBENCH_SUPPRESS_CLI_OUTPUT") == "1"):
        lines = [f"Suite: {summary.suite.name}", f"Hardware Profile: {summary.context.hardware_profile.name}",
                 summary.profile_note, _runtime_line(summary.run_metadata),
                 f"Records: {len(summary.records)}" + (f" ({failed} failed)" if failed else "")]
        lines += [f"{fmt.upper()}: {path}" for fmt, path in summary.outputs.items()]
        for line in filter(None, lines):
            typer.echo(line)
    if failed:
        raise typer.Exit(code=1)


@app.command("list-benchmarks")
def list_benchmarks_command() -> None:
    typer.echo("\n".join(list_benchmarks()))


@app.command("list-metrics")
def list_metrics_command() -> None:
    typer.echo("\n".join(list_metrics()))


@app.command("list-native-kernels")
def list_native_kernels_command(benchmark: str | None = typer.Option(None, help="Optional benchmark filter.")) -> None:
    for kernel in list_native_kernels(benchmark=benchmark):
        aliases = f" (aliases: {', '.join(kernel.aliases)})" if kernel.aliases else ""
        typer.echo(f"{kernel.name} [{kernel.benchmark}] abi={kernel.abi}{aliases}")


@app.command("list-profile-engines")
def list_profile_engines_command() -> None:
    for engine in list_profile_engines():
        typer.echo(f"{engine.name}: {engine.description}")


@app.command("list-dtypes")
def list_dtypes_command() -> None:
    typer.echo("\n".join(sorted(discover_dtypes(load_torch()))))


@app.command("clean-native-cache")
def clean_native_cache_command(
    cache_dir: Path | None = typer.Option(None, help="Override native kernel cache directory."),
) -> None:
    cleared, removed = clear_native_cache(native_cache_dir(cache_dir.resolve() if cache_dir else None))
    typer.echo(f"Native cache: {cleared}")
    typer.echo(f"Removed entries: {removed}")


@app.command("build-native")
def build_native_command() -> None:
    """Compile libmi355bench.so for gfx950 in-tree."""
    from teamredbench_amd.native import build

    typer.echo(str(build.build(verbose=True)))


@app.command()
def discover(
    device_id: int = typer.Option(0, help="GPU index."),
    as_json: bool = typer.Option(False, "--json", help="Emit JSON instead of YAML."),
) -> None:
    payload = discover_environment(load_torch(), device_id=device_id)
    typer.echo(json.dumps(payload, indent=2) if as_json else yaml.safe_dump(payload, sort_keys=False))
