"""Command line (the ``teamredbench`` commands of src/teamredbench/cli.py:85-163
that drive this path): run, list-benchmarks, list-metrics, list-native-kernels,
list-profile-engines, list-dtypes, clean-native-cache, build-native, discover."""
from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Any

import typer
import yaml

from teamredbench_amd import builtin as _builtin  # noqa: F401
from teamredbench_amd.benchmarks.base import BenchmarkRecord
from teamredbench_amd.device import discover_environment, load_torch
from teamredbench_amd.dtypes import discover_dtypes
from teamredbench_amd.native.registry import list_native_kernels
from teamredbench_amd.native.runtime import clear_native_cache, native_cache_dir
from teamredbench_amd.profiling.registry import list_profile_engines
from teamredbench_amd.profiling.runtime import profiling_active
from teamredbench_amd.registry import list_benchmarks, list_metrics
from teamredbench_amd.runner import run_suite

app = typer.Typer(no_args_is_help=True)


def _fmt(name: str, value: Any) -> str:
    if value is None:
        return "n/a"
    if isinstance(value, float):
        text = f"{value:.6g}"
        return text + "%" if name.endswith("_pct") else text
    return str(value)


def format_record(record: BenchmarkRecord) -> str:
    head = f"[{record.status.upper()}] {record.benchmark} case={record.case} dtype={record.dtype}"
    if record.status != "ok":
        return f"{head} error={record.error}"
    values = record.metrics or record.raw_metrics
    body = ", ".join(f"{k}={_fmt(k, v)}" for k, v in sorted(values.items()))
    return f"{head} {body}" if body else head


@app.command()
def run(
    suite: Path = typer.Argument(..., help="Path to suite YAML."),
    output_dir: Path | None = typer.Option(None, help="Override result directory."),
    device_id: int = typer.Option(0, help="GPU index."),
    print_records: bool = typer.Option(True, "--print-records/--quiet-records", help="Print each result record."),
) -> None:
    summary = run_suite(
        suite_path=suite,
        output_dir=output_dir,
        device_id=device_id,
        record_callback=(lambda r: typer.echo(format_record(r))) if print_records else None,
    )
    if profiling_active() or os.environ.get("TEAMREDBENCH_SUPPRESS_CLI_OUTPUT") == "1":
        return
    typer.echo(f"Suite: {summary.suite.name}")
    typer.echo(f"Hardware Profile: {summary.context.hardware_profile.name}")
    if summary.profile_note:
        typer.echo(summary.profile_note)
    typer.echo(f"Records: {len(summary.records)}")
    for fmt, path in summary.outputs.items():
        typer.echo(f"{fmt.upper()}: {path}")


@app.command("list-benchmarks")
def list_benchmarks_command() -> None:
    for name in list_benchmarks():
        typer.echo(name)


@app.command("list-metrics")
def list_metrics_command() -> None:
    for name in list_metrics():
        typer.echo(name)


@app.command("list-native-kernels")
def list_native_kernels_command(benchmark: str | None = typer.Option(None, help="Optional benchmark filter.")) -> None:
    for d in list_native_kernels(benchmark=benchmark):
        alias = f" (aliases: {', '.join(d.aliases)})" if d.aliases else ""
        typer.echo(f"{d.name} [{d.benchmark}] abi={d.abi}{alias}")


@app.command("list-profile-engines")
def list_profile_engines_command() -> None:
    for d in list_profile_engines():
        typer.echo(f"{d.name}: {d.description}")


@app.command("list-dtypes")
def list_dtypes_command() -> None:
    for name in sorted(discover_dtypes(load_torch())):
        typer.echo(name)


@app.command("clean-native-cache")
def clean_native_cache_command(
    cache_dir: Path | None = typer.Option(None, help="Override native kernel cache directory."),
) -> None:
    resolved = native_cache_dir(cache_dir.resolve() if cache_dir else None)
    cleared, removed = clear_native_cache(resolved)
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
