"""Suite and profile YAML loading (schema of src/teamredbench/config.py:10-150).

A suite names a hardware profile (peaks: the denominators of every % metric),
a runtime profile, output settings, an optional profiling block, plugin
modules and a list of benchmark invocations. Profile and output paths are
resolved relative to the suite file.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import yaml


@dataclass
class HardwareProfile:
    name: str
    family: str
    peak_hbm_bandwidth_gbps: float | None = None
    peak_link_bandwidth_gbps: dict[str, float] = field(default_factory=dict)
    peak_compute_tops: dict[str, float] = field(default_factory=dict)
    notes: list[str] = field(default_factory=list)
    path: Path | None = None
    raw: dict[str, Any] = field(default_factory=dict)


@dataclass
class RuntimeProfile:
    name: str
    rocm_version: str = "unknown"
    libraries: dict[str, str] = field(default_factory=dict)
    env: dict[str, str] = field(default_factory=dict)
    notes: list[str] = field(default_factory=list)
    path: Path | None = None
    raw: dict[str, Any] = field(default_factory=dict)


@dataclass
class OutputConfig:
    directory: Path
    formats: list[str] = field(default_factory=lambda: ["json", "csv"])


@dataclass
class ProfilingConfig:
    enabled: bool = False
    engine: str | None = None
    params: dict[str, Any] = field(default_factory=dict)
    raw: dict[str, Any] = field(default_factory=dict)


@dataclass
class BenchmarkInvocation:
    benchmark: str
    params: dict[str, Any] = field(default_factory=dict)
    metrics: list[str] = field(default_factory=list)


@dataclass
class SuiteConfig:
    name: str
    benchmarks: list[BenchmarkInvocation]
    hardware_profile: HardwareProfile
    runtime_profile: RuntimeProfile
    outputs: OutputConfig
    profiling: ProfilingConfig = field(default_factory=ProfilingConfig)
    plugins: list[str] = field(default_factory=list)
    path: Path | None = None
    raw: dict[str, Any] = field(default_factory=dict)


def _read_mapping(path: Path) -> dict[str, Any]:
    data = yaml.safe_load(path.read_text(encoding="utf-8")) or {}
    if not isinstance(data, dict):
        raise ValueError(f"Expected mapping in {path}")
    return data


def resolve_relative(base_dir: Path, target: str) -> Path:
    path = Path(target)
    return path if path.is_absolute() else (base_dir / path).resolve()


def load_hardware_profile(path: Path) -> HardwareProfile:
    data = _read_mapping(path)
    return HardwareProfile(
        name=str(data["name"]),
        family=str(data["family"]),
        peak_hbm_bandwidth_gbps=data.get("peak_hbm_bandwidth_gbps"),
        peak_link_bandwidth_gbps=dict(data.get("peak_link_bandwidth_gbps") or {}),
        peak_compute_tops={str(k): float(v) for k, v in (data.get("peak_compute_tops") or {}).items()},
        notes=list(data.get("notes") or []),
        path=path,
        raw=data,
    )


def load_runtime_profile(path: Path) -> RuntimeProfile:
    data = _read_mapping(path)
    return RuntimeProfile(
        name=str(data["name"]),
        rocm_version=str(data.get("rocm_version", "unknown")),
        libraries={str(k): str(v) for k, v in (data.get("libraries") or {}).items()},
        env={str(k): str(v) for k, v in (data.get("env") or {}).items()},
        notes=list(data.get("notes") or []),
        path=path,
        raw=data,
    )


def _profiling_config(block: Any, suite_path: Path) -> ProfilingConfig:
    if block is None:
        block = {}
    if not isinstance(block, dict):
        raise ValueError(f"Expected mapping for profiling config in {suite_path}")
    engine = block.get("engine")
    return ProfilingConfig(
        enabled=bool(block.get("enabled", bool(engine))),
        engine=None if engine is None else str(engine),
        params=dict(block.get("params") or {}),
        raw=dict(block),
    )


def load_suite(path: str | Path) -> SuiteConfig:
    suite_path = Path(path).resolve()
    data = _read_mapping(suite_path)
    base = suite_path.parent
    outputs = data.get("outputs") or {}
    return SuiteConfig(
        name=str(data.get("name", suite_path.stem)),
        benchmarks=[
            BenchmarkInvocation(
                benchmark=str(item["benchmark"]),
                params=dict(item.get("params") or {}),
                metrics=list(item.get("metrics") or []),
            )
            for item in data.get("benchmarks") or []
        ],
        hardware_profile=load_hardware_profile(resolve_relative(base, str(data["device"]["profile"]))),
        runtime_profile=load_runtime_profile(resolve_relative(base, str(data["runtime"]["profile"]))),
        outputs=OutputConfig(
            directory=resolve_relative(base, str(outputs.get("directory", "../../results"))),
            formats=list(outputs.get("formats", ["json", "csv"])),
        ),
        profiling=_profiling_config(data.get("profiling"), suite_path),
        plugins=list(data.get("plugins") or []),
        path=suite_path,
        raw=data,
    )
