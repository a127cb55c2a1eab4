"""Suite and profile files.

The YAML schema is the reference's (src/teamredbench/config.py:10-150), so a
suite written for it loads here unchanged:

    name: <suite name>                      # default: the file's stem
    device:  {profile: <hardware profile yaml>}
    runtime: {profile: <runtime profile yaml>}
    outputs: {directory: <dir>, formats: [json, csv]}
    profiling: {enabled: <bool>, engine: <name>, params: {...}}
    plugins: [<module>, ...]
    benchmarks:
      - {benchmark: <name>, params: {...}, metrics: [<metric>, ...]}

Relative paths are taken from the directory of the file that names them.
Every value is read through :class:`_Section`, which knows where in which
file it is, so a malformed file fails with a ``ConfigError`` naming the key
(``suite.yaml: benchmarks[2].params must be a mapping``) rather than with a
``KeyError`` or a half-loaded suite.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import yaml


class ConfigError(ValueError):
    """A suite or profile file that does not follow the schema."""


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


_MISSING = object()


class _Section:
    """A mapping read from `origin` at `where` (a dotted key path)."""

    def __init__(self, data: Any, origin: Path, where: str = ""):
        if not isinstance(data, dict):
            raise ConfigError(f"{origin.name}: {where or 'the document'} must be a mapping")
        self.data, self.origin, self.where = data, origin, where

    @classmethod
    def read(cls, path: Path) -> "_Section":
        try:
            data = yaml.safe_load(path.read_text(encoding="utf-8"))
        except OSError as exc:
            raise ConfigError(f"cannot read {path}: {exc}") from exc
        return cls({} if data is None else data, path)

    def _key(self, key: str) -> str:
        return f"{self.where}.{key}" if self.where else key

    def _fail(self, key: str, what: str) -> ConfigError:
        return ConfigError(f"{self.origin.name}: {self._key(key)} {what}")

    def get(self, key: str, default: Any = _MISSING) -> Any:
        value = self.data.get(key, _MISSING)
        if value is _MISSING or value is None:
            if default is _MISSING:
                raise self._fail(key, "is required")
            return default
        return value

    def text(self, key: str, default: Any = _MISSING) -> str:
        value = self.get(key, default)
        if isinstance(value, (dict, list)):
            raise self._fail(key, "must be a scalar")
        return str(value)

    def number(self, key: str) -> float | None:
        value = self.get(key, None)
        if value is None:
            return None
        try:
            return float(value)
        except (TypeError, ValueError):
            raise self._fail(key, f"must be a number (got {value!r})") from None

    def section(self, key: str) -> "_Section":
        return _Section(self.get(key, {}), self.origin, self._key(key))

    def mapping(self, key: str, convert=lambda v: v) -> dict[str, Any]:
        sub = self.section(key)
        try:
            return {str(k): convert(v) for k, v in sub.data.items()}
        except (TypeError, ValueError):
            raise self._fail(key, "holds a value of the wrong type") from None

    def items(self, key: str) -> list[Any]:
        value = self.get(key, [])
        if not isinstance(value, list):
            raise self._fail(key, "must be a list")
        return value

    def path(self, key: str, default: Any = _MISSING) -> Path:
        target = Path(self.text(key, default)).expanduser()
        return target if target.is_absolute() else (self.origin.parent / target).resolve()


def load_hardware_profile(path: Path) -> HardwareProfile:
    """A hardware profile: the peaks every efficiency metric divides by."""
    doc = _Section.read(Path(path))
    return HardwareProfile(
        name=doc.text("name"),
        family=doc.text("family"),
        peak_hbm_bandwidth_gbps=doc.number("peak_hbm_bandwidth_gbps"),
        peak_link_bandwidth_gbps=doc.mapping("peak_link_bandwidth_gbps"),
        peak_compute_tops=doc.mapping("peak_compute_tops", float),
        notes=[str(n) for n in doc.items("notes")],
        path=Path(path),
        raw=doc.data,
    )


def load_runtime_profile(path: Path) -> RuntimeProfile:
    """A runtime profile: the ROCm stack a run was meant for (recorded, not enforced)."""
    doc = _Section.read(Path(path))
    return RuntimeProfile(
        name=doc.text("name"),
        rocm_version=doc.text("rocm_version", "unknown"),
        libraries=doc.mapping("libraries", str),
        env=doc.mapping("env", str),
        notes=[str(n) for n in doc.items("notes")],
        path=Path(path),
        raw=doc.data,
    )


def _invocation(doc: _Section, index: int) -> BenchmarkInvocation:
    entry = _Section(doc.items("benchmarks")[index], doc.origin, f"benchmarks[{index}]")
    return BenchmarkInvocation(
        benchmark=entry.text("benchmark"),
        params=dict(entry.section("params").data),
        metrics=[str(m) for m in entry.items("metrics")],
    )


def _profiling(doc: _Section) -> ProfilingConfig:
    block = doc.section("profiling")
    engine = block.get("engine", None)
    return ProfilingConfig(
        # a named engine switches profiling on unless the block says otherwise
        enabled=bool(block.get("enabled", engine is not None)),
        engine=None if engine is None else str(engine),
        params=dict(block.section("params").data),
        raw=dict(block.data),
    )


def load_suite(path: str | Path) -> SuiteConfig:
    suite_path = Path(path).resolve()
    doc = _Section.read(suite_path)
    outputs = doc.section("outputs")
    return SuiteConfig(
        name=doc.text("name", suite_path.stem),
        benchmarks=[_invocation(doc, i) for i in range(len(doc.items("benchmarks")))],
        hardware_profile=load_hardware_profile(doc.section("device").path("profile")),
        runtime_profile=load_runtime_profile(doc.section("runtime").path("profile")),
        outputs=OutputConfig(
            directory=outputs.path("directory", "../../results"),
            formats=[str(f) for f in outputs.get("formats", ["json", "csv"])],
        ),
        profiling=_profiling(doc),
        plugins=[str(p) for p in doc.items("plugins")],
        path=suite_path,
        raw=doc.data,
    )
