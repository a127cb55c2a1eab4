"""Profile-engine registry (API of src/teamredbench/profiling/registry.py:8-51).

An engine turns (params, child command, artifact dir, suite dir) into a
:class:`ProfilingLaunch`. ``command`` is the run whose records are kept;
``extra_passes`` are further runs of the same child under the profiler (one
per hardware-counter group -- rocprofv3 collects a limited number of counters
per pass) whose records are discarded and whose artifacts are parsed.
``standalone_passes`` are complete commands run once each after those (for
example a calibration workload of known traffic under the same counters).
``collect`` (optional) parses the artifact directory into a JSON-able
summary that the runner attaches to the metadata sidecar.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable


@dataclass(frozen=True)
class ProfilingLaunch:
    command: tuple[str, ...]
    artifact_dir: Path
    env: dict[str, str] = field(default_factory=dict)
    metadata: dict[str, Any] = field(default_factory=dict)
    extra_passes: tuple[tuple[str, ...], ...] = ()
    standalone_passes: tuple[tuple[str, ...], ...] = ()
    collect: Callable[[Path], dict[str, Any]] | None = None


BuildProfileCommand = Callable[[dict[str, Any], list[str], Path, "Path | None"], ProfilingLaunch]


@dataclass(frozen=True)
class ProfilingEngineDefinition:
    name: str
    description: str
    build_command: BuildProfileCommand


PROFILE_ENGINE_REGISTRY: dict[str, ProfilingEngineDefinition] = {}


def register_profile_engine(*, name: str, description: str, build_command: BuildProfileCommand) -> ProfilingEngineDefinition:
    definition = ProfilingEngineDefinition(name=name, description=description, build_command=build_command)
    PROFILE_ENGINE_REGISTRY[name] = definition
    return definition


def get_profile_engine(name: str) -> ProfilingEngineDefinition:
    if name not in PROFILE_ENGINE_REGISTRY:
        raise KeyError(f"Unknown profile engine: {name}")
    return PROFILE_ENGINE_REGISTRY[name]


def list_profile_engines() -> list[ProfilingEngineDefinition]:
    return sorted(PROFILE_ENGINE_REGISTRY.values(), key=lambda d: d.name)
