"""Benchmark and metric registries (API of src/teamredbench/registry.py:9-56).

``register_benchmark(name)`` / ``register_metric(name, description)`` are
decorators; ``load_plugins`` imports modules named in a suite's ``plugins:``
list so their decorators run.
"""
from __future__ import annotations

import importlib
from typing import Any, Callable

from teamredbench_amd.metrics.base import MetricDefinition

BENCHMARK_REGISTRY: dict[str, type] = {}
METRIC_REGISTRY: dict[str, MetricDefinition] = {}


def register_benchmark(name: str) -> Callable[[type], type]:
    def decorate(cls: type) -> type:
        cls.name = name
        BENCHMARK_REGISTRY[name] = cls
        return cls

    return decorate


def register_metric(name: str, description: str) -> Callable:
    def decorate(fn: Callable[[dict[str, Any]], float | None]):
        METRIC_REGISTRY[name] = MetricDefinition(name=name, description=description, compute=fn)
        return fn

    return decorate


def _lookup(table: dict, kind: str, name: str):
    try:
        return table[name]
    except KeyError:
        raise KeyError(f"Unknown {kind}: {name}") from None


def get_benchmark(name: str) -> type:
    return _lookup(BENCHMARK_REGISTRY, "benchmark", name)


def get_metric(name: str) -> MetricDefinition:
    return _lookup(METRIC_REGISTRY, "metric", name)


def list_benchmarks() -> list[str]:
    return sorted(BENCHMARK_REGISTRY)


def list_metrics() -> list[str]:
    return sorted(METRIC_REGISTRY)


def load_plugins(module_names: list[str]) -> None:
    for module_name in module_names:
        importlib.import_module(module_name)
