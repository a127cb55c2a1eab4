from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable


@dataclass(frozen=True)
class MetricDefinition:
    """A derived metric: raw counters of one record -> value or None
    (src/teamredbench/metrics/base.py:7-12)."""

    name: str
    description: str
    compute: Callable[[dict[str, Any]], float | None]
