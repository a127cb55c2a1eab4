"""What a benchmark plugin sees and what it produces.

The names and fields here are the plugin interface of the reference
(src/teamredbench/benchmarks/base.py:13-86): a benchmark class takes a
:class:`BenchmarkContext`, its suite ``params`` and an optional record sink,
and ``run()`` returns :class:`BenchmarkRecord`s, each passed to the sink as
it is emitted. Third-party plugins written against that interface run here
unchanged.

Record lifecycle, as this package implements it:
  * ``ok``      -- measured; the runner derives the metrics from raw_metrics.
  * ``skipped`` -- the case could not run here (no device, no peak for the
                   dtype, a kernel that does not build); ``error`` says why.
  * ``failed``  -- the case ran but its in-run correctness check did not
                   pass (``metadata["parity"]["passed"]`` is false): the
                   timing is kept in raw_metrics for diagnosis, but no metric
                   is derived, so a wrong kernel never publishes a rate.
The JSON / CSV forms of a record (``to_dict`` / ``to_row``) are the
reference's result-file formats.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable

from teamredbench_amd.config import HardwareProfile, RuntimeProfile
from teamredbench_amd.device import DeviceInfo, rocm_device, rocm_device_available, set_rocm_device
from teamredbench_amd.dtypes import DTypeSpec, resolve_dtype_names

STATUS_OK, STATUS_SKIPPED, STATUS_FAILED = "ok", "skipped", "failed"


@dataclass
class BenchmarkContext:
    hardware_profile: HardwareProfile
    runtime_profile: RuntimeProfile
    device_info: DeviceInfo | None
    torch_module: Any
    dtype_specs: dict[str, DTypeSpec]
    device_id: int = 0
    repo_root: Path | None = None
    suite_path: Path | None = None


@dataclass
class BenchmarkRecord:
    benchmark: str
    case: str
    dtype: str
    raw_metrics: dict[str, Any] = field(default_factory=dict)
    metadata: dict[str, Any] = field(default_factory=dict)
    metrics: dict[str, float | None] = field(default_factory=dict)
    status: str = STATUS_OK
    error: str | None = None

    @property
    def ok(self) -> bool:
        return self.status == STATUS_OK

    # ---- result-file forms ----------------------------------------------
    _JSON_KEYS = ("benchmark", "case", "dtype", "status", "error", "metrics", "raw_metrics", "metadata")

    def to_dict(self) -> dict[str, Any]:
        """The object written for this record in the JSON results file."""
        return {key: getattr(self, key) for key in self._JSON_KEYS}

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> "BenchmarkRecord":
        """Inverse of :meth:`to_dict` (reloading a results file)."""
        error = payload.get("error")
        return cls(
            benchmark=str(payload["benchmark"]),
            case=str(payload["case"]),
            dtype=str(payload["dtype"]),
            status=str(payload.get("status", STATUS_OK)),
            error=None if error is None else str(error),
            metrics=dict(payload.get("metrics") or {}),
            raw_metrics=dict(payload.get("raw_metrics") or {}),
            metadata=dict(payload.get("metadata") or {}),
        )

    def to_row(self) -> dict[str, Any]:
        """The flat CSV row: identity columns, then metric_* / raw_* / meta_* in key order. Values go to
        the CSV writer as they are, so a nested one (a parity dict, a shape list) is written as its Python
        text, str(value), the form the reference's CSV holds (src/teamredbench/io.py:25-39)."""
        row: dict[str, Any] = {"benchmark": self.benchmark, "case": self.case, "dtype": self.dtype,
                               "status": self.status, "error": self.error or ""}
        for prefix, values in (("metric", self.metrics), ("raw", self.raw_metrics), ("meta", self.metadata)):
            for key in sorted(values):
                row[f"{prefix}_{key}"] = values[key]
        return row


def parity_failure(record: BenchmarkRecord) -> str | None:
    """Why the record's in-run correctness check failed, or None if it passed or was not run."""
    parity = record.metadata.get("parity")
    if not isinstance(parity, dict) or parity.get("passed", True):
        return None
    figures = ", ".join(f"{k}={v}" for k, v in parity.items() if k != "passed")
    return f"in-run parity check failed ({figures})"


class Benchmark(ABC):
    """Base class of the registered benchmarks (``@register_benchmark(name)`` sets ``name``)."""

    name = "benchmark"
    default_metrics: list[str] = []

    def __init__(self, context: BenchmarkContext, params: dict[str, Any],
                 record_sink: Callable[[BenchmarkRecord], None] | None = None):
        self.context = context
        self.params = params
        self.record_sink = record_sink

    # ---- device ----------------------------------------------------------
    @property
    def torch(self) -> Any:
        if self.context.torch_module is None:
            raise RuntimeError("PyTorch is required for GPU benchmarks.")
        return self.context.torch_module

    @property
    def device(self) -> Any:
        return rocm_device(self.torch, self.context.device_id)

    def set_device(self) -> None:
        if rocm_device_available(self.context.torch_module):
            set_rocm_device(self.context.torch_module, self.context.device_id)

    def selected_dtype_specs(self) -> list[DTypeSpec]:
        specs = self.context.dtype_specs
        return [specs[name] for name in resolve_dtype_names(self.params.get("dtypes"), specs)]

    # ---- records -----------------------------------------------------------
    def emit_record(self, record: BenchmarkRecord) -> BenchmarkRecord:
        """Hand a finished record to the sink. An ``ok`` record whose in-run parity check failed
        is turned into a ``failed`` one first."""
        if record.ok:
            why = parity_failure(record)
            if why is not None:
                record.status, record.error = STATUS_FAILED, why
        if self.record_sink is not None:
            self.record_sink(record)
        return record

    def skipped_record(self, *, case: str, dtype: str, error: str,
                       metadata: dict[str, Any] | None = None) -> BenchmarkRecord:
        return BenchmarkRecord(benchmark=self.name, case=case, dtype=dtype, metadata=dict(metadata or {}),
                               status=STATUS_SKIPPED, error=error)

    def skip(self, *, case: str, dtype: str, error: str, metadata: dict[str, Any] | None = None) -> BenchmarkRecord:
        """Build and emit a skipped record."""
        return self.emit_record(self.skipped_record(case=case, dtype=dtype, error=error, metadata=metadata))

    def measured(self, *, case: str, dtype: str, raw_metrics: dict[str, Any],
                 metadata: dict[str, Any]) -> BenchmarkRecord:
        """Build and emit the record of a case that ran."""
        return self.emit_record(BenchmarkRecord(benchmark=self.name, case=case, dtype=dtype,
                                                raw_metrics=raw_metrics, metadata=metadata))

    @abstractmethod
    def run(self) -> list[BenchmarkRecord]:
        raise NotImplementedError
