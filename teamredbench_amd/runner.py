"""Running a suite: load it, set up the device context, run every benchmark
invocation, derive metrics, write the result files.

``run_suite``, ``build_context`` and ``RunSummary`` keep the reference's
signatures (src/teamredbench/runner.py:21-179); :class:`SuiteRun` holds the
steps. Two behaviours carried over:
  * the device index is ``LOCAL_RANK`` when that is set, else ``device_id``;
  * a hardware profile with no peak data (hbm bandwidth and at least one
    compute peak) is replaced by a profile whose SKU token (``mi355x`` ...)
    matches the detected device name (torch's, or, when that carries no
    SKU, the product names amdsmi and rocm-smi report for the device:
    device.product_names), found by :class:`ProfileCatalog` in
    the suite tree's ``configs/profiles/hardware`` or among this package's
    profiles; the replacement is reported in ``profile_note``.
Metrics are derived only for ``ok`` records; a skipped or failed record keeps
its raw metrics and error and gets none.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from datetime import datetime, timezone
import os
from pathlib import Path
import re
from typing import Callable, Iterable

from teamredbench_amd import builtin as _builtin  # noqa: F401  (registers the built-in benchmarks and metrics)
from teamredbench_amd.benchmarks.base import BenchmarkContext, BenchmarkRecord
from teamredbench_amd.config import HardwareProfile, SuiteConfig, load_hardware_profile, load_suite
from teamredbench_amd.device import detect_device, load_torch, product_names
from teamredbench_amd.dtypes import discover_dtypes
from teamredbench_amd.io import write_results
from teamredbench_amd.profiling.runtime import (
    effective_output_formats,
    inherited_hardware_profile,
    profiling_enabled,
    run_profiled_suite,
)
from teamredbench_amd.provenance import build_run_metadata
from teamredbench_amd.registry import get_benchmark, get_metric, load_plugins

PACKAGED_HARDWARE_DIR = Path(__file__).resolve().parent / "configs" / "profiles" / "hardware"
_SKU_PATTERN = re.compile(r"mi\d{3,4}x", re.IGNORECASE)


def sku_tokens(text: str | None) -> set[str]:
    """Instinct SKU names in a device or profile name ("AMD Instinct MI355X" -> {"mi355x"})."""
    return {token.lower() for token in _SKU_PATTERN.findall(text or "")}


def has_peak_data(profile: HardwareProfile) -> bool:
    hbm = profile.peak_hbm_bandwidth_gbps
    return bool(hbm and hbm > 0) and any(v is not None and v > 0 for v in profile.peak_compute_tops.values())


@dataclass
class ProfileCatalog:
    """Hardware profiles that can stand in for one without peak data."""

    directories: list[Path] = field(default_factory=list)

    @classmethod
    def packaged(cls) -> "ProfileCatalog":
        return cls([PACKAGED_HARDWARE_DIR])

    @classmethod
    def for_suite(cls, repo_root: Path | None) -> "ProfileCatalog":
        dirs = [repo_root / "configs" / "profiles" / "hardware"] if repo_root is not None else []
        return cls(dirs + [PACKAGED_HARDWARE_DIR])

    def candidates(self) -> Iterable[tuple[Path, HardwareProfile]]:
        seen: set[Path] = set()
        for directory in self.directories:
            for path in sorted(directory.glob("*.yaml")) if directory.is_dir() else []:
                if path.resolve() not in seen:
                    seen.add(path.resolve())
                    yield path, load_hardware_profile(path)

    def match(self, device_name: str | None) -> HardwareProfile | None:
        wanted = sku_tokens(device_name)
        if not wanted:
            return None
        for path, profile in self.candidates():
            if sku_tokens(f"{profile.name} {path.stem}") & wanted and has_peak_data(profile):
                return profile
        return None


@dataclass
class RunSummary:
    suite: SuiteConfig
    context: BenchmarkContext
    records: list[BenchmarkRecord]
    outputs: dict[str, Path]
    run_metadata: dict[str, object]
    profile_note: str | None = None


def _suite_repo_root(suite: SuiteConfig) -> Path | None:
    # <root>/configs/suites/<suite>.yaml, the layout both trees use
    return suite.path.parent.parent.parent if suite.path else None


def build_context(suite: SuiteConfig, device_id: int = 0) -> tuple[BenchmarkContext, str | None]:
    index = int(os.environ.get("LOCAL_RANK", device_id))
    torch_module = load_torch()
    device = detect_device(torch_module, device_id=index)
    profile, note = suite.hardware_profile, None
    inherited = inherited_hardware_profile() if not has_peak_data(profile) else None
    if inherited is not None:
        # the child of a profiled run measures against the profile its parent resolved
        profile, note = load_hardware_profile(inherited[0]), inherited[1]
    elif not has_peak_data(profile) and device is not None:
        # torch's device name carries the SKU where the platform's marketing-name table is installed;
        # otherwise the board's own product name (amdsmi, rocm-smi) does
        detected = device.name
        if not sku_tokens(detected):
            detected = " / ".join([device.name, *product_names(torch_module, index)])
        stand_in = ProfileCatalog.for_suite(_suite_repo_root(suite)).match(detected)
        if stand_in is not None:
            note = (f"Auto-selected hardware profile {stand_in.name} from detected device {detected!r} "
                    f"because {profile.name} has no theoretical peak data.")
            profile = stand_in
    context = BenchmarkContext(
        hardware_profile=profile,
        runtime_profile=suite.runtime_profile,
        device_info=device,
        torch_module=torch_module,
        dtype_specs=discover_dtypes(torch_module),
        device_id=index,
        repo_root=_suite_repo_root(suite),
        suite_path=suite.path,
    )
    return context, note


class SuiteRun:
    """One execution of a suite file."""

    def __init__(self, suite_path: str | Path, output_dir: str | Path | None, device_id: int,
                 record_callback: Callable[[BenchmarkRecord], None] | None):
        self.started = datetime.now(timezone.utc)
        self.suite = load_suite(suite_path)
        load_plugins(self.suite.plugins)
        self.output_dir = (Path(output_dir) if output_dir else self.suite.outputs.directory).resolve()
        self.device_id = device_id
        self.record_callback = record_callback
        self.context, self.profile_note = build_context(self.suite, device_id=device_id)
        self.suite.hardware_profile = self.context.hardware_profile
        self.records: list[BenchmarkRecord] = []

    def _sink_for(self, metric_names: list[str]) -> Callable[[BenchmarkRecord], None]:
        metrics = [get_metric(name) for name in metric_names]

        def sink(record: BenchmarkRecord) -> None:
            if record.ok:
                for metric in metrics:
                    record.metrics[metric.name] = metric.compute(record.raw_metrics)
            if self.record_callback is not None:
                self.record_callback(record)

        return sink

    def execute(self) -> None:
        for invocation in self.suite.benchmarks:
            cls = get_benchmark(invocation.benchmark)
            sink = self._sink_for(invocation.metrics or list(cls.default_metrics))
            self.records.extend(cls(context=self.context, params=invocation.params, record_sink=sink).run())

    def finish(self) -> RunSummary:
        formats = effective_output_formats(self.suite.outputs.formats)
        run_metadata = build_run_metadata(
            suite=self.suite, context=self.context, requested_device_id=self.device_id,
            output_dir=self.output_dir, output_formats=formats, profile_note=self.profile_note,
            started_at=self.started, finished_at=datetime.now(timezone.utc),
        )
        outputs = write_results(records=self.records, suite_name=self.suite.name, output_dir=self.output_dir,
                                formats=formats, run_metadata=run_metadata)
        return RunSummary(suite=self.suite, context=self.context, records=self.records, outputs=outputs,
                          run_metadata=run_metadata, profile_note=self.profile_note)


def run_suite(suite_path: str | Path, output_dir: str | Path | None = None, device_id: int = 0,
              record_callback: Callable[[BenchmarkRecord], None] | None = None) -> RunSummary:
    run = SuiteRun(suite_path, output_dir, device_id, record_callback)
    if profiling_enabled(run.suite.profiling):
        # the whole suite runs again in a child process under the profiler
        return run_profiled_suite(suite=run.suite, context=run.context, output_dir=run.output_dir,
                                  device_id=device_id, record_callback=record_callback,
                                  profile_note=run.profile_note)
    run.execute()
    return run.finish()
