"""Suite execution (src/teamredbench/runner.py:31-179).

``run_suite`` loads the suite, imports its plugins, builds the context
(device from ``LOCAL_RANK`` or ``device_id``; a hardware profile without peak
data is replaced by the packaged profile whose SKU token -- ``mi355x`` etc. --
matches the detected device name), runs every invocation with a record sink
that derives metrics for ``ok`` records, and writes JSON / CSV / metadata.
If the suite enables profiling, the run is re-executed under the profiler
(teamredbench_amd.profiling.runtime).
"""
from __future__ import annotations

from dataclasses import dataclass
from datetime import datetime, timezone
import os
from pathlib import Path
import re
from typing import Callable

from teamredbench_amd import builtin as _builtin  # noqa: F401
from teamredbench_amd.benchmarks.base import BenchmarkContext, BenchmarkRecord
from teamredbench_amd.config import HardwareProfile, SuiteConfig, load_hardware_profile, load_suite
from teamredbench_amd.device import detect_device, load_torch
from teamredbench_amd.dtypes import discover_dtypes
from teamredbench_amd.io import write_results
from teamredbench_amd.profiling.runtime import effective_output_formats, profiling_enabled, run_profiled_suite
from teamredbench_amd.provenance import build_run_metadata
from teamredbench_amd.registry import get_benchmark, get_metric, load_plugins


@dataclass
class RunSummary:
    suite: SuiteConfig
    context: BenchmarkContext
    records: list[BenchmarkRecord]
    outputs: dict[str, Path]
    run_metadata: dict[str, object]
    profile_note: str | None = None


def _apply_metrics(record: BenchmarkRecord, metric_names: list[str]) -> None:
    if record.status != "ok":
        return
    for name in metric_names:
        record.metrics[name] = get_metric(name).compute(record.raw_metrics)


_SKU = re.compile(r"mi\d{3,4}x", re.IGNORECASE)


def _sku_tokens(text: str | None) -> set[str]:
    return {t.lower() for t in _SKU.findall(text or "")}


def _has_peaks(profile: HardwareProfile) -> bool:
    hbm = profile.peak_hbm_bandwidth_gbps
    compute = any(v is not None and float(v) > 0 for v in profile.peak_compute_tops.values())
    return hbm is not None and float(hbm) > 0 and compute


def _resolve_hardware_profile(profile: HardwareProfile, *, device_name: str | None,
                              repo_root: Path | None) -> tuple[HardwareProfile, str | None]:
    if _has_peaks(profile) or repo_root is None:
        return profile, None
    wanted = _sku_tokens(device_name)
    hardware_dir = repo_root / "configs" / "profiles" / "hardware"
    if not wanted or not hardware_dir.exists():
        return profile, None
    for path in sorted(hardware_dir.glob("*.yaml")):
        candidate = load_hardware_profile(path)
        if _sku_tokens(f"{candidate.name} {path.stem}") & wanted and _has_peaks(candidate):
            note = (f"Auto-selected hardware profile {candidate.name} from detected device {device_name!r} "
                    f"because {profile.name} has no theoretical peak data.")
            return candidate, note
    return profile, None


def build_context(suite: SuiteConfig, device_id: int = 0) -> tuple[BenchmarkContext, str | None]:
    resolved_id = int(os.environ.get("LOCAL_RANK", device_id))
    torch_module = load_torch()
    device_info = detect_device(torch_module, device_id=resolved_id)
    repo_root = suite.path.parent.parent.parent if suite.path else None
    profile, note = _resolve_hardware_profile(
        suite.hardware_profile, device_name=device_info.name if device_info else None, repo_root=repo_root
    )
    context = BenchmarkContext(
        hardware_profile=profile,
        runtime_profile=suite.runtime_profile,
        device_info=device_info,
        torch_module=torch_module,
        dtype_specs=discover_dtypes(torch_module),
        device_id=resolved_id,
        repo_root=repo_root,
        suite_path=suite.path,
    )
    return context, note


def run_suite(
    suite_path: str | Path,
    output_dir: str | Path | None = None,
    device_id: int = 0,
    record_callback: Callable[[BenchmarkRecord], None] | None = None,
) -> RunSummary:
    started = datetime.now(timezone.utc)
    suite = load_suite(suite_path)
    load_plugins(suite.plugins)
    target = Path(output_dir).resolve() if output_dir else suite.outputs.directory
    context, note = build_context(suite, device_id=device_id)
    suite.hardware_profile = context.hardware_profile
    if profiling_enabled(suite.profiling):
        return run_profiled_suite(suite=suite, context=context, output_dir=target.resolve(), device_id=device_id,
                                  record_callback=record_callback)

    records: list[BenchmarkRecord] = []
    for invocation in suite.benchmarks:
        cls = get_benchmark(invocation.benchmark)
        metric_names = invocation.metrics or list(cls.default_metrics)

        def sink(record: BenchmarkRecord, metric_names: list[str] = metric_names) -> None:
            _apply_metrics(record, metric_names)
            if record_callback is not None:
                record_callback(record)

        records.extend(cls(context=context, params=invocation.params, record_sink=sink).run())

    formats = effective_output_formats(suite.outputs.formats)
    run_metadata = build_run_metadata(
        suite=suite,
        context=context,
        requested_device_id=device_id,
        output_dir=target.resolve(),
        output_formats=formats,
        profile_note=note,
        started_at=started,
        finished_at=datetime.now(timezone.utc),
    )
    outputs = write_results(records=records, suite_name=suite.name, output_dir=target.resolve(), formats=formats,
                            run_metadata=run_metadata)
    return RunSummary(suite=suite, context=context, records=records, outputs=outputs, run_metadata=run_metadata,
                      profile_note=note)
