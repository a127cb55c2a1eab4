"""Result writers: JSON records, flattened CSV and the metadata sidecar
(formats of src/teamredbench/io.py:12-87; sidecar schema_version 1)."""
from __future__ import annotations

import csv
from datetime import datetime, timezone
import json
from pathlib import Path
from typing import Iterable

from teamredbench_amd.benchmarks.base import BenchmarkRecord


def record_to_dict(record: BenchmarkRecord) -> dict[str, object]:
    return {
        "benchmark": record.benchmark,
        "case": record.case,
        "dtype": record.dtype,
        "status": record.status,
        "error": record.error,
        "metrics": record.metrics,
        "raw_metrics": record.raw_metrics,
        "metadata": record.metadata,
    }


def record_to_row(record: BenchmarkRecord) -> dict[str, object]:
    row: dict[str, object] = {
        "benchmark": record.benchmark,
        "case": record.case,
        "dtype": record.dtype,
        "status": record.status,
        "error": record.error or "",
    }
    for prefix, mapping in (("metric", record.metrics), ("raw", record.raw_metrics), ("meta", record.metadata)):
        for key in sorted(mapping):
            value = mapping[key]
            row[f"{prefix}_{key}"] = json.dumps(value) if isinstance(value, (dict, list)) else value
    return row


def write_results(
    records: Iterable[BenchmarkRecord],
    suite_name: str,
    output_dir: Path,
    formats: list[str],
    run_metadata: dict[str, object] | None = None,
) -> dict[str, Path]:
    records = list(records)
    output_dir.mkdir(parents=True, exist_ok=True)
    stamp = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%SZ")
    stem = output_dir / f"{suite_name}-{stamp}"
    outputs: dict[str, Path] = {}

    if "json" in formats:
        path = stem.with_name(stem.name + ".json")
        path.write_text(json.dumps([record_to_dict(r) for r in records], indent=2), encoding="utf-8")
        outputs["json"] = path

    if "csv" in formats:
        path = stem.with_name(stem.name + ".csv")
        rows = [record_to_row(r) for r in records]
        columns = sorted({key for row in rows for key in row})
        with path.open("w", encoding="utf-8", newline="") as handle:
            writer = csv.DictWriter(handle, fieldnames=columns)
            writer.writeheader()
            writer.writerows(rows)
        outputs["csv"] = path

    meta_path = stem.with_name(stem.name + ".metadata.json")
    outputs["metadata"] = meta_path
    counts: dict[str, int] = {}
    for record in records:
        counts[record.status] = counts.get(record.status, 0) + 1
    payload = {
        "schema_version": 1,
        "suite_name": suite_name,
        "generated_at_utc": datetime.now(timezone.utc).isoformat().replace("+00:00", "Z"),
        "record_count": len(records),
        "record_status_counts": counts,
        "outputs": {name: str(path) for name, path in outputs.items()},
        "run": run_metadata or {},
    }
    meta_path.write_text(json.dumps(payload, indent=2), encoding="utf-8")
    return outputs
