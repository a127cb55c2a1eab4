"""Result files of a suite run.

Three files share one stem, ``<suite>-<UTC timestamp>``, in the output
directory: ``.json`` (a list of record objects), ``.csv`` (one flat row per
record) and ``.metadata.json`` (the sidecar: schema_version 1, counts by
status, the paths written, and the run's provenance under ``run``). These
are the reference's formats (src/teamredbench/io.py:12-87) -- tools that read
its results read these. The record forms themselves are
``BenchmarkRecord.to_dict`` / ``to_row``. The sidecar is always written;
JSON and CSV only when the suite's ``outputs.formats`` asks for them, and a
format this writer does not know is listed in the sidecar under
``ignored_formats`` instead of failing the run after its measurements.
"""
from __future__ import annotations

from collections import Counter
import csv
from datetime import datetime, timezone
import json
from pathlib import Path
from typing import Any, Callable, Iterable

from teamredbench_amd.benchmarks.base import BenchmarkRecord

SIDECAR_SCHEMA_VERSION = 1


def _utc_stamp(moment: datetime) -> str:
    return moment.strftime("%Y%m%dT%H%M%SZ")


def _iso_utc(moment: datetime) -> str:
    return moment.isoformat().replace("+00:00", "Z")


class ResultWriter:
    """Writes one run's records under ``<output_dir>/<suite>-<stamp>.*``."""

    def __init__(self, output_dir: Path, suite_name: str, now: datetime | None = None):
        self.output_dir = Path(output_dir)
        self.created = now or datetime.now(timezone.utc)
        self.stem = f"{suite_name}-{_utc_stamp(self.created)}"
        self.suite_name = suite_name

    def path(self, suffix: str) -> Path:
        return self.output_dir / f"{self.stem}{suffix}"

    def write_json(self, records: list[BenchmarkRecord]) -> Path:
        target = self.path(".json")
        target.write_text(json.dumps([r.to_dict() for r in records], indent=2), encoding="utf-8")
        return target

    def write_csv(self, records: list[BenchmarkRecord]) -> Path:
        target = self.path(".csv")
        rows = [r.to_row() for r in records]
        columns = sorted(set().union(*rows)) if rows else ["benchmark", "case", "dtype", "error", "status"]
        with target.open("w", encoding="utf-8", newline="") as handle:
            writer = csv.DictWriter(handle, fieldnames=columns)
            writer.writeheader()
            writer.writerows(rows)
        return target

    WRITERS: dict[str, Callable[["ResultWriter", list[BenchmarkRecord]], Path]] = {
        "json": write_json,
        "csv": write_csv,
    }

    def write(self, records: Iterable[BenchmarkRecord], formats: list[str],
              run_metadata: dict[str, Any] | None = None) -> dict[str, Path]:
        records = list(records)
        self.output_dir.mkdir(parents=True, exist_ok=True)
        outputs = {fmt: self.WRITERS[fmt](self, records) for fmt in self.WRITERS if fmt in formats}
        outputs["metadata"] = self.path(".metadata.json")
        sidecar: dict[str, Any] = {
            "schema_version": SIDECAR_SCHEMA_VERSION,
            "suite_name": self.suite_name,
            "generated_at_utc": _iso_utc(datetime.now(timezone.utc)),
            "record_count": len(records),
            "record_status_counts": dict(Counter(r.status for r in records)),
            "outputs": {name: str(path) for name, path in outputs.items()},
            "run": run_metadata or {},
        }
        unknown = [fmt for fmt in formats if fmt not in self.WRITERS]
        if unknown:
            sidecar["ignored_formats"] = unknown
        outputs["metadata"].write_text(json.dumps(sidecar, indent=2), encoding="utf-8")
        return outputs


def write_results(records: Iterable[BenchmarkRecord], suite_name: str, output_dir: Path, formats: list[str],
                  run_metadata: dict[str, object] | None = None) -> dict[str, Path]:
    """Write the result files of one run; returns {"json"|"csv"|"metadata": path}."""
    return ResultWriter(output_dir, suite_name).write(records, formats, run_metadata)


def read_results(sidecar_path: Path) -> tuple[dict[str, Any], list[BenchmarkRecord]]:
    """The sidecar of a run and the records of the JSON file it names."""
    sidecar = json.loads(Path(sidecar_path).read_text(encoding="utf-8"))
    json_path = sidecar.get("outputs", {}).get("json")
    if json_path is None or not Path(json_path).exists():
        raise FileNotFoundError(f"{sidecar_path} names no JSON results file")
    payload = json.loads(Path(json_path).read_text(encoding="utf-8"))
    return sidecar, [BenchmarkRecord.from_dict(item) for item in payload]
