"""The reference's own suite files, run unchanged through run_suite (-m gpu).

tests/golden/reference_suites/ holds byte-for-byte copies of the reference's
configs/suites/native_smoke.yaml, native_gemm_smoke.yaml and
rocprof_hbm_smoke.yaml (tests/golden/copy_reference_suites.py made them).
Each test lays out a tree the way the reference's repository is laid out --
configs/suites/<suite>.yaml beside configs/profiles/hardware/cdna_generic.yaml
and configs/profiles/rocm/rocm_generic.yaml, the profiles this package
ships under those names -- and runs the suite file as it is:

  * every record comes back ``ok`` with the reference's result fields;
  * the generic hardware profile (no peak figures) is replaced by the MI355X
    profile found for the detected device, so hbm_efficiency_pct and mfu_pct
    are percentages of the MI355X peaks;
  * the reference's kernel names (hbm_hip, mfu_hipblas) run the gfx950
    library in-process, with its in-run parity check passed;
  * the profiled suite runs under the ``rocprof`` engine name with the v1
    parameters it sets (stats, hip_trace), and its sidecar carries the
    rocprofv3 kernel trace and counters.
"""
from __future__ import annotations

import json
import math
from pathlib import Path
import shutil

import pytest

from teamredbench_amd.runner import PACKAGED_HARDWARE_DIR, run_suite

pytestmark = pytest.mark.gpu

FIXTURES = Path(__file__).resolve().parent / "golden" / "reference_suites"
FIELDS = {"hbm": ("hbm_bandwidth_gbps", "hbm_efficiency_pct", "latency_us"),
          "mfu": ("achieved_tops", "mfu_pct", "latency_us")}


def _reference_tree(tmp: Path, suite: str) -> Path:
    """<tmp>/configs/suites/<suite> with the two profiles the suite names at their relative paths."""
    profiles = tmp / "configs" / "profiles"
    (profiles / "hardware").mkdir(parents=True)
    (profiles / "rocm").mkdir(parents=True)
    shutil.copyfile(PACKAGED_HARDWARE_DIR / "cdna_generic.yaml", profiles / "hardware" / "cdna_generic.yaml")
    shutil.copyfile(PACKAGED_HARDWARE_DIR.parent / "rocm" / "rocm_generic.yaml", profiles / "rocm" / "rocm_generic.yaml")
    suites = tmp / "configs" / "suites"
    suites.mkdir(parents=True)
    shutil.copyfile(FIXTURES / suite, suites / suite)
    return suites / suite


def _check_records(summary, expected: int) -> None:
    assert summary.profile_note and "amd-instinct-mi355x" in summary.profile_note, summary.profile_note
    assert summary.context.hardware_profile.name == "amd-instinct-mi355x"
    assert len(summary.records) == expected
    for record in summary.records:
        assert record.status == "ok", (record.benchmark, record.case, record.dtype, record.error)
        for name in FIELDS[record.benchmark]:
            value = record.metrics.get(name)
            assert value is not None and math.isfinite(value) and value > 0, (record.case, record.dtype, name, value)
        assert record.metadata["parity"]["passed"] is True, (record.case, record.dtype, record.metadata["parity"])


def test_reference_native_smoke_suite(tmp_path: Path):
    # 4 dtypes x copy / scale / triad at 2048 MiB per array, and 4 dtypes of 4096^3 GEMM
    print("[reference-suite] native_smoke.yaml", flush=True)
    summary = run_suite(_reference_tree(tmp_path, "native_smoke.yaml"))
    _check_records(summary, 12 + 4)
    assert {r.dtype for r in summary.records if r.benchmark == "hbm"} == {"float16", "bfloat16", "float32", "float64"}
    assert (tmp_path / "results" / "native_smoke").is_dir()   # ../../results, as in the reference's tree


def test_reference_native_gemm_smoke_suite(tmp_path: Path):
    print("[reference-suite] native_gemm_smoke.yaml", flush=True)
    summary = run_suite(_reference_tree(tmp_path, "native_gemm_smoke.yaml"))
    _check_records(summary, 4)
    for record in summary.records:    # the suite's own metric list
        assert set(record.metrics) == {"achieved_tops", "mfu_pct", "latency_us"}


def test_reference_rocprof_hbm_smoke_suite(tmp_path: Path):
    print("[reference-suite] rocprof_hbm_smoke.yaml under the rocprof engine", flush=True)
    summary = run_suite(_reference_tree(tmp_path, "rocprof_hbm_smoke.yaml"))
    _check_records(summary, 1)
    sidecar = json.loads(summary.outputs["metadata"].read_text(encoding="utf-8"))
    profiling = sidecar["run"]["profiling"]
    crashes = profiling.get("profiler_teardown_crashes", [])
    print(f"[reference-suite] profiler_teardown_crashes: {crashes}", flush=True)
    assert profiling["engine"] == "rocprof"
    trace = profiling["command"][:profiling["command"].index("--")]
    assert "--stats" in trace and "--hip-trace" in trace
    copy = [v for k, v in profiling["counters"].items() if "stream_vec_kernel<0, 0" in k]
    assert len(copy) == 1 and copy[0]["dispatches"] >= 5, sorted(profiling["counters"])
    # calibrated DRAM bytes of the copy against its algorithmic 2 x 256 MiB (the 512 MiB it touches is
    # about twice the Infinity Cache, so most of it streams from HBM; a parse or calibration failure
    # would be off by a factor)
    ratio = (copy[0]["dram_fetch_bytes"] + copy[0]["dram_write_bytes"]) / (2 * 256 * (1 << 20))
    print(f"[reference-suite] copy DRAM bytes / algorithmic = {ratio:.4f}", flush=True)
    assert 0.75 <= ratio <= 1.25
