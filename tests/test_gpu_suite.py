"""The product API on the GPU (-m gpu): suites run through ``run_suite`` with
``backend: native`` (libmi355bench.so in-process) and ``backend: torch``
(PyTorch's own kernels, the reference torch path), and a profiled suite
whose metadata sidecar carries the rocprofv3 counters.

Each record must come back ``ok`` with the reference's result fields
(hbm_bandwidth_gbps / hbm_efficiency_pct / latency_us for ``hbm``,
achieved_tops / mfu_pct / latency_us for ``mfu``); native records also carry
the in-run parity check against the torch op on the same arrays, passed.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import yaml

from teamredbench_amd.runner import PACKAGED_HARDWARE_DIR, run_suite

pytestmark = pytest.mark.gpu

RUNTIME_PROFILE = PACKAGED_HARDWARE_DIR.parent / "rocm" / "rocm_7.yaml"
HARDWARE_PROFILE = PACKAGED_HARDWARE_DIR / "amd_instinct_mi355x.yaml"
HBM_FIELDS = ("hbm_bandwidth_gbps", "hbm_efficiency_pct", "latency_us")
MFU_FIELDS = ("achieved_tops", "mfu_pct", "latency_us")


def _write_suite(tmp: Path, name: str, benchmarks: list, profiling: dict | None = None) -> Path:
    doc = {"name": name, "device": {"profile": str(HARDWARE_PROFILE)}, "runtime": {"profile": str(RUNTIME_PROFILE)},
           "outputs": {"directory": str(tmp / "results"), "formats": ["json", "csv"]}, "benchmarks": benchmarks}
    if profiling is not None:
        doc["profiling"] = profiling
    path = tmp / f"{name}.yaml"
    path.write_text(yaml.safe_dump(doc), encoding="utf-8")
    return path


def _benchmarks(backend: str) -> list[dict]:
    hbm = {"backend": backend, "dtypes": ["float32", "bfloat16", "float16"], "modes": ["copy", "scale", "triad"],
           "elements": [(1 << 20) + 3], "scale": 3.0, "warmup": 2, "iterations": 5}
    mfu = {"backend": backend, "dtypes": ["bfloat16", "float16", "float8_e4m3fn"],
           "shapes": [[512, 512, 512], [16, 8192, 1024]], "warmup": 2, "iterations": 5}
    return [{"benchmark": "hbm", "params": hbm}, {"benchmark": "mfu", "params": mfu}]


@pytest.mark.parametrize("backend", ["native", "torch"])
def test_suite_runs_end_to_end(tmp_path: Path, backend: str):
    print(f"[suite] run_suite backend={backend}", flush=True)
    summary = run_suite(_write_suite(tmp_path, f"api-{backend}", _benchmarks(backend)))
    records = summary.records
    assert len(records) == 9 + 6
    for record in records:
        assert record.status == "ok", (record.benchmark, record.case, record.dtype, record.error)
        fields = HBM_FIELDS if record.benchmark == "hbm" else MFU_FIELDS
        for name in fields:
            value = record.metrics[name]
            assert value is not None and math.isfinite(value) and value > 0, (record.case, name, value)
        assert record.metadata["backend"] == backend
        if backend == "native":
            assert record.metadata["parity"]["passed"] is True, (record.case, record.metadata["parity"])
    skinny = [r for r in records if r.case == "gemm_16x8192x1024"]
    # memory-bound and cache-sized: both backends time it over operand copies that exceed the Infinity Cache
    assert all(r.metadata["operand_sets"] > 1 and r.metadata["cache_resident_b"] is False
               and r.metadata["operand_footprint_bytes"] >= 3 * 256 * (1 << 20) for r in skinny)
    if backend == "torch":
        fp8 = next(r for r in skinny if r.dtype == "float8_e4m3fn")
        assert fp8.metadata["torch_op"] == "_scaled_mm"
    for fmt in ("json", "csv", "metadata"):
        assert summary.outputs[fmt].exists()
    sidecar = json.loads(summary.outputs["metadata"].read_text(encoding="utf-8"))
    assert sidecar["record_status_counts"] == {"ok": 15}


def test_profiled_suite_attaches_counters(tmp_path: Path):
    # The rocprofv3 engine: a kernel-trace run whose records are kept, counter passes (FETCH_SIZE,
    # WRITE_SIZE, MFMA busy) over the same suite, and a calibration copy of known traffic; the parsed
    # per-kernel summary lands in the sidecar under run.profiling.counters.
    n = 1 << 28
    benchmarks = [
        {"benchmark": "hbm", "params": {"backend": "native", "dtypes": ["float32"], "modes": ["triad"],
                                        "elements": [n], "scale": 3.0, "warmup": 2, "iterations": 5}},
        {"benchmark": "mfu", "params": {"backend": "native", "dtypes": ["bfloat16"], "shapes": [[4096, 4096, 4096]],
                                        "warmup": 2, "iterations": 5}},
    ]
    profiling = {"enabled": True, "engine": "rocprofv3",
                 "params": {"kernel_include_regex": "stream_|gemm_",
                            "counter_passes": [["FETCH_SIZE"], ["WRITE_SIZE"],
                                               ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]]}}
    print("[suite] profiled run under rocprofv3 (trace, 3 counter passes, 2 calibration passes)", flush=True)
    summary = run_suite(_write_suite(tmp_path, "profiled", benchmarks, profiling))
    assert [r.status for r in summary.records] == ["ok", "ok"], [r.error for r in summary.records]
    sidecar = json.loads(summary.outputs["metadata"].read_text(encoding="utf-8"))
    # A profiler exit by SIGSEGV after complete output is tolerated and recorded, never silent.
    crashes = sidecar["run"]["profiling"].get("profiler_teardown_crashes", [])
    print(f"[suite] profiler_teardown_crashes: {crashes}", flush=True)
    assert all(c["exit_status"] in (-11, 139) and c["step"] for c in crashes), crashes
    counters = sidecar["run"]["profiling"]["counters"]
    assert set(counters["_calibration"]) == {"FETCH_SIZE", "WRITE_SIZE"}
    triad = [v for k, v in counters.items() if "stream_vec_kernel<2, 0" in k]
    assert len(triad) == 1, sorted(counters)
    algorithmic = 3 * 4 * n
    dram = triad[0]["dram_fetch_bytes"] + triad[0]["dram_write_bytes"]
    print(f"[suite] triad DRAM bytes {dram:.0f} vs algorithmic {algorithmic}", flush=True)
    assert abs(dram / algorithmic - 1) <= 0.02
    gemm = [v for k, v in counters.items() if "gemm_tiled_kernel" in k]
    assert gemm and all(0 < g["mfma_busy_pct"] <= 100 for g in gemm), gemm


def test_external_executable_runs_through_the_registry(tmp_path: Path):
    # A third-party kernel in the reference's executable contract: native/examples/stream_exec.hip,
    # built by hipcc for gfx950 through the content-keyed cache (build() prebuilt it, so the suite finds
    # it there), run once per case with the reference's argv, its last stdout line parsed as the record.
    from teamredbench_amd.native import build

    source = build.EXAMPLES_DIR / "stream_exec.hip"
    params = {"backend": "native", "dtypes": ["float32", "bfloat16"], "modes": ["copy", "scale", "triad"],
              "size_mib": 256, "scale": 3.0, "warmup": 2, "iterations": 10, **build.example_params(source)}
    print("[suite] external executable example", flush=True)
    summary = run_suite(_write_suite(tmp_path, "external", [{"benchmark": "hbm", "params": params}]))
    f32 = [r for r in summary.records if r.dtype == "float32"]
    assert len(f32) == 3
    for record in f32:
        assert record.status == "ok", record.error
        assert record.metadata["implementation"] == "example_stream_exec"
        assert record.metadata["arch"].startswith("gfx950")
        assert record.metrics["hbm_bandwidth_gbps"] > 100 and record.raw_metrics["moved_bytes"] > 0
    # the example takes float32 only: other dtypes come back as the executable's own skip
    bf16 = [r for r in summary.records if r.dtype == "bfloat16"]
    assert len(bf16) == 3 and all(r.status == "skipped" and "float32" in r.error for r in bf16)
