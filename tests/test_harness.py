"""The registry/suite/record/metric harness around the native path (CPU only).

Mirrors the reference's own unit and integration tests
(tests/test_metrics.py, test_registry.py, test_runner.py, test_native.py,
test_autoprofile.py, test_config.py, test_profiles.py): the metric
known-answer values are the reference's numbers, and the external-executable
contract is driven through fake executables written by the test.
"""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import yaml

import teamredbench_amd.builtin  # noqa: F401
from teamredbench_amd import runner as runner_mod
from teamredbench_amd.benchmarks.base import Benchmark, BenchmarkRecord
from teamredbench_amd.config import load_hardware_profile, load_suite
from teamredbench_amd.device import DeviceInfo
from teamredbench_amd.metrics.common import (
    achieved_tops,
    bus_bandwidth_gbps,
    gemm_bandwidth_gbps,
    hbm_bandwidth_gbps,
    hbm_efficiency_pct,
    latency_us,
    link_efficiency_pct,
    mfu_pct,
    payload_bandwidth_gbps,
)
from teamredbench_amd.native import runtime as native_runtime
from teamredbench_amd.native.registry import get_native_kernel, list_native_kernels, registered_names
from teamredbench_amd.native.runtime import ResolvedNativeKernel
from teamredbench_amd.registry import get_benchmark, list_benchmarks, list_metrics, register_benchmark
from teamredbench_amd.runner import run_suite

PACKAGE = Path(teamredbench_amd.builtin.__file__).resolve().parent
HW_DIR = PACKAGE / "configs" / "profiles" / "hardware"


# ---------------------------------------------------------------- metrics
def test_hbm_metrics_known_answers():
    raw = {"elapsed_s": 0.5, "moved_bytes": 1_000_000_000, "peak_bandwidth_gbps": 4.0}
    assert hbm_bandwidth_gbps(raw) == 2.0
    assert hbm_efficiency_pct(raw) == 50.0
    assert latency_us(raw) == 500000.0


def test_mfu_metrics_known_answers():
    raw = {"elapsed_s": 0.1, "achieved_ops": 5_000_000_000_000, "peak_tops": 100.0}
    assert achieved_tops(raw) == 50.0
    assert mfu_pct(raw) == 50.0


def test_collective_metrics_known_answers():
    raw = {"elapsed_s": 0.25, "payload_bytes": 500_000_000, "bus_factor": 1.5, "peak_link_bandwidth_gbps": 4.0}
    assert payload_bandwidth_gbps(raw) == 2.0
    assert bus_bandwidth_gbps(raw) == 3.0
    assert link_efficiency_pct(raw) == 75.0


def test_metrics_are_none_without_inputs():
    assert mfu_pct({"elapsed_s": 0.001, "achieved_ops": 1e9}) is None
    assert hbm_efficiency_pct({"elapsed_s": 0.001, "moved_bytes": 1e9, "peak_bandwidth_gbps": 0}) is None
    assert hbm_bandwidth_gbps({"moved_bytes": 1e9}) is None
    assert gemm_bandwidth_gbps({"elapsed_s": 2.0, "gemm_bytes": 4e9}) == 2.0


# ---------------------------------------------------------------- registries
def test_builtin_benchmarks_metrics_and_native_kernels():
    assert {"hbm", "mfu"} <= set(list_benchmarks())
    assert {"latency_us", "hbm_bandwidth_gbps", "hbm_efficiency_pct", "achieved_tops", "mfu_pct"} <= set(list_metrics())
    # the reference's built-in kernel names resolve to the gfx950 kernels
    assert {"hbm_hip", "mfu_hipblas", "hbm_gfx950", "mfu_gfx950"} <= registered_names()
    assert get_native_kernel("hbm_hip").name == "hbm_gfx950"
    assert get_native_kernel("mfu_hipblas").benchmark == "mfu"
    assert {d.name for d in list_native_kernels()} >= {"hbm_gfx950", "mfu_gfx950"}


# ---------------------------------------------------------------- suite plumbing
def _write_profiles(tmp: Path, compute: dict | None = None, hbm: float = 4000) -> tuple[Path, Path]:
    hardware, runtime = tmp / "hardware.yaml", tmp / "runtime.yaml"
    hardware.write_text(yaml.safe_dump({
        "name": "test-hw", "family": "cdna", "peak_hbm_bandwidth_gbps": hbm,
        "peak_link_bandwidth_gbps": {"xgmi": 1, "network": 1},
        "peak_compute_tops": compute if compute is not None else {"float32": 100},
    }), encoding="utf-8")
    runtime.write_text(yaml.safe_dump({"name": "test-runtime", "rocm_version": "test", "libraries": {}, "env": {}}),
                       encoding="utf-8")
    return hardware, runtime


def _write_suite(tmp: Path, name: str, benchmarks: list, formats=("json",), compute=None, hbm=4000) -> Path:
    hardware, runtime = _write_profiles(tmp, compute, hbm)
    suite = tmp / "suite.yaml"
    suite.write_text(yaml.safe_dump({
        "name": name, "device": {"profile": str(hardware)}, "runtime": {"profile": str(runtime)},
        "outputs": {"directory": str(tmp / "results"), "formats": list(formats)}, "benchmarks": benchmarks,
    }), encoding="utf-8")
    return suite


@register_benchmark("test_dummy_callback")
class DummyCallbackBenchmark(Benchmark):
    default_metrics = ["latency_us", "mfu_pct"]

    def run(self) -> list[BenchmarkRecord]:
        return [self.emit_record(BenchmarkRecord(benchmark=self.name, case="single", dtype="float32",
                                                 raw_metrics={"elapsed_s": 0.001, "achieved_ops": 1e9}))]


def test_run_suite_invokes_record_callback_with_metrics(tmp_path: Path):
    suite = _write_suite(tmp_path, "callback-suite", [{"benchmark": "test_dummy_callback"}], formats=("json", "csv"),
                         compute={"float32": 1}, hbm=1)
    seen: list[BenchmarkRecord] = []
    summary = run_suite(suite, record_callback=seen.append)
    assert len(summary.records) == 1 and len(seen) == 1
    assert seen[0].metrics["latency_us"] == 1000.0
    assert seen[0].metrics["mfu_pct"] is None          # no peak_tops in the raw metrics
    for key in ("json", "csv", "metadata"):
        assert summary.outputs[key].exists()
    records = json.loads(summary.outputs["json"].read_text(encoding="utf-8"))
    meta = json.loads(summary.outputs["metadata"].read_text(encoding="utf-8"))
    assert records[0]["benchmark"] == "test_dummy_callback"
    assert meta["record_count"] == 1
    assert meta["outputs"]["json"] == str(summary.outputs["json"])
    assert meta["run"]["configs"]["suite"]["raw"]["name"] == "callback-suite"
    assert meta["run"]["configs"]["hardware_profile"]["raw"]["name"] == "test-hw"


# ---------------------------------------------------------------- executable contract
def _fake_executable(path: Path, seen: Path, payload: dict | str, exit_code: int = 0) -> None:
    line = payload if isinstance(payload, str) else json.dumps(payload)
    path.write_text("\n".join([
        "#!/usr/bin/env python3",
        "import json, sys",
        f"open({str(seen)!r}, 'w', encoding='utf-8').write(json.dumps(sys.argv[1:]))",
        "print('noise before the contract line')",
        f"print({line!r})",
        f"sys.exit({exit_code})",
    ]), encoding="utf-8")
    path.chmod(0o755)


def test_hbm_native_backend_runs_an_external_binary(tmp_path: Path):
    seen = tmp_path / "args.json"
    _fake_executable(tmp_path / "fake_hbm.py", seen,
                     {"status": "ok", "raw_metrics": {"elapsed_s": 0.002}, "metadata": {"executor": "fake"}})
    suite = _write_suite(tmp_path, "native-hbm", [{"benchmark": "hbm", "params": {
        "backend": "native", "dtypes": ["float32"], "modes": ["copy"], "size_mib": 1024, "warmup": 2,
        "iterations": 5, "native": {"binary": "./fake_hbm.py"}}}])
    record = run_suite(suite).records[0]
    assert record.status == "ok" and record.metadata["executor"] == "fake"
    assert record.metrics["hbm_bandwidth_gbps"] == pytest.approx(1073.741824)
    assert record.metrics["hbm_efficiency_pct"] == pytest.approx(26.8435456)
    argv = json.loads(seen.read_text(encoding="utf-8"))
    for token in ("--dtype", "float32", "--mode", "copy", "--size-mib", "1024", "--warmup", "2", "--iterations", "5"):
        assert token in argv


def test_mfu_native_backend_runs_an_external_binary(tmp_path: Path):
    seen = tmp_path / "args.json"
    _fake_executable(tmp_path / "fake_mfu.py", seen,
                     {"status": "ok", "raw_metrics": {"elapsed_s": 0.001}, "metadata": {"executor": "fake"}})
    suite = _write_suite(tmp_path, "native-mfu", [{"benchmark": "mfu", "params": {
        "backend": "native", "dtypes": ["float32"], "shapes": [[1024, 1024, 1024]], "warmup": 2, "iterations": 5,
        "native": {"binary": "./fake_mfu.py"}}}], compute={"float32": 20})
    record = run_suite(suite).records[0]
    assert record.status == "ok"
    assert record.metrics["achieved_tops"] == pytest.approx(2.147483648)
    assert record.metrics["mfu_pct"] == pytest.approx(10.73741824)
    argv = json.loads(seen.read_text(encoding="utf-8"))
    for flag in ("--m", "--n", "--k", "--dtype"):
        assert flag in argv
    assert argv.count("1024") == 3


@pytest.mark.parametrize("payload, code, error", [
    ({"status": "ok", "raw_metrics": {"elapsed_s": 0.001}}, 3, "exit"),
    ("this is not json", 0, "JSON"),
    ({"status": "skipped", "error": "unsupported dtype"}, 0, "unsupported dtype"),
    ({"status": "ok", "raw_metrics": {}}, 0, "elapsed_s"),
])
def test_executable_failures_become_skipped_records(tmp_path: Path, payload, code, error):
    _fake_executable(tmp_path / "fake.py", tmp_path / "args.json", payload, exit_code=code)
    suite = _write_suite(tmp_path, "failing", [{"benchmark": "hbm", "params": {
        "backend": "native", "dtypes": ["float32"], "modes": ["copy", "triad"], "size_mib": 1,
        "native": {"binary": "./fake.py"}}}])
    records = run_suite(suite).records
    assert len(records) == 2
    for record in records:
        assert record.status == "skipped"
        assert error.lower() in (record.error or "").lower()
        assert record.metrics == {}


def test_elapsed_seconds_alias_is_accepted(tmp_path: Path):
    _fake_executable(tmp_path / "fake.py", tmp_path / "args.json",
                     {"status": "ok", "raw_metrics": {"elapsed_seconds": 0.5, "moved_bytes": 1e9}})
    suite = _write_suite(tmp_path, "alias", [{"benchmark": "hbm", "params": {
        "backend": "native", "dtypes": ["float32"], "modes": ["copy"], "size_mib": 1,
        "native": {"binary": "./fake.py"}}}])
    record = run_suite(suite).records[0]
    assert record.status == "ok" and record.metrics["hbm_bandwidth_gbps"] == 2.0


def test_missing_binary_skips_every_case(tmp_path: Path):
    suite = _write_suite(tmp_path, "missing", [{"benchmark": "mfu", "params": {
        "backend": "native", "dtypes": ["float32"], "shapes": [[64, 64, 64], [128, 128, 128]],
        "native": {"binary": "./does_not_exist"}}}], compute={"float32": 1})
    records = run_suite(suite).records
    assert [r.status for r in records] == ["skipped", "skipped"]


def test_mfu_gates_dtypes_without_a_peak(tmp_path: Path):
    _fake_executable(tmp_path / "fake.py", tmp_path / "args.json",
                     {"status": "ok", "raw_metrics": {"elapsed_s": 0.001}})
    suite = _write_suite(tmp_path, "gate", [{"benchmark": "mfu", "params": {
        "backend": "native", "dtypes": ["float16"], "shapes": [[64, 64, 64]],
        "native": {"binary": "./fake.py"}}}], compute={"float32": 1})
    record = run_suite(suite).records[0]
    assert record.status == "skipped" and "peak" in record.error.lower()


# ---------------------------------------------------------------- built-in C-ABI kernels on a host without a GPU
class _TorchWithoutDevice:
    """The real torch module with no visible GPU."""

    def __init__(self):
        import torch

        self._torch = torch
        self.cuda = SimpleNamespace(is_available=lambda: False)

    def __getattr__(self, name):
        return getattr(self._torch, name)


def test_builtin_kernels_skip_cleanly_without_a_device(tmp_path: Path, monkeypatch):
    monkeypatch.setattr(runner_mod, "load_torch", _TorchWithoutDevice)
    suite = _write_suite(tmp_path, "builtin", [
        {"benchmark": "hbm", "params": {"backend": "native", "dtypes": ["float32"], "modes": ["copy", "triad"],
                                        "size_mib": 1}},
        {"benchmark": "mfu", "params": {"backend": "native", "dtypes": ["float32"], "shapes": [[64, 64, 64]]}},
    ], compute={"float32": 1})
    records = run_suite(suite).records
    assert len(records) == 3
    assert all(r.status == "skipped" for r in records)
    assert all(r.metadata.get("kernel") in ("hbm_gfx950", "mfu_gfx950") for r in records)


# ---------------------------------------------------------------- native cache
def test_prepare_native_kernel_binary_rebuilds_when_local_include_changes(tmp_path: Path, monkeypatch):
    source, include = tmp_path / "kernel.hip.cpp", tmp_path / "kernel_impl.hip.hpp"
    source.write_text('#include "kernel_impl.hip.hpp"\nint main() { return kValue; }\n', encoding="utf-8")
    include.write_text("static constexpr int kValue = 0;\n", encoding="utf-8")
    monkeypatch.setattr(native_runtime, "_find_hip_compiler", lambda preferred=None: "/opt/rocm/bin/hipcc")
    outputs: list[Path] = []

    def fake_run(command, **_):
        out = Path(command[command.index("-o") + 1])
        out.write_text("fake-binary", encoding="utf-8")
        outputs.append(out)
        return SimpleNamespace(returncode=0, stderr="", stdout="")

    monkeypatch.setattr(native_runtime.subprocess, "run", fake_run)
    kernel = ResolvedNativeKernel(benchmark="mfu", name="unit-test-kernel", description="cache test",
                                  source_path=source, cache_dir=tmp_path / "cache")
    first = native_runtime.prepare_native_kernel_binary(kernel)
    assert native_runtime.prepare_native_kernel_binary(kernel) == first and len(outputs) == 1  # cached
    include.write_text("static constexpr int kValue = 1;\n", encoding="utf-8")
    second = native_runtime.prepare_native_kernel_binary(kernel)
    assert first != second and len(outputs) == 2 and first.exists() and second.exists()
    # each build lands under a temporary name first and is renamed into place
    assert all(not out.exists() and out.name.endswith(".tmp") for out in outputs)


def test_clean_native_cache_command_removes_entries(tmp_path: Path):
    from typer.testing import CliRunner

    from teamredbench_amd.cli import app

    cache = tmp_path / "native-cache"
    cache.mkdir()
    (cache / "kernel-a").write_text("a", encoding="utf-8")
    (cache / "kernel-b").mkdir()
    (cache / "kernel-b" / "payload").write_text("b", encoding="utf-8")
    result = CliRunner().invoke(app, ["clean-native-cache", "--cache-dir", str(cache)])
    assert result.exit_code == 0
    assert f"Native cache: {cache}" in result.stdout and "Removed entries: 2" in result.stdout
    assert list(cache.iterdir()) == []


def test_cli_lists_native_kernels():
    from typer.testing import CliRunner

    from teamredbench_amd.cli import app

    result = CliRunner().invoke(app, ["list-native-kernels"])
    assert result.exit_code == 0 and "hbm_gfx950" in result.stdout and "mfu_gfx950" in result.stdout


# ---------------------------------------------------------------- profiles
def test_mi355x_profile_peaks():
    profile = load_hardware_profile(HW_DIR / "amd_instinct_mi355x.yaml")
    assert profile.peak_hbm_bandwidth_gbps == 8000.0
    assert profile.peak_compute_tops["bfloat16"] == 2500.0
    assert profile.peak_compute_tops["float16"] == 2500.0
    assert profile.peak_compute_tops["float8_e4m3fn"] == 5000.0


def test_packaged_suites_load():
    for suite_path in sorted((PACKAGE / "configs" / "suites").glob("*.yaml")):
        suite = load_suite(suite_path)
        assert suite.benchmarks, suite_path
        for inv in suite.benchmarks:
            assert get_benchmark(inv.benchmark)


def test_generic_profile_is_replaced_by_the_detected_sku(monkeypatch):
    monkeypatch.setattr(runner_mod, "load_torch", lambda: object())
    monkeypatch.setattr(runner_mod, "detect_device",
                        lambda torch_module, device_id=0: DeviceInfo(index=0, name="AMD Instinct MI355X"))
    suite = load_suite(PACKAGE / "configs" / "suites" / "native_smoke.yaml")
    context, note = runner_mod.build_context(suite)
    assert context.hardware_profile.name == "amd-instinct-mi355x"
    assert note and "Auto-selected" in note


# ---------------------------------------------------------------- record status and result files
@register_benchmark("test_parity_outcomes")
class ParityOutcomeBenchmark(Benchmark):
    """Emits one record whose in-run parity check passed and one whose check failed."""

    default_metrics = ["latency_us", "hbm_bandwidth_gbps"]

    def run(self) -> list[BenchmarkRecord]:
        raw = {"elapsed_s": 0.002, "moved_bytes": 2e9, "peak_bandwidth_gbps": 8000.0}
        return [self.measured(case=case, dtype="float32", raw_metrics=dict(raw),
                              metadata={"parity": {"vs": "torch", "max_ulp": ulp, "bound_ulp": 1, "passed": ulp <= 1}})
                for case, ulp in (("good", 0), ("bad", 7))]


def test_a_failed_parity_check_fails_the_record_and_the_cli(tmp_path: Path):
    from typer.testing import CliRunner

    from teamredbench_amd.cli import app

    suite = _write_suite(tmp_path, "parity", [{"benchmark": "test_parity_outcomes"}], formats=("json", "csv"))
    good, bad = run_suite(suite).records
    assert good.status == "ok" and good.metrics["hbm_bandwidth_gbps"] == pytest.approx(1000.0)
    # the wrong kernel keeps its timing for diagnosis but publishes no rate
    assert bad.status == "failed" and bad.metrics == {} and bad.raw_metrics["elapsed_s"] == 0.002
    assert "parity" in bad.error and "max_ulp=7" in bad.error
    result = CliRunner().invoke(app, ["run", str(suite)])
    assert result.exit_code == 1
    assert "[FAILED] test_parity_outcomes case=bad" in result.stdout and "(1 failed)" in result.stdout
    sidecar = json.loads(next((tmp_path / "results").glob("parity-*.metadata.json")).read_text(encoding="utf-8"))
    assert sidecar["record_status_counts"] == {"ok": 1, "failed": 1}


def test_record_round_trips_through_its_result_forms():
    record = BenchmarkRecord(benchmark="mfu", case="gemm_8x8x8", dtype="bfloat16", raw_metrics={"elapsed_s": 1e-6},
                             metadata={"parity": {"passed": True}, "shape": [8, 8, 8]}, metrics={"mfu_pct": 1.5})
    assert BenchmarkRecord.from_dict(json.loads(json.dumps(record.to_dict()))) == record
    row = record.to_row()
    assert row["metric_mfu_pct"] == 1.5 and row["error"] == ""
    # nested values reach the CSV as the reference writes them: str(value), Python's text of the value
    import ast
    import csv
    import io as _io

    buf = _io.StringIO()
    writer = csv.DictWriter(buf, fieldnames=list(row))
    writer.writeheader()
    writer.writerow(row)
    cells = next(csv.DictReader(_io.StringIO(buf.getvalue())))
    assert cells["meta_parity"] == "{'passed': True}" and ast.literal_eval(cells["meta_shape"]) == [8, 8, 8]


def test_unknown_output_formats_are_reported_not_fatal(tmp_path: Path):
    suite = _write_suite(tmp_path, "formats", [{"benchmark": "test_dummy_callback"}], formats=("json", "parquet"))
    summary = run_suite(suite)
    sidecar = json.loads(summary.outputs["metadata"].read_text(encoding="utf-8"))
    assert set(summary.outputs) == {"json", "metadata"} and sidecar["ignored_formats"] == ["parquet"]


@pytest.mark.parametrize("mutate, message", [
    (lambda doc: doc.update(benchmarks=[{"benchmark": "hbm", "params": [1, 2]}]), "benchmarks[0].params must be a mapping"),
    (lambda doc: doc.update(benchmarks=[{"params": {}}]), "benchmarks[0].benchmark is required"),
    (lambda doc: doc.update(device={}), "device.profile is required"),
    (lambda doc: doc.update(plugins="not-a-list"), "plugins must be a list"),
])
def test_malformed_suites_name_the_offending_key(tmp_path: Path, mutate, message):
    from teamredbench_amd.config import ConfigError

    suite = _write_suite(tmp_path, "broken", [{"benchmark": "test_dummy_callback"}])
    doc = yaml.safe_load(suite.read_text(encoding="utf-8"))
    mutate(doc)
    suite.write_text(yaml.safe_dump(doc), encoding="utf-8")
    with pytest.raises(ConfigError, match=message.replace("[", r"\[").replace("]", r"\]")):
        load_suite(suite)


def test_discover_suggests_the_packaged_profile_of_the_detected_sku(monkeypatch):
    from teamredbench_amd import device

    monkeypatch.setattr(device, "detect_device", lambda torch_module, device_id=0: DeviceInfo(index=0, name="AMD Instinct MI355X"))
    monkeypatch.setattr(device, "_run_command", lambda command: None)
    payload = device.discover_environment(None)
    assert payload["suggested_hardware_profile"]["name"] == "amd-instinct-mi355x"
    assert payload["suggested_hardware_profile"]["peak_hbm_bandwidth_gbps"] == 8000
    assert payload["runtime"]["hipcc_version"] is None and "cuda_api_version" not in payload["runtime"]["torch"]


def test_example_executable_is_prebuilt_under_the_key_a_suite_resolves():
    # build() builds native/examples/*.hip into the in-tree cache under the content key that a suite
    # selecting the example resolves to, so the GPU box runs it without compiling.
    import teamredbench_amd.native.builtin  # noqa: F401
    from teamredbench_amd.native import build

    source = build.EXAMPLES_DIR / "stream_exec.hip"
    kernel = native_runtime.resolve_native_kernel(benchmark="hbm", params=build.example_params(source),
                                                  suite_path=Path("/elsewhere/suite.yaml"), repo_root=None,
                                                  default_kernel="hbm_hip")
    assert kernel.abi == "executable" and kernel.source_path == source and kernel.cache_dir == build.EXAMPLE_CACHE_DIR
    cache = native_runtime.KernelCache(kernel.cache_dir)
    expected = cache.directory / f"{kernel.name}-{cache.key(kernel, native_runtime._find_hip_compiler())}"
    assert expected in build.build_examples() and expected.exists()


# ---------------------------------------------------------------- mfu operand sets
def _mfu(params: dict):
    from teamredbench_amd.benchmarks.mfu import MfuBenchmark

    profile = load_hardware_profile(HW_DIR / "amd_instinct_mi355x.yaml")
    return MfuBenchmark(context=SimpleNamespace(hardware_profile=profile), params=params)


def _spec(name: str, size: int):
    return SimpleNamespace(name=name, bytes_per_element=size, matmul_ops_factor=2)


def test_operand_sets_span_three_infinity_caches_counting_a_b_and_c():
    from teamredbench_amd.benchmarks.mfu import INFINITY_CACHE_BYTES, OPERAND_FOOTPRINT_TARGET, gemm_bytes

    bench = _mfu({})
    # 64 x 1024 x 1024 bf16: 2.25 MiB per set (A + B + C), far under the cache; memory-bound
    sets, info = bench._operand_sets(_spec("bfloat16", 2), 64, 1024, 1024, 2, 2500.0)
    per_set = gemm_bytes(64, 1024, 1024, 2, 2)
    assert sets == -(-OPERAND_FOOTPRINT_TARGET // per_set) and sets > 64
    assert info["operand_footprint_bytes"] == sets * per_set >= OPERAND_FOOTPRINT_TARGET
    assert info["cache_resident_b"] is False and "operand_footprint_short_of_target" not in info
    # small K, large M x N: C dominates the set, so fewer copies reach the target (no 64 copies of C)
    sets, info = bench._operand_sets(_spec("bfloat16", 2), 8192, 8192, 16, 2, 2500.0)
    assert sets == -(-OPERAND_FOOTPRINT_TARGET // gemm_bytes(8192, 8192, 16, 2, 2)) <= 7
    # compute-bound: one set; the footprint decides residency (8192^3 bf16 spans 384 MiB)
    sets, info = bench._operand_sets(_spec("bfloat16", 2), 4096, 4096, 4096, 2, 2500.0)
    assert (sets, info["cache_resident_b"]) == (1, True)
    sets, info = bench._operand_sets(_spec("bfloat16", 2), 8192, 8192, 8192, 2, 2500.0)
    assert (sets, info["cache_resident_b"]) == (1, False)
    # a set beyond the target is already streamed from HBM
    assert bench._operand_sets(_spec("bfloat16", 2), 1, 32768, 16384, 2, 2500.0)[0] == 1
    assert INFINITY_CACHE_BYTES == 256 << 20


def test_operand_sets_cap_is_reported_and_a_count_is_taken_as_given():
    from teamredbench_amd.benchmarks.mfu import MAX_OPERAND_SETS

    sets, info = _mfu({})._operand_sets(_spec("bfloat16", 2), 16, 256, 256, 2, 2500.0)   # 144 KiB per set
    assert sets == MAX_OPERAND_SETS and info["operand_footprint_short_of_target"] is True
    sets, info = _mfu({"operand_sets": 1})._operand_sets(_spec("bfloat16", 2), 64, 1024, 1024, 2, 2500.0)
    assert sets == 1 and info["cache_resident_b"] is True
    assert _mfu({"operand_sets": 5})._operand_sets(_spec("float8_e4m3fn", 1), 8, 8, 8, 2, 5000.0)[0] == 5


def test_generic_profile_found_from_the_board_name_when_torch_has_none(monkeypatch):
    # Where libdrm's marketing-name table is missing, torch names the device without its SKU; the board's
    # product name (amdsmi / rocm-smi) then identifies it.
    monkeypatch.setattr(runner_mod, "load_torch", lambda: object())
    monkeypatch.setattr(runner_mod, "detect_device",
                        lambda torch_module, device_id=0: DeviceInfo(index=0, name="AMD Radeon Graphics"))
    monkeypatch.setattr(runner_mod, "product_names", lambda torch_module, index: ["AMD Instinct MI355X OAM"])
    context, note = runner_mod.build_context(load_suite(PACKAGE / "configs" / "suites" / "native_smoke.yaml"))
    assert context.hardware_profile.name == "amd-instinct-mi355x"
    assert "MI355X OAM" in note
    monkeypatch.setattr(runner_mod, "product_names", lambda torch_module, index: [])
    context, note = runner_mod.build_context(load_suite(PACKAGE / "configs" / "suites" / "native_smoke.yaml"))
    assert context.hardware_profile.name == "cdna-generic" and note is None


def test_amdsmi_names_include_the_gfx950_sku_of_the_peak_clock(monkeypatch):
    import sys as _sys

    from teamredbench_amd import device as device_mod

    class FakeSmi:
        class AmdSmiClkType:
            GFX = "gfx"

        max_clk = 2400

        def amdsmi_init(self):
            pass

        def amdsmi_shut_down(self):
            pass

        def amdsmi_get_processor_handles(self):
            return ["h0", "h1"]

        def amdsmi_get_gpu_device_bdf(self, h):
            return {"h0": "0000:11:00.0", "h1": "0000:f1:00.0"}[h]

        def amdsmi_get_gpu_board_info(self, h):
            return {"product_name": "N/A"}

        def amdsmi_get_gpu_asic_info(self, h):
            return {"market_name": "AMD Radeon Graphics"}

        def amdsmi_get_clock_info(self, h, kind):
            assert h == "h1"
            return {"max_clk": self.max_clk}

    fake = FakeSmi()
    props = SimpleNamespace(pci_domain_id=0, pci_bus_id=0xF1, pci_device_id=0, gcnArchName="gfx950:sramecc+:xnack-")
    torch_like = SimpleNamespace(cuda=SimpleNamespace(get_device_properties=lambda i: props))
    monkeypatch.setitem(_sys.modules, "amdsmi", fake)
    names = device_mod._amdsmi_names(torch_like, 0)
    assert names[0] == "AMD Radeon Graphics" and "MI355X" in names[1]
    fake.max_clk = 2200
    assert "MI350X" in device_mod._amdsmi_names(torch_like, 0)[-1]
    fake.max_clk = 2100
    assert device_mod._amdsmi_names(torch_like, 0) == ["AMD Radeon Graphics"]
