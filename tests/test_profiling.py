"""Profiling engine on the CPU (the reference's tests/test_profiling_runtime.py
and tests/test_autoprofile.py cover the same plumbing).

The rocprofv3 launch is built and checked without running rocprofv3; the
counter parser and the calibration are fed synthetic CSV files laid out as
rocprofv3 writes them; an end-to-end profiled suite runs under a stand-in
profiler script that writes such CSV files and runs the command after `--`.
"""
from __future__ import annotations

import csv
import json
import os
from pathlib import Path
import sys

import pytest
import yaml

from teamredbench_amd.profiling import builtin
from teamredbench_amd.profiling.registry import get_profile_engine
from teamredbench_amd.runner import run_suite

COPY = "void stream_vec_kernel<0, float, 4, true>(float*, float const*, float const*, unsigned long, float, int)"
TRIAD = "void stream_vec_kernel<2, float, 2, true>(float*, float const*, float const*, unsigned long, float, int)"
GEMM = "void gemm_tiled_kernel<1, 256, 256>(...)"


def _write_csv(path: Path, rows: list[dict]) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", newline="", encoding="utf-8") as handle:
        writer = csv.DictWriter(handle, fieldnames=list(rows[0]))
        writer.writeheader()
        writer.writerows(rows)


def _counter_rows(kernel: str, counter: str, per_dispatch: float, dispatches: int, first_id: int = 1,
                  split: int = 4) -> list[dict]:
    """rocprofv3 reports one row per counter dimension; the parser sums them per dispatch."""
    return [{"Dispatch_Id": first_id + d, "Kernel_Name": kernel, "Counter_Name": counter,
             "Counter_Value": per_dispatch / split} for d in range(dispatches) for _ in range(split)]


def _trace_rows(kernel: str, duration_ns: int, dispatches: int) -> list[dict]:
    return [{"Kernel_Name": kernel, "Start_Timestamp": 1000 * d, "End_Timestamp": 1000 * d + duration_ns}
            for d in range(dispatches)]


def test_rocprofv3_launch_calibrates_each_traffic_pass(tmp_path: Path):
    engine = get_profile_engine("rocprofv3")
    launch = engine.build_command({"binary": "/opt/rocm/bin/rocprofv3"}, ["python", "-m", "x"], tmp_path, None)
    assert launch.command[:2] == ("/opt/rocm/bin/rocprofv3", "--kernel-trace")
    assert launch.command[-3:] == ("python", "-m", "x")
    assert len(launch.extra_passes) == 3
    # counter passes never carry a trace domain
    for prefix in launch.extra_passes:
        assert "--pmc" in prefix and not any(a.endswith("-trace") for a in prefix)
    # one calibration run per pass that reads FETCH_SIZE or WRITE_SIZE, none for the MFMA pass
    assert len(launch.standalone_passes) == 2
    for i, (command, counter) in enumerate(zip(launch.standalone_passes, ("FETCH_SIZE", "WRITE_SIZE"))):
        assert command[command.index("--pmc") + 1] == counter
        assert command[command.index("-d") + 1] == str(tmp_path / f"cal{i + 1}")
        tail = command[command.index("--") + 1:]
        assert tail[:3] == (sys.executable, "-m", "teamredbench_amd.profiling.stream_probe")
        assert tail[tail.index("--ops") + 1] == "copy"
        assert not any(a.endswith("-trace") for a in command)
    spec = json.loads((tmp_path / "calibration.json").read_text(encoding="utf-8"))
    assert spec["read_bytes"] == spec["write_bytes"] == 4 * builtin.CALIBRATION_ELEMENTS

    off = engine.build_command({"calibrate": False, "counter_passes": [["FETCH_SIZE"]]}, ["x"], tmp_path / "o", None)
    assert off.standalone_passes == () and len(off.extra_passes) == 1


def test_collect_scales_traffic_by_the_copy_calibration(tmp_path: Path):
    engine = get_profile_engine("rocprofv3")
    engine.build_command({}, ["x"], tmp_path, None)        # writes calibration.json
    known = 4 * builtin.CALIBRATION_ELEMENTS
    n = 1 << 28
    # the copy reads `known` bytes but FETCH_SIZE says half of it; WRITE_SIZE is exact
    _write_csv(tmp_path / "cal1" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(COPY, "FETCH_SIZE", known / 2 / 1024, 3))
    _write_csv(tmp_path / "cal2" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(COPY, "WRITE_SIZE", known / 1024, 3))
    # the triad moves 8n read + 4n written bytes in 500 us
    _write_csv(tmp_path / "trace" / "host" / "1" / "run_kernel_trace.csv",
               _trace_rows(TRIAD, 500_000, 5) + _trace_rows(GEMM, 1_000_000, 2))
    _write_csv(tmp_path / "pmc1" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(TRIAD, "FETCH_SIZE", 8 * n / 2 / 1024, 5))
    _write_csv(tmp_path / "pmc2" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(TRIAD, "WRITE_SIZE", 4 * n / 1024, 5))
    # GEMM: 8 XCDs each active 2e6 cycles (GRBM_GUI_ACTIVE sums them); 256 CUs x 4 SIMDs busy 60 %
    busy = 0.6 * 2e6 * 256 * 4
    _write_csv(tmp_path / "pmc3" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(GEMM, "SQ_VALU_MFMA_BUSY_CYCLES", busy, 2)
               + _counter_rows(GEMM, "GRBM_GUI_ACTIVE", 8 * 2e6, 2, first_id=1, split=8))

    summary = builtin.collect(tmp_path, cu_count=256, xcd_count=8)
    assert summary["_calibration"] == {"FETCH_SIZE": pytest.approx(2.0), "WRITE_SIZE": pytest.approx(1.0)}
    triad = summary[TRIAD]
    assert triad["dispatches"] == 5 and triad["avg_duration_ns"] == 500_000
    assert triad["dram_fetch_bytes"] == pytest.approx(8 * n)
    assert triad["dram_write_bytes"] == pytest.approx(4 * n)
    assert triad["dram_gbps"] == pytest.approx(12 * n / 500_000)
    assert triad["calibrated"] is True
    gemm = summary[GEMM]
    assert gemm["mfma_busy_pct"] == pytest.approx(60.0)
    assert gemm["clock_ghz"] == pytest.approx(2.0)       # 2e6 cycles per XCD in 1 ms
    assert COPY not in summary                             # calibration kernels stay out of the result


def test_collect_without_calibration_reports_raw_counters(tmp_path: Path):
    _write_csv(tmp_path / "pmc1" / "host" / "1" / "run_counter_collection.csv",
               _counter_rows(TRIAD, "FETCH_SIZE", 1000.0, 2) + _counter_rows(TRIAD, "WRITE_SIZE", 500.0, 2))
    summary = builtin.collect(tmp_path)
    assert "_calibration" not in summary
    assert summary[TRIAD]["dram_fetch_bytes"] == 1000.0 * 1024
    assert summary[TRIAD]["dram_write_bytes"] == 500.0 * 1024
    assert "calibrated" not in summary[TRIAD] and "dram_gbps" not in summary[TRIAD]   # no trace, no duration


FAKE_PROFILER = r'''#!/usr/bin/env python3
"""Stand-in for rocprofv3: writes CSV files where rocprofv3 would and runs the program after --."""
import csv, os, subprocess, sys
argv = sys.argv[1:]
cmd = argv[argv.index("--") + 1:]
out = argv[argv.index("-d") + 1]
counters = []
if "--pmc" in argv:
    i = argv.index("--pmc") + 1
    while not argv[i].startswith("-"):
        counters.append(argv[i]); i += 1
os.makedirs(os.path.join(out, "host", "1"), exist_ok=True)
calibration = "teamredbench_amd.profiling.stream_probe" in cmd
kernel = COPY if calibration else TRIAD
if not calibration:
    rc = subprocess.call(cmd)
    if rc:
        sys.exit(rc)
if "--kernel-trace" in argv:
    with open(os.path.join(out, "host", "1", "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.writer(f); w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writerow([kernel, 0, 400000])
if counters:
    moved = {"FETCH_SIZE": 2.0 ** 28 / 2 / 1024, "WRITE_SIZE": 2.0 ** 28 / 1024} if calibration else \
            {"FETCH_SIZE": 4.0 * 2 ** 20 / 1024, "WRITE_SIZE": 4.0 * 2 ** 20 / 1024}
    with open(os.path.join(out, "host", "1", "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f); w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for c in counters:
            w.writerow([1, kernel, c, moved[c]])
'''


def test_profiled_suite_attaches_calibrated_counters(tmp_path: Path):
    profiler = tmp_path / "fake_rocprofv3.py"
    profiler.write_text(FAKE_PROFILER.replace("COPY if", f"{COPY!r} if").replace("else TRIAD", f"else {TRIAD!r}"),
                        encoding="utf-8")
    profiler.chmod(0o755)
    executable = tmp_path / "fake_hbm.py"
    executable.write_text("#!/usr/bin/env python3\nimport json\n"
                          "print(json.dumps({'status': 'ok', 'raw_metrics': {'elapsed_s': 0.001}}))\n",
                          encoding="utf-8")
    executable.chmod(0o755)
    hardware = tmp_path / "hardware.yaml"
    hardware.write_text(yaml.safe_dump({"name": "test-hw", "family": "cdna", "peak_hbm_bandwidth_gbps": 8000,
                                        "peak_link_bandwidth_gbps": {"xgmi": 1, "network": 1},
                                        "peak_compute_tops": {"float32": 100}}), encoding="utf-8")
    runtime = tmp_path / "runtime.yaml"
    runtime.write_text(yaml.safe_dump({"name": "rt", "rocm_version": "test", "libraries": {}, "env": {}}),
                       encoding="utf-8")
    suite = tmp_path / "suite.yaml"
    suite.write_text(yaml.safe_dump({
        "name": "profiled", "device": {"profile": str(hardware)}, "runtime": {"profile": str(runtime)},
        "profiling": {"enabled": True, "engine": "rocprofv3",
                      "params": {"binary": str(profiler), "counter_passes": [["FETCH_SIZE"], ["WRITE_SIZE"]]}},
        "outputs": {"directory": str(tmp_path / "results"), "formats": ["json"]},
        "benchmarks": [{"benchmark": "hbm", "params": {"backend": "native", "dtypes": ["float32"],
                                                        "modes": ["copy"], "size_mib": 1,
                                                        "native": {"binary": str(executable)}}}],
    }), encoding="utf-8")
    summary = run_suite(suite)
    assert [r.status for r in summary.records] == ["ok"]
    profiling = summary.run_metadata["profiling"]
    assert len(profiling["extra_passes"]) == 2 and len(profiling["standalone_passes"]) == 2
    counters = profiling["counters"]
    assert counters["_calibration"] == {"FETCH_SIZE": pytest.approx(2.0), "WRITE_SIZE": pytest.approx(1.0)}
    assert counters[TRIAD]["dram_fetch_bytes"] == pytest.approx(2 * 4.0 * 2 ** 20)
    assert counters[TRIAD]["dram_write_bytes"] == pytest.approx(4.0 * 2 ** 20)
    assert counters[TRIAD]["dram_gbps"] == pytest.approx(3 * 4.0 * 2 ** 20 / 400000)


def test_suite_summary_formats_gemm_records(tmp_path: Path):
    # `summarize suite` reads a suite's CSV output: one line per ok GEMM record, stream records skipped.
    from teamredbench_amd.profiling import summarize

    fields = ["benchmark", "case", "dtype", "status", "meta_tile_m", "meta_tile_n", "meta_split_k",
              "metric_latency_us", "metric_achieved_tops", "metric_mfu_pct", "metric_gemm_bandwidth_gbps",
              "metric_hbm_bandwidth_gbps", "metric_hbm_efficiency_pct", "meta_cache_resident"]
    rows = [
        ["mfu", "gemm_16x8192x8192", "bfloat16", "ok", "128", "256", "4", "26.25", "81.8", "3.27", "5133.0", "", "", ""],
        ["mfu", "gemm_2048x2048x2048", "bfloat16", "ok", "128", "128", "1", "21.3", "806.5", "32.26", "", "", "", ""],
        ["mfu", "gemm_1x1x1", "bfloat16", "skipped", "", "", "", "", "", "", "", "", "", ""],
        ["hbm", "triad_268435456el", "float32", "ok", "", "", "", "512.5", "", "", "", "6285.3", "78.57", "False"],
    ]
    path = tmp_path / "suite.csv"
    with path.open("w", newline="") as handle:
        w = csv.writer(handle)
        w.writerow(fields)
        w.writerows(rows)
    hbm, gemm = [t.splitlines() for t in summarize.suite([path]).split("\n\n")]
    assert hbm[1].split() == ["triad_268435456el", "float32", "512.50", "6285", "78.6", "False"]
    assert len(gemm) == 3
    assert gemm[1].split() == ["gemm_16x8192x8192", "bfloat16", "128x256", "4", "26.25", "81.8", "3.3", "5133"]
    assert gemm[2].split() == ["gemm_2048x2048x2048", "bfloat16", "128x128", "1", "21.30", "806.5", "32.3", "-"]


def test_waits_summary_shares_of_wave_cycles(tmp_path: Path):
    # `summarize waits` divides each SQ wait / issue counter by SQ_WAVE_CYCLES of the same kernel; other
    # counters are printed without a share, and kernels not matching --kernel are left out.
    from teamredbench_amd.profiling import summarize

    rows = (_counter_rows(GEMM, "SQ_WAVE_CYCLES", 2.0e8, 3) + _counter_rows(GEMM, "SQ_WAIT_ANY", 2.5e7, 3)
            + _counter_rows(GEMM, "SQ_WAIT_INST_LDS", 1.0e7, 3) + _counter_rows(GEMM, "GRBM_GUI_ACTIVE", 5.0e6, 3)
            + _counter_rows(TRIAD, "SQ_WAVE_CYCLES", 1.0e6, 2, first_id=10))
    _write_csv(tmp_path / "sq" / "host" / "1" / "run_counter_collection.csv", rows)
    lines = summarize.waits(tmp_path / "sq", "gemm_").splitlines()
    assert lines[0].startswith("kernel: ") and "gemm_tiled_kernel" in lines[0] and len(lines) == 5
    by_name = {line.split(":")[0].strip(): line for line in lines[1:]}
    assert by_name["SQ_WAIT_ANY"].endswith("(12.5% of SQ_WAVE_CYCLES)")
    assert by_name["SQ_WAIT_INST_LDS"].endswith("(5.0% of SQ_WAVE_CYCLES)")
    assert "%" not in by_name["GRBM_GUI_ACTIVE"]
    with pytest.raises(SystemExit):
        summarize.waits(tmp_path / "sq", "no_such_kernel")


# ---- the reference engine's v1 parameters under the `rocprof` name (src/teamredbench/profiling/builtin.py:37-143)
def test_rocprof_name_translates_the_reference_smoke_params(tmp_path: Path):
    # configs/suites/rocprof_hbm_smoke.yaml: engine rocprof, params {stats: true, hip_trace: true}
    launch = get_profile_engine("rocprof").build_command({"stats": True, "hip_trace": True}, ["x"], tmp_path, None)
    assert launch.command[1] == "--kernel-trace"
    assert "--stats" in launch.command and "--hip-trace" in launch.command
    assert launch.metadata["binary"].endswith("rocprofv3")
    for prefix in launch.extra_passes:     # the API trace stays off the counter passes
        assert "--hip-trace" not in prefix and "--stats" not in prefix


def test_rocprof_name_translates_trace_toggles(tmp_path: Path):
    params = {"roctx_trace": True, "hsa_trace": True, "sys_trace": True, "basenames": True, "timestamp": True,
              "env": {"A": "1"}, "extra_args": ["--minimum-output-data", "0"]}
    launch = get_profile_engine("rocprof").build_command(params, ["x"], tmp_path, None)
    trace = launch.command[:launch.command.index("--")]
    for flag in ("--marker-trace", "--hsa-trace", "--sys-trace", "--truncate-kernels", "--minimum-output-data"):
        assert flag in trace
    assert launch.env["A"] == "1"
    for prefix in launch.extra_passes:
        assert not any(a.endswith("-trace") for a in prefix)


def test_rocprof_name_reads_a_v1_counter_input_file(tmp_path: Path):
    suite_dir = tmp_path / "suites"
    suite_dir.mkdir()
    (suite_dir / "counters.txt").write_text(
        "# v1 input\npmc: FETCH_SIZE\npmc : WRITE_SIZE, GRBM_GUI_ACTIVE\nkernel: stream_vec_kernel gemm_tiled\n",
        encoding="utf-8")
    launch = get_profile_engine("rocprof").build_command({"input": "counters.txt"}, ["x"], tmp_path / "a", suite_dir)
    passes = [list(p[p.index("--pmc") + 1:p.index("-d")]) for p in launch.extra_passes]
    assert passes == [["FETCH_SIZE"], ["WRITE_SIZE", "GRBM_GUI_ACTIVE"]]
    assert launch.command[launch.command.index("--kernel-include-regex") + 1] == "stream_vec_kernel|gemm_tiled"
    (suite_dir / "bad.txt").write_text("pmc: FETCH_SIZE\nrange: 0:10\ngpu: 0\n", encoding="utf-8")
    with pytest.raises(ValueError) as err:
        get_profile_engine("rocprof").build_command({"input": "bad.txt"}, ["x"], tmp_path / "b", suite_dir)
    assert "'range: 0:10'" in str(err.value) and "'gpu: 0'" in str(err.value)


def test_rocprof_name_refuses_what_rocprofv3_cannot_honour(tmp_path: Path):
    params = {name: ("x" if name in ("tool_version", "metric_file", "output", "data_dir", "temporary_dir") else True)
              for name in builtin.V1_REFUSED}
    params.update({"timestamp": False, "binary": "rocprof"})
    with pytest.raises(ValueError) as err:
        get_profile_engine("rocprof").build_command(params, ["x"], tmp_path, None)
    message = str(err.value)
    for name in [*builtin.V1_REFUSED, "timestamp", "binary"]:
        assert name in message, name
    # the rocprofv3 engine itself takes its own parameters only
    assert get_profile_engine("rocprofv3").build_command({"stats": False}, ["x"], tmp_path / "v3", None)


def test_clock_summary_pairs_stamps_cu_by_cu():
    from teamredbench_amd.profiling.clock import clock_summary

    # two XCDs x 4 CUs, counters offset per CU by ~1e8 cycles; XCD 0 at 1500 MHz, XCD 1 at 2000 MHz over
    # 10 ms (1e6 ticks of the 100 MHz counter); the second stamp lands its blocks in another order
    def stamp(t_real: int, order: list[int]) -> list[list[int]]:
        rows = []
        for i in order:
            xcd, cu = divmod(i, 4)
            offset = 10**8 * (i + 1)
            shader = offset + (1500 if xcd == 0 else 2000) * t_real // 100
            rows.append([shader, 5_000_000 + t_real, xcd, (cu << 8) | 0x25])
        return rows

    before = stamp(0, list(range(8)) + [0, 5])         # CU 0 and CU 5 ran two blocks
    after = stamp(1_000_000, [7, 6, 5, 4, 3, 2, 1])   # CU 0 missing from the second stamp
    out = clock_summary(before, after)
    assert out["gfxclk_mhz_per_xcd"] == {"0": 1500.0, "1": 2000.0}
    assert out["cus_paired"] == 7 and out["cu_spread_mhz"] == 0.0 and out["window_s"] == 0.01
    assert clock_summary(before, [])["available"] is False


def test_profiled_child_measures_against_the_profile_its_parent_resolved(tmp_path: Path, monkeypatch):
    # The parent auto-selects the MI355X profile for a suite whose own profile has no peaks; the child under
    # the profiler (a separate process, which here sees no device at all) measures against the same one.
    from teamredbench_amd import runner as runner_mod
    from teamredbench_amd.device import DeviceInfo

    profiler = tmp_path / "fake_rocprofv3.py"
    profiler.write_text(FAKE_PROFILER.replace("COPY if", f"{COPY!r} if").replace("else TRIAD", f"else {TRIAD!r}"),
                        encoding="utf-8")
    profiler.chmod(0o755)
    executable = tmp_path / "fake_hbm.py"
    executable.write_text("#!/usr/bin/env python3\nimport json\n"
                          "print(json.dumps({'status': 'ok', 'raw_metrics': {'elapsed_s': 0.001}}))\n",
                          encoding="utf-8")
    executable.chmod(0o755)
    generic = runner_mod.PACKAGED_HARDWARE_DIR / "cdna_generic.yaml"
    runtime = runner_mod.PACKAGED_HARDWARE_DIR.parent / "rocm" / "rocm_generic.yaml"
    suite = tmp_path / "suite.yaml"
    suite.write_text(yaml.safe_dump({
        "name": "inherit", "device": {"profile": str(generic)}, "runtime": {"profile": str(runtime)},
        "profiling": {"enabled": True, "engine": "rocprof",
                      "params": {"binary": str(profiler), "calibrate": False, "counter_passes": [["FETCH_SIZE"]]}},
        "outputs": {"directory": str(tmp_path / "results"), "formats": ["json"]},
        "benchmarks": [{"benchmark": "hbm", "params": {"backend": "native", "dtypes": ["float32"],
                                                        "modes": ["copy"], "size_mib": 1,
                                                        "native": {"binary": str(executable)}}}],
    }), encoding="utf-8")
    monkeypatch.setattr(runner_mod, "load_torch", lambda: object())
    monkeypatch.setattr(runner_mod, "detect_device",
                        lambda torch_module, device_id=0: DeviceInfo(index=0, name="AMD Instinct MI355X"))
    summary = run_suite(suite)
    assert summary.profile_note and "amd-instinct-mi355x" in summary.profile_note
    (record,) = summary.records
    assert record.status == "ok" and record.raw_metrics["peak_bandwidth_gbps"] == 8000.0
    assert record.metrics["hbm_efficiency_pct"] > 0
