"""Text summaries of rocprofv3 CSV output (kernel statistics and counters).

    python -m teamredbench_amd.profiling.summarize stats <dir> [--top N]
        per-kernel calls / average / total duration from *_kernel_stats.csv
    python -m teamredbench_amd.profiling.summarize traffic --fetch <dir> --write <dir>
            --kernel <regex> --calibrate <regex> --calibrate-read B --calibrate-write B
            [--algorithmic-bytes B]
        DRAM bytes per dispatch of the kernel matching --kernel, from
        FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by the factor
        that makes the calibration kernel (a plain copy of known size) read
        and write exactly its known bytes; prints a `traffic_bytes_per_launch:`
        line that bench.py reads.

    python -m teamredbench_amd.profiling.summarize mfma <dir> --kernel <regex> [--duration-us T ...]
        SQ_VALU_MFMA_BUSY_CYCLES against GRBM_GUI_ACTIVE (summed over the
        XCDs) for each matching kernel: the fraction of SIMD cycles the MFMA
        units were busy, and the clock it ran at over the dispatch duration
        (the counter run's own timestamps unless --duration-us is given).

    python -m teamredbench_amd.profiling.summarize waits <dir> --kernel <regex>
        each SQ_WAIT* / SQ_ACTIVE_INST* / SQ_INST_CYCLES* / SQ_LDS* counter of
        a counter run as a share of SQ_WAVE_CYCLES (the wave-cycles the
        kernel's waves existed), per matching kernel: SQ_WAIT_ANY is time in
        s_waitcnt and barriers, SQ_WAIT_INST_ANY time with an instruction that
        could not issue yet.

    python -m teamredbench_amd.profiling.summarize suite <results.csv> [...]
        one line per record of a suite run's CSV output: for GEMM records the
        shape, dtype, kernel configuration (tile, K splits), latency, TFLOP/s,
        MFU and the effective bandwidth where the suite asked for it; for
        stream records the latency, GB/s, % of peak and cache residency.

The directories are rocprofv3 output directories written with `-f csv`.
"""
from __future__ import annotations

import argparse
import csv
from pathlib import Path
import re
import sys

from teamredbench_amd.profiling.builtin import parse_counter_durations, parse_counters


def _kernel_stats(directory: Path) -> list[dict[str, str]]:
    rows: list[dict[str, str]] = []
    for path in sorted(directory.rglob("*kernel_stats.csv")):
        with path.open(newline="", encoding="utf-8", errors="replace") as handle:
            rows.extend(csv.DictReader(handle))
    return rows


def _short(name: str, width: int = 110) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def stats(directory: Path, top: int) -> str:
    rows = _kernel_stats(directory)
    if not rows:
        raise SystemExit(f"no *kernel_stats.csv under {directory}")
    rows.sort(key=lambda r: -float(r.get("TotalDurationNs", 0) or 0))
    lines = [f"{'calls':>6} {'avg_us':>11} {'total_us':>12} {'pct':>6}  kernel"]
    for r in rows[:top]:
        lines.append(
            f"{int(float(r['Calls'])):6d} {float(r['AverageNs']) / 1e3:11.2f} {float(r['TotalDurationNs']) / 1e3:12.1f}"
            f" {float(r['Percentage']):6.2f}  {_short(r['Name'])}"
        )
    return "\n".join(lines)


def suite(paths: list[Path]) -> str:
    gemm = [f"{'case':<22} {'dtype':<14} {'tile':>9} {'split':>5} {'latency_us':>11} {'TFLOP/s':>9} {'MFU%':>6} {'GB/s':>7}"]
    hbm = [f"{'case':<22} {'dtype':<9} {'latency_us':>11} {'GB/s':>8} {'% peak':>7}  cache-resident"]
    for path in paths:
        with path.open(newline="", encoding="utf-8") as handle:
            for r in csv.DictReader(handle):
                if r.get("status") != "ok":
                    continue
                if r.get("benchmark") == "mfu":
                    tile = f"{r.get('meta_tile_m', '?')}x{r.get('meta_tile_n', '?')}"
                    gbps = r.get("metric_gemm_bandwidth_gbps") or ""
                    gemm.append(
                        f"{r['case']:<22} {r['dtype']:<14} {tile:>9} {r.get('meta_split_k', '1') or '1':>5}"
                        f" {float(r['metric_latency_us']):11.2f} {float(r['metric_achieved_tops']):9.1f}"
                        f" {float(r['metric_mfu_pct']):6.1f} {(f'{float(gbps):7.0f}' if gbps else '-'):>7}"
                    )
                elif r.get("benchmark") == "hbm":
                    hbm.append(
                        f"{r['case']:<22} {r['dtype']:<9} {float(r['metric_latency_us']):11.2f}"
                        f" {float(r['metric_hbm_bandwidth_gbps']):8.0f} {float(r['metric_hbm_efficiency_pct']):7.1f}"
                        f"  {r.get('meta_cache_resident', '')}"
                    )
    parts = [t for t in (hbm, gemm) if len(t) > 1]
    return "\n\n".join("\n".join(t) for t in parts)


def _match(counters: dict[str, dict[str, float]], pattern: str, counter: str) -> tuple[str, float]:
    rx = re.compile(pattern)
    hits = [(k, v[counter]) for k, v in counters.items() if rx.search(k) and counter in v]
    if len(hits) != 1:
        raise SystemExit(f"pattern {pattern!r} matched {len(hits)} kernels with {counter}: {[h[0] for h in hits]}")
    return hits[0]


def traffic(fetch_dir: Path, write_dir: Path, kernel: str, calibrate: str, cal_read: float, cal_write: float,
            algorithmic: float | None) -> str:
    fetch = parse_counters(fetch_dir)
    write = parse_counters(write_dir)
    k_name, k_fetch = _match(fetch, kernel, "FETCH_SIZE")
    _, k_write = _match(write, kernel, "WRITE_SIZE")
    c_name, c_fetch = _match(fetch, calibrate, "FETCH_SIZE")
    _, c_write = _match(write, calibrate, "WRITE_SIZE")
    f_fetch = cal_read / (c_fetch * 1024.0)
    f_write = cal_write / (c_write * 1024.0)
    total = k_fetch * 1024.0 * f_fetch + k_write * 1024.0 * f_write
    lines = [
        f"kernel: {_short(k_name)}",
        f"calibration kernel: {_short(c_name)} (known read {cal_read:.0f} B, write {cal_write:.0f} B)",
        f"FETCH_SIZE per dispatch: kernel {k_fetch:.1f} KiB, calibration {c_fetch:.1f} KiB -> factor {f_fetch:.4f}",
        f"WRITE_SIZE per dispatch: kernel {k_write:.1f} KiB, calibration {c_write:.1f} KiB -> factor {f_write:.4f}",
        f"dram_read_bytes_per_launch: {k_fetch * 1024.0 * f_fetch:.0f}",
        f"dram_write_bytes_per_launch: {k_write * 1024.0 * f_write:.0f}",
        f"traffic_bytes_per_launch: {total:.0f}",
    ]
    if algorithmic:
        lines.append(f"algorithmic_bytes_per_launch: {algorithmic:.0f} (traffic / algorithmic = {total / algorithmic:.4f})")
    return "\n".join(lines)


def mfma(directory: Path, kernel: str, durations_us: list[float], xcds: int, cus: int) -> str:
    rx = re.compile(kernel)
    counters = {k: v for k, v in parse_counters(directory).items() if rx.search(k)}
    if not counters:
        raise SystemExit(f"no kernel matching {kernel!r} under {directory}")
    own = parse_counter_durations(directory)
    lines = []
    for idx, (name, values) in enumerate(sorted(counters.items())):
        busy, gui = values.get("SQ_VALU_MFMA_BUSY_CYCLES"), values.get("GRBM_GUI_ACTIVE")
        lines.append(f"kernel: {_short(name)}")
        for key in sorted(values):
            lines.append(f"  {key}: {values[key]:.6g}")
        if busy is not None and gui:
            per_xcd = gui / xcds
            lines.append(f"  mfma_busy_pct (busy / (GUI_ACTIVE/{xcds} * {cus} CUs * 4 SIMDs)): "
                         f"{100.0 * busy / (per_xcd * cus * 4):.2f}")
            span_us = durations_us[idx] if idx < len(durations_us) else own.get(name, 0.0) / 1e3
            if span_us:
                source = "given" if idx < len(durations_us) else "this run's timestamps"
                lines.append(f"  average dispatch duration ({source}): {span_us:.2f} us")
                lines.append(f"  clock over the dispatch (GUI_ACTIVE/{xcds} / duration): "
                             f"{per_xcd / span_us / 1e3:.3f} GHz")
    return "\n".join(lines)


def waits(directory: Path, kernel: str) -> str:
    rx = re.compile(kernel)
    counters = {k: v for k, v in parse_counters(directory).items() if rx.search(k)}
    if not counters:
        raise SystemExit(f"no kernel matching {kernel!r} under {directory}")
    shares = ("SQ_WAIT", "SQ_ACTIVE_INST", "SQ_INST_CYCLES", "SQ_LDS", "SQ_BUSY_CYCLES")
    lines = []
    for name, values in sorted(counters.items()):
        lines.append(f"kernel: {_short(name)}")
        wave = values.get("SQ_WAVE_CYCLES")
        for key in sorted(values):
            share = f"  ({100.0 * values[key] / wave:.1f}% of SQ_WAVE_CYCLES)" if wave and key.startswith(shares) else ""
            lines.append(f"  {key}: {values[key]:.6g}{share}")
    return "\n".join(lines)


def sidecar(path: Path, match: str | None = None) -> str:
    """The rocprofv3 counter summary a profiled suite run attached to its metadata sidecar
    (run.profiling.counters), one line per kernel (those matching `match`, a regex, if given)."""
    import json

    doc = json.loads(path.read_text(encoding="utf-8"))
    block = doc.get("run", {}).get("profiling", {})
    counters = block.get("counters")
    if not counters:
        raise SystemExit(f"{path} carries no run.profiling.counters ({block.get('counters_error', 'no profiling')})")
    lines = [f"suite: {doc.get('suite_name')}  records: {doc.get('record_count')}  engine: {block.get('engine')}",
             f"calibration factors: {counters.get('_calibration', {})}"]
    for name, entry in sorted(counters.items()):
        if name.startswith("_") or (match and not re.search(match, name)):
            continue
        parts = [f"{entry.get('dispatches', 0):4d} x {entry.get('avg_duration_ns', 0) / 1e3:9.2f} us"]
        if "dram_fetch_bytes" in entry and "dram_write_bytes" in entry:
            parts.append(f"DRAM read {entry['dram_fetch_bytes']:.4g} B write {entry['dram_write_bytes']:.4g} B")
        if "dram_gbps" in entry:
            parts.append(f"{entry['dram_gbps']:.1f} GB/s")
        if "mfma_busy_pct" in entry:
            parts.append(f"MFMA busy {entry['mfma_busy_pct']:.1f}%")
        if "clock_ghz" in entry:
            parts.append(f"{entry['clock_ghz']:.2f} GHz")
        lines.append(f"{'  '.join(parts)}  {_short(name, 90)}")
    return "\n".join(lines)


def _by_launch_shape(pmc_dir: Path) -> tuple[dict[str, dict[str, float]], dict[str, float]]:
    """Counters (median per dispatch) and dispatch durations, keyed by kernel name plus launch shape,
    so the same kernel launched with other block sizes or grids stays apart."""
    from statistics import median

    per: dict[tuple[str, str], dict[str, float]] = {}
    spans: dict[tuple[str, str], int] = {}
    for path in sorted(pmc_dir.rglob("*counter_collection.csv")):
        with path.open(newline="", encoding="utf-8", errors="replace") as handle:
            for row in csv.DictReader(handle):
                key = (f"{row.get('Kernel_Name', '?')} [{row.get('Workgroup_Size')} x "
                       f"{int(row.get('Grid_Size') or 0) // max(int(row.get('Workgroup_Size') or 1), 1)}]",
                       row.get("Dispatch_Id", "?"))
                counters = per.setdefault(key, {})
                counters[row["Counter_Name"]] = counters.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
                spans[key] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    grouped: dict[str, dict[str, list[float]]] = {}
    for (name, dispatch), counters in per.items():
        entry = grouped.setdefault(name, {})
        for counter, value in counters.items():
            entry.setdefault(counter, []).append(value)
        entry.setdefault("_ns", []).append(spans[(name, dispatch)])
    values = {k: {c: median(v) for c, v in cs.items() if c != "_ns"} for k, cs in grouped.items()}
    return values, {k: median(cs["_ns"]) for k, cs in grouped.items()}


def traffic_mix(latency_dir: Path, stall_dir: Path, xcds: int, channels: int) -> str:
    """Memory-side behaviour per kernel from two counter passes: (1) TCC_EA0_RDREQ_LEVEL_sum,
    TCC_EA0_RDREQ_sum, TCC_EA0_WRREQ_LEVEL_sum, TCC_EA0_WRREQ_sum, GRBM_GUI_ACTIVE; (2)
    TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum, TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum, GRBM_GUI_ACTIVE. Average
    EA read / write latency = LEVEL / requests (cycles); requests in flight = LEVEL / cycles; a credit
    stall is the fraction of channel-cycles (channels per XCD x XCDs) a request waited for DRAM credit."""
    lat, durations = _by_launch_shape(latency_dir)
    stall, _ = _by_launch_shape(stall_dir)
    lines = [f"{'us':>8} {'rd req':>9} {'wr req':>9} {'rd lat':>7} {'wr lat':>7} {'rd fly':>7} {'wr fly':>7} "
             f"{'GHz':>5} {'rdstall':>7} {'wrstall':>7}  kernel"]
    for name in sorted(lat):
        a, b = lat[name], stall.get(name, {})
        if not a.get("GRBM_GUI_ACTIVE"):
            continue
        cycles = a["GRBM_GUI_ACTIVE"] / xcds
        rd, wr = a.get("TCC_EA0_RDREQ_sum", 0.0), a.get("TCC_EA0_WRREQ_sum", 0.0)
        rdl, wrl = a.get("TCC_EA0_RDREQ_LEVEL_sum", 0.0), a.get("TCC_EA0_WRREQ_LEVEL_sum", 0.0)
        ns = durations.get(name, 0.0)
        per_channel = cycles * xcds * channels
        lines.append(
            f"{ns / 1e3:8.1f} {rd:9.3g} {wr:9.3g} {rdl / rd if rd else 0:7.0f} {wrl / wr if wr else 0:7.0f} "
            f"{rdl / cycles:7.0f} {wrl / cycles:7.0f} {cycles / ns if ns else 0:5.2f} "
            f"{b.get('TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum', 0.0) / per_channel:7.3f} "
            f"{b.get('TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum', 0.0) / per_channel:7.3f}  {_short(name, 60)}"
            f"{name[name.rindex(' ['):] if ' [' in name else ''}")
    return "\n".join(lines)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = parser.add_subparsers(dest="cmd", required=True)
    p_stats = sub.add_parser("stats")
    p_stats.add_argument("directory", type=Path)
    p_stats.add_argument("--top", type=int, default=12)
    p_tr = sub.add_parser("traffic")
    p_tr.add_argument("--fetch", type=Path, required=True)
    p_tr.add_argument("--write", type=Path, required=True)
    p_tr.add_argument("--kernel", required=True)
    p_tr.add_argument("--calibrate", required=True)
    p_tr.add_argument("--calibrate-read", type=float, required=True)
    p_tr.add_argument("--calibrate-write", type=float, required=True)
    p_tr.add_argument("--algorithmic-bytes", type=float)
    p_mfma = sub.add_parser("mfma")
    p_mfma.add_argument("directory", type=Path)
    p_mfma.add_argument("--kernel", required=True)
    p_mfma.add_argument("--duration-us", type=float, nargs="*", default=[],
                        help="average duration of each matching kernel, in name order")
    p_mfma.add_argument("--xcds", type=int, default=8)
    p_mfma.add_argument("--cus", type=int, default=256)
    p_waits = sub.add_parser("waits", help="SQ wait and issue counters as shares of SQ_WAVE_CYCLES")
    p_waits.add_argument("directory", type=Path)
    p_waits.add_argument("--kernel", required=True)
    p_suite = sub.add_parser("suite")
    p_suite.add_argument("csv", type=Path, nargs="+")
    p_mix = sub.add_parser("mix", help="EA read / write latency, requests in flight and DRAM credit stalls")
    p_mix.add_argument("latency_dir", type=Path)
    p_mix.add_argument("stall_dir", type=Path)
    p_mix.add_argument("--xcds", type=int, default=8)
    p_mix.add_argument("--channels", type=int, default=16, help="TCC channels per XCD")
    p_side = sub.add_parser("sidecar", help="counter summary of a profiled suite run's metadata sidecar")
    p_side.add_argument("path", type=Path)
    p_side.add_argument("--match", help="only kernels whose name matches this regex")
    args = parser.parse_args(argv)
    if args.cmd == "suite":
        print(suite(args.csv))
    elif args.cmd == "mfma":
        print(mfma(args.directory, args.kernel, args.duration_us, args.xcds, args.cus))
    elif args.cmd == "waits":
        print(waits(args.directory, args.kernel))
    elif args.cmd == "stats":
        print(stats(args.directory, args.top))
    elif args.cmd == "mix":
        print(traffic_mix(args.latency_dir, args.stall_dir, args.xcds, args.channels))
    elif args.cmd == "sidecar":
        print(sidecar(args.path, args.match))
    else:
        print(traffic(args.fetch, args.write, args.kernel, args.calibrate, args.calibrate_read,
                      args.calibrate_write, args.algorithmic_bytes))
    return 0


if __name__ == "__main__":
    sys.exit(main())
