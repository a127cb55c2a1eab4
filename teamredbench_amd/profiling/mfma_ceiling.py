"""Sustained MFMA ceiling of the part under its power limit (no memory traffic).

Runs the `mfma_ceiling` probe that `teamredbench_amd.native.build` compiles
next to libmi355bench.so (source: mfma_ceiling.hip beside this file) and
prints its per-instruction sustained TFLOP/s with random operands. These
figures bound what any GEMM kernel's MFMA work can reach on the part: a GEMM
that also moves data draws more power and runs below them.

    python -m teamredbench_amd.profiling.mfma_ceiling [--scale S] [--json]
"""
from __future__ import annotations

import argparse
import json
import subprocess
import sys
from typing import Any


def parse(output: str) -> list[dict[str, Any]]:
    """The probe's JSON lines (one per instruction), other lines ignored."""
    rows = []
    for line in output.splitlines():
        line = line.strip()
        if line.startswith("{") and line.endswith("}"):
            row = json.loads(line)
            if "instruction" in row and "sustained_tflops" in row:
                rows.append(row)
    return rows


def format_table(rows: list[dict[str, Any]]) -> str:
    lines = [f"{'instruction':36s} {'dtype':14s} {'sustained TFLOP/s':>18s} {'peak':>8s} {'fraction':>9s}"]
    for r in rows:
        lines.append(f"{r['instruction']:36s} {r['dtype']:14s} {r['sustained_tflops']:18.1f} "
                     f"{r['peak_tflops']:8.1f} {100.0 * r['fraction_of_peak']:8.1f}%")
    return "\n".join(lines)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--scale", type=float, default=1.0, help="iterations per launch, relative to ~5 ms")
    parser.add_argument("--json", action="store_true", help="print the probe's JSON lines instead of a table")
    args = parser.parse_args(argv)
    from teamredbench_amd.native import build

    exe = build.probe_path("mfma_ceiling")
    if not exe.exists():
        print(f"{exe} is not built; run `python -m teamredbench_amd.native.build`", file=sys.stderr)
        return 1
    proc = subprocess.run([str(exe), str(args.scale)], capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        print(proc.stdout + proc.stderr, file=sys.stderr)
        return proc.returncode
    rows = parse(proc.stdout)
    print("\n".join(json.dumps(r) for r in rows) if args.json else format_table(rows))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
