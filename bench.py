#!/usr/bin/env python3
"""Headline benchmark of the gfx950 stream and GEMM kernels on one MI355X.

One step is one launch of the stream triad a = b + 3*c over 2^28 fp32
elements per array (3 GiB of algorithmic traffic), through the C ABI of
libmi355bench.so on torch's current stream, with the inputs already resident
in HBM. The printed JSON line carries:

  value / ms_per_step  whole-job triad GB/s and the wall-clock time per step
                       (K launches between two device synchronisations);
  roofline             the triad kernel's algorithmic GB/s from HIP events
                       recorded on the launch stream, against 8000 GB/s;
                       `traffic` is the HBM bytes per launch from the committed
                       rocprofv3 FETCH_SIZE/WRITE_SIZE summary, when present;
                       `launch_us` the min / median / max of the per-launch
                       event durations and `clock` the shader clock each XCD
                       ran at over the timed loop (clock stamps on its stream);
  gemm                 bf16 and fp8 e4m3 GEMM TFLOPS and MFU at 8192^3
                       (event-timed per launch, same library, with the same
                       `launch_us` spread and `clock`), a sampled parity check,
                       and each one's CPU baseline: torch.mm on CPU tensors over
                       a 512-row slab of the same problem (bf16 operands for
                       bf16; for fp8, whose torch.mm has no CPU kernel, the
                       dequantised fp32 operands the oracle multiplies);
  mfma_ceiling         the sustained TFLOP/s of the MFMA instructions those
                       GEMMs run, with no memory traffic, in the same process
                       (each GEMM's frac_of_mfma_ceiling divides by it);
  cpu_baseline         the reference torch op (torch.add(b, c, alpha=3.0,
                       out=a)) on CPU tensors on this host's cores: the CPU
                       triad configuration (2^24 elements, seed 0, 5 warmup +
                       20 timed), plus the same op at the GPU step's size.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-gemm]
                       [--no-mfma-ceiling] [--cpu-iterations I] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
from pathlib import Path
import sys
import time

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"bfloat16": 2500.0, "float16": 2500.0, "float8_e4m3fn": 5000.0}
GEMM_WARMUP_S = 0.25
TRIAD_ELEMENTS = 1 << 28
TRAFFIC_SUMMARY = ROOT / "profiles" / "stream_triad_f32_2p28_traffic.txt"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def launch_spread(seconds: list[float]) -> dict:
    """Min / median / max / mean of per-launch HIP-event durations, in microseconds."""
    ordered = sorted(seconds)
    mid = len(ordered) // 2
    median = ordered[mid] if len(ordered) % 2 else 0.5 * (ordered[mid - 1] + ordered[mid])
    return {"min": round(ordered[0] * 1e6, 2), "median": round(median * 1e6, 2), "max": round(ordered[-1] * 1e6, 2),
            "mean": round(sum(ordered) / len(ordered) * 1e6, 2), "launches": len(ordered)}


def read_traffic() -> dict | None:
    """HBM bytes per triad launch from the committed rocprofv3 counter summary.

    The summary holds a line `traffic_bytes_per_launch: <int>` derived from
    FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel calibration factor.
    """
    if not TRAFFIC_SUMMARY.exists():
        return None
    for line in TRAFFIC_SUMMARY.read_text(encoding="utf-8").splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return {"bytes": int(float(line.split(":", 1)[1])), "source": str(TRAFFIC_SUMMARY.relative_to(ROOT))}
    return None


def bench_triad(torch, lib, capi, steps: int, warmup: int) -> dict:
    from teamredbench_amd.profiling.clock import ClockWindow

    n = TRIAD_ELEMENTS
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    b = torch.empty(n, device=dev, dtype=torch.float32).uniform_(-1.0, 1.0, generator=gen)
    c = torch.empty(n, device=dev, dtype=torch.float32).uniform_(-1.0, 1.0, generator=gen)
    a = torch.empty_like(b)
    stream = torch.cuda.current_stream(dev)
    handle = stream.cuda_stream

    def step() -> None:
        lib.stream(capi.OP_TRIAD, capi.DT_FLOAT32, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, 3.0, 0, handle)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # One event before the first launch and one after each: launch i spans events i .. i + 1, and the
    # first and last bracket the whole loop, which the wall clock brackets too.
    # The clock stamps bracket the loop on its stream (two one-wave kernels of a few microseconds, the
    # second inside the wall-clock window).
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    clock = ClockWindow(torch, lib, handle)
    clock.start()
    t0 = time.perf_counter()
    events[0].record(stream)
    for i in range(steps):
        step()
        events[i + 1].record(stream)
    clock.stop()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    event_s = events[0].elapsed_time(events[-1]) / 1000.0 / steps
    per_launch = [events[i].elapsed_time(events[i + 1]) / 1000.0 for i in range(steps)]

    # in-run parity against the torch GPU op (1 ulp bound of the stream configuration)
    from teamredbench_amd.parity import stream_parity

    ref = torch.add(b, c, alpha=3.0)
    parity = stream_parity(torch, "triad", a, ref)
    del ref
    moved = 3 * 4 * n
    return {
        "wall_s_per_step": wall / steps,
        "event_s_per_launch": event_s,
        "launch_us": launch_spread(per_launch),
        "clock": clock.summary(),
        "moved_bytes": moved,
        "parity": parity,
        "info": lib.stream_info(capi.OP_TRIAD, capi.DT_FLOAT32, n),
    }


def bench_gemm(torch, lib, capi, dtype: str, size: int, warmup: int, iterations: int) -> dict:
    from teamredbench_amd.parity import gemm_parity
    from teamredbench_amd.profiling.clock import ClockWindow
    from teamredbench_amd.utils import seeded_gemm_operands

    dev = torch.device("cuda:0")
    m = n = k = size
    a, b, sa, sb = seeded_gemm_operands(torch, m, n, k, dtype, dev, seed=0)
    out_dtype = torch.float16 if dtype == "float16" else torch.bfloat16
    c = torch.empty((m, n), device=dev, dtype=out_dtype)
    dt = capi.DTYPES[dtype]
    ws_bytes = lib.gemm_workspace_size(dt, m, n, k)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    handle = torch.cuda.current_stream(dev).cuda_stream
    # The part leaves its low-power clock state only after tens of milliseconds of sustained MFMA work
    # (a 3-launch warmup measures ~10% low), so the untimed warmup lasts WARMUP_S seconds.
    est = lib.time_gemm(dt, a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, sa, sb, ws.data_ptr(), ws_bytes,
                        0, 2, handle)
    warmup = max(warmup, int(GEMM_WARMUP_S / est) + 1)
    lib.time_gemm(dt, a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, sa, sb, ws.data_ptr(), ws_bytes,
                  warmup, 1, handle)
    stream = torch.cuda.current_stream(dev)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(iterations + 1)]
    clock = ClockWindow(torch, lib, handle)
    clock.start()
    events[0].record(stream)
    for i in range(iterations):
        lib.gemm(dt, a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, sa, sb, ws.data_ptr(), ws_bytes, handle)
        events[i + 1].record(stream)
    clock.stop()
    torch.cuda.synchronize()
    secs = events[0].elapsed_time(events[-1]) / 1000.0 / iterations
    per_launch = [events[i].elapsed_time(events[i + 1]) / 1000.0 for i in range(iterations)]
    rows = torch.randperm(m, generator=torch.Generator().manual_seed(0))[:256].to(dev)
    ref = (a[rows].float() * sa) @ (b.float() * sb)
    parity = gemm_parity(torch, dtype, c[rows].float(), ref)
    flops = 2.0 * m * n * k
    tflops = flops / secs / 1e12
    info = lib.gemm_info(dt, m, n, k)
    del a, b, c, ws, ref
    torch.cuda.empty_cache()
    return {
        "shape": [m, n, k],
        "latency_us": secs * 1e6,
        "launch_us": launch_spread(per_launch),
        "clock": clock.summary(),
        "achieved_tflops": tflops,
        "mfu_pct": 100.0 * tflops / MFMA_PEAK_TFLOPS[dtype],
        "parity": {**parity, "rows_checked": 256},
        "warmup_launches": warmup,
        "implementation": info.get("implementation"),
    }


CEILING_INSTRUCTIONS = ("v_mfma_f32_32x32x16_bf16", "v_mfma_scale_f32_16x16x128_f8f6f4",
                        "v_mfma_scale_f32_32x32x64_f8f6f4")
# The instruction each 8192^3 GEMM kernel runs: its sustained rate bounds what the GEMM's MFMA work can reach.
GEMM_INSTRUCTION = {"bfloat16": "v_mfma_f32_32x32x16_bf16", "float8_e4m3fn": "v_mfma_scale_f32_16x16x128_f8f6f4"}


def bench_mfma_ceiling(torch, lib, capi, names=CEILING_INSTRUCTIONS, launch_s: float = 2e-3,
                       warmup_s: float = GEMM_WARMUP_S, launches: int = 20) -> dict:
    """Sustained TFLOP/s of each MFMA instruction with no memory traffic (mb_mfma_ceiling): one 256-thread
    block per CU issuing 8 independent MFMAs per wave per round on random operands of the instruction's type,
    about launch_s per launch, an untimed warmup of warmup_s (the clock settles under the power limit), then
    `launches` event-timed launches bracketed by clock stamps."""
    from teamredbench_amd.profiling.clock import ClockWindow

    dev = torch.device("cuda:0")
    handle = torch.cuda.current_stream(dev).cuda_stream
    blocks = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(256 * blocks, device=dev, dtype=torch.float32)
    gen = torch.Generator().manual_seed(0)
    result = {}
    for name in names:
        code, flop, dtype = capi.MFMA_INSTRUCTIONS[name]
        values = torch.randn(capi.MFMA_CEILING_OPERAND_BYTES, generator=gen)
        if dtype == "bfloat16":
            raw = values[: capi.MFMA_CEILING_OPERAND_BYTES // 2].to(torch.bfloat16).view(torch.uint8)
        elif dtype == "float8_e4m3fn":
            raw = values.to(torch.float8_e4m3fn).view(torch.uint8)
        else:
            raw = values[: capi.MFMA_CEILING_OPERAND_BYTES // 4].view(torch.uint8)
        ops = raw.to(dev)
        per_round = blocks * 4 * capi.MFMA_CEILING_CHAINS * flop
        probe = lib.mfma_ceiling(code, ops.data_ptr(), out.data_ptr(), blocks, 256, 1, 2, handle)
        iterations = max(2, int(launch_s / probe * 256))
        per_launch = lib.mfma_ceiling(code, ops.data_ptr(), out.data_ptr(), blocks, iterations, 0, 1, handle)
        warmup = max(1, int(warmup_s / per_launch))
        lib.mfma_ceiling(code, ops.data_ptr(), out.data_ptr(), blocks, iterations, warmup, 1, handle)
        clock = ClockWindow(torch, lib, handle)
        clock.start()
        secs = lib.mfma_ceiling(code, ops.data_ptr(), out.data_ptr(), blocks, iterations, 0, launches, handle)
        clock.stop()
        torch.cuda.synchronize()
        rounds = (iterations + 1) // 2 * 2
        tflops = per_round * rounds / secs / 1e12
        result[name] = {"tflops": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS.get(dtype, 157.3),
                        "frac_of_peak": round(tflops / MFMA_PEAK_TFLOPS.get(dtype, 157.3), 4),
                        "launch_us": round(secs * 1e6, 1), "clock": clock.summary()}
    return result


def _cpu_quota() -> float | None:
    """CPUs the cgroup quota allows this process (cpu.max), or None when unlimited or unreadable."""
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text(encoding="utf-8").split()[:2]
        return None if quota == "max" else int(quota) / int(period)
    except (OSError, ValueError):
        return None


def _time_triad_cpu(rp, n: int, warmup: int, iterations: int) -> float:
    """Mean wall-clock seconds of torch.add(b, c, alpha=3.0, out=a) on CPU tensors, b then c drawn
    uniform[-1, 1] fp32 from one generator seeded 0 (the reference path, hbm.py:36-38, timed as
    utils.py:14-29 times it, without a device synchronisation)."""
    import torch

    b, c = rp.stream_inputs(n, "float32", seed=0)
    a = torch.empty_like(b)
    for _ in range(warmup):
        rp.run_mode("triad", b, a, c, 3.0)
    t0 = time.perf_counter()
    for _ in range(iterations):
        rp.run_mode("triad", b, a, c, 3.0)
    return (time.perf_counter() - t0) / iterations


def cpu_baseline(large_iterations: int) -> dict:
    """The CPU triad configuration, timed as configured: 2^24 fp32 elements per array, seed 0, 5 warmup +
    20 timed iterations, torch threads = every CPU this process may run on (sched_getaffinity), that
    count recorded. The same op at the GPU step's 2^28 elements is reported beside it."""
    import torch

    from oracle import reference_path as rp

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    n = 1 << 24
    per = _time_triad_cpu(rp, n, warmup=5, iterations=20)
    out = {
        "value": 3 * 4 * n / per / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": ("fp32 triad a = b + 3*c over 2^24 elements per array (b, c uniform[-1, 1] from seed 0), "
                   "torch.add(b, c, alpha=3.0, out=a) on CPU tensors, 5 warmup + 20 timed iterations, "
                   f"{per * 1e3:.3f} ms per iteration"),
        "cpu_quota_cores": _cpu_quota(),
    }
    if large_iterations > 0:
        big = TRIAD_ELEMENTS
        per_big = _time_triad_cpu(rp, big, warmup=2, iterations=large_iterations)
        out["at_gpu_step_size"] = {
            "value": 3 * 4 * big / per_big / 1e9, "unit": "GB/s", "elements": big,
            "sample": f"the same op over 2^28 elements per array, 2 warmup + {large_iterations} timed iterations",
        }
    return out


GEMM_CPU_ROWS = 512


def cpu_gemm_baseline(dtype: str, size: int, rows: int = GEMM_CPU_ROWS, min_seconds: float = 2.0) -> dict:
    """torch.mm on CPU tensors (the reference torch path, mfu.py:229-238) over a rows x size slab of A
    against the whole size x size B: 1 untimed call, then timed calls until min_seconds have passed (at
    most 5). bf16 multiplies bf16 tensors; fp8 e4m3 multiplies fp32 tensors, the dequantised values the
    oracle uses, since torch.mm has no CPU kernel for float8. Threads: every CPU this process may use."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    a = torch.randn(rows, size, generator=gen) / math.sqrt(size)
    b = torch.randn(size, size, generator=gen) / math.sqrt(size)
    if dtype == "bfloat16":
        a, b = a.to(torch.bfloat16), b.to(torch.bfloat16)
    c = torch.empty(rows, size, dtype=a.dtype)
    torch.mm(a, b, out=c)
    calls, t0 = 0, time.perf_counter()
    while calls < 1 or (time.perf_counter() - t0 < min_seconds and calls < 5):
        torch.mm(a, b, out=c)
        calls += 1
    per = (time.perf_counter() - t0) / calls
    operands = "bf16" if dtype == "bfloat16" else "fp32 (dequantised fp8)"
    return {
        "value": 2.0 * rows * size * size / per / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"torch.mm on {operands} CPU tensors, a {rows} x {size} slab of A against the {size} x {size} B "
                   f"({2.0 * rows * size * size / 1e9:.1f} GFLOP per call), 1 untimed + {calls} timed calls, "
                   f"{per * 1e3:.1f} ms per call"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--no-gemm", action="store_true", help="skip the 8192^3 GEMM measurements")
    parser.add_argument("--gemm-iterations", type=int, default=50)
    parser.add_argument("--cpu-iterations", type=int, default=20,
                        help="timed CPU iterations at the GPU step's 2^28 size, beside the 2^24 CPU triad "
                             "configuration (0 = that configuration only); --no-cpu skips the CPU baseline")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-mfma-ceiling", action="store_true",
                        help="skip the sustained-rate measurement of the MFMA instructions the GEMMs run")
    parser.add_argument("--calibration-copy", action="store_true",
                        help="before the triad, launch the fp32 copy kernel 3 times over 2^28 elements (1 GiB read, "
                             "1 GiB written per launch, untimed): the known traffic that scales FETCH_SIZE / "
                             "WRITE_SIZE when rocprofv3 counter passes run over this command")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the stream and GEMM paths shard "
              "with no exchange, so N GPUs = N independent single-GPU runs.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        parser.error("--steps must be >= 1 and --warmup >= 0")

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a visible MI355X (torch.cuda.is_available() is False)", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    from teamredbench_amd.native import capi

    lib = capi.load_library()  # raises if the HIP library is missing or stale: no fallback

    if args.calibration_copy:
        _log("calibration: 3 copy launches over 2^28 fp32 elements")
        src = torch.zeros(TRIAD_ELEMENTS, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            lib.stream(capi.OP_COPY, capi.DT_FLOAT32, dst.data_ptr(), src.data_ptr(), None, TRIAD_ELEMENTS, 1.0, 0,
                       torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    _log(f"triad fp32 2^28: warmup {args.warmup}, steps {args.steps}")
    triad = bench_triad(torch, lib, capi, args.steps, args.warmup)
    value = triad["moved_bytes"] / triad["wall_s_per_step"] / 1e9
    achieved = triad["moved_bytes"] / triad["event_s_per_launch"] / 1e9
    _log(f"triad: {value:.1f} GB/s wall, {achieved:.1f} GB/s events, parity {triad['parity']}")
    torch.cuda.empty_cache()

    gemm = {}
    if not args.no_gemm:
        for dtype in ("bfloat16", "float8_e4m3fn"):
            _log(f"gemm {dtype} 8192^3")
            gemm[dtype] = bench_gemm(torch, lib, capi, dtype, 8192, warmup=3, iterations=args.gemm_iterations)
            _log(f"gemm {dtype}: {gemm[dtype]['achieved_tflops']:.1f} TFLOPS ({gemm[dtype]['mfu_pct']:.1f}% MFU)")

    ceiling = None
    if not args.no_gemm and not args.no_mfma_ceiling:
        _log("mfma ceiling: " + ", ".join(CEILING_INSTRUCTIONS))
        ceiling = bench_mfma_ceiling(torch, lib, capi)
        for dtype, entry in gemm.items():
            top = ceiling[GEMM_INSTRUCTION[dtype]]["tflops"]
            entry["mfma_instruction"] = GEMM_INSTRUCTION[dtype]
            entry["frac_of_mfma_ceiling"] = round(entry["achieved_tflops"] / top, 4)
        _log("mfma ceiling: " + ", ".join(f"{k} {v['tflops']} TFLOPS" for k, v in ceiling.items()))

    baseline = None
    if not args.no_cpu:
        _log("cpu baseline: 2^24 fp32 triad, 5 warmup + 20 timed")
        baseline = cpu_baseline(args.cpu_iterations)
        _log(f"cpu baseline: {baseline['value']:.1f} GB/s on {baseline['cores']} threads")
        for dtype, entry in gemm.items():
            _log(f"cpu baseline: torch.mm {dtype}, {GEMM_CPU_ROWS} x 8192 x 8192 slab")
            entry["cpu_baseline"] = cpu_gemm_baseline(dtype, 8192)
            _log(f"cpu baseline: {entry['cpu_baseline']['value']:.3f} TFLOPS ({entry['cpu_baseline']['sample']})")

    traffic = read_traffic()
    line = {
        "metric": "triad HBM GB/s & % peak; bf16/fp8 GEMM TFLOPS & MFU% at 8192^3",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": triad["wall_s_per_step"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: b, c ~ uniform[-1, 1] fp32 from seed 0, resident in HBM",
        "config": {
            "workload": "stream triad a = b + 3*c, fp32, 2^28 elements per array (3 GiB moved per step)",
            "elements": TRIAD_ELEMENTS,
            "element_dtype": "float32",
            "scale": 3.0,
        },
        "hbm_efficiency_pct": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "algorithmic_bytes": triad["moved_bytes"],
            "kernel": triad["info"].get("implementation"),
            "launch_us": triad["launch_us"],
            "clock": triad["clock"],
        },
        "parity": triad["parity"],
        "kernel_info": triad["info"],
        "gemm": gemm or None,
        "mfma_ceiling": ceiling,
        "cpu_baseline": baseline,
    }
    if traffic:
        line["roofline"]["traffic_source"] = traffic["source"]
    print(json.dumps(line), flush=True)
    ok = triad["parity"]["passed"] and all(g["parity"]["passed"] for g in gemm.values())
    return 0 if ok else 3


if __name__ == "__main__":
    sys.exit(main())
