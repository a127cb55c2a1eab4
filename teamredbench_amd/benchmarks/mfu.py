"""``mfu`` benchmark: dense GEMM C = A * B and its model-FLOPs utilisation.

API and record shape follow src/teamredbench/benchmarks/mfu.py:
  params: backend (torch|native), dtypes, shapes [[m, n, k], ...] (default
          4096^3 and 8192^3), warmup (10), iterations (50), native.{...}
  extension params: seed (default 0), verify (compare against torch,
          default true; at most `verify_max_rows` rows of C, default 4096),
          warmup_seconds (default 0: untimed warmup lasts at least this
          long, more launches than `warmup` if need be -- the part leaves
          its low-power clock state only after tens of ms of MFMA work),
          operand_sets ("auto", or a count: the timed loop, native and torch
          alike, cycles through that many copies of A, B and C; "auto" takes
          enough copies to span three times the 256 MB Infinity Cache (at
          most 1024) for a memory-bound shape -- arithmetic intensity below
          the dtype's ridge point, peak_tops / peak HBM bandwidth -- whose
          operands would otherwise stay cache-resident between launches, and
          1 otherwise; 1 times a single set, as the reference does)
  record: case "gemm_<m>x<n>x<k>"; raw_metrics elapsed_s / achieved_ops
          (= matmul_ops_factor * m * n * k) / peak_tops, plus gemm_bytes
          ((mk + kn) * in_bytes + mn * out_bytes) for the effective-GB/s metric.
A dtype with matmul_ops_factor 0, or without a peak in the hardware profile,
yields a skipped record (mfu.py:81-104).

backend "native" with a built-in kernel calls libmi355bench.so (mb_time_gemm,
event-timed on torch's current stream). B is consumed row-major as given:
unlike the reference executable there is no untimed re-layout of B
(native/kernels/mfu_gemm_lowp.hip.hpp:396-409). Inputs are seeded:
bf16/fp16/fp32/fp64 ~ normal(0, 1/sqrt(k)); fp8 e4m3fn / e5m2 ~ normal(0, 1)
quantised per tensor with amax -> the format's largest finite value (448 /
57344), bf16 output with the dequantisation scales applied in the fp32
epilogue. fp32 and fp64 produce C in their own type.
"""
from __future__ import annotations

from typing import Any

from teamredbench_amd.benchmarks.base import Benchmark, BenchmarkRecord
from teamredbench_amd.benchmarks.native_exec import ExecutableCase, run_executable_cases
from teamredbench_amd.device import rocm_device_available
from teamredbench_amd.native import capi
from teamredbench_amd.native.runtime import resolve_native_kernel
from teamredbench_amd.parity import gemm_parity
from teamredbench_amd.registry import register_benchmark
from teamredbench_amd.utils import seeded_gemm_operands, timed_iterations

DEFAULT_SHAPES = [
    [4096, 4096, 4096],
    [8192, 8192, 8192],
]

INFINITY_CACHE_BYTES = 256 * 1024 * 1024
# Bytes the cycled operand sets of a memory-bound shape span (three times the Infinity Cache), and the
# most sets "auto" takes to get there.
OPERAND_FOOTPRINT_TARGET = 3 * INFINITY_CACHE_BYTES
MAX_OPERAND_SETS = 1024


def gemm_bytes(m: int, n: int, k: int, in_bytes: int, out_bytes: int) -> int:
    """Algorithmic bytes of one GEMM: read A and B once, write C once."""
    return (m * k + k * n) * in_bytes + m * n * out_bytes


@register_benchmark("mfu")
class MfuBenchmark(Benchmark):
    default_metrics = ["achieved_tops", "mfu_pct", "latency_us"]

    def _common_params(self) -> tuple[int, int, list[list[int]]]:
        warmup = int(self.params.get("warmup", 10))
        iterations = int(self.params.get("iterations", 50))
        shapes = list(self.params.get("shapes", DEFAULT_SHAPES))
        return warmup, iterations, shapes

    def _gate(self, spec, peak_tops) -> str | None:
        if spec.matmul_ops_factor == 0:
            return "MFU is not defined for this dtype."
        if peak_tops is None:
            return "Missing peak_compute_tops entry for dtype in hardware profile."
        return None

    # ------------------------------------------------------------ native
    def _run_native(self) -> list[BenchmarkRecord]:
        kernel = resolve_native_kernel(
            benchmark=self.name,
            params=self.params,
            suite_path=self.context.suite_path,
            repo_root=self.context.repo_root,
            default_kernel="mfu_hipblas",
        )
        if kernel.in_process:
            return self._run_capi(kernel.name)
        return self._run_executable(kernel)

    def _run_executable(self, kernel) -> list[BenchmarkRecord]:
        warmup, iterations, shapes = self._common_params()
        cases: list[ExecutableCase] = []
        for spec in self.selected_dtype_specs():
            peak_tops = self.context.hardware_profile.peak_compute_tops.get(spec.name)
            for shape in shapes:
                m, n, k = (int(d) for d in shape)
                metadata = {"backend": "native", "kernel": kernel.name, "m": m, "n": n, "k": k}
                gate = self._gate(spec, peak_tops)
                argv = None if gate else [
                    "--dtype", spec.name, "--m", str(m), "--n", str(n), "--k", str(k), "--warmup", str(warmup),
                    "--iterations", str(iterations), "--device-id", str(self.context.device_id),
                ]
                ops = spec.matmul_ops_factor * m * n * k

                def defaults(raw: dict[str, Any], ops: int = ops, peak=peak_tops) -> None:
                    raw.setdefault("achieved_ops", ops)
                    raw.setdefault("peak_tops", peak)

                cases.append(ExecutableCase(f"gemm_{m}x{n}x{k}", spec.name, metadata, argv, defaults, gate))
        return run_executable_cases(self, kernel, cases)

    def _run_capi(self, kernel_name: str) -> list[BenchmarkRecord]:
        warmup, iterations, shapes = self._common_params()
        seed = int(self.params.get("seed", 0))
        verify = bool(self.params.get("verify", True))
        verify_rows = int(self.params.get("verify_max_rows", 4096))
        plan = []
        for spec in self.selected_dtype_specs():
            peak_tops = self.context.hardware_profile.peak_compute_tops.get(spec.name)
            for shape in shapes:
                m, n, k = (int(d) for d in shape)
                meta = {"backend": "native", "kernel": kernel_name, "m": m, "n": n, "k": k}
                plan.append((spec, peak_tops, m, n, k, f"gemm_{m}x{n}x{k}", meta))

        try:
            lib = capi.load_library()
        except capi.NativeLibraryError as exc:
            return [self.skip(case=c, dtype=s.name, error=str(exc), metadata=md) for s, _, _, _, _, c, md in plan]
        torch = self.context.torch_module
        if not rocm_device_available(torch):
            return [self.skip(case=c, dtype=s.name, error="No ROCm device visible to PyTorch.", metadata=md)
                    for s, _, _, _, _, c, md in plan]
        self.set_device()

        records: list[BenchmarkRecord] = []
        for spec, peak_tops, m, n, k, case, meta in plan:
            gate = self._gate(spec, peak_tops)
            if gate is None and spec.name not in capi.GEMM_DTYPES:
                gate = f"unsupported dtype for native GEMM kernel: {spec.name}"
            if gate:
                records.append(self.skip(case=case, dtype=spec.name, error=gate, metadata=meta))
                continue
            try:
                records.append(self._capi_case(lib, torch, spec, peak_tops, m, n, k, case, meta, warmup, iterations,
                                               seed, verify, verify_rows))
            except (capi.NativeLibraryError, RuntimeError) as exc:
                records.append(self.skip(case=case, dtype=spec.name, error=str(exc), metadata=meta))
            finally:
                torch.cuda.empty_cache()
        return records

    def _operand_sets(self, spec, m: int, n: int, k: int, out_bytes: int,
                      peak_tops: float | None) -> tuple[int, dict[str, Any]]:
        """(operand sets to cycle through, metadata describing them).

        One set is A, B and C. ``operand_sets: auto`` takes one set for a compute-bound shape (arithmetic
        intensity at or above the dtype's ridge point, peak_tops / peak HBM bandwidth) or one whose set
        already spans OPERAND_FOOTPRINT_TARGET, else enough sets to span that target (at most
        MAX_OPERAND_SETS); an integer takes that many. The metadata gives the sets' total footprint,
        ``cache_resident_b`` (true when that footprint fits the Infinity Cache, so the operands are re-read
        from the cache rather than HBM) and, when ``auto`` stopped at MAX_OPERAND_SETS short of the target,
        ``operand_footprint_short_of_target``."""
        per_set = gemm_bytes(m, n, k, spec.bytes_per_element, out_bytes)
        requested = self.params.get("operand_sets", "auto")
        if requested != "auto":
            sets = max(1, int(requested))
        else:
            sets = 1
            hbm = self.context.hardware_profile.peak_hbm_bandwidth_gbps
            if peak_tops and hbm and per_set < OPERAND_FOOTPRINT_TARGET:
                intensity = spec.matmul_ops_factor * m * n * k / per_set
                if intensity < peak_tops * 1e12 / (hbm * 1e9):
                    sets = min(MAX_OPERAND_SETS, -(-OPERAND_FOOTPRINT_TARGET // per_set))
        footprint = sets * per_set
        info: dict[str, Any] = {"operand_sets": sets, "operand_footprint_bytes": footprint,
                                "cache_resident_b": footprint <= INFINITY_CACHE_BYTES}
        if requested == "auto" and sets > 1 and footprint < OPERAND_FOOTPRINT_TARGET:
            info["operand_footprint_short_of_target"] = True
        return sets, info

    def _capi_case(self, lib, torch, spec, peak_tops, m, n, k, case, meta, warmup, iterations, seed, verify,
                   verify_rows) -> BenchmarkRecord:
        device = self.device
        a, b, sa, sb = seeded_gemm_operands(torch, m, n, k, spec.name, device, seed)
        out_dtype = getattr(torch, capi.GEMM_OUTPUT_DTYPES[spec.name])
        c = torch.empty((m, n), device=device, dtype=out_dtype)
        dt = capi.DTYPES[spec.name]
        sets, set_info = self._operand_sets(spec, m, n, k, c.element_size(), peak_tops)
        ws_bytes = lib.gemm_workspace_size(dt, m, n, k)
        ws = torch.empty(ws_bytes, device=device, dtype=torch.uint8) if ws_bytes else None
        stream = torch.cuda.current_stream(device).cuda_stream
        ws_ptr = ws.data_ptr() if ws is not None else None
        warmup_s = float(self.params.get("warmup_seconds", 0.0))
        if warmup_s > 0:
            est = lib.time_gemm(dt, a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, sa, sb, ws_ptr, ws_bytes, 0, 2,
                                stream)
            warmup = max(warmup, int(warmup_s / est) + 1)
            meta["warmup_launches"] = warmup
        if sets > 1:
            # copies of A, B and C; C of set 0 is the one checked below
            copies = [(a, b, c)] + [(a.clone(), b.clone(), torch.empty_like(c)) for _ in range(sets - 1)]
            elapsed = lib.time_gemm_rotating(dt, [x.data_ptr() for x, _, _ in copies],
                                             [y.data_ptr() for _, y, _ in copies],
                                             [z.data_ptr() for _, _, z in copies], m, n, k, sa, sb, ws_ptr, ws_bytes,
                                             warmup, iterations, stream)
            del copies
        else:
            elapsed = lib.time_gemm(dt, a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, sa, sb, ws_ptr, ws_bytes,
                                    warmup, iterations, stream)
        meta = {**meta, **lib.gemm_info(dt, m, n, k), **set_info}
        if spec.name in capi.FP8_DTYPES:
            meta["scale_a"], meta["scale_b"] = sa, sb
        in_bytes = spec.bytes_per_element
        moved = gemm_bytes(m, n, k, in_bytes, c.element_size())
        if verify:
            rows = min(m, verify_rows)
            if spec.name == "float64":
                ref = a[:rows] @ b
                got = c[:rows]
            else:
                ref = (a[:rows].float() * sa) @ (b.float() * sb)
                got = c[:rows].float()
            meta["parity"] = gemm_parity(torch, spec.name, got, ref)
            meta["parity"]["rows_checked"] = rows
            del ref
        return self.measured(case=case, dtype=spec.name, metadata=meta, raw_metrics={
            "elapsed_s": elapsed, "achieved_ops": spec.matmul_ops_factor * m * n * k, "peak_tops": peak_tops,
            "gemm_bytes": moved})

    # ------------------------------------------------------------- torch
    # The reference torch path (mfu.py:183-268): the GEMM through PyTorch's
    # library kernels (hipBLASLt), timed by wall clock between device
    # synchronisations (utils.timed_iterations). It runs on the native path's
    # seeded operands (the reference draws unseeded randn). fp8, which
    # torch.mm does not take, goes through torch._scaled_mm with the same
    # per-tensor scales and bf16 output; that routine requires B column-major,
    # so B is laid out so once, outside the timed region (recorded as b_layout).
    def _torch_gemm(self, torch, spec, a, b, sa, sb, out, sets: int = 1):
        """(callable that runs one GEMM, metadata naming the torch routine). With `sets` > 1 the callable
        cycles through that many copies of A, B and C, one per call, as the native timed loop does."""
        copies = [(a, b, out)] + [(a.clone(), b.clone(), torch.empty_like(out)) for _ in range(sets - 1)]
        turn = [0]

        def next_set():
            i = turn[0]
            turn[0] = (i + 1) % sets
            return copies[i]

        if spec.name in capi.FP8_DTYPES:
            copies = [(x, y.t().contiguous().t(), z) for x, y, z in copies]
            scale_a = torch.tensor(sa, dtype=torch.float32, device=a.device)
            scale_b = torch.tensor(sb, dtype=torch.float32, device=a.device)

            def run_fp8():
                x, y, _ = next_set()
                return torch._scaled_mm(x, y, scale_a=scale_a, scale_b=scale_b, out_dtype=torch.bfloat16)
            return run_fp8, {"torch_op": "_scaled_mm", "b_layout": "column_major"}

        def run():
            x, y, z = next_set()
            return torch.mm(x, y, out=z)
        return run, {"torch_op": "mm", "b_layout": "row_major"}

    def _run_torch(self) -> list[BenchmarkRecord]:
        torch = self.context.torch_module
        if torch is None:
            return [self.skip(case="global", dtype="n/a", error="PyTorch is not installed.")]
        if not rocm_device_available(torch):
            return [self.skip(case="global", dtype="n/a", error="No ROCm device visible to PyTorch.")]
        self.set_device()
        warmup, iterations, shapes = self._common_params()
        seed = int(self.params.get("seed", 0))
        records: list[BenchmarkRecord] = []
        for spec in self.selected_dtype_specs():
            peak_tops = self.context.hardware_profile.peak_compute_tops.get(spec.name)
            for shape in shapes:
                m, n, k = (int(d) for d in shape)
                case, meta = f"gemm_{m}x{n}x{k}", {"backend": "torch", "m": m, "n": n, "k": k}
                gate = self._gate(spec, peak_tops)
                if gate:
                    records.append(self.skip(case=case, dtype=spec.name, error=gate, metadata=meta))
                    continue
                try:
                    a, b, sa, sb = seeded_gemm_operands(torch, m, n, k, spec.name, self.device, seed)
                    out_dtype = getattr(torch, capi.GEMM_OUTPUT_DTYPES.get(spec.name, spec.torch_attr))
                    out = torch.empty((m, n), device=self.device, dtype=out_dtype)
                    sets, set_info = self._operand_sets(spec, m, n, k, out.element_size(), peak_tops)
                    gemm, routine = self._torch_gemm(torch, spec, a, b, sa, sb, out, sets)
                    elapsed = timed_iterations(gemm, torch_module=torch, warmup=warmup, iterations=iterations)
                    del gemm
                except Exception as exc:  # noqa: BLE001 -- a dtype torch cannot multiply skips this case only
                    records.append(self.skip(case=case, dtype=spec.name, error=str(exc), metadata=meta))
                    continue
                finally:
                    torch.cuda.empty_cache()
                meta.update(routine, timing="wall_clock", **set_info)
                records.append(self.measured(case=case, dtype=spec.name, metadata=meta, raw_metrics={
                    "elapsed_s": elapsed, "achieved_ops": spec.matmul_ops_factor * m * n * k, "peak_tops": peak_tops,
                    "gemm_bytes": gemm_bytes(m, n, k, spec.bytes_per_element, out.element_size())}))
        return records

    def run(self) -> list[BenchmarkRecord]:
        backend = str(self.params.get("backend", "torch")).lower()
        if backend == "torch":
            return self._run_torch()
        if backend == "native":
            return self._run_native()
        raise KeyError(f"Unknown MFU backend: {backend}")
