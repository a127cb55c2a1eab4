"""``hbm`` benchmark: STREAM copy / scale / triad.

API and record shape follow src/teamredbench/benchmarks/hbm.py:
  params: backend (torch|native), dtypes, modes [copy|scale|triad],
          size_mib (bytes per array, default 1024), warmup (10),
          iterations (50), scale (1.0), blocks_per_cu (optional override),
          native.{kernel|source|binary|...}
  extension params: elements (list of element counts; overrides size_mib,
          one case per count), seed (input seed, default 0), verify
          (compare against the torch op, default true), allocations (native
          backend: time the case on this many sets of arrays, each allocated
          while the earlier ones are still held, so each lands elsewhere in
          HBM, and report the median; default 1, the reference's single
          allocation -- where the arrays sit moves a 2^28-element case by up
          to ~5%)
  record: case "<mode>_<size_mib>MiB" (or "<mode>_<n>el"), raw_metrics
          elapsed_s / moved_bytes / peak_bandwidth_gbps
  moved_bytes = MODE_BYTE_FACTORS[mode] * numel * bytes_per_element.

backend "native" with a built-in kernel runs libmi355bench.so in-process
(mb_time_stream: warmup launches, then an event-timed loop on torch's current
stream, like run_kernel<T> in the reference executable,
native/kernels/hbm_bandwidth.hip.cpp:390-425). External executables keep the
reference's subprocess contract.
"""
from __future__ import annotations

import statistics
from typing import Any

from teamredbench_amd.benchmarks.base import Benchmark, BenchmarkRecord
from teamredbench_amd.benchmarks.native_exec import ExecutableCase, run_executable_cases
from teamredbench_amd.device import rocm_device_available
from teamredbench_amd.native import capi
from teamredbench_amd.native.runtime import resolve_native_kernel
from teamredbench_amd.parity import stream_parity
from teamredbench_amd.registry import register_benchmark
from teamredbench_amd.utils import make_tensor, seeded_uniform, timed_iterations

MODE_BYTE_FACTORS = {
    "copy": 2,
    "scale": 2,
    "triad": 3,
}

# MI355X Infinity Cache (MALL): working sets at or below this stay cache-resident
# across timed iterations, so their GB/s is not an HBM figure.
INFINITY_CACHE_BYTES = 256 * 1024 * 1024


@register_benchmark("hbm")
class HbmBandwidthBenchmark(Benchmark):
    default_metrics = ["hbm_bandwidth_gbps", "hbm_efficiency_pct", "latency_us"]

    # ------------------------------------------------------------ shared
    # The reference's stream ops (hbm.py:29-39) as PyTorch computes them: the
    # torch backend times these, and the native backend checks its output
    # against them on the same arrays.
    TORCH_OPS = {
        "copy": lambda torch, dst, src, aux, s: dst.copy_(src),
        "scale": lambda torch, dst, src, aux, s: torch.mul(src, s, out=dst),
        "triad": lambda torch, dst, src, aux, s: torch.add(src, aux, alpha=s, out=dst),
    }

    def _device_problem(self) -> str | None:
        """Why no GPU case can run here, or None."""
        if self.context.torch_module is None:
            return "PyTorch is not installed."
        if not rocm_device_available(self.context.torch_module):
            return "No ROCm device visible to PyTorch."
        return None

    def _inputs(self, spec, mode: str, numel: int, seed: int):
        """(src, aux or None): uniform[-1, 1] from `seed` / `seed + 1` for the float types and int8
        (drawn on the device), torch's generic random fill for any other type."""
        torch = self.torch
        if spec.kind == "float" or spec.name == "int8":
            make = lambda s: seeded_uniform(torch, numel, spec.name, self.device, s)  # noqa: E731
        else:
            make = lambda s: make_tensor(torch, spec, (numel,), self.device)  # noqa: E731
        return make(seed), (make(seed + 1) if mode == "triad" else None)

    def _common_params(self) -> tuple[int, int, int, list[str], float]:
        size_mib = int(self.params.get("size_mib", 1024))
        warmup = int(self.params.get("warmup", 10))
        iterations = int(self.params.get("iterations", 50))
        modes = list(self.params.get("modes", ["copy"]))
        scale = float(self.params.get("scale", 1.0))
        return size_mib, warmup, iterations, modes, scale

    def _sizes(self, spec) -> list[tuple[int, str, dict[str, Any]]]:
        """(numel, case suffix, size metadata) per case for one dtype."""
        elements = self.params.get("elements")
        if elements is not None:
            counts = [int(x) for x in (elements if isinstance(elements, list) else [elements])]
            return [(n, f"{n}el", {"elements": n}) for n in counts]
        size_mib = int(self.params.get("size_mib", 1024))
        numel = max(size_mib * 1024 * 1024 // spec.bytes_per_element, 1)
        return [(numel, f"{size_mib}MiB", {"size_mib": size_mib, "elements": numel})]

    # ------------------------------------------------------------ native
    def _run_native(self) -> list[BenchmarkRecord]:
        kernel = resolve_native_kernel(
            benchmark=self.name,
            params=self.params,
            suite_path=self.context.suite_path,
            repo_root=self.context.repo_root,
            default_kernel="hbm_hip",
        )
        if kernel.in_process:
            return self._run_capi(kernel.name)
        return self._run_executable(kernel)

    def _run_executable(self, kernel) -> list[BenchmarkRecord]:
        size_mib, warmup, iterations, modes, scale = self._common_params()
        peak = self.context.hardware_profile.peak_hbm_bandwidth_gbps
        cases: list[ExecutableCase] = []
        for spec in self.selected_dtype_specs():
            numel = max(size_mib * 1024 * 1024 // spec.bytes_per_element, 1)
            for mode in modes:
                metadata = {"backend": "native", "kernel": kernel.name, "mode": mode, "size_mib": size_mib,
                            "elements": numel}
                argv = ["--dtype", spec.name, "--mode", mode, "--size-mib", str(size_mib), "--warmup", str(warmup),
                        "--iterations", str(iterations), "--device-id", str(self.context.device_id),
                        "--scale", str(scale)]
                if self.params.get("blocks_per_cu") is not None:
                    argv += ["--blocks-per-cu", str(int(self.params["blocks_per_cu"]))]
                    metadata["blocks_per_cu"] = int(self.params["blocks_per_cu"])
                moved = MODE_BYTE_FACTORS[mode] * numel * spec.bytes_per_element

                def defaults(raw: dict[str, Any], moved: int = moved) -> None:
                    raw.setdefault("moved_bytes", moved)
                    raw.setdefault("peak_bandwidth_gbps", peak)

                cases.append(ExecutableCase(f"{mode}_{size_mib}MiB", spec.name, metadata, argv, defaults))
        return run_executable_cases(self, kernel, cases)

    def _run_capi(self, kernel_name: str) -> list[BenchmarkRecord]:
        _, warmup, iterations, modes, scale = self._common_params()
        seed = int(self.params.get("seed", 0))
        verify = bool(self.params.get("verify", True))
        bpc = int(self.params.get("blocks_per_cu") or 0)
        peak = self.context.hardware_profile.peak_hbm_bandwidth_gbps

        plan: list[tuple[Any, str, int, str, dict[str, Any]]] = []
        for spec in self.selected_dtype_specs():
            for numel, suffix, size_meta in self._sizes(spec):
                for mode in modes:
                    meta = {"backend": "native", "kernel": kernel_name, "mode": mode, **size_meta}
                    if bpc:
                        meta["blocks_per_cu"] = bpc
                    plan.append((spec, mode, numel, f"{mode}_{suffix}", meta))

        def skip_all(error: str) -> list[BenchmarkRecord]:
            return [self.skip(case=case, dtype=spec.name, error=error, metadata=meta)
                    for spec, _, _, case, meta in plan]

        try:
            lib = capi.load_library()
        except capi.NativeLibraryError as exc:
            return skip_all(str(exc))
        problem = self._device_problem()
        if problem is not None:
            return skip_all(problem)
        torch = self.torch
        self.set_device()

        records: list[BenchmarkRecord] = []
        for spec, mode, numel, case, meta in plan:
            if mode not in MODE_BYTE_FACTORS:
                records.append(self.skip(case=case, dtype=spec.name, error=f"Unknown HBM mode: {mode}", metadata=meta))
                continue
            supported = spec.name in capi.STREAM_DTYPES and (spec.name != "int8" or mode == "copy")
            if not supported:
                records.append(self.skip(case=case, dtype=spec.name, metadata=meta,
                                         error=f"unsupported dtype or mode for native HBM kernel: {spec.name}/{mode}"))
                continue
            try:
                records.append(self._capi_case(lib, torch, spec, mode, numel, case, meta, scale, bpc, warmup,
                                               iterations, seed, verify, peak))
            except (capi.NativeLibraryError, RuntimeError) as exc:
                records.append(self.skip(case=case, dtype=spec.name, error=str(exc), metadata=meta))
            finally:
                torch.cuda.empty_cache()
        return records

    def _capi_case(self, lib, torch, spec, mode, numel, case, meta, scale, bpc, warmup, iterations, seed, verify,
                   peak) -> BenchmarkRecord:
        device = self.device
        src, aux = self._inputs(spec, mode, numel, seed)
        dst = torch.empty_like(src)
        op, dt = capi.OPS[mode], capi.DTYPES[spec.name]
        stream = torch.cuda.current_stream(device).cuda_stream
        allocations = max(1, int(self.params.get("allocations", 1)))
        held = []          # the earlier sets stay allocated, so every set gets its own placement
        timings = []
        for index in range(allocations):
            if index:
                held.append((src, aux, dst))
                src, aux = src.clone(), (aux.clone() if aux is not None else None)
                dst = torch.empty_like(src)
            timings.append(lib.time_stream(op, dt, dst.data_ptr(), src.data_ptr(),
                                           aux.data_ptr() if aux is not None else None, numel, scale, bpc, warmup,
                                           iterations, stream))
        elapsed = statistics.median(timings)
        del held
        meta = {**meta, **lib.stream_info(op, dt, numel, bpc)}
        if allocations > 1:
            meta["allocations"] = allocations
            meta["allocation_elapsed_s"] = timings
        moved = MODE_BYTE_FACTORS[mode] * numel * spec.bytes_per_element
        working_set = (3 if mode == "triad" else 2) * numel * spec.bytes_per_element
        meta["working_set_bytes"] = working_set
        meta["cache_resident"] = working_set <= INFINITY_CACHE_BYTES
        if verify:
            ref = torch.empty_like(src)
            self.TORCH_OPS[mode](torch, ref, src, aux, scale)
            meta["parity"] = stream_parity(torch, mode, dst, ref)
            del ref
        return self.measured(case=case, dtype=spec.name, metadata=meta,
                             raw_metrics={"elapsed_s": elapsed, "moved_bytes": moved, "peak_bandwidth_gbps": peak})

    # ------------------------------------------------------------- torch
    # The reference torch path (hbm.py:174-240): the op through PyTorch's own
    # kernels, timed by wall clock between device synchronisations
    # (utils.timed_iterations), the reference's timing for this backend. It
    # runs on the native path's seeded inputs (the reference draws unseeded
    # randn), so the two backends' records time the same data; cases and
    # sizes follow the same params (size_mib or elements).
    def _run_torch(self) -> list[BenchmarkRecord]:
        problem = self._device_problem()
        if problem is not None:
            return [self.skip(case="global", dtype="n/a", error=problem)]
        self.set_device()
        _, warmup, iterations, modes, scale = self._common_params()
        seed = int(self.params.get("seed", 0))
        peak = self.context.hardware_profile.peak_hbm_bandwidth_gbps
        return [self._torch_case(spec, mode, numel, suffix, size_meta, scale, warmup, iterations, seed, peak)
                for spec in self.selected_dtype_specs()
                for numel, suffix, size_meta in self._sizes(spec)
                for mode in modes]

    def _torch_case(self, spec, mode, numel, suffix, size_meta, scale, warmup, iterations, seed,
                    peak) -> BenchmarkRecord:
        torch = self.torch
        case, meta = f"{mode}_{suffix}", {"backend": "torch", "mode": mode, **size_meta}
        if mode not in self.TORCH_OPS:
            return self.skip(case=case, dtype=spec.name, error=f"Unknown HBM mode: {mode}", metadata=meta)
        op = self.TORCH_OPS[mode]
        try:
            src, aux = self._inputs(spec, mode, numel, seed)
            dst = torch.empty_like(src)
            elapsed = timed_iterations(lambda: op(torch, dst, src, aux, scale), torch_module=torch, warmup=warmup,
                                       iterations=iterations)
        except Exception as exc:  # noqa: BLE001 -- an op torch cannot run for this dtype skips this case only
            return self.skip(case=case, dtype=spec.name, error=str(exc), metadata=meta)
        finally:
            torch.cuda.empty_cache()
        working_set = (3 if mode == "triad" else 2) * numel * spec.bytes_per_element
        meta.update(working_set_bytes=working_set, cache_resident=working_set <= INFINITY_CACHE_BYTES,
                    timing="wall_clock")
        moved = MODE_BYTE_FACTORS[mode] * numel * spec.bytes_per_element
        return self.measured(case=case, dtype=spec.name, metadata=meta,
                             raw_metrics={"elapsed_s": elapsed, "moved_bytes": moved, "peak_bandwidth_gbps": peak})

    def run(self) -> list[BenchmarkRecord]:
        backend = str(self.params.get("backend", "torch")).lower()
        if backend == "torch":
            return self._run_torch()
        if backend == "native":
            return self._run_native()
        raise KeyError(f"Unknown HBM backend: {backend}")
