"""Input generation and the torch backend's timing.

``timed_iterations`` is the torch backend's clock (the semantics of
src/teamredbench/utils.py:14-29): run the op `warmup` times, synchronise the
device, then report the wall-clock mean of `iterations` calls bracketed by
device synchronisations. The native backend times with hipEvents inside the
library instead (mb_time_stream / mb_time_gemm).
"""
from __future__ import annotations

import math
import time
from typing import Any, Callable

from teamredbench_amd.device import synchronize_rocm_device
from teamredbench_amd.dtypes import DTypeSpec


def synchronize(torch_module: Any) -> None:
    synchronize_rocm_device(torch_module)


def timed_iterations(fn: Callable[[], None], *, torch_module: Any, warmup: int, iterations: int) -> float:
    """Mean seconds per call of `fn`, after `warmup` untimed calls."""
    calls = max(iterations, 1)
    for _ in range(max(warmup, 0)):
        fn()
    synchronize(torch_module)
    began = time.perf_counter()
    for _ in range(calls):
        fn()
    synchronize(torch_module)
    return (time.perf_counter() - began) / calls


def _random_of_kind(torch: Any, kind: str, shape: tuple[int, ...], device: Any, dtype: Any):
    """Unseeded random values for one dtype kind, in a type torch can draw them in."""
    if kind == "bool":
        return torch.randint(0, 2, shape, device=device, dtype=torch.uint8)
    if kind == "integer":
        return torch.randint(0, 17, shape, device=device, dtype=dtype)
    if kind == "complex":
        part = torch.float32 if dtype == torch.complex64 else torch.float64
        return torch.complex(torch.randn(shape, device=device, dtype=part), torch.randn(shape, device=device, dtype=part))
    return torch.randn(shape, device=device, dtype=torch.float32)


def make_tensor(torch_module: Any, spec: DTypeSpec, shape: tuple[int, ...], device: Any):
    """An unseeded random tensor of `spec` (for dtypes the seeded generators below do not cover)."""
    dtype = getattr(torch_module, spec.torch_attr)
    return _random_of_kind(torch_module, spec.kind, shape, device, dtype).to(dtype=dtype)


def seeded_uniform(torch_module: Any, numel: int, dtype_name: str, device: Any, seed: int):
    """uniform[-1, 1] drawn in fp32 from a device generator seeded `seed`, cast to the dtype."""
    torch = torch_module
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    values = torch.empty(numel, device=device, dtype=torch.float32).uniform_(-1.0, 1.0, generator=gen)
    if dtype_name == "int8":
        return (values * 100).to(torch.int8)
    return values.to(getattr(torch, dtype_name))


# Largest finite value of each fp8 format (the per-tensor quantisation target).
FP8_MAX = {"float8_e4m3fn": 448.0, "float8_e5m2": 57344.0}


def seeded_gemm_operands(torch_module: Any, m: int, n: int, k: int, dtype_name: str, device: Any, seed: int):
    """GEMM operands on the device: normal(0, 1/sqrt(k)) for bf16/f16/f32/f64;
    for fp8 normal(0, 1) scaled per tensor so amax maps to the format's
    largest finite value (448 for e4m3fn, 57344 for e5m2) and cast.
    Returns (a, b, scale_a, scale_b)."""
    torch = torch_module
    ga = torch.Generator(device=device)
    ga.manual_seed(seed)
    gb = torch.Generator(device=device)
    gb.manual_seed(seed + 1)
    a = torch.randn(m, k, device=device, dtype=torch.float32, generator=ga)
    b = torch.randn(k, n, device=device, dtype=torch.float32, generator=gb)
    if dtype_name in FP8_MAX:
        fp8 = getattr(torch, dtype_name)
        sa = float(a.abs().max()) / FP8_MAX[dtype_name]
        sb = float(b.abs().max()) / FP8_MAX[dtype_name]
        return (a / sa).to(fp8), (b / sb).to(fp8), sa, sb
    if dtype_name == "float64":
        a, b = a.double(), b.double()
    dtype = getattr(torch, dtype_name)
    std = 1.0 / math.sqrt(k)
    return (a * std).to(dtype), (b * std).to(dtype), 1.0, 1.0


def tensor_nbytes(tensor: Any) -> int:
    return int(tensor.numel() * tensor.element_size())
