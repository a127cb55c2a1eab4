"""Native-kernel registry (API of src/teamredbench/native/registry.py:7-48).

A definition names a kernel, the benchmark it serves and how it is reached:
  * ``abi="capi"``        -- an entry of libmi355bench.so called in-process
                             through the C ABI (include/mi355bench.h);
  * ``abi="executable"``  -- the reference's contract: a HIP source compiled
                             by hipcc into an executable that takes argv and
                             prints one JSON line (third-party plugins).
``aliases`` registers the same definition under extra names, so suites that
select the reference's built-ins (``hbm_hip``, ``mfu_hipblas``) resolve to
the gfx950 kernels.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

ABI_CAPI = "capi"
ABI_EXECUTABLE = "executable"


@dataclass(frozen=True)
class NativeKernelDefinition:
    name: str
    benchmark: str
    description: str
    source_path: Path | None = None
    compile_args: tuple[str, ...] = ()
    abi: str = ABI_EXECUTABLE
    aliases: tuple[str, ...] = field(default_factory=tuple)


NATIVE_KERNEL_REGISTRY: dict[str, NativeKernelDefinition] = {}


def register_native_kernel(
    *,
    name: str,
    benchmark: str,
    description: str,
    source_path: Path | None = None,
    compile_args: tuple[str, ...] = (),
    abi: str = ABI_EXECUTABLE,
    aliases: tuple[str, ...] = (),
) -> NativeKernelDefinition:
    if abi not in (ABI_CAPI, ABI_EXECUTABLE):
        raise ValueError(f"unknown native kernel abi {abi!r}")
    definition = NativeKernelDefinition(
        name=name,
        benchmark=benchmark,
        description=description,
        source_path=source_path,
        compile_args=tuple(compile_args),
        abi=abi,
        aliases=tuple(aliases),
    )
    for key in (name, *aliases):
        NATIVE_KERNEL_REGISTRY[key] = definition
    return definition


def get_native_kernel(name: str) -> NativeKernelDefinition:
    if name not in NATIVE_KERNEL_REGISTRY:
        raise KeyError(f"Unknown native kernel: {name}")
    return NATIVE_KERNEL_REGISTRY[name]


def list_native_kernels(benchmark: str | None = None) -> list[NativeKernelDefinition]:
    """Registered definitions (each once, aliases folded), sorted by name."""
    unique = {d.name: d for d in NATIVE_KERNEL_REGISTRY.values()}
    found = sorted(unique.values(), key=lambda d: d.name)
    return [d for d in found if benchmark is None or d.benchmark == benchmark]


def registered_names() -> set[str]:
    """Every selectable name, aliases included."""
    return set(NATIVE_KERNEL_REGISTRY)
