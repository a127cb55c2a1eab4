"""The GPU and ROCm stack this process runs on, as seen through PyTorch-ROCm.

PyTorch's ROCm build exposes HIP devices through the ``torch.cuda``
namespace (``cuda:N`` is HIP device N); nothing here needs CUDA. The public
names are the reference's (src/teamredbench/device.py:9-127), since
benchmark plugins call them. Two probes are table-driven:
  * :func:`detect_device` copies the device-property attributes listed in
    ``_PROPERTY_SOURCES`` (first attribute present wins);
  * :func:`detect_runtime` runs the tools listed in ``_TOOL_PROBES`` and
    keeps what each prints (None when a tool is missing or fails).
:func:`discover_environment` suggests a hardware profile for the device:
the packaged profile of its SKU when one matches (so its peaks are filled
in), else a skeleton to complete by hand.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
import os
import shutil
import subprocess
from typing import Any, Callable


@dataclass
class DeviceInfo:
    index: int
    name: str
    total_memory_bytes: int | None = None
    multiprocessor_count: int | None = None
    clock_rate_khz: int | None = None
    gcn_arch_name: str | None = None


def load_torch():
    """The torch module, or None where PyTorch is not installed."""
    try:
        import torch
    except ImportError:
        return None
    return torch


def rocm_device_available(torch_module: Any) -> bool:
    return torch_module is not None and bool(torch_module.cuda.is_available())


def rocm_device(torch_module: Any, device_id: int):
    return torch_module.device(f"cuda:{device_id}")


def set_rocm_device(torch_module: Any, device_id: int) -> None:
    if rocm_device_available(torch_module):
        torch_module.cuda.set_device(device_id)


def synchronize_rocm_device(torch_module: Any) -> None:
    if rocm_device_available(torch_module):
        torch_module.cuda.synchronize()


def host_cores() -> int:
    """CPU cores this process may run on (its affinity mask; the CPU baseline's thread count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# DeviceInfo field -> device-property attributes that may carry it, in order of preference.
_PROPERTY_SOURCES: dict[str, tuple[str, ...]] = {
    "total_memory_bytes": ("total_memory",),
    "multiprocessor_count": ("multi_processor_count",),
    "clock_rate_khz": ("clock_rate",),
    "gcn_arch_name": ("gcnArchName", "gcn_arch_name", "arch"),
}


def detect_device(torch_module: Any, device_id: int = 0) -> DeviceInfo | None:
    if not rocm_device_available(torch_module):
        return None
    props = torch_module.cuda.get_device_properties(device_id)
    found: dict[str, Any] = {}
    for field_name, attributes in _PROPERTY_SOURCES.items():
        values = (getattr(props, a, None) for a in attributes)
        found[field_name] = next((v for v in values if v), None)
    if found["gcn_arch_name"] is not None:
        found["gcn_arch_name"] = str(found["gcn_arch_name"])
    return DeviceInfo(index=device_id, name=str(props.name), **found)


def _run_command(command: list[str]) -> str | None:
    """stdout of a tool, stripped; None when the tool is absent, fails or prints nothing."""
    if shutil.which(command[0]) is None:
        return None
    try:
        proc = subprocess.run(command, capture_output=True, text=True, timeout=60, check=False)
    except (OSError, subprocess.TimeoutExpired):
        return None
    return (proc.stdout.strip() or None) if proc.returncode == 0 else None


def _first_lines(count: int) -> Callable[[str], str]:
    return lambda text: "\n".join(text.splitlines()[:count])


# runtime key -> (command, post-processing of its output)
_TOOL_PROBES: dict[str, tuple[list[str], Callable[[str], str]]] = {
    "hipcc_version": (["hipcc", "--version"], str),
    "rocminfo_head": (["rocminfo"], _first_lines(40)),
    "rocm_smi_product": (["rocm-smi", "--showproductname"], str),
}


def detect_runtime(torch_module: Any) -> dict[str, Any]:
    """torch / HIP versions (no CUDA fields) and what the ROCm tools report."""
    runtime: dict[str, Any] = {"torch": {}}
    if torch_module is not None:
        runtime["torch"] = {
            "torch_version": getattr(torch_module, "__version__", "unknown"),
            "hip_version": getattr(getattr(torch_module, "version", None), "hip", None),
        }
    for key, (command, post) in _TOOL_PROBES.items():
        text = _run_command(command)
        runtime[key] = None if text is None else post(text)
    return runtime


def _packaged_profile_for(device_name: str | None) -> dict[str, Any] | None:
    """The packaged hardware profile whose SKU matches the device name, as a mapping."""
    if not device_name:
        return None
    from teamredbench_amd.runner import ProfileCatalog

    match = ProfileCatalog.packaged().match(device_name)
    return None if match is None else dict(match.raw)


def discover_environment(torch_module: Any, device_id: int = 0) -> dict[str, Any]:
    device = detect_device(torch_module, device_id=device_id)
    suggested = _packaged_profile_for(device.name if device else None) or {
        "name": device.name if device else "fill-me",
        "family": "cdna-or-rdna",
        "peak_hbm_bandwidth_gbps": None,
        "peak_link_bandwidth_gbps": {"xgmi": None, "network": None},
        "peak_compute_tops": {},
        "notes": ["Fill in theoretical peak values before using MFU or efficiency metrics."],
    }
    return {
        "device": asdict(device) if device else None,
        "runtime": detect_runtime(torch_module),
        "suggested_hardware_profile": suggested,
    }
