"""Device discovery through torch's ROCm build (src/teamredbench/device.py:9-127).

PyTorch exposes ROCm GPUs through the ``torch.cuda`` namespace; ``cuda:N``
is the N-th HIP device.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
import os
import shutil
import subprocess
from typing import Any


@dataclass
class DeviceInfo:
    index: int
    name: str
    total_memory_bytes: int | None = None
    multiprocessor_count: int | None = None
    clock_rate_khz: int | None = None
    gcn_arch_name: str | None = None


def load_torch():
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


def _run_command(command: list[str]) -> str | None:
    if shutil.which(command[0]) is None:
        return None
    try:
        proc = subprocess.run(command, capture_output=True, text=True, timeout=60)
    except (OSError, subprocess.TimeoutExpired):
        return None
    if proc.returncode != 0:
        return None
    return proc.stdout.strip() or None


def detect_device(torch_module: Any, device_id: int = 0) -> DeviceInfo | None:
    if not rocm_device_available(torch_module):
        return None
    props = torch_module.cuda.get_device_properties(device_id)
    arch = None
    for attr in ("gcnArchName", "gcn_arch_name", "arch"):
        value = getattr(props, attr, None)
        if value:
            arch = str(value)
            break
    return DeviceInfo(
        index=device_id,
        name=str(props.name),
        total_memory_bytes=getattr(props, "total_memory", None),
        multiprocessor_count=getattr(props, "multi_processor_count", None),
        clock_rate_khz=getattr(props, "clock_rate", None),
        gcn_arch_name=arch,
    )


def detect_runtime(torch_module: Any) -> dict[str, Any]:
    torch_info: dict[str, Any] = {}
    if torch_module is not None:
        torch_info = {
            "torch_version": getattr(torch_module, "__version__", "unknown"),
            "hip_version": getattr(getattr(torch_module, "version", None), "hip", None),
        }
    rocminfo = _run_command(["rocminfo"])
    return {
        "torch": torch_info,
        "hipcc_version": _run_command(["hipcc", "--version"]),
        "rocminfo_head": "\n".join(rocminfo.splitlines()[:40]) if rocminfo else None,
        "rocm_smi_product": _run_command(["rocm-smi", "--showproductname"]),
    }


def host_cores() -> int:
    """CPU cores this process may run on (the CPU-baseline thread count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def discover_environment(torch_module: Any, device_id: int = 0) -> dict[str, Any]:
    device = detect_device(torch_module, device_id=device_id)
    return {
        "device": asdict(device) if device else None,
        "runtime": detect_runtime(torch_module),
        "suggested_hardware_profile": {
            "name": device.name if device else "fill-me",
            "family": "cdna-or-rdna",
            "peak_hbm_bandwidth_gbps": None,
            "peak_link_bandwidth_gbps": {"xgmi": None, "network": None},
            "peak_compute_tops": {},
            "notes": ["Fill in theoretical peak values before using MFU or efficiency metrics."],
        },
    }
