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


# Peak engine clock (MHz) -> SKU, for gfx950 parts whose marketing name the platform does not report
# (the device name comes from libdrm's amdgpu.ids table, which a container may lack). MI355X and MI350X
# are both gfx950 with 256 CUs; their published peak engine clocks differ.
_GFX950_SKU_BY_MAX_CLOCK = {2400: "AMD Instinct MI355X", 2200: "AMD Instinct MI350X"}


def _amdsmi_names(torch_module: Any, device_id: int) -> list[str]:
    """The board's FRU product name, the ASIC's market name and, for gfx950, the SKU its peak engine clock
    identifies, as amdsmi reports them for the device with torch device `device_id`'s PCI address."""
    try:
        import amdsmi
    except Exception:  # noqa: BLE001 -- absent or broken: no names
        return []
    names: list[str] = []
    try:
        amdsmi.amdsmi_init()
    except Exception:  # noqa: BLE001
        return []
    try:
        props = torch_module.cuda.get_device_properties(device_id)
        bdf = f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}.0"
        handles = amdsmi.amdsmi_get_processor_handles()
        handle = next((h for h in handles if str(amdsmi.amdsmi_get_gpu_device_bdf(h)).lower() == bdf), None)
        if handle is None and len(handles) == 1:
            handle = handles[0]
        if handle is None:
            return []
        for getter, key in ((amdsmi.amdsmi_get_gpu_board_info, "product_name"),
                            (amdsmi.amdsmi_get_gpu_asic_info, "market_name")):
            try:
                value = getter(handle).get(key)
            except Exception:  # noqa: BLE001
                continue
            if isinstance(value, str) and value.strip() and value != "N/A":
                names.append(value.strip())
        arch = str(getattr(props, "gcnArchName", "") or "")
        if arch.startswith("gfx950"):
            try:
                top = int(amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX)["max_clk"])
            except Exception:  # noqa: BLE001
                top = None
            if top in _GFX950_SKU_BY_MAX_CLOCK:
                names.append(f"{_GFX950_SKU_BY_MAX_CLOCK[top]} (gfx950, peak engine clock {top} MHz)")
    except Exception:  # noqa: BLE001
        return names
    finally:
        try:
            amdsmi.amdsmi_shut_down()
        except Exception:  # noqa: BLE001
            pass
    return names


def product_names(torch_module: Any, device_id: int = 0) -> list[str]:
    """Other names of the device than torch's: amdsmi's (see _amdsmi_names) and the product lines
    ``rocm-smi --showproductname`` prints. Used to find the SKU when torch's name does not carry it."""
    names = _amdsmi_names(torch_module, device_id)
    text = _run_command(["rocm-smi", "--showproductname"])
    if text:
        names += [line.split(":", 2)[-1].strip() for line in text.splitlines()
                  if "card series" in line.lower() or "card sku" in line.lower() or "card model" in line.lower()]
    return [n for n in names if n]


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
