"""Run metadata for the sidecar: configs, versions, device, host cores and a
command that reproduces the run (the subset of src/teamredbench/provenance.py
that results need to be interpretable; keys keep the reference's names)."""
from __future__ import annotations

from dataclasses import asdict
from datetime import datetime
import os
import platform
import socket
import sys
from pathlib import Path
from typing import Any

from teamredbench_amd.benchmarks.base import BenchmarkContext
from teamredbench_amd.config import SuiteConfig
from teamredbench_amd.device import host_cores

_ENV_PREFIXES = ("HIP_", "HSA_", "ROCR_", "ROCM_", "RCCL_", "NCCL_", "GPU_", "AMD_", "MB_", "TEAMREDBENCH_", "OMP_")


def _filtered_env() -> dict[str, str]:
    return {k: v for k, v in sorted(os.environ.items()) if k.startswith(_ENV_PREFIXES)}


def _native_library() -> dict[str, Any]:
    from teamredbench_amd.native import build

    path = build.library_path()
    stamp = path.parent / "BUILD_DIGEST"
    return {
        "path": str(path),
        "present": path.exists(),
        "build_digest": stamp.read_text(encoding="utf-8").strip() if stamp.exists() else None,
        "offload_arch": build.OFFLOAD_ARCH,
    }


def build_run_metadata(
    *,
    suite: SuiteConfig,
    context: BenchmarkContext,
    requested_device_id: int,
    output_dir: Path,
    output_formats: list[str],
    profile_note: str | None,
    started_at: datetime,
    finished_at: datetime,
) -> dict[str, Any]:
    torch = context.torch_module
    torch_info: dict[str, Any] = {}
    if torch is not None:
        torch_info = {
            "version": getattr(torch, "__version__", "unknown"),
            "hip_version": getattr(getattr(torch, "version", None), "hip", None),
        }
    from teamredbench_amd.profiling.runtime import run_token

    hw = context.hardware_profile
    return {
        "run_token": run_token(),
        "started_at_utc": started_at.isoformat().replace("+00:00", "Z"),
        "finished_at_utc": finished_at.isoformat().replace("+00:00", "Z"),
        "duration_s": (finished_at - started_at).total_seconds(),
        "system": {
            "hostname": socket.gethostname(),
            "platform": platform.platform(),
            "cpu_cores_available": host_cores(),
        },
        "python": {"version": platform.python_version(), "executable": sys.executable},
        "torch": torch_info,
        "rocm": {"profile_version": context.runtime_profile.rocm_version},
        "device": asdict(context.device_info) if context.device_info else None,
        "device_id": context.device_id,
        "native_library": _native_library(),
        "env": _filtered_env(),
        "configs": {
            "suite": {"path": str(suite.path) if suite.path else None, "raw": suite.raw},
            "hardware_profile": {"path": str(hw.path) if hw.path else None, "raw": hw.raw},
            "runtime_profile": {
                "path": str(context.runtime_profile.path) if context.runtime_profile.path else None,
                "raw": context.runtime_profile.raw,
            },
            "profile_note": profile_note,
            "output_formats": output_formats,
        },
        "reproduce": {
            "run_command": [sys.executable, "-m", "teamredbench_amd", "run", str(suite.path),
                            "--device-id", str(requested_device_id), "--output-dir", str(output_dir)],
        },
    }
