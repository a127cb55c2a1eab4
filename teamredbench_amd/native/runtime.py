"""Resolution of ``params.native`` and the external-executable contract.

``resolve_native_kernel`` reads ``params.native.{kernel, source, binary,
compiler, compile_args, run_args, env, cache_dir}`` exactly as the reference
does (src/teamredbench/native/runtime.py:65-119); relative paths resolve
against the suite file.

Built-in kernels (abi "capi") need nothing more: the benchmark calls
libmi355bench.so through :mod:`teamredbench_amd.native.capi`. A
user-supplied ``source`` or ``binary`` -- or a plugin kernel registered with
abi "executable" -- keeps the reference's process contract
(docs/extending.md:155-175): hipcc builds the source into a cache keyed by a
sha256 over the source, its local ``#include "..."`` closure, the compiler
and the flags; the executable receives argv and its last non-empty stdout
line must be a JSON object ``{status, raw_metrics, metadata, error}``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
import hashlib
import json
import os
from pathlib import Path
import re
import shutil
import subprocess
from typing import Any

from teamredbench_amd.native.registry import ABI_CAPI, ABI_EXECUTABLE, get_native_kernel


class NativeKernelError(RuntimeError):
    pass


@dataclass(frozen=True)
class ResolvedNativeKernel:
    benchmark: str
    name: str
    description: str
    source_path: Path | None = None
    binary_path: Path | None = None
    compiler: str | None = None
    compile_args: tuple[str, ...] = ()
    run_args: tuple[str, ...] = ()
    env: dict[str, str] = field(default_factory=dict)
    cache_dir: Path | None = None
    abi: str = ABI_EXECUTABLE

    @property
    def in_process(self) -> bool:
        return self.abi == ABI_CAPI


@dataclass(frozen=True)
class NativeKernelResult:
    status: str
    raw_metrics: dict[str, Any]
    metadata: dict[str, Any]
    error: str | None = None


def _as_str_list(value: Any, label: str) -> list[str]:
    if value is None:
        return []
    if not isinstance(value, list):
        raise ValueError(f"{label} must be a list of strings.")
    return [str(v) for v in value]


def _as_str_map(value: Any, label: str) -> dict[str, str]:
    if value is None:
        return {}
    if not isinstance(value, dict):
        raise ValueError(f"{label} must be a mapping.")
    return {str(k): str(v) for k, v in value.items()}


def _user_path(base: Path, value: str) -> Path:
    path = Path(value)
    return path if path.is_absolute() else (base / path).resolve()


def resolve_native_kernel(
    *,
    benchmark: str,
    params: dict[str, Any],
    suite_path: Path | None,
    repo_root: Path | None,
    default_kernel: str | None = None,
) -> ResolvedNativeKernel:
    native = params.get("native") or {}
    if not isinstance(native, dict):
        raise ValueError("benchmark params.native must be a mapping.")
    base = suite_path.parent if suite_path else (repo_root or Path.cwd())

    kernel_name = str(native.get("kernel", default_kernel or "")).strip() or None
    definition = get_native_kernel(kernel_name) if kernel_name else None
    if definition is not None and definition.benchmark != benchmark:
        raise ValueError(f"Native kernel {definition.name} is registered for {definition.benchmark}, not {benchmark}.")

    source = definition.source_path if definition is not None else None
    binary = _user_path(base, str(native["binary"])) if native.get("binary") else None
    user_source = _user_path(base, str(native["source"])) if native.get("source") else None
    if user_source is not None:
        source = user_source
    # A user-supplied source or binary always goes through the executable contract.
    abi = definition.abi if definition is not None and binary is None and user_source is None else ABI_EXECUTABLE

    compile_args = list(definition.compile_args if definition is not None else ())
    compile_args += _as_str_list(native.get("compile_args"), "native.compile_args")
    if abi == ABI_EXECUTABLE and source is None and binary is None:
        if kernel_name is None:
            raise ValueError(
                "No native kernel configured. Set params.native.kernel, params.native.source, or params.native.binary."
            )
        raise ValueError(f"Native kernel {kernel_name} does not define a source or binary path.")

    if definition is not None and abi == ABI_CAPI:
        name = definition.name
    else:
        name = kernel_name or (source.stem if source is not None else binary.stem)
    return ResolvedNativeKernel(
        benchmark=benchmark,
        name=name,
        description=definition.description if definition is not None else "external native kernel",
        source_path=source,
        binary_path=binary,
        compiler=str(native["compiler"]) if native.get("compiler") else None,
        compile_args=tuple(compile_args),
        run_args=tuple(_as_str_list(native.get("run_args"), "native.run_args")),
        env=_as_str_map(native.get("env"), "native.env"),
        cache_dir=_user_path(base, str(native["cache_dir"])) if native.get("cache_dir") else None,
        abi=abi,
    )


# ------------------------------------------------------------------ cache
def native_cache_dir(explicit: Path | None = None) -> Path:
    if explicit is not None:
        return explicit
    xdg = os.environ.get("XDG_CACHE_HOME")
    root = Path(xdg).expanduser().resolve() if xdg else Path.home().resolve() / ".cache"
    return root / "teamredbench" / "native"


def clear_native_cache(explicit: Path | None = None) -> tuple[Path, int]:
    cache = native_cache_dir(explicit)
    if not cache.exists():
        return cache, 0
    removed = 0
    for entry in cache.iterdir():
        if entry.is_dir():
            shutil.rmtree(entry)
        else:
            entry.unlink()
        removed += 1
    return cache, removed


def _find_hip_compiler(preferred: str | None = None) -> str:
    for candidate in (
        preferred,
        os.environ.get("TEAMREDBENCH_HIPCC"),
        "hipcc",
        "/opt/rocm/bin/hipcc",
        "amdclang++",
        "/opt/rocm/bin/amdclang++",
    ):
        if not candidate:
            continue
        if Path(candidate).is_absolute():
            if Path(candidate).exists():
                return candidate
            continue
        found = shutil.which(candidate)
        if found:
            return found
    raise NativeKernelError("No HIP compiler found. Set TEAMREDBENCH_HIPCC, params.native.compiler, or params.native.binary.")


_INCLUDE = re.compile(r'^\s*#\s*include\s*"([^"]+)"', re.MULTILINE)


def _hash_sources(digest: "hashlib._Hash", path: Path, seen: set[Path]) -> None:
    """Feed `path` and, depth-first, every local include that exists into `digest`."""
    path = path.resolve()
    if path in seen:
        return
    seen.add(path)
    data = path.read_bytes()
    digest.update(str(path).encode() + b"\0" + data)
    for name in _INCLUDE.findall(data.decode("utf-8", errors="ignore")):
        candidate = (path.parent / name).resolve()
        if candidate.exists():
            _hash_sources(digest, candidate, seen)


def prepare_native_kernel_binary(kernel: ResolvedNativeKernel) -> Path:
    """Executable for an abi="executable" kernel: the given binary, or a cached hipcc build."""
    if kernel.binary_path is not None:
        if not kernel.binary_path.exists():
            raise NativeKernelError(f"Native kernel binary does not exist: {kernel.binary_path}")
        return kernel.binary_path
    if kernel.source_path is None:
        raise NativeKernelError(f"Native kernel {kernel.name} is missing both source_path and binary_path.")
    if not kernel.source_path.exists():
        raise NativeKernelError(f"Native kernel source does not exist: {kernel.source_path}")

    compiler = _find_hip_compiler(kernel.compiler)
    cache = native_cache_dir(kernel.cache_dir)
    cache.mkdir(parents=True, exist_ok=True)
    digest = hashlib.sha256()
    _hash_sources(digest, kernel.source_path, set())
    for part in (kernel.benchmark, kernel.name, compiler, *kernel.compile_args):
        digest.update(part.encode())
    binary = cache / f"{kernel.name}-{digest.hexdigest()[:16]}"
    if binary.exists():
        return binary

    command = [compiler, "-O3", "-std=c++17"]
    if Path(compiler).name.endswith("clang++"):
        command += ["-x", "hip"]
    command += [str(kernel.source_path), "-o", str(binary), *kernel.compile_args]
    proc = subprocess.run(command, check=False, capture_output=True, text=True)
    if proc.returncode != 0:
        detail = proc.stderr.strip() or proc.stdout.strip() or "unknown compiler failure"
        raise NativeKernelError(f"Failed to compile native kernel {kernel.name}: {detail}")
    binary.chmod(0o755)
    return binary


def parse_native_result(stdout: str) -> NativeKernelResult:
    lines = [line.strip() for line in stdout.splitlines() if line.strip()]
    if not lines:
        raise NativeKernelError("Native kernel produced no JSON output.")
    try:
        payload = json.loads(lines[-1])
    except json.JSONDecodeError as exc:
        raise NativeKernelError(f"Native kernel output was not valid JSON: {exc}") from exc
    if not isinstance(payload, dict):
        raise NativeKernelError("Native kernel output JSON must be an object.")
    raw = payload.get("raw_metrics", {})
    meta = payload.get("metadata", {})
    if not isinstance(raw, dict):
        raise NativeKernelError("Native kernel raw_metrics must be a JSON object.")
    if not isinstance(meta, dict):
        raise NativeKernelError("Native kernel metadata must be a JSON object.")
    error = payload.get("error")
    return NativeKernelResult(
        status=str(payload.get("status", "ok")),
        raw_metrics=dict(raw),
        metadata=dict(meta),
        error=None if error is None else str(error),
    )


def run_native_kernel(kernel: ResolvedNativeKernel, args: list[str], timeout_s: float | None = None) -> NativeKernelResult:
    binary = prepare_native_kernel_binary(kernel)
    env = {**os.environ, **kernel.env}
    try:
        proc = subprocess.run(
            [str(binary), *args, *kernel.run_args],
            check=False,
            capture_output=True,
            text=True,
            env=env,
            timeout=timeout_s,
        )
    except subprocess.TimeoutExpired as exc:
        raise NativeKernelError(f"Native kernel {kernel.name} timed out after {timeout_s} s") from exc
    if proc.returncode != 0:
        detail = proc.stderr.strip() or proc.stdout.strip() or "native kernel process failed"
        raise NativeKernelError(f"Native kernel {kernel.name} failed (exit status {proc.returncode}): {detail}")
    return parse_native_result(proc.stdout)
