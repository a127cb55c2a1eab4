"""``params.native``: which native kernel a benchmark runs, and how.

Selection (the keys of src/teamredbench/native/runtime.py:65-119, so suites
written for the reference resolve the same way):
  params.native.kernel        a registered name (default: the benchmark's
                              built-in, e.g. ``hbm_hip`` -> the gfx950 stream
                              kernels of libmi355bench.so)
  params.native.source        a HIP source to build (overrides the kernel's)
  params.native.binary        a ready executable (no build)
  params.native.compiler / compile_args / run_args / env / cache_dir
Relative paths are taken from the suite file's directory.

Built-in kernels (abi "capi") run in-process through the C ABI
(:mod:`teamredbench_amd.native.capi`). A user ``source`` or ``binary``, or
a plugin registered with abi "executable", keeps the reference's process
contract: argv in, and the last non-empty stdout line is a JSON object
``{status, raw_metrics, metadata, error}`` (docs/extending.md:155-175).

Sources are built by :class:`KernelCache`: one executable per content key,
a sha256 over the source, every local ``#include "..."`` it reaches (so
editing a header rebuilds), the compiler and the flags. Builds target
gfx950 (``--offload-arch=gfx950``) unless the flags name an offload arch,
and land under a temporary name first, so an interrupted build never leaves
a truncated executable under its final name.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
import hashlib
import json
import os
from pathlib import Path
import re
import shutil
import subprocess
from typing import Any

from teamredbench_amd.config import ConfigError, _Section
from teamredbench_amd.native.registry import ABI_CAPI, ABI_EXECUTABLE, get_native_kernel

DEFAULT_OFFLOAD_ARCH = "gfx950"


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

    @classmethod
    def from_stdout(cls, stdout: str) -> "NativeKernelResult":
        """The contract line: the last non-empty line of the executable's stdout."""
        line = next((text.strip() for text in reversed(stdout.splitlines()) if text.strip()), None)
        if line is None:
            raise NativeKernelError("Native kernel produced no JSON output.")
        try:
            payload = json.loads(line)
        except json.JSONDecodeError as exc:
            raise NativeKernelError(f"Native kernel output was not valid JSON: {exc}") from exc
        if not isinstance(payload, dict):
            raise NativeKernelError("Native kernel output JSON must be an object.")
        parts = {}
        for key in ("raw_metrics", "metadata"):
            value = payload.get(key, {})
            if not isinstance(value, dict):
                raise NativeKernelError(f"Native kernel {key} must be a JSON object.")
            parts[key] = dict(value)
        error = payload.get("error")
        return cls(status=str(payload.get("status", "ok")), error=None if error is None else str(error), **parts)


def parse_native_result(stdout: str) -> NativeKernelResult:
    return NativeKernelResult.from_stdout(stdout)


def _string_list(block: _Section, key: str) -> list[str]:
    values = block.get(key, [])
    if not isinstance(values, list):
        raise ConfigError(f"{block.origin.name}: {block.where}.{key} must be a list of strings.")
    return [str(v) for v in values]


def resolve_native_kernel(*, benchmark: str, params: dict[str, Any], suite_path: Path | None,
                          repo_root: Path | None, default_kernel: str | None = None) -> ResolvedNativeKernel:
    base = suite_path.parent if suite_path else (repo_root or Path.cwd())
    origin = suite_path or base / "params"
    if not isinstance(params.get("native") or {}, dict):
        raise ConfigError(f"{origin.name}: benchmark params.native must be a mapping.")
    block = _Section(params.get("native") or {}, origin, "params.native")   # paths resolve against `base`

    name = str(block.get("kernel", default_kernel or "")).strip() or None
    definition = get_native_kernel(name) if name else None
    if definition is not None and definition.benchmark != benchmark:
        raise ValueError(f"Native kernel {definition.name} is registered for {definition.benchmark}, not {benchmark}.")
    user_source = block.path("source") if block.get("source", None) else None
    binary = block.path("binary") if block.get("binary", None) else None
    source = user_source or (definition.source_path if definition is not None else None)
    # a user-supplied source or binary always goes through the executable contract
    abi = definition.abi if definition is not None and user_source is None and binary is None else ABI_EXECUTABLE
    if abi == ABI_EXECUTABLE and source is None and binary is None:
        raise ValueError("No native kernel configured. Set params.native.kernel, params.native.source, or "
                         "params.native.binary." if name is None else
                         f"Native kernel {name} does not define a source or binary path.")
    if definition is not None and abi == ABI_CAPI:
        resolved_name = definition.name
    else:
        resolved_name = name or (source or binary).stem
    env = block.get("env", {})
    if not isinstance(env, dict):
        raise ConfigError(f"{origin.name}: params.native.env must be a mapping.")
    return ResolvedNativeKernel(
        benchmark=benchmark,
        name=resolved_name,
        description=definition.description if definition is not None else "external native kernel",
        source_path=source,
        binary_path=binary,
        compiler=block.text("compiler") if block.get("compiler", None) else None,
        compile_args=tuple((definition.compile_args if definition is not None else ()) +
                           tuple(_string_list(block, "compile_args"))),
        run_args=tuple(_string_list(block, "run_args")),
        env={str(k): str(v) for k, v in env.items()},
        cache_dir=block.path("cache_dir") if block.get("cache_dir", None) else None,
        abi=abi,
    )


# ------------------------------------------------------------------ builds
def native_cache_dir(explicit: Path | None = None) -> Path:
    """Where external kernels are built: ``$XDG_CACHE_HOME/teamredbench/native`` (or ~/.cache/...)."""
    if explicit is not None:
        return Path(explicit)
    root = os.environ.get("XDG_CACHE_HOME")
    return (Path(root).expanduser() if root else Path.home() / ".cache").resolve() / "teamredbench" / "native"


def _find_hip_compiler(preferred: str | None = None) -> str:
    for candidate in (preferred, os.environ.get("TEAMREDBENCH_HIPCC"), "hipcc", "/opt/rocm/bin/hipcc",
                      "amdclang++", "/opt/rocm/bin/amdclang++"):
        if not candidate:
            continue
        path = Path(candidate)
        found = str(path) if path.is_absolute() and path.exists() else (None if path.is_absolute()
                                                                       else shutil.which(candidate))
        if found:
            return found
    raise NativeKernelError("No HIP compiler found. Set TEAMREDBENCH_HIPCC, params.native.compiler, or "
                            "params.native.binary.")


_LOCAL_INCLUDE = re.compile(r'^\s*#\s*include\s*"([^"]+)"', re.MULTILINE)


def source_closure(source: Path) -> list[Path]:
    """The source and every local include it reaches that exists, breadth first, each once."""
    order: list[Path] = []
    pending = deque([source.resolve()])
    while pending:
        path = pending.popleft()
        if path in order:
            continue
        order.append(path)
        text = path.read_text(encoding="utf-8", errors="ignore")
        pending.extend(p for p in ((path.parent / inc).resolve() for inc in _LOCAL_INCLUDE.findall(text))
                       if p.exists())
    return order


class KernelCache:
    """Content-keyed hipcc builds of external kernel sources."""

    def __init__(self, directory: Path | None = None):
        self.directory = native_cache_dir(directory)

    def build_command(self, compiler: str, source: Path, output: Path, flags: tuple[str, ...]) -> list[str]:
        command = [compiler, "-O3", "-std=c++17"]
        if Path(compiler).name.endswith("clang++"):
            command += ["-x", "hip"]
        if not any(flag.startswith("--offload-arch") for flag in flags):
            command.append(f"--offload-arch={DEFAULT_OFFLOAD_ARCH}")
        return command + [str(source), "-o", str(output), *flags]

    def key(self, kernel: ResolvedNativeKernel, compiler: str) -> str:
        # paths relative to the source's directory: a moved tree keeps its builds
        digest = hashlib.sha256()
        root = kernel.source_path.resolve().parent
        for path in source_closure(kernel.source_path):
            digest.update(f"{os.path.relpath(path, root)}\0".encode() + path.read_bytes() + b"\0")
        for part in (kernel.benchmark, kernel.name, compiler, *kernel.compile_args):
            digest.update(part.encode() + b"\0")
        return digest.hexdigest()[:16]

    def executable(self, kernel: ResolvedNativeKernel) -> Path:
        compiler = _find_hip_compiler(kernel.compiler)
        self.directory.mkdir(parents=True, exist_ok=True)
        target = self.directory / f"{kernel.name}-{self.key(kernel, compiler)}"
        if target.exists():
            return target
        staging = target.with_name(f".{target.name}.{os.getpid()}.tmp")
        proc = subprocess.run(self.build_command(compiler, kernel.source_path, staging, kernel.compile_args),
                              check=False, capture_output=True, text=True)
        if proc.returncode != 0 or not staging.exists():
            detail = proc.stderr.strip() or proc.stdout.strip() or "unknown compiler failure"
            raise NativeKernelError(f"Failed to compile native kernel {kernel.name}: {detail}")
        staging.chmod(0o755)
        staging.replace(target)
        return target

    def clear(self) -> int:
        if not self.directory.exists():
            return 0
        entries = list(self.directory.iterdir())
        for entry in entries:
            shutil.rmtree(entry) if entry.is_dir() else entry.unlink()
        return len(entries)


def clear_native_cache(explicit: Path | None = None) -> tuple[Path, int]:
    cache = KernelCache(explicit)
    return cache.directory, cache.clear()


def prepare_native_kernel_binary(kernel: ResolvedNativeKernel) -> Path:
    """The executable of an abi="executable" kernel: its binary, or a cached build of its source."""
    if kernel.binary_path is not None:
        if not kernel.binary_path.exists():
            raise NativeKernelError(f"Native kernel binary does not exist: {kernel.binary_path}")
        return kernel.binary_path
    if kernel.source_path is None:
        raise NativeKernelError(f"Native kernel {kernel.name} is missing both source_path and binary_path.")
    if not kernel.source_path.exists():
        raise NativeKernelError(f"Native kernel source does not exist: {kernel.source_path}")
    return KernelCache(kernel.cache_dir).executable(kernel)


def run_native_kernel(kernel: ResolvedNativeKernel, args: list[str],
                      timeout_s: float | None = None) -> NativeKernelResult:
    executable = prepare_native_kernel_binary(kernel)
    try:
        proc = subprocess.run([str(executable), *args, *kernel.run_args], check=False, capture_output=True,
                              text=True, env={**os.environ, **kernel.env}, timeout=timeout_s)
    except subprocess.TimeoutExpired as exc:
        raise NativeKernelError(f"Native kernel {kernel.name} timed out after {timeout_s} s") from exc
    if proc.returncode != 0:
        detail = proc.stderr.strip() or proc.stdout.strip() or "native kernel process failed"
        raise NativeKernelError(f"Native kernel {kernel.name} failed (exit status {proc.returncode}): {detail}")
    return NativeKernelResult.from_stdout(proc.stdout)
