"""Build libmi355bench.so in-tree with hipcc for gfx950.

The reference compiles one standalone executable per kernel with
``hipcc -O3 -std=c++17 src -o bin`` into a content-hashed cache
(src/teamredbench/native/runtime.py:201-246). This package instead builds a
single shared library from ``teamredbench_amd/csrc/*.hip`` into
``teamredbench_amd/lib/`` so the built object ships with the source tree and
is loaded in-process through ctypes (teamredbench_amd/native/capi.py).

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
instruction selection disabled (``-packed-fp32-ops``).
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
from pathlib import Path
import shutil
import subprocess
import sys

PACKAGE_DIR = Path(__file__).resolve().parent.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "lib"
BUILD_DIR = PACKAGE_DIR.parent / "_build" / "mi355bench"
LIB_NAME = "libmi355bench.so"
OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


class BuildError(RuntimeError):
    pass


def find_hipcc() -> str:
    for candidate in (os.environ.get("TEAMREDBENCH_HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return str(candidate)
    raise BuildError("hipcc not found (set TEAMREDBENCH_HIPCC or install ROCm)")


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def source_digest() -> str:
    """sha256 over every csrc file and the public header, in name order."""
    digest = hashlib.sha256()
    header = PACKAGE_DIR.parent / "include" / "mi355bench.h"
    for path in sorted(CSRC_DIR.glob("*")) + [header]:
        if path.is_file():
            digest.update(path.name.encode())
            digest.update(b"\0")
            digest.update(path.read_bytes())
    return digest.hexdigest()


def _compile(hipcc: str, src: Path, obj: Path) -> tuple[Path, int, str]:
    cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name; that warning is expected.
    noise = "packed-fp32-ops"
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line and line.strip()
    )
    return src, proc.returncode, log


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libmi355bench.so. Always rebuilds."""
    hipcc = find_hipcc()
    digest = source_digest()   # of the sources as compiled: an edit made during the build leaves it stale
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise BuildError(f"no HIP sources under {CSRC_DIR}")
    objs = [BUILD_DIR / (src.stem + ".o") for src in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2) // 2))
    failures = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for src, rc, log in pool.map(lambda so: _compile(hipcc, *so), zip(srcs, objs)):
            if verbose and log:
                print(f"[{src.name}]\n{log}", file=sys.stderr)
            if rc != 0:
                failures.append(f"{src.name}:\n{log}")
    if failures:
        raise BuildError("hipcc failed:\n" + "\n".join(failures))
    out = library_path()
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise BuildError("link failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, out)
    (LIB_DIR / "BUILD_DIGEST").write_text(digest + "\n", encoding="utf-8")
    return out


EXAMPLES_DIR = PACKAGE_DIR / "native" / "examples"
EXAMPLE_CACHE_DIR = LIB_DIR / "exec_cache"


def example_params(source: Path) -> dict:
    """The `hbm` suite params that select an example executable and its in-tree build cache."""
    return {"native": {"source": str(source), "cache_dir": str(EXAMPLE_CACHE_DIR)}}


def build_examples() -> list[Path]:
    """Build the example external kernels (native/examples/*.hip) through the same content-keyed
    cache a suite selecting them uses, so a suite run finds them built (and rebuilds one only if
    its source or compiler changed). Returns the executables."""
    import teamredbench_amd.native.builtin  # noqa: F401  (the built-in names the benchmark defaults to)
    from teamredbench_amd.native.runtime import prepare_native_kernel_binary, resolve_native_kernel

    built = []
    for source in sorted(EXAMPLES_DIR.glob("*.hip")):
        kernel = resolve_native_kernel(benchmark="hbm", params=example_params(source), suite_path=None,
                                       repo_root=PACKAGE_DIR.parent, default_kernel="hbm_hip")
        built.append(prepare_native_kernel_binary(kernel))
    return built


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)
    for exe in build_examples():
        print(exe)
