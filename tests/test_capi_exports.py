"""The C-ABI library loads on a host without a GPU and exports exactly what
include/mi355bench.h declares (no compute calls here)."""
from __future__ import annotations

import re
import subprocess

import pytest

from teamredbench_amd.native import build, capi

HEADER = build.PACKAGE_DIR.parent / "include" / "mi355bench.h"


def _declared() -> set[str]:
    text = HEADER.read_text(encoding="utf-8")
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(mb_[a-z_0-9]+)\s*\(", text))


def test_header_declares_the_bound_signatures():
    assert _declared() == set(capi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    path = build.library_path()
    assert path.exists(), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = _declared() - exported
    assert not missing, f"not exported: {sorted(missing)}"
    # nothing else escapes under the mb_ prefix
    assert {s for s in exported if s.startswith("mb_")} == _declared()


def test_library_loads_and_reports_its_abi():
    lib = capi.load_library()
    assert lib.handle.mb_abi_version() == capi.ABI_VERSION
    assert lib.handle.mb_last_error() == b""


def test_stale_build_is_refused(tmp_path, monkeypatch):
    monkeypatch.setattr(capi._build, "source_digest", lambda: "0" * 64)
    capi._cache.clear()
    try:
        with pytest.raises(capi.NativeLibraryError, match="different sources"):
            capi.load_library()
    finally:
        capi._cache.clear()


def test_missing_library_is_an_error_not_a_fallback(tmp_path):
    with pytest.raises(capi.NativeLibraryError, match="not built"):
        capi.load_library(tmp_path / "libmissing.so")


def test_abi_constants_match_the_header():
    text = HEADER.read_text(encoding="utf-8")
    consts = dict(re.findall(r"#define (MB_[A-Z0-9_]+) (-?\d+)", text))
    assert int(consts["MB_ABI_VERSION"]) == capi.ABI_VERSION
    assert int(consts["MB_OP_TRIAD"]) == capi.OP_TRIAD and int(consts["MB_OP_SCALE"]) == capi.OP_SCALE
    for name, value in capi.DTYPES.items():
        assert int(consts["MB_DT_" + name.upper()]) == value
    assert int(consts["MB_ERR_SHAPE"]) == capi.MB_ERR_SHAPE
    assert int(consts["MB_ERR_WORKSPACE"]) == capi.MB_ERR_WORKSPACE
    for name, value in capi.TUNING_KNOBS.items():
        assert int(consts["MB_TUNE_" + name.upper()]) == value
    assert int(consts["MB_TUNE_COUNT"]) == len(capi.TUNING_KNOBS)
    shift = re.search(r"#define MB_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert shift and int(shift.group(1)) << int(shift.group(2)) == capi.NOALLOC_SCRATCH_BYTES
    assert int(consts["MB_CLOCK_BLOCKS"]) == capi.CLOCK_BLOCKS
    assert int(consts["MB_CLOCK_REALTIME_HZ"]) == capi.CLOCK_REALTIME_HZ
    assert int(consts["MB_MFMA_CEILING_OPERAND_BYTES"]) == capi.MFMA_CEILING_OPERAND_BYTES
    codes = {name: code for name, (code, _, _) in capi.MFMA_INSTRUCTIONS.items()}
    assert codes == {"v_mfma_f32_32x32x16_bf16": int(consts["MB_MFMA_BF16_32X32X16"]),
                     "v_mfma_f32_16x16x32_bf16": int(consts["MB_MFMA_BF16_16X16X32"]),
                     "v_mfma_scale_f32_32x32x64_f8f6f4": int(consts["MB_MFMA_FP8_32X32X64"]),
                     "v_mfma_scale_f32_16x16x128_f8f6f4": int(consts["MB_MFMA_FP8_16X16X128"]),
                     "v_mfma_f32_32x32x2_f32": int(consts["MB_MFMA_F32_32X32X2"])}


def test_tuning_knobs_validate_and_restore_without_a_gpu():
    # mb_set_tuning / mb_get_tuning touch no device: they run here.
    lib = capi.load_library()
    assert all(lib.get_tuning(name) is None for name in capi.TUNING_KNOBS)
    with lib.tuned(gemm_splits=4, stream_unroll=8):
        assert lib.get_tuning("gemm_splits") == 4 and lib.get_tuning("stream_unroll") == 8
    assert lib.get_tuning("gemm_splits") is None and lib.get_tuning("stream_unroll") is None
    for name, bad in (("stream_unroll", 3), ("stream_threads", 96), ("stream_threads", 2048),
                      ("gemm_tiled_config", 5), ("gemm_splits", 0), ("gemm_splits", 513), ("gemm_fp8_mfma", 8),
                      ("gemm_force_generic", 2)):
        with pytest.raises(capi.NativeLibraryError, match="cannot take") as err:
            lib.set_tuning(name, bad)
        assert err.value.status == capi.MB_ERR_INVALID_ARG
        assert lib.get_tuning(name) is None          # a rejected value leaves the knob as it was
    assert lib.handle.mb_set_tuning(capi.TUNING_KNOBS["gemm_splits"] + 100, 1) == capi.MB_ERR_INVALID_ARG
    assert lib.handle.mb_get_tuning(-1) == -1
