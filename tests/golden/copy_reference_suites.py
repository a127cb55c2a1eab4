"""Copies the reference's own suite files for the single-GPU native path into
tests/golden/reference_suites/, byte for byte, as test fixtures (data, not code):

  configs/suites/native_smoke.yaml       hbm + mfu, backend native, the cdna_generic
                                         hardware profile and the rocm_generic runtime profile
  configs/suites/native_gemm_smoke.yaml  mfu, backend native, fp16/bf16/fp32/fp64 at 4096^3
  configs/suites/rocprof_hbm_smoke.yaml  hbm copy under the rocprof profile engine

tests/test_gpu_reference_suites.py runs them unchanged through run_suite. Run
this in a tree where the reference is checked out at /root/reference:

    python tests/golden/copy_reference_suites.py
"""
from __future__ import annotations

from pathlib import Path
import shutil

REFERENCE_SUITES = Path("/root/reference/configs/suites")
NAMES = ("native_smoke.yaml", "native_gemm_smoke.yaml", "rocprof_hbm_smoke.yaml")
OUT = Path(__file__).resolve().parent / "reference_suites"


def main() -> None:
    OUT.mkdir(exist_ok=True)
    for name in NAMES:
        shutil.copyfile(REFERENCE_SUITES / name, OUT / name)
        print(OUT / name)


if __name__ == "__main__":
    main()
