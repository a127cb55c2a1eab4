"""The MFMA ceiling measurement (mb_mfma_ceiling) on the GPU (-m gpu): every instruction runs and sustains a
rate between a tenth of its peak and the peak (the power limit holds the 16-bit and fp8 forms below it)."""
from __future__ import annotations

import pytest
import torch

from teamredbench_amd.native import capi

pytestmark = pytest.mark.gpu

PEAK = {"bfloat16": 2500.0, "float8_e4m3fn": 5000.0, "float32": 157.3}


@pytest.mark.parametrize("name", sorted(capi.MFMA_INSTRUCTIONS))
def test_mfma_ceiling_runs_within_the_peak(lib, name):
    code, flop, dtype = capi.MFMA_INSTRUCTIONS[name]
    blocks = torch.cuda.get_device_properties(0).multi_processor_count
    ops = torch.randint(0, 120, (capi.MFMA_CEILING_OPERAND_BYTES,), dtype=torch.uint8, device="cuda")  # finite values
    out = torch.full((256 * blocks,), float("nan"), device="cuda")
    print(f"[mfma-ceiling] {name}", flush=True)
    secs = lib.mfma_ceiling(code, ops.data_ptr(), out.data_ptr(), blocks, 2000, 2, 3,
                            torch.cuda.current_stream().cuda_stream)
    tflops = blocks * 4 * capi.MFMA_CEILING_CHAINS * flop * 2000 / secs / 1e12
    print(f"[mfma-ceiling] {name}: {tflops:.1f} TFLOP/s", flush=True)
    assert 0.1 * PEAK[dtype] < tflops <= 1.02 * PEAK[dtype]
    assert not torch.isnan(out).any()      # every thread wrote its sum


def test_mfma_ceiling_rejects_bad_arguments(lib):
    with pytest.raises(capi.NativeLibraryError) as err:
        lib.mfma_ceiling(99, 1, 1, 1, 1, 0, 1)
    assert err.value.status == capi.MB_ERR_INVALID_ARG
