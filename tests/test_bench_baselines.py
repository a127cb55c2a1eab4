"""bench.py's CPU baselines on the CPU: the GEMM baseline's record (a small slab, so it runs in
milliseconds) carries the fields and units the JSON line reports, and its FLOP count follows the slab."""
from __future__ import annotations

import bench


def test_cpu_gemm_baseline_record():
    for dtype, operands in (("bfloat16", "bf16"), ("float8_e4m3fn", "fp32 (dequantised fp8)")):
        rec = bench.cpu_gemm_baseline(dtype, 256, rows=32, min_seconds=0.0)
        assert set(rec) == {"value", "unit", "cores", "kind", "sample"}
        assert rec["unit"] == "TFLOP/s" and rec["kind"] == "port" and rec["value"] > 0
        assert rec["cores"] >= 1
        assert f"torch.mm on {operands} CPU tensors" in rec["sample"]
        assert "a 32 x 256 slab of A against the 256 x 256 B (0.0 GFLOP per call), 1 untimed + 1 timed" in rec["sample"]
