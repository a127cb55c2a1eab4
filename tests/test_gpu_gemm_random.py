"""GEMM on seeded random shapes, each taking whatever plan the library picks (-m gpu).

The fixed-shape tests pin each kernel and plan branch; these shapes are drawn
at random (M 1..2000, N and K multiples of 128 / 64, of 8, or arbitrary) so that
the plan's choices -- small-M stream kernel, tile configuration, K split count
up to 32, bounds-checked generic kernel -- are exercised where no test chose
them. Every element of C is checked against an fp64 matmul of the same
operands (the fp8 codes' exact values, times scale_a * scale_b) within its
rounding bound: the output rounding of C's type, the fp32 rounding of the fp8
scale product, and summation in any order, (K + 2) * u * (|A| @ |B|) with u the
unit roundoff of the accumulation (fp32, or fp64 for fp64 operands).

fp8 adds one more term. The f8f6f4 MFMA sums the products of one instruction
(a 128- or 64-deep K block) aligned to the largest of them, keeping about 14
bits below it: with 448 * 448 - 448 * 448 in the same block, an added product
of 1 or 4 comes back as 0 and one of 16 as 16, while the same small product in
another K block comes back exact (the instructions accumulate in fp32). On
random operands the error reached 2^-14.5 of sum |a * b| (K = 16, one block)
and 2^-18.5 or less for K >= 1000, the same on the generic kernel and both
tiled fp8 kernels; the bound allows 2^-11 * (|A| @ |B|). An element taken
from a wrong row, column or K range is off by about |C| ~ sum |a * b| / sqrt(K).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gemm_bounds import elementwise_bound
from oracle import reference_path as rp
from teamredbench_amd.native import capi

pytestmark = pytest.mark.gpu

IMPLEMENTATIONS = {"gfx950_gemv_stream", "gfx950_mfma16_lds_dma", "gfx950_mfma32_lds_dma", "gfx950_mfma_generic",
                   "gfx950_mfma_f32_32x32x2", "gfx950_mfma_f32_32x32x2_lds_dma", "gfx950_mfma_f64_16x16x4",
                   "gfx950_mfma_f64_16x16x4_lds_dma"}
DTYPES = ["bfloat16", "float16", "float8_e4m3fn", "float8_e5m2", "float32", "float64"]
def _dim(rng: np.random.Generator, aligned: int, hi: int) -> int:
    kind = rng.random()
    if kind < 0.85:
        return aligned * int(rng.integers(1, hi // aligned + 1))
    if kind < 0.93:
        return 8 * int(rng.integers(1, hi // 8 + 1))
    return int(rng.integers(1, hi // 2 + 1))


def random_shape(dtype: str, case: int) -> tuple[int, int, int]:
    rng = np.random.default_rng(1000 * case + len(dtype))
    m = int(np.exp(rng.uniform(0.0, np.log(2000.0))))
    n = _dim(rng, 128, 4096)
    k = _dim(rng, 64, 4096)
    while m * n * k > 3_000_000_000:
        k = max(1, k // 2)
    return max(m, 1), n, k


def pytest_generate_tests(metafunc):
    # 20 seeded cases per input type; `--gemm-random-cases N` runs N (a wider sweep of the same draws)
    if "case" in metafunc.fixturenames:
        metafunc.parametrize("case", range(metafunc.config.getoption("--gemm-random-cases")))


@pytest.mark.parametrize("dtype", DTYPES)
def test_planned_gemm_on_random_shapes(lib, dtype, case):
    m, n, k = random_shape(dtype, case)
    dt = capi.DTYPES[dtype]
    info = lib.gemm_info(dt, m, n, k)
    print(f"[gemm-random] {dtype} {m}x{n}x{k} case {case}: {info['implementation']} "
          f"{info['tile_m']}x{info['tile_n']} split {info['split_k']}", flush=True)
    assert info["implementation"] in IMPLEMENTATIONS, info
    ops = rp.gemm_inputs(m, n, k, dtype, seed=case)
    da, db = ops["a"].cuda(), ops["b"].cuda()
    dc = torch.full((m, n), float("nan"), dtype=rp.gemm_output_dtype(dtype), device="cuda")
    ws_bytes = lib.gemm_workspace_size(dt, m, n, k)
    ws = torch.full((max(ws_bytes, 1),), 0x7F, dtype=torch.uint8, device="cuda")   # stale contents
    lib.gemm(dt, da.data_ptr(), db.data_ptr(), dc.data_ptr(), m, n, k, ops["scale_a"], ops["scale_b"],
             ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = dc.cpu().double().numpy()
    a64, b64 = ops["a"].double().numpy(), ops["b"].double().numpy()   # exact: every input value is an fp64
    scale = float(ops["scale_a"]) * float(ops["scale_b"])
    ref = scale * (a64 @ b64)
    mag = scale * (np.abs(a64) @ np.abs(b64))
    bound = elementwise_bound(dtype, k, np.abs(ref), mag)
    assert not np.isnan(got).any(), "C has unwritten (NaN-filled) elements"
    excess = np.abs(got - ref) - bound
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess.max() <= 0.0, (f"{dtype} {m}x{n}x{k}: C{tuple(int(v) for v in worst)} = {got[worst]!r}, "
                                 f"fp64 {ref[worst]!r}, bound {bound[worst]:.3e}")
