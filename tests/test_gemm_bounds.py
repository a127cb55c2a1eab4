"""The per-element GEMM bound (tests/gemm_bounds.py) on the CPU: a correctly
rounded product passes it, and the mistakes it is there to catch fail it.

The GPU tests hold the kernels' output to this bound at the benchmark
configurations' sizes. Here the "kernel" is the oracle's own fp32 product,
rounded to the output type as the kernels round it, with a mistake planted in
one tile: one 32-deep K stage left out (16-bit), one 64-deep stage left out
(fp8), or a column tile taken from its neighbour. The relative-Frobenius gate
of the configurations lets the first through (8 of the 64 checked rows cross
the faulty tile, as about 8 of 256 sampled rows cross one 256-row tile at
8192^3); the element bound does not.
"""
from __future__ import annotations

import torch

from gemm_bounds import elementwise_bound
from oracle import reference_path as rp

M, N, K = 64, 8192, 8192
TILE = 256
FAULTY_ROWS = 8


def _check(dtype: str, got: torch.Tensor, ops: dict) -> float:
    """Largest excess of |got - fp64 product| over the bound (<= 0 means every element passes)."""
    s = float(ops["scale_a"]) * float(ops["scale_b"])
    ref64 = s * (ops["a"].double() @ ops["b"].double())
    mag = s * (ops["a"].float().abs() @ ops["b"].float().abs()).double() * (1.0 + 2.0**-8)
    bound = elementwise_bound(dtype, K, ref64.abs(), mag)
    return float(((got.double() - ref64).abs() - bound).max())


def _kernel_like(dtype: str, ops: dict, skip: tuple[int, int] | None = None, shift_tile: bool = False):
    """The fp32 product of the dequantised operands, rounded to C's type; `skip` = (first, last) K rows left
    out of the first FAULTY_ROWS rows of the first column tile, `shift_tile` = those rows of the second column
    tile copied from the first."""
    a = ops["a"].float() * float(ops["scale_a"])
    b = ops["b"].float() * float(ops["scale_b"])
    c = a @ b
    if skip is not None:
        lo, hi = skip
        c[:FAULTY_ROWS, :TILE] -= a[:FAULTY_ROWS, lo:hi] @ b[lo:hi, :TILE]
    if shift_tile:
        c[:FAULTY_ROWS, TILE:2 * TILE] = c[:FAULTY_ROWS, :TILE]
    return c.to(rp.gemm_output_dtype(dtype))


def test_correct_product_passes_bound():
    for dtype in ("bfloat16", "float16", "float8_e4m3fn"):
        ops = rp.gemm_inputs(M, N, K, dtype, seed=3)
        assert _check(dtype, _kernel_like(dtype, ops), ops) <= 0.0, dtype


def test_skipped_k_stage_fails_bound_but_not_frobenius():
    for dtype, stage in (("bfloat16", 32), ("float16", 32), ("float8_e4m3fn", 64)):
        ops = rp.gemm_inputs(M, N, K, dtype, seed=4)
        got = _kernel_like(dtype, ops, skip=(4096, 4096 + stage))
        ref = rp.gemm_reference(ops["a"], ops["b"], ops["scale_a"], ops["scale_b"])
        # the configurations' gate alone would pass this tile
        assert rp.rel_frobenius(got.float(), ref) <= {"float8_e4m3fn": 5e-2}.get(dtype, 1e-2), dtype
        assert _check(dtype, got, ops) > 0.0, dtype


def test_tile_from_wrong_place_fails_bound():
    ops = rp.gemm_inputs(M, N, K, "bfloat16", seed=5)
    assert _check("bfloat16", _kernel_like("bfloat16", ops, shift_tile=True), ops) > 0.0
