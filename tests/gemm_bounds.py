"""Per-element rounding bound of a GEMM output against an fp64 matmul of the same operands.

Shared by the GPU tests that check C element by element. Every input value
(bf16, fp16, the fp8 codes, fp32, fp64) is exact in fp64, so an fp64 matmul of
the operands, times scale_a * scale_b, is the exact product up to fp64
rounding. A correct kernel differs from it by

  * the rounding of C to its output type: half an ulp of |C|;
  * the fp32 rounding of the fp8 scale product applied to the accumulator;
  * summation in any order in the accumulator's precision: (K + 2) * u *
    (|A| @ |B|), u the accumulation's unit roundoff (fp32, or fp64 for fp64
    operands, doubled there because numpy's fp64 reference errs as much);
  * for fp8, the f8f6f4 MFMA's block sum: the products of one instruction (a
    64- or 128-deep K block) are aligned to the largest of them and kept to
    about 14 bits below it, so the bound allows 2^-11 * (|A| @ |B|);
  * fp16 output subnormals: one fp16 subnormal step.

An element taken from a wrong row, column, tile or K range is off by about
|C| ~ sum |a * b| / sqrt(K), orders of magnitude past this bound.
"""
from __future__ import annotations

OUT_HALF_ULP = {"bfloat16": 2.0**-8, "float16": 2.0**-11, "float8_e4m3fn": 2.0**-8, "float8_e5m2": 2.0**-8,
                "float32": 0.0, "float64": 0.0}   # C is bf16 for fp8; fp32 / fp64 C is the accumulator itself
SUBNORMAL_SLACK = {"float16": 2.0**-24}
MFMA_BLOCK_SUM = {"float8_e4m3fn": 2.0**-11, "float8_e5m2": 2.0**-11}   # x (|A| @ |B|)
SCALE_ROUND = {"float8_e4m3fn": 2.0**-22, "float8_e5m2": 2.0**-22}     # fp32 scale_a * scale_b, then x acc
SUM_UNIT = {"float32": 2.0**-24, "float64": 2 * 2.0**-53}


def elementwise_bound(dtype: str, k: int, ref_abs, mag):
    """The bound above for each element, given |C_fp64| (`ref_abs`) and scale * (|A| @ |B|) (`mag`).

    Works on numpy arrays and torch tensors alike (only +, * and scalars)."""
    return (ref_abs * (OUT_HALF_ULP[dtype] + SCALE_ROUND.get(dtype, 0.0)) + SUBNORMAL_SLACK.get(dtype, 0.0)
            + ((k + 2) * SUM_UNIT.get(dtype, 2.0**-24) + MFMA_BLOCK_SUM.get(dtype, 0.0)) * mag)
