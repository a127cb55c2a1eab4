"""ORACLE -- CPU restatement of the reference torch path (test infrastructure).

Follows, on CPU tensors:
  * src/teamredbench/benchmarks/hbm.py:18-22  MODE_BYTE_FACTORS
  * src/teamredbench/benchmarks/hbm.py:29-39  _run_mode (copy_ / mul / add(alpha))
  * src/teamredbench/benchmarks/hbm.py:85,192 numel = size_mib * 2**20 // bytes
  * src/teamredbench/benchmarks/mfu.py:229-238 torch.mm(a, b, out=out)
The reference draws unseeded ``randn`` inputs (utils.py:32-48); the
benchmark configurations measured here fix seeded distributions instead, generated here with a CPU ``torch.Generator`` so the GPU and the CPU
see identical bits.
"""
from __future__ import annotations

import math

import numpy as np
import torch

MODE_BYTE_FACTORS = {"copy": 2, "scale": 2, "triad": 3}

TORCH_DTYPES = {
    "float32": torch.float32,
    "bfloat16": torch.bfloat16,
    "float16": torch.float16,
    "float64": torch.float64,
    "int8": torch.int8,
    "float8_e4m3fn": torch.float8_e4m3fn,
    "float8_e5m2": torch.float8_e5m2,
}

FP8_E4M3_MAX = 448.0
FP8_E5M2_MAX = 57344.0
FP8_MAX = {"float8_e4m3fn": FP8_E4M3_MAX, "float8_e5m2": FP8_E5M2_MAX}


# ---------------------------------------------------------------- stream path
def run_mode(mode: str, src: torch.Tensor, dst: torch.Tensor, aux: torch.Tensor | None, scale: float) -> None:
    """hbm.py:29-39 on whatever device the tensors live on."""
    if mode == "copy":
        dst.copy_(src)
        return
    if mode == "scale":
        torch.mul(src, scale, out=dst)
        return
    if mode == "triad":
        torch.add(src, aux, alpha=scale, out=dst)
        return
    raise KeyError(f"Unknown HBM mode: {mode}")


def stream_reference(mode: str, b: torch.Tensor, c: torch.Tensor | None, scale: float) -> torch.Tensor:
    """Expected stream output, computed by the reference op on CPU."""
    dst = torch.empty_like(b)
    run_mode(mode, b, dst, c, scale)
    return dst


def numel_for(size_mib: int, bytes_per_element: int) -> int:
    """hbm.py:85 -- elements per array for a size in MiB."""
    return max(size_mib * 1024 * 1024 // bytes_per_element, 1)


def stream_inputs(n: int, dtype: str, seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """b, c ~ uniform[-1, 1] in fp32 from one CPU generator seeded `seed`, then cast.

    For float32 with n = 2**24 and seed 0 this is exactly the CPU triad
    configuration's input (b first, then c from the same generator).
    """
    g = torch.Generator().manual_seed(seed)
    b = torch.empty(n, dtype=torch.float32).uniform_(-1.0, 1.0, generator=g)
    c = torch.empty(n, dtype=torch.float32).uniform_(-1.0, 1.0, generator=g)
    if dtype == "int8":
        return (b * 100).to(torch.int8), (c * 100).to(torch.int8)
    return b.to(TORCH_DTYPES[dtype]), c.to(TORCH_DTYPES[dtype])


# ------------------------------------------------------------------ GEMM path
def gemm_inputs(m: int, n: int, k: int, dtype: str, seed: int = 0) -> dict:
    """Seeded GEMM operands as CPU tensors.

    bfloat16 / float16 / float32 / float64: A (m x k) ~ normal(0, 1/sqrt(k))
    from seed, B (k x n) from seed + 1, drawn in fp32 and cast.
    float8_e4m3fn / float8_e5m2: A, B ~ normal(0, 1) from the same seeds; each
    is scaled so its amax maps to the format's largest finite value (448,
    57344) and cast; scale_a / scale_b are the dequantisation factors.
    """
    ga = torch.Generator().manual_seed(seed)
    gb = torch.Generator().manual_seed(seed + 1)
    a32 = torch.randn(m, k, generator=ga, dtype=torch.float32)
    b32 = torch.randn(k, n, generator=gb, dtype=torch.float32)
    if dtype in FP8_MAX:
        qa, sa = quantize_fp8(a32, dtype)
        qb, sb = quantize_fp8(b32, dtype)
        return {"a": qa, "b": qb, "scale_a": sa, "scale_b": sb}
    std = 1.0 / math.sqrt(k)
    return {
        "a": (a32 * std).to(TORCH_DTYPES[dtype]),
        "b": (b32 * std).to(TORCH_DTYPES[dtype]),
        "scale_a": 1.0,
        "scale_b": 1.0,
    }


def quantize_fp8(x: torch.Tensor, dtype: str = "float8_e4m3fn") -> tuple[torch.Tensor, float]:
    """Per-tensor fp8 quantisation with amax -> the format's largest finite
    value; returns (q, scale) with x ~= q * scale."""
    amax = float(x.abs().max())
    scale = amax / FP8_MAX[dtype] if amax > 0 else 1.0
    q = (x / scale).to(TORCH_DTYPES[dtype])
    return q, scale


def gemm_reference(a: torch.Tensor, b: torch.Tensor, scale_a: float = 1.0, scale_b: float = 1.0,
                   rows: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 CPU matmul of the dequantised operands (mfu.py:234 with fp32
    accumulation); fp64 operands are multiplied in fp64.

    `rows` optionally restricts the check to a subset of C's rows (large shapes).
    """
    if a.dtype == torch.float64:
        return (a if rows is None else a[rows]) @ b
    af = a.float()
    if rows is not None:
        af = af[rows]
    if scale_a != 1.0:
        af = af * scale_a
    bf = b.float()
    if scale_b != 1.0:
        bf = bf * scale_b
    return af @ bf


def gemm_output_dtype(dtype: str) -> torch.dtype:
    """C's element type: fp8 inputs produce bf16, the others their own type."""
    return {"float16": torch.float16, "float32": torch.float32, "float64": torch.float64}.get(dtype, torch.bfloat16)


# ---------------------------------------------------------------- comparators
_INT_VIEW = {
    torch.float32: torch.int32,
    torch.float64: torch.int64,
    torch.bfloat16: torch.int16,
    torch.float16: torch.int16,
}


def ordered_bits(x: torch.Tensor) -> torch.Tensor:
    """Map floats to int64 keys whose difference counts representable steps (ulps)."""
    bits = x.contiguous().view(_INT_VIEW[x.dtype]).to(torch.int64)
    width = x.element_size() * 8
    sign_bit = 1 << (width - 1)
    mag = bits & (sign_bit - 1)
    return torch.where(bits < 0, -mag, mag)


def ulp_distance(out: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Per-element ulp distance; 0 where both are NaN; huge where exactly one is NaN."""
    if out.dtype != ref.dtype or out.shape != ref.shape:
        raise ValueError(f"mismatched tensors {out.dtype}{tuple(out.shape)} vs {ref.dtype}{tuple(ref.shape)}")
    d = (ordered_bits(out) - ordered_bits(ref)).abs()
    out_nan, ref_nan = torch.isnan(out), torch.isnan(ref)
    d = torch.where(out_nan & ref_nan, torch.zeros_like(d), d)
    return torch.where(out_nan ^ ref_nan, torch.full_like(d, 1 << 62), d)


def bits_equal(out: torch.Tensor, ref: torch.Tensor) -> bool:
    """Bit-for-bit equality (copy parity)."""
    a = out.contiguous().view(torch.uint8)
    b = ref.contiguous().view(torch.uint8)
    return a.shape == b.shape and bool(torch.equal(a, b))


def rel_frobenius(out: torch.Tensor, ref: torch.Tensor) -> float:
    """||out - ref||_F / ||ref||_F in float64."""
    o = out.double()
    r = ref.double()
    denom = float(torch.linalg.vector_norm(r))
    num = float(torch.linalg.vector_norm(o - r))
    return num / denom if denom > 0 else num


def max_abs_over_max_ref(out: torch.Tensor, ref: torch.Tensor) -> float:
    """The reference parity harness's criterion: max|out-ref| / max|ref|
    (tests/native/gemm_parity.hip.cpp:160-178)."""
    o = out.double()
    r = ref.double()
    return float((o - r).abs().max()) / max(float(r.abs().max()), 1e-12)


def to_numpy_bits(x: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a tensor as a numpy unsigned array (for fixtures)."""
    view = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[x.element_size()]
    np_dtype = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[x.element_size()]
    return x.contiguous().view(view).numpy().view(np_dtype)
