"""In-run correctness evidence for the native backend: the native result is
compared with the reference torch op on the same device and inputs, and the
distance goes into the record's metadata (``parity``). Copy must match bit
for bit, scale/triad within 1 ulp, GEMM within a relative Frobenius bound."""
from __future__ import annotations

from typing import Any

STREAM_ULP_BOUND = 1
GEMM_REL_FROBENIUS_BOUND = {"bfloat16": 1e-2, "float16": 1e-2, "float8_e4m3fn": 5e-2, "float8_e5m2": 5e-2,
                            "float32": 1e-5, "float64": 1e-12}


def _ordered(torch: Any, x: Any) -> Any:
    view = {1: torch.int8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[x.element_size()]
    bits = x.contiguous().view(view).to(torch.int64)
    sign = 1 << (x.element_size() * 8 - 1)
    mag = bits & (sign - 1)
    return torch.where(bits < 0, -mag, mag)


def max_ulp(torch: Any, out: Any, ref: Any) -> int:
    """Largest ulp distance between two float tensors (NaN == NaN)."""
    d = (_ordered(torch, out) - _ordered(torch, ref)).abs()
    if out.is_floating_point():
        both_nan = torch.isnan(out) & torch.isnan(ref)
        d = torch.where(both_nan, torch.zeros_like(d), d)
        one_nan = torch.isnan(out) ^ torch.isnan(ref)
        d = torch.where(one_nan, torch.full_like(d, 1 << 62), d)
    return int(d.max()) if d.numel() else 0


def stream_parity(torch: Any, mode: str, out: Any, ref: Any) -> dict[str, Any]:
    if mode == "copy":
        equal = bool(torch.equal(out.view(torch.uint8), ref.view(torch.uint8)))
        return {"vs": "torch", "bit_exact": equal, "passed": equal}
    worst = max_ulp(torch, out, ref)
    return {"vs": "torch", "max_ulp": worst, "bound_ulp": STREAM_ULP_BOUND, "passed": worst <= STREAM_ULP_BOUND}


def gemm_parity(torch: Any, dtype: str, out: Any, ref: Any) -> dict[str, Any]:
    o = out.double()
    r = ref.double()
    denom = float(torch.linalg.vector_norm(r))
    err = float(torch.linalg.vector_norm(o - r)) / denom if denom > 0 else float("inf")
    bound = GEMM_REL_FROBENIUS_BOUND[dtype]
    return {"vs": "torch", "rel_frobenius": err, "bound": bound, "passed": err <= bound}
