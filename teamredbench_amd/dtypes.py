"""Element-type catalogue (the table of src/teamredbench/dtypes.py:7-31).

``matmul_ops_factor`` is the ops counted per multiply-accumulate for MFU
(2 for real types, 8 for complex, 0 where MFU is undefined).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class DTypeSpec:
    name: str
    torch_attr: str
    bytes_per_element: int
    kind: str
    matmul_ops_factor: int


def _spec(name: str, nbytes: int, kind: str, factor: int) -> DTypeSpec:
    return DTypeSpec(name, name, nbytes, kind, factor)


DTYPE_CANDIDATES: list[DTypeSpec] = [
    _spec("bool", 1, "bool", 0),
    _spec("uint8", 1, "integer", 2),
    _spec("int8", 1, "integer", 2),
    _spec("int16", 2, "integer", 2),
    _spec("int32", 4, "integer", 2),
    _spec("int64", 8, "integer", 2),
    _spec("float8_e4m3fn", 1, "float", 2),
    _spec("float8_e5m2", 1, "float", 2),
    _spec("float16", 2, "float", 2),
    _spec("bfloat16", 2, "float", 2),
    _spec("float32", 4, "float", 2),
    _spec("float64", 8, "float", 2),
    _spec("complex64", 8, "complex", 8),
    _spec("complex128", 16, "complex", 8),
]


def discover_dtypes(torch_module: Any) -> dict[str, DTypeSpec]:
    """All candidates without torch; with torch, those torch defines."""
    return {
        spec.name: spec
        for spec in DTYPE_CANDIDATES
        if torch_module is None or hasattr(torch_module, spec.torch_attr)
    }


def resolve_dtype_names(requested: list[str] | None, available: dict[str, DTypeSpec]) -> list[str]:
    """Empty or containing "all" -> every available dtype; unknown names raise KeyError."""
    if not requested or "all" in requested:
        return list(available)
    unknown = [name for name in requested if name not in available]
    if unknown:
        raise KeyError(f"Unknown dtypes requested: {', '.join(unknown)}")
    return list(requested)
