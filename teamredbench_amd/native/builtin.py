"""Built-in native kernels: the gfx950 stream and GEMM families of
libmi355bench.so. They answer to the reference's built-in names too
(src/teamredbench/native/builtin.py:11-23: ``hbm_hip``, ``mfu_hipblas``)."""
from __future__ import annotations

from teamredbench_amd.native.build import CSRC_DIR
from teamredbench_amd.native.registry import ABI_CAPI, register_native_kernel

register_native_kernel(
    name="hbm_gfx950",
    benchmark="hbm",
    description="gfx950 stream kernels (copy/scale/triad, 16-byte nontemporal grid-stride) via the C ABI.",
    source_path=CSRC_DIR / "stream.hip",
    abi=ABI_CAPI,
    aliases=("hbm_hip",),
)

register_native_kernel(
    name="mfu_gfx950",
    benchmark="mfu",
    description="gfx950 MFMA GEMM (bf16/fp16/fp8 e4m3 and e5m2 with fp32 accumulate; fp32; fp64) via the C ABI.",
    source_path=CSRC_DIR / "gemm.hip",
    abi=ABI_CAPI,
    aliases=("mfu_hipblas",),
)
