"""GPU parity at the benchmark configurations' own sizes, against the oracle (-m gpu).

The other GPU test files check every kernel family on small and medium
shapes. This one runs the exact sizes the benchmark configurations time, so
the plans those sizes select (256 x 256 rounds at 8192^3 and 16384^3, the
128-row tiles and fill rule of the rectangular shapes, the split-K skinny
plans) have oracle-checked output:

  * stream: copy / scale / triad x fp32 / bf16 / fp16 at 2^28 elements per
    array (1 GiB fp32), bit for bit against the C oracle;
  * GEMM bf16 8192^3 and fp8 e4m3 8192^3 / 16384^3, and the rectangular
    shapes 8192 x 1024 x 8192 and 4096 x 14336 x 4096 in bf16 and fp16: a
    seeded subset of C's rows (every column) against the fp32 CPU matmul of
    the same (dequantised) operands, with the relative-Frobenius gates of the
    configurations (1e-2 bf16/fp16, 5e-2 fp8), and every element of those
    rows within its rounding bound of an fp64 matmul of the same operands
    (tests/gemm_bounds.py: output half-ulp, (K + 2) fp32 summation steps of
    |A| @ |B|, the fp8 MFMA block term), which a tile that skipped one of its
    K stages, or took one from the wrong place, fails;
  * the reference's own numerical parity case
    (tests/native/gemm_parity.hip.cpp:126-130, 174-178;
    tests/test_native_gemm_parity.py:69): A from std::mt19937(0xA1), B from
    std::mt19937(0xB2), uniform(+-0.05) for fp16, +-0.10 for bf16, +-1 for
    fp32/fp64, cast with round-to-nearest-even, at 512^3 (the reference
    test's size) and 1024^3 (the harness default); pass when
    max|C - C_ref| <= tol * max|C_ref| with tol 1e-2 fp16, 2e-2 bf16,
    1e-4 fp32, 1e-10 fp64. The reference compares against hipBLAS with fp32
    compute; here C_ref is the oracle's CPU matmul (fp32, fp64 for fp64)
    rounded to the output type, as the reference reads hipBLAS's C back in T.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gemm_bounds import elementwise_bound
from oracle import clib
from oracle import reference_path as rp
from teamredbench_amd.native import capi

pytestmark = pytest.mark.gpu

REL_FROB = {"bfloat16": 1e-2, "float16": 1e-2, "float8_e4m3fn": 5e-2}
ROWS_CHECKED = 256

_STREAM_INPUTS: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}


def _stream_inputs(dtype: str) -> tuple[torch.Tensor, torch.Tensor]:
    # One seeded draw per dtype at 2^28, shared by the three modes (the draw takes seconds).
    if dtype not in _STREAM_INPUTS:
        _STREAM_INPUTS.clear()
        _STREAM_INPUTS[dtype] = rp.stream_inputs(1 << 28, dtype, seed=0)
    return _STREAM_INPUTS[dtype]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("mode", ["copy", "scale", "triad"])
def test_stream_2p28_matches_oracle(lib, dtype, mode):
    n = 1 << 28
    print(f"[config] stream {mode} {dtype} n=2^28", flush=True)
    b, c = _stream_inputs(dtype)
    db, dc = b.cuda(), c.cuda()
    dst = torch.full_like(db, 7)
    lib.stream(capi.OPS[mode], capi.DTYPES[dtype], dst.data_ptr(), db.data_ptr(),
               dc.data_ptr() if mode == "triad" else None, n, 3.0, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = rp.to_numpy_bits(dst.cpu())
    del db, dc, dst
    expected = clib.stream(mode, dtype, rp.to_numpy_bits(b), rp.to_numpy_bits(c), 3.0)
    mismatches = int(np.count_nonzero(got != expected))
    assert mismatches == 0, f"{mode} {dtype} 2^28: {mismatches} elements differ from the oracle"


def _run_gemm(lib, dtype: str, ops: dict) -> torch.Tensor:
    a, b = ops["a"], ops["b"]
    m, k = a.shape
    n = b.shape[1]
    dt = capi.DTYPES[dtype]
    da, db = a.cuda(), b.cuda()
    dc = torch.full((m, n), float("nan"), dtype=rp.gemm_output_dtype(dtype), device="cuda")
    ws_bytes = lib.gemm_workspace_size(dt, m, n, k)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    lib.gemm(dt, da.data_ptr(), db.data_ptr(), dc.data_ptr(), m, n, k, ops["scale_a"], ops["scale_b"],
             ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = dc.cpu()
    del da, db, dc, ws
    torch.cuda.empty_cache()
    return out


@pytest.mark.parametrize("dtype, shape", [
    ("bfloat16", (8192, 8192, 8192)),
    ("float8_e4m3fn", (8192, 8192, 8192)),
    ("float8_e4m3fn", (16384, 16384, 16384)),
    ("bfloat16", (8192, 1024, 8192)),
    ("float16", (8192, 1024, 8192)),
    ("bfloat16", (4096, 14336, 4096)),
    ("float16", (4096, 14336, 4096)),
])
def test_gemm_configuration_shape_matches_oracle(lib, dtype, shape):
    m, n, k = shape
    info = lib.gemm_info(capi.DTYPES[dtype], m, n, k)
    print(f"[config] gemm {dtype} {m}x{n}x{k} plan {info['implementation']} "
          f"{info['tile_m']}x{info['tile_n']} split {info['split_k']}", flush=True)
    assert info["implementation"].endswith("lds_dma"), info   # the pipelined kernel, not the generic one
    ops = rp.gemm_inputs(m, n, k, dtype, seed=0)
    got = _run_gemm(lib, dtype, ops)
    assert not torch.isnan(got).any(), "C has unwritten (NaN-filled) elements"
    # rows: a seeded sample plus the first and last rows of C
    gen = torch.Generator().manual_seed(m + n + k)
    rows = torch.cat([torch.randperm(m, generator=gen)[:ROWS_CHECKED - 4],
                      torch.tensor([0, 127, m - 128, m - 1])]).unique()
    ref = rp.gemm_reference(ops["a"][rows], ops["b"], ops["scale_a"], ops["scale_b"])
    out = got[rows].float()
    err = rp.rel_frobenius(out, ref)
    assert err <= REL_FROB[dtype], f"{dtype} {shape}: rel-Frobenius {err:.3e} over {rows.numel()} rows"
    # Every checked element within its rounding bound of the fp64 product of the same operands (exact
    # inputs, so only fp64 rounding separates it from the true sum). The magnitude term |A_rows| @ |B| is
    # taken in fp32 (every term is positive, so its own rounding is below (K + 2) * 2^-24 relative: the
    # bound's slack factor 1 + 2^-8 covers it at K <= 16384).
    s = float(ops["scale_a"]) * float(ops["scale_b"])
    ref64 = s * (ops["a"][rows].double() @ ops["b"].double())
    mag = s * (ops["a"][rows].float().abs() @ ops["b"].float().abs()).double() * (1.0 + 2.0**-8)
    bound = elementwise_bound(dtype, k, ref64.abs(), mag)
    excess = (got[rows].double() - ref64).abs() - bound
    worst = int(torch.argmax(excess))
    wr, wc = divmod(worst, n)
    assert float(excess.max()) <= 0.0, (
        f"{dtype} {shape}: C[{int(rows[wr])}, {wc}] = {float(got[rows][wr, wc])!r}, fp64 {float(ref64[wr, wc])!r}, "
        f"bound {float(bound[wr, wc]):.3e}")


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32", "float64"])
@pytest.mark.parametrize("size", [512, 1024])
def test_reference_gemm_parity_case(lib, dtype, size):
    m = n = k = size
    amp = {"float16": 0.05, "bfloat16": 0.10, "float32": 1.0, "float64": 1.0}[dtype]
    tol = {"float16": 1e-2, "bfloat16": 2e-2, "float32": 1e-4, "float64": 1e-10}[dtype]
    tdt = rp.TORCH_DTYPES[dtype]
    a = torch.from_numpy(clib.fill_uniform_mt19937(m * k, 0xA1, -amp, amp)).view(m, k).to(tdt)
    b = torch.from_numpy(clib.fill_uniform_mt19937(k * n, 0xB2, -amp, amp)).view(k, n).to(tdt)
    print(f"[config] reference parity case {dtype} {size}^3", flush=True)
    got = _run_gemm(lib, dtype, {"a": a, "b": b, "scale_a": 1.0, "scale_b": 1.0})
    ref = rp.gemm_reference(a, b).to(tdt)
    ratio = rp.max_abs_over_max_ref(got, ref)
    assert not torch.isnan(got).any()
    assert ratio <= tol, f"{dtype} {size}^3: max|d| / max|ref| = {ratio:.3e} > {tol}"
