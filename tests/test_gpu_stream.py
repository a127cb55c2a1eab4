"""GPU parity of the gfx950 stream kernels against the oracle (-m gpu).

Every case builds its inputs on the host with the oracle's seeded generator
(uniform[-1, 1] fp32 from one CPU generator, cast to the element type),
copies them to the GPU, runs one mb_stream launch through the C ABI on the
current stream and compares the bytes that come back with the C oracle
(oracle/stream_oracle.c) on the same inputs. The kernels and the oracle share
one definition (copy = bit copy, scale = RNE(s*b), triad = RNE(fma(s, c, b))
in fp32, fp64 for float64), so every op is checked bit for bit; the looser
1-ulp bound of the benchmark configuration is the in-run check against the
torch GPU op.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import clib
from oracle import reference_path as rp
from teamredbench_amd.native import capi

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "bfloat16", "float16", "float64"]
MODES = ["copy", "scale", "triad"]


def _bits(x: torch.Tensor) -> np.ndarray:
    return rp.to_numpy_bits(x.cpu())


def _run(lib, mode: str, dtype: str, b: torch.Tensor, c: torch.Tensor, s: float, *, offset: int = 0,
         blocks_per_cu: int = 0) -> torch.Tensor:
    """mb_stream on device copies of b/c (optionally shifted by `offset` elements)."""
    n = b.numel() - offset
    db = b.cuda()
    dc = c.cuda()
    dst = torch.full((b.numel(),), 7, dtype=b.dtype, device="cuda") if dtype != "int8" else \
        torch.full((b.numel(),), 7, dtype=torch.int8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    lib.stream(capi.OPS[mode], capi.DTYPES[dtype], dst[offset:].data_ptr(), db[offset:].data_ptr(),
               dc[offset:].data_ptr() if mode == "triad" else None, n, s, blocks_per_cu, stream)
    torch.cuda.synchronize()
    return dst.cpu()


def _expect(mode: str, dtype: str, b: torch.Tensor, c: torch.Tensor, s: float) -> np.ndarray:
    return clib.stream(mode, dtype, _bits(b), _bits(c), s)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 4099, (1 << 20) + 3, 1 << 20])
def test_stream_matches_oracle(lib, mode, dtype, n):
    print(f"[stream] {mode} {dtype} n={n}", flush=True)
    b, c = rp.stream_inputs(n, dtype, seed=n % 97)
    got = _run(lib, mode, dtype, b, c, 3.0)
    assert np.array_equal(_bits(got), _expect(mode, dtype, b, c, 3.0))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", MODES)
def test_stream_configuration_sizes(lib, mode, dtype):
    # The stream sweep's 2^24 point, checked element for element.
    n = 1 << 24
    print(f"[stream] {mode} {dtype} n=2^24", flush=True)
    b, c = rp.stream_inputs(n, dtype, seed=0)
    got = _run(lib, mode, dtype, b, c, 3.0)
    assert np.array_equal(_bits(got), _expect(mode, dtype, b, c, 3.0))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("offset", [1, 3])
def test_unaligned_buffers_take_the_scalar_kernel(lib, mode, dtype, offset):
    n = 50_001
    print(f"[stream] unaligned {mode} {dtype} offset={offset}", flush=True)
    b, c = rp.stream_inputs(n, dtype, seed=offset)
    got = _run(lib, mode, dtype, b, c, 3.0, offset=offset)
    exp = _expect(mode, dtype, b[offset:], c[offset:], 3.0)
    assert np.array_equal(_bits(got)[offset:], exp)
    # elements before the window are untouched
    untouched = _bits(torch.full((offset,), 7, dtype=b.dtype))
    assert np.array_equal(_bits(got)[:offset], untouched)


def test_int8_copy(lib):
    b, c = rp.stream_inputs(100_003, "int8", seed=2)
    got = _run(lib, "copy", "int8", b, c, 1.0)
    assert np.array_equal(got.numpy(), b.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_copy_keeps_every_bit_pattern(lib, dtype):
    # NaN payloads, infinities, -0 and subnormals survive the copy unchanged.
    width = {"float32": 4, "bfloat16": 2, "float16": 2}[dtype]
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, 65536 * width + 6 * width, dtype=np.uint8)
    b = torch.from_numpy(raw).view(rp.TORCH_DTYPES[dtype])
    got = _run(lib, "copy", dtype, b, b, 1.0)
    assert rp.bits_equal(got, b)


@pytest.mark.parametrize("bpc", [1, 3, 16])
def test_blocks_per_cu_override_keeps_results(lib, bpc):
    b, c = rp.stream_inputs((1 << 20) + 5, "float32", seed=9)
    got = _run(lib, "triad", "float32", b, c, 3.0, blocks_per_cu=bpc)
    assert np.array_equal(got.numpy().view(np.uint32), _expect("triad", "float32", b, c, 3.0).view(np.uint32))


def test_zero_length_is_a_noop(lib):
    dst = torch.full((4,), 5.0, device="cuda")
    lib.stream(capi.OP_TRIAD, capi.DT_FLOAT32, dst.data_ptr(), dst.data_ptr(), dst.data_ptr(), 0, 3.0)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), torch.full((4,), 5.0))


def test_rejections_carry_an_error_string(lib):
    x = torch.zeros(16, device="cuda")
    with pytest.raises(capi.NativeLibraryError, match="int8 supports only copy") as err:
        lib.stream(capi.OP_SCALE, capi.DT_INT8, x.data_ptr(), x.data_ptr(), None, 16, 2.0)
    assert err.value.status == capi.MB_ERR_UNSUPPORTED
    with pytest.raises(capi.NativeLibraryError, match="null buffer") as err:
        lib.stream(capi.OP_TRIAD, capi.DT_FLOAT32, x.data_ptr(), x.data_ptr(), None, 16, 2.0)
    assert err.value.status == capi.MB_ERR_INVALID_ARG
    with pytest.raises(capi.NativeLibraryError, match="unknown stream op"):
        lib.stream(7, capi.DT_FLOAT32, x.data_ptr(), x.data_ptr(), None, 16, 2.0)


def test_timed_loop_reports_positive_time_and_keeps_results(lib):
    n = 1 << 22
    b, c = rp.stream_inputs(n, "float32", seed=1)
    db, dc = b.cuda(), c.cuda()
    dst = torch.empty_like(db)
    stream = torch.cuda.current_stream().cuda_stream
    t = lib.time_stream(capi.OP_TRIAD, capi.DT_FLOAT32, dst.data_ptr(), db.data_ptr(), dc.data_ptr(), n, 3.0, 0,
                        2, 5, stream)
    assert 0 < t < 1.0
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), _expect("triad", "float32", b, c, 3.0).view(np.uint32))


def test_kernel_info_keys(lib):
    info = lib.stream_info(capi.OP_TRIAD, capi.DT_FLOAT32, 1 << 28)
    for key in ("implementation", "threads_per_block", "vector_unroll", "blocks_per_cu", "arch"):
        assert key in info
    assert info["arch"].startswith("gfx950")


@pytest.mark.parametrize("mode, dtype, n, nontemporal", [
    ("triad", "float32", 1 << 28, True),     # 3 GiB a pass: streams past the Infinity Cache
    ("triad", "float32", 1 << 24, False),    # 192 MiB: fits, ordinary accesses keep it there
    ("copy", "float32", 1 << 24, False),     # 128 MiB
    ("copy", "bfloat16", 1 << 24, False),    # 64 MiB, the copy / scale window's lower edge
    ("scale", "bfloat16", (1 << 24) - 8, True),   # just below it
    ("triad", "float32", 6990507, False),    # 80 MiB + 4 bytes, the triad's lower edge
    ("triad", "float32", 6990506, True),     # 8 bytes below it
    ("copy", "float32", 1 << 25, False),     # 256 MiB, the upper edge
    ("scale", "float32", (1 << 25) + 8, True),    # just above it
    ("triad", "float32", 1 << 25, True),     # 384 MiB
    ("copy", "float32", 1 << 20, True),
])
def test_nontemporal_hint_follows_the_pass_size(lib, mode, dtype, n, nontemporal):
    info = lib.stream_info(capi.OPS[mode], capi.DTYPES[dtype], n)
    assert info["nontemporal"] is nontemporal, info
    with lib.tuned(stream_nontemporal=0 if nontemporal else 1):    # the knob still overrides it
        assert lib.stream_info(capi.OPS[mode], capi.DTYPES[dtype], n)["nontemporal"] is not nontemporal


def test_triad_and_copy_past_2_31_elements(lib):
    # n = 2^31 + 13 bf16 elements (4 GiB per array): element indexes and byte offsets past 32 bits. Checked
    # on the device in slices: the triad against fp32 fma then RNE to bf16 (for bf16 inputs b + 3c is exact
    # in fp64, so rounding it to fp32 is the fma), the copy bit for bit; a guard after dst stays untouched.
    n, guard = (1 << 31) + 13, 4096
    print(f"[stream] triad/copy bfloat16 n=2^31+13", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    b = torch.rand(n, device="cuda", dtype=torch.bfloat16, generator=gen) * 2 - 1
    c = torch.rand(n, device="cuda", dtype=torch.bfloat16, generator=gen) * 2 - 1
    flat = torch.full((n + guard,), 7, dtype=torch.bfloat16, device="cuda")
    dst = flat[:n]
    stream = torch.cuda.current_stream().cuda_stream
    step = 1 << 28
    for mode in ("triad", "copy"):
        lib.stream(capi.OPS[mode], capi.DTYPES["bfloat16"], dst.data_ptr(), b.data_ptr(),
                   c.data_ptr() if mode == "triad" else None, n, 3.0, 0, stream)
        torch.cuda.synchronize()
        assert (flat[n:] == 7).all(), f"{mode} wrote past the end of dst"
        for i in range(0, n, step):
            if mode == "triad":
                want = (b[i:i + step].double() + 3.0 * c[i:i + step].double()).float().bfloat16()
            else:
                want = b[i:i + step]
            assert torch.equal(dst[i:i + step].view(torch.int16), want.view(torch.int16)), (mode, i)
