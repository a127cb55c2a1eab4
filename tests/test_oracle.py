"""Pinning the oracle (CPU only).

Each oracle function is checked against something other than its own
formula: the torch library routine the reference path calls, exhaustive
enumeration of a format's codes, exact rational arithmetic, closed forms, an
independent MT19937 implementation, or a float64 brute force. A planted
mistake (an unfused triad, a truncating bf16 encoder, a transposed GEMM
operand) is shown to fail the same checks.
"""
from __future__ import annotations

from fractions import Fraction
import math

import numpy as np
import pytest
import torch

from oracle import clib
from oracle import reference_path as rp


# ---------------------------------------------------------------- codecs
def test_bf16_decode_matches_torch_for_every_code():
    codes = np.arange(1 << 16, dtype=np.uint16)
    ours = clib.decode_bf16(codes)
    theirs = torch.from_numpy(codes.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_f16_decode_matches_torch_for_every_code():
    codes = np.arange(1 << 16, dtype=np.uint16)
    ours = clib.decode_f16(codes)
    theirs = torch.from_numpy(codes.view(np.int16).copy()).view(torch.float16).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(nan, np.isnan(ours))
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def _encode_probe_values() -> np.ndarray:
    rng = np.random.default_rng(7)
    wide = rng.standard_normal(400_000).astype(np.float32) * (
        np.float32(10.0) ** rng.integers(-40, 38, 400_000).astype(np.float32))
    raw = rng.integers(0, 1 << 32, 400_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # exact ties for bf16 (low 16 bits 0x8000) and fp16 (bit 12 set, lower clear)
    ties_bf = (rng.integers(0, 1 << 16, 4096, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 2.0**-14, 2.0**-24,
                         2.0**-25, 3 * 2.0**-26, 1e-45, 3.4028235e38], dtype=np.float32)
    x = np.concatenate([wide, raw, ties_bf, specials, -specials])
    return x[~np.isnan(x)]


def test_bf16_and_f16_encode_match_torch_rne():
    x = _encode_probe_values()
    t = torch.from_numpy(x)
    assert np.array_equal(clib.encode_bf16(x), t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(clib.encode_f16(x), t.to(torch.float16).view(torch.int16).numpy().view(np.uint16))


def test_truncating_bf16_encoder_is_caught():
    x = _encode_probe_values()
    truncated = (x.view(np.uint32) >> 16).astype(np.uint16)
    expected = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert not np.array_equal(truncated, expected)


def test_e4m3_decode_matches_torch_and_format_kats():
    codes = np.arange(256, dtype=np.uint8)
    ours = clib.decode_e4m3(codes)
    theirs = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(nan, np.isnan(ours))
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert set(codes[nan].tolist()) == {0x7F, 0xFF}
    assert ours[0x7E] == 448.0 and ours[0xFE] == -448.0   # max finite
    assert ours[0x01] == 2.0**-9                          # min subnormal
    assert ours[0x08] == 2.0**-6                          # min normal
    assert ours[0x38] == 1.0


def test_e5m2_decode_matches_torch_and_format_kats():
    codes = np.arange(256, dtype=np.uint8)
    ours = clib.decode_e5m2(codes)
    theirs = torch.from_numpy(codes.copy()).view(torch.float8_e5m2).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(nan, np.isnan(ours))
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert set(codes[nan].tolist()) == {0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF}
    assert ours[0x7C] == np.inf and ours[0xFC] == -np.inf
    assert ours[0x7B] == 57344.0 and ours[0xFB] == -57344.0   # max finite
    assert ours[0x01] == 2.0**-16                             # min subnormal
    assert ours[0x04] == 2.0**-14                             # min normal
    assert ours[0x3C] == 1.0 and ours[0x3D] == 1.25


def test_e5m2_quantisation_rounds_to_nearest_even_and_saturates_to_inf():
    # 1.125 lies halfway between 1.0 and 1.25: ties go to the even mantissa (1.0);
    # 1.375 lies between 1.25 and 1.5: to 1.5 (even). Beyond 61440 the cast overflows.
    x = torch.tensor([1.125, 1.375, 57344.0, 61440.0, -2.0**-17, 2.0**-17 * 3])
    q = x.to(torch.float8_e5m2)
    got = clib.decode_e5m2(q.view(torch.uint8).numpy())
    assert got[0] == 1.0 and got[1] == 1.5 and got[2] == 57344.0
    assert np.isinf(got[3])
    assert got[4] == 0.0 and np.signbit(got[4])    # -2^-17 ties to -0
    assert got[5] == 2.0**-15                        # 1.5 * 2^-16 ties to 2 * 2^-16


def test_e5m2_gemm_inputs_round_trip():
    ops = rp.gemm_inputs(64, 48, 128, "float8_e5m2", seed=0)
    for key, scale in (("a", ops["scale_a"]), ("b", ops["scale_b"])):
        q = ops[key]
        assert q.dtype == torch.float8_e5m2
        deq = clib.decode_e5m2(q.view(torch.uint8).numpy())
        assert np.isfinite(deq).all() and np.abs(deq).max() == 57344.0
    # the oracle product is the fp64 product of the decoded operands, scaled
    a = clib.decode_e5m2(ops["a"].view(torch.uint8).numpy()).astype(np.float64) * ops["scale_a"]
    b = clib.decode_e5m2(ops["b"].view(torch.uint8).numpy()).astype(np.float64) * ops["scale_b"]
    ref = rp.gemm_reference(ops["a"], ops["b"], ops["scale_a"], ops["scale_b"]).numpy().astype(np.float64)
    assert np.abs(ref - a @ b).max() <= 1e-5 * np.abs(a @ b).max()


def test_float64_gemm_reference_stays_in_float64():
    ops = rp.gemm_inputs(16, 8, 32, "float64", seed=3)
    assert ops["a"].dtype == torch.float64
    ref = rp.gemm_reference(ops["a"], ops["b"])
    assert ref.dtype == torch.float64
    exact = clib.gemm_f64(ops["a"].numpy(), ops["b"].numpy())
    assert np.allclose(ref.numpy(), exact, rtol=1e-13, atol=1e-15)


# ---------------------------------------------------------------- stream
STREAM_DTYPES = ["float32", "bfloat16", "float16", "float64"]


def _np(x: torch.Tensor) -> np.ndarray:
    return rp.to_numpy_bits(x) if x.dtype in (torch.bfloat16, torch.float16) else x.numpy()


def _torch(arr: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype in ("bfloat16", "float16"):
        return torch.from_numpy(arr.view(np.int16).copy()).view(rp.TORCH_DTYPES[dtype])
    return torch.from_numpy(arr.copy())


@pytest.mark.parametrize("dtype", STREAM_DTYPES)
@pytest.mark.parametrize("mode", ["copy", "scale", "triad"])
def test_stream_oracle_vs_reference_torch_op(dtype, mode):
    b, c = rp.stream_inputs(100_003, dtype, seed=3)
    expected = rp.stream_reference(mode, b, c, 3.0)
    got = _torch(clib.stream(mode, dtype, _np(b), _np(c), 3.0), dtype)
    if mode != "triad" or dtype in ("float32", "float64"):
        assert rp.bits_equal(got, expected)
        return
    # torch's CPU half-precision add(alpha) computes in fp32 in its vector
    # body (equal to ours) but, in the scalar remainder of each thread's
    # chunk, rounds alpha*c to the element type before the add: two extra
    # roundings, up to 2 ulp off on those few elements only.
    dist = rp.ulp_distance(got, expected)
    assert int(dist.max()) <= 2
    assert int((dist != 0).sum()) <= 64
    # Against the composition of library routines this build's semantics
    # name -- fp32 fused add(alpha), then one RNE cast -- it is bit-exact.
    composed = torch.add(b.float(), c.float(), alpha=3.0).to(b.dtype)
    assert rp.bits_equal(got, composed)


def test_torch_cpu_fp32_add_alpha_is_fused():
    # The composition above relies on torch's fp32 add(alpha) being one fma;
    # the correctly-rounded check below (exact rationals) pins that.
    b, c = rp.stream_inputs(4000, "float32", seed=4)
    t = torch.add(b, c, alpha=3.0)
    for i in range(0, 4000, 13):
        exact = Fraction(float(b[i])) + 3 * Fraction(float(c[i]))
        lo = np.float32(float(exact))
        cands = [lo, np.nextafter(lo, np.float32(-np.inf)), np.nextafter(lo, np.float32(np.inf))]
        best = min(cands, key=lambda f: (abs(Fraction(float(f)) - exact), int(np.array(f).view(np.uint32)) & 1))
        assert float(t[i]) == float(best)


def test_int8_copy_oracle():
    b, _ = rp.stream_inputs(4097, "int8", seed=1)
    got = clib.stream("copy", "int8", b.numpy(), None, 1.0)
    assert np.array_equal(got, b.numpy())


def test_fp32_triad_is_the_correctly_rounded_b_plus_sc():
    b, c = rp.stream_inputs(2000, "float32", seed=11)
    s = 3.0
    got = clib.stream("triad", "float32", b.numpy(), c.numpy(), s)
    for i in range(0, 2000, 7):
        exact = Fraction(float(b[i])) + Fraction(s) * Fraction(float(c[i]))
        # the nearest float32 to `exact`: the rounding of the two neighbours' midpoint test
        lo = np.float32(float(exact))
        cand = [lo, np.nextafter(lo, np.float32(-np.inf)), np.nextafter(lo, np.float32(np.inf))]
        best = min(cand, key=lambda f: (abs(Fraction(float(f)) - exact), int(np.array(f).view(np.uint32)) & 1))
        assert got[i] == best


def test_unfused_triad_would_fail_the_bit_exact_check():
    b, c = rp.stream_inputs(1 << 16, "float32", seed=0)
    unfused = (b.numpy() + np.float32(3.0) * c.numpy()).astype(np.float32)  # two roundings
    expected = rp.stream_reference("triad", b, c, 3.0).numpy()
    assert not np.array_equal(unfused.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("dtype", STREAM_DTYPES)
def test_stream_closed_forms(dtype):
    b, c = rp.stream_inputs(5000, dtype, seed=5)
    bn, cn = _np(b), _np(c)
    # scale by 1 is a copy; triad with s = 0 or c = 0 returns b (b is finite, so b + 0 == b)
    assert np.array_equal(clib.stream("scale", dtype, bn, None, 1.0), bn)
    assert np.array_equal(clib.stream("triad", dtype, bn, cn, 0.0), bn)
    assert np.array_equal(clib.stream("triad", dtype, bn, np.zeros_like(cn), 3.0), bn)
    # scale by 0 gives zeros carrying the sign of b; scale by -1 flips exactly the sign bit
    zero = _torch(clib.stream("scale", dtype, bn, None, 0.0), dtype)
    assert torch.all(zero == 0) and torch.equal(torch.signbit(zero), torch.signbit(b))
    neg = _torch(clib.stream("scale", dtype, bn, None, -1.0), dtype)
    assert torch.equal(neg, -b)


def test_stream_inputs_follow_the_configured_generator():
    # uniform[-1, 1) fp32 from one generator, b then c
    b, c = rp.stream_inputs(1 << 12, "float32", seed=0)
    g = torch.Generator().manual_seed(0)
    b2 = torch.rand(1 << 12, generator=g)
    assert b.min() >= -1 and b.max() <= 1 and not torch.equal(b, c)
    assert abs(float(b.mean())) < 0.05 and abs(float(b2.mean()) - 0.5) < 0.05


# ---------------------------------------------------------------- comparators
def test_ulp_distance_known_values():
    one = torch.tensor([1.0], dtype=torch.float32)
    nxt = torch.tensor([np.nextafter(np.float32(1), np.float32(2))])
    assert int(rp.ulp_distance(one, nxt)) == 1
    z = torch.tensor([0.0]), torch.tensor([-0.0])
    assert int(rp.ulp_distance(*z)) == 0
    tiny = torch.tensor([np.float32(1e-45)]), torch.tensor([-np.float32(1e-45)])
    assert int(rp.ulp_distance(*tiny)) == 2
    nan = torch.tensor([float("nan")])
    assert int(rp.ulp_distance(nan, nan)) == 0 and int(rp.ulp_distance(nan, one)) > 1 << 60
    bf = torch.tensor([1.0], dtype=torch.bfloat16)
    assert int(rp.ulp_distance(bf, bf * (1 + 2**-7))) == 1


def test_rel_frobenius_known_value():
    ref = torch.tensor([3.0, 4.0])
    assert rp.rel_frobenius(torch.tensor([3.0, 4.5]), ref) == pytest.approx(0.1)


def test_max_abs_over_max_ref_known_values():
    # The reference harness's criterion (tests/native/gemm_parity.hip.cpp:160-178): the largest
    # absolute difference over the largest |reference| entry. Chosen so that the plausible slips give
    # other numbers: max(ref) instead of max|ref| gives 0.25 / 1, max|out| instead of max|ref| gives
    # 0.25 / 3.75, the mean difference instead of the max gives 0.25 / 4 / 4, a signed max gives 0.
    ref = torch.tensor([[1.0, -4.0], [2.0, 0.5]])
    out = torch.tensor([[1.0, -3.75], [2.0, 0.5]])
    assert rp.max_abs_over_max_ref(out, ref) == 0.0625
    assert rp.max_abs_over_max_ref(ref, ref) == 0.0
    # half-precision inputs are compared as their exact values (no rounding of the difference):
    # 1 + 2^-7 and 1 are both bf16 values; the difference 2^-7 over max|ref| = 2 is 2^-8 exactly
    r16 = torch.tensor([1.0, 2.0], dtype=torch.bfloat16)
    o16 = torch.tensor([1.0 + 2.0**-7, 2.0], dtype=torch.bfloat16)
    assert rp.max_abs_over_max_ref(o16, r16) == 2.0**-8
    # an all-zero reference divides by the harness's 1e-12 floor
    assert rp.max_abs_over_max_ref(torch.tensor([1e-13]), torch.tensor([0.0])) == pytest.approx(0.1)


# ---------------------------------------------------------------- GEMM
def test_gemm_reference_matches_float64_brute_force():
    for m, n, k in [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 48, 96)]:
        a = torch.randn(m, k, generator=torch.Generator().manual_seed(m))
        b = torch.randn(k, n, generator=torch.Generator().manual_seed(n))
        ref = rp.gemm_reference(a, b).double().numpy()
        brute = clib.gemm_f64(a.numpy(), b.numpy())
        assert np.max(np.abs(ref - brute)) <= 1e-5 * max(1.0, np.max(np.abs(brute)))


def test_transposed_operand_is_caught():
    a = torch.randn(32, 32, generator=torch.Generator().manual_seed(1))
    b = torch.randn(32, 32, generator=torch.Generator().manual_seed(2))
    brute = torch.from_numpy(clib.gemm_f64(a.numpy(), b.numpy()))
    assert rp.rel_frobenius(rp.gemm_reference(a, b.t().contiguous()), brute) > 0.5


def test_gemm_constant_fill_kat():
    # The reference executable fills A = B = 0.03125: every C entry is K / 1024 exactly.
    for k in (32, 1024, 8192):
        a = torch.full((4, k), 0.03125, dtype=torch.bfloat16)
        b = torch.full((k, 3), 0.03125, dtype=torch.bfloat16)
        assert torch.all(rp.gemm_reference(a, b) == k / 1024)


def test_gemm_identity_and_outer_product():
    a = torch.randn(16, 16).to(torch.bfloat16)
    assert torch.equal(rp.gemm_reference(a, torch.eye(16, dtype=torch.bfloat16)), a.float())
    u = torch.randn(9, 1).to(torch.bfloat16)
    v = torch.randn(1, 11).to(torch.bfloat16)
    assert torch.equal(rp.gemm_reference(u, v), u.float() * v.float())


def test_fp8_quantisation_properties():
    ops = rp.gemm_inputs(64, 48, 128, "float8_e4m3fn", seed=0)
    for key, scale_key, seed in (("a", "scale_a", 0), ("b", "scale_b", 1)):
        q, s = ops[key], ops[scale_key]
        assert q.dtype == torch.float8_e4m3fn
        deq = q.float()
        assert float(deq.abs().max()) == 448.0                       # amax maps onto the max code
        assert not torch.isnan(deq).any()
        x = torch.randn(*q.shape, generator=torch.Generator().manual_seed(seed))
        # relative error of e4m3 with 3 mantissa bits is <= 2^-4 for normals
        err = (deq * s - x).abs()
        assert float((err - (x.abs() * 2.0**-4 + 2.0**-9 * s)).max()) <= 1e-6


def test_gemm_inputs_distribution():
    ops = rp.gemm_inputs(256, 256, 1024, "bfloat16", seed=0)
    a = ops["a"].float()
    assert ops["a"].dtype == torch.bfloat16 and ops["b"].shape == (1024, 256)
    assert abs(float(a.std()) - 1 / math.sqrt(1024)) < 0.05 / math.sqrt(1024)


# ---------------------------------------------------------------- parity harness inputs
def test_mt19937_uniform_fill_matches_an_independent_mt19937():
    # numpy's legacy RandomState seeds MT19937 with init_genrand like std::mt19937;
    # libstdc++ uniform_real_distribution<float> uses one 32-bit draw:
    # (hi - lo) * (float(x) / 2^32) + lo, computed in float.
    n, seed, lo, hi = 4096, 0xA1, -0.1, 0.1
    raw = np.random.RandomState(seed).randint(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    canon = raw.astype(np.float32) / np.float32(2.0**32)
    canon = np.where(canon >= 1.0, np.nextafter(np.float32(1), np.float32(0)), canon).astype(np.float32)
    expected = (np.float32(hi) - np.float32(lo)) * canon + np.float32(lo)
    got = clib.fill_uniform_mt19937(n, seed, lo, hi)
    assert np.array_equal(got, expected.astype(np.float32))


def test_mode_byte_factors_and_numel():
    assert rp.MODE_BYTE_FACTORS == {"copy": 2, "scale": 2, "triad": 3}
    assert rp.numel_for(1024, 4) == 1 << 28
    assert rp.numel_for(2, 2) == 1 << 20
