"""Pins the oracle's fp16 / bf16 conversions.

fp16: Swift's Float16(Float) is IEEE round-to-nearest-even; numpy's float32 ->
float16 cast is the same IEEE operation, so the oracle must agree with it on
every input class: normals, ties, subnormal results, overflow, inf and zero.
bf16: Quantization.swift:70-77 rounds the top 16 bits half-to-even; torch's
bfloat16 cast does the same for finite values.
"""
import numpy as np
import pytest


def _random_floats(n, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    return f[np.isfinite(f)]


def test_f16_matches_numpy_rne_on_random_bits(oracle):
    f = _random_floats(2_000_000, 1)
    got = oracle.f16_bits(f)
    want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_matches_numpy_in_the_fp16_range_incl_ties_and_subnormals(oracle):
    # Every fp32 value whose exponent lands near the fp16 range, and exact ties.
    rng = np.random.default_rng(2)
    exps = rng.integers(127 - 30, 127 + 17, size=1_000_000)
    mant = rng.integers(0, 2**23, size=exps.size)
    sign = rng.integers(0, 2, size=exps.size)
    bits = ((sign << 31) | (exps << 23) | mant).astype(np.uint32)
    f = bits.view(np.float32)
    assert np.array_equal(oracle.f16_bits(f), f.astype(np.float16).view(np.uint16))
    # ties: fp16 value +/- half an ulp
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    base = h.view(np.float16).astype(np.float32)
    nxt = (h + 1).view(np.float16).astype(np.float32)
    mid = ((base.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    assert np.array_equal(oracle.f16_bits(mid), mid.astype(np.float16).view(np.uint16))


def test_f16_special_values(oracle):
    vals = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e9,
                     2.0**-24, 2.0**-25, 2.0**-25 * 1.0001, 2.0**-14, 6e-8],
                    np.float32)
    assert np.array_equal(oracle.f16_bits(vals), vals.astype(np.float16).view(np.uint16))


def test_f16_to_float_is_exact_for_every_finite_half(oracle):
    h = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(h.view(np.float16))
    got = oracle.f16_to_float(h[finite])
    want = h[finite].view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_matches_round_half_even_and_torch(oracle):
    torch = pytest.importorskip("torch")
    f = _random_floats(1_000_000, 3)
    f = f[np.abs(f) < 3e38]
    got = oracle.bf16_bits(f)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # a scalar through the C entry point agrees with the vectorised numpy one
    for v in f[:2000]:
        assert oracle.lib().tsgo_bf16_bits(float(v)) == int(oracle.bf16_bits([v])[0])


def test_sym_bias_is_minus_eight_scale_bit_exact(oracle):
    # MoEPackAffineV1.swift:20-25: -8*scale is a pure exponent shift in bf16.
    s = np.arange(0x0080, 0x7F00, 7, dtype=np.uint16)  # positive normal bf16 scales
    for bits in s[:4000]:
        b = oracle.sym_bias_bits(int(bits))
        assert oracle.bf16_to_float([b])[0] == np.float32(-8.0) * oracle.bf16_to_float([bits])[0]
