"""Pins the oracle's int4 quantisers and dequantisers.

- nibble order: low nibble = even element, high = odd
  (QuantizationTests.swift:35, dequant_int4.metal:4-18);
- round-trip bounds |w - w_hat| <= scale/2 (+ bf16 rounding of the scale);
- `sym` rows carry bias == symmetricBiasBits(scale) bit for bit, and the
  sym/affine dequantisers agree on them exactly;
- the fp16 staging value equals numpy's float16 rounding of the exact fp32
  product (q-8)*s.
"""
import numpy as np


def test_nibble_order_low_is_even(oracle):
    # A row whose even elements are the group minimum and odd elements the
    # maximum quantises to q=0 (low nibbles) and q=15 (high nibbles).
    row = np.tile(np.array([-1.0, 1.0], np.float32), 16)[None, :]
    packed, scales, biases = oracle.quantize_int4(row, 32, symmetric=False)
    assert np.all(packed == 0xF0)
    deq = oracle.dequantize_int4(packed, scales, biases, 32, 32)
    assert deq[0, 0] < deq[0, 1]


def test_affine_round_trip_bound(oracle):
    rng = oracle.SplitMix64(11)
    for group in (32, 64):
        w = rng.uniforms(-0.5, 0.5, 16 * 256).reshape(16, 256)
        packed, scales, biases = oracle.quantize_int4(w, group, symmetric=False)
        deq = oracle.dequantize_int4(packed, scales, biases, 256, group)
        s = oracle.bf16_to_float(scales).repeat(group, axis=1)
        b = oracle.bf16_to_float(biases).repeat(group, axis=1)
        # bias is rounded to bf16 too, so allow its rounding on top of s/2
        bound = s / 2 + np.abs(b) * 2.0**-8 + 1e-7
        assert np.all(np.abs(deq - w) <= bound + s * 2.0**-8)


def test_sym_round_trip_and_bias_identity(oracle):
    rng = oracle.SplitMix64(12)
    for group in (32, 64):
        w = rng.uniforms(-0.5, 0.5, 16 * 256).reshape(16, 256)
        packed, scales, biases = oracle.quantize_int4(w, group, symmetric=True)
        for s, b in zip(scales.ravel(), biases.ravel()):
            assert oracle.sym_bias_bits(int(s)) == int(b)
        deq_affine = oracle.dequantize_int4(packed, scales, biases, 256, group)
        deq_sym = oracle.dequantize_int4(packed, scales, None, 256, group)
        assert np.array_equal(deq_affine.view(np.uint32), deq_sym.view(np.uint32))
        s = oracle.bf16_to_float(scales).repeat(group, axis=1)
        assert np.all(np.abs(deq_sym - w) <= s / 2 * (1 + 2.0**-7) + 1e-9)
        # values sit on the lattice s * (q - 8), q in [0, 15]
        q = deq_sym / s + 8
        assert np.allclose(q, np.round(q)) and q.min() >= 0 and q.max() <= 15


def test_quantize_rounding_is_half_away_from_zero(oracle):
    # Swift Float.rounded() rounds 0.5 away from zero: a value exactly half a
    # step above the bias goes up. Scale 1 (bf16 exact) via a 0..15 ramp.
    row = np.zeros((1, 32), np.float32)
    row[0, :16] = np.arange(16, dtype=np.float32)
    row[0, 16:] = np.arange(16, dtype=np.float32)
    row[0, 3] = 2.5  # exactly between q=2 and q=3
    packed, scales, biases = oracle.quantize_int4(row, 32, symmetric=False)
    assert oracle.bf16_to_float(scales)[0, 0] == 1.0
    deq = oracle.dequantize_int4(packed, scales, biases, 32, 32)
    assert deq[0, 3] == 3.0


def test_f16_staging_is_rne_of_exact_product(oracle):
    rng = oracle.SplitMix64(13)
    w = rng.uniforms(-0.125, 0.125, 64 * 704).reshape(64, 704)
    for symmetric in (True, False):
        packed, scales, biases = oracle.quantize_int4(w, 32, symmetric)
        got = oracle.dequantize_int4_f16(packed, scales, biases, 704, 32, symmetric)
        exact = oracle.dequantize_int4(packed, scales, None if symmetric else biases, 704, 32)
        if symmetric:
            # (q-8)*s is exact in fp32, so fp16 staging is one RNE of it
            want = exact.astype(np.float16).view(np.uint16)
            assert np.array_equal(got, want)
        else:
            # affine: fma(q, s, b) rounds once to fp32, then half() to fp16.
            # q*s + b is exact in fp64 (4 + 8 + 8 significant bits).
            q = np.empty((64, 704), np.float64)
            q[:, 0::2] = packed & 0x0F
            q[:, 1::2] = packed >> 4
            sf = oracle.bf16_to_float(scales).repeat(32, axis=1).astype(np.float64)
            bf = oracle.bf16_to_float(biases).repeat(32, axis=1).astype(np.float64)
            want = (q * sf + bf).astype(np.float32).astype(np.float16).view(np.uint16)
            assert np.array_equal(got, want)
