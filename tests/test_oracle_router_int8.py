"""Pins the oracle's INT8-affine restatement (Quantization.swift:243-303) and its
router logits in the MI355X kernel's order against closed forms, exact
arithmetic, fp64 brute force and the reference's own router test cases."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc

STEP = 2.0 ** -7  # a bf16-exact scale: (wmax - wmin) = 255 * STEP


def ramp_group(group, codes, half=False):
    """A group whose min is -1 and max -1 + 255 * STEP (so scale = STEP and
    bias = -1 exactly); the other elements sit at code k (or k + 1/2)."""
    row = np.empty(group, np.float32)
    row[0], row[1] = -1.0, -1.0 + 255 * STEP
    for j in range(2, group):
        row[j] = -1.0 + (codes[j] + (0.5 if half else 0.0)) * STEP
    return row


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_int8_exact_ramp(group):
    codes = [0, 255] + [(7 * j + 3) % 255 for j in range(2, group)]
    row = ramp_group(group, codes)
    packed, scales, biases = oracle.quantize_int8_affine(row[None, :], group)
    assert scales[0, 0] == 0x3C00 and biases[0, 0] == 0xBF80  # bf16 2^-7 and -1
    assert packed[0].tolist() == codes
    back = oracle.dequantize_int8_affine(packed, scales, biases, group)
    np.testing.assert_array_equal(back[0], row)


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_int8_half_steps_round_away_from_zero(group):
    # (w - bias) / scale = k + 1/2 exactly: Swift's rounded() takes k + 1, even
    # for even k (round-half-even would not)
    codes = [0, 255] + [(2 * j) % 254 for j in range(2, group)]
    row = ramp_group(group, codes, half=True)
    packed, _, _ = oracle.quantize_int8_affine(row[None, :], group)
    assert packed[0, 2:].tolist() == [k + 1 for k in codes[2:]]


def test_quantize_int8_constant_group_and_clamps():
    # wmax == wmin: scale 1 and bias bf16(w); the codes are round(w - bias) = 0
    const = np.full(64, 0.3, np.float32)
    p, s, b = oracle.quantize_int8_affine(const[None, :], 64)
    assert s[0, 0] == 0x3F80 and b[0, 0] == oracle.bf16_bits(np.float32(0.3))
    assert (p == 0).all()
    # bf16(wmin) above wmin: the min element's code would be negative -> 0
    row = np.linspace(1.0 + 3 * 2.0 ** -9, 2.0, 64, dtype=np.float32)
    p, s, b = oracle.quantize_int8_affine(row[None, :], 64)
    assert oracle.bf16_to_float(b[0, 0]) > row[0]
    assert p[0, 0] == 0 and p[0, -1] in (254, 255)


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_int8_round_trip_bound(group):
    rng = oracle.SplitMix64(0x1A7E)
    w = rng.uniforms(-0.2, 0.2, 16 * 256).reshape(16, 256)
    p, s, b = oracle.quantize_int8_affine(w, group)
    back = oracle.dequantize_int8_affine(p, s, b, group).reshape(16, 256 // group, group)
    wg = w.reshape(16, 256 // group, group)
    scale = oracle.bf16_to_float(s)[..., None]
    bias_err = np.abs(oracle.bf16_to_float(b) - wg.min(axis=2))[..., None]
    # half a step, plus the bias rounding, plus the bf16 scale's rounding
    # carried over up to 255 steps at the top of the range
    assert (np.abs(back - wg) <= 0.5 * scale + bias_err + 255 * scale * 2.0 ** -8 + 1e-7).all()
    assert np.abs(back - wg).max() < 0.003


def test_dequantize_int8_closed_form():
    # float(q) * scale + bias: an 8-bit code times a bf16 scale is exact in
    # fp32, so the one rounding is the sum's (fused or not, the same bits)
    rng = np.random.default_rng(5)
    q = rng.integers(0, 256, (8, 128), dtype=np.uint8)
    s_bits = oracle.bf16_bits(rng.uniform(1e-4, 2e-3, (8, 2)).astype(np.float32))
    b_bits = oracle.bf16_bits(rng.uniform(-0.3, 0.0, (8, 2)).astype(np.float32))
    got = oracle.dequantize_int8_affine(q, s_bits, b_bits, 64)
    s = np.repeat(oracle.bf16_to_float(s_bits), 64, axis=1).astype(np.float32)
    b = np.repeat(oracle.bf16_to_float(b_bits), 64, axis=1).astype(np.float32)
    want = (q.astype(np.float32) * s).astype(np.float32) + b
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, (q.astype(np.float64) * s + b).astype(np.float32))


@pytest.mark.parametrize("group", [32, 64])
def test_router_int8_logits_exact_arithmetic(group):
    """Inputs on which every product and partial sum is exact in fp32: any
    order gives the fp64 sum, so a dropped term, a wrong group index or a
    swapped scale/bias fails bit for bit."""
    rng = np.random.default_rng(11 + group)
    ne, d = 12, 512
    q = rng.integers(0, 256, (ne, d), dtype=np.uint8)
    hidden = oracle.f16_bits((rng.integers(-64, 65, d) / 64.0).astype(np.float32))
    es = oracle.bf16_bits(rng.choice([0.5, 1.0, 2.0], d).astype(np.float32))
    s_bits = oracle.bf16_bits(rng.choice([2.0 ** -7, 2.0 ** -8], (ne, d // group)).astype(np.float32))
    b_bits = oracle.bf16_bits((rng.integers(-8, 9, (ne, d // group)) / 8.0).astype(np.float32))
    got = oracle.router_logits_int8_canonical(q, s_bits, b_bits, hidden, es, ne, d, group)
    x = oracle.f16_to_float(hidden).astype(np.float64) * oracle.bf16_to_float(es)
    wf = (q.astype(np.float64) * np.repeat(oracle.bf16_to_float(s_bits), group, axis=1)
          + np.repeat(oracle.bf16_to_float(b_bits), group, axis=1))
    want = wf @ x
    np.testing.assert_array_equal(got.astype(np.float64), want)


def test_router_int8_logits_fp32_bound():
    c = kc.router_int8_case(2816, 32, 64, 0xD1, 0)
    got = oracle.router_logits_int8_canonical(c["packed"], c["scales"], c["biases"],
                                              c["hidden"], c["es_bits"], 32, 2816, 64)
    x = oracle.f16_to_float(c["hidden"]).astype(np.float64) * oracle.bf16_to_float(c["es_bits"])
    wf = oracle.dequantize_int8_affine(c["packed"], c["scales"], c["biases"], 64)
    terms = np.abs(wf.astype(np.float64) * x)
    want = wf.astype(np.float64) @ x
    assert (np.abs(got - want) <= 4e-6 * terms.sum(axis=1) + 1e-7).all()


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("draw", range(4))
def test_router_int8_kernelcheck_selection(group, draw):
    """checkRouter(weightBits: 8, d: 2816, experts: 128, seed: 0xD1): the
    kernel-order logits select routerReference's experts, weights within
    Tolerance.fp16Reduction."""
    c = kc.router_int8_case(2816, 128, group, 0xD1, draw)
    logits = oracle.router_logits_int8_canonical(c["packed"], c["scales"], c["biases"],
                                                 c["hidden"], c["es_bits"], 128, 2816, group)
    idx, w_bits = oracle.topk_softmax(logits, 8, oracle.bf16_to_float(c["pes_bits"]))
    assert idx.tolist() == c["idx"].tolist()
    assert oracle.relative_error(oracle.f16_to_float(w_bits), c["wts"]) <= kc.FP16_REDUCTION


@pytest.mark.parametrize("kind", ["spread", "near_tie"])
def test_router_int8_reference_test_cases(kind):
    """RouterTopKTests (RouterTopKTests.swift:17-69): same indices, weights
    within 5e-3 absolute."""
    c = kc.router_topk_test_case(kind)
    logits = oracle.router_logits_int8_canonical(c["packed"], c["scales"], c["biases"],
                                                 c["hidden"], c["es_bits"], c["ne"], c["d"], 64)
    idx, w_bits = oracle.topk_softmax(logits, 8, oracle.bf16_to_float(c["pes_bits"]))
    assert idx.tolist() == c["idx"].tolist()
    assert np.abs(oracle.f16_to_float(w_bits) - c["wts"]).max() < 5e-3
