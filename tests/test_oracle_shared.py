"""Pins the oracle's Qwen shared-expert restatement (qwen.metal:33-34, 432-455,
466; QwenForwardRunner.swift:1548-1578). The reference's tests hold no
shared-expert vectors, so the checks are closed forms, special cases that fix
each rounding point, and a composition over weights whose outputs are known
exactly (one nonzero per row), which a transposed operand, a wrong sub-tensor
offset or a missing fp16 rounding fails. Also Gemma's dense-MLP pieces
(gelu_mul_fp16, utility.metal:7-18; SharedExpertInt4.encode): the reference's
literal GELU points, the odd symmetry of the tanh form, and the composition
over the oracle's own pinned GEMV steps."""
import math

import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc


def h(x):
    return np.array(x, np.float16).view(np.uint16)


def test_sigmoid_closed_forms():
    assert oracle.sigmoid(0.0) == 0.5
    for x in (0.25, 1.0, 3.5, 9.0):
        assert abs(oracle.sigmoid(x) + oracle.sigmoid(-x) - 1.0) < 1e-6
        assert abs(oracle.sigmoid(x) - 1.0 / (1.0 + np.exp(-x))) < 1e-6
    assert oracle.sigmoid(100.0) == 1.0
    assert oracle.sigmoid(-100.0) == 0.0


def test_silu_mul_special_cases():
    # silu(0) = 0; up = 0 gives 0; silu(20) * 1 rounds to 20 in fp16; silu(-20)
    # = -4.12e-8 is 0.69 of fp16's smallest subnormal 2^-24, so it rounds to -2^-24.
    got = oracle.f16_to_float(oracle.silu_mul_f16(h([0.0, 3.0, 20.0, -20.0]),
                                                  h([5.0, 0.0, 1.0, 1.0])))
    assert list(got[:3]) == [0.0, 0.0, 20.0]
    assert got[3] == -(2.0 ** -24)
    # the gate is rounded to fp16 first (the GEMV stores it): silu(g) * u with
    # g = 2 exactly: 2 * sigmoid(2) = 1.7615942 -> times 2 -> 3.5231884 -> fp16 3.523438
    got = oracle.f16_to_float(oracle.silu_mul_f16(h([2.0]), h([2.0])))
    assert got[0] == np.float16(2.0 * 2.0 / (1.0 + np.exp(-2.0)))


def test_shared_gate_special_cases():
    y = h([1.0, -3.0, 0.5, 1000.0])
    x = h(np.ones(4))
    # zero weights: sigmoid(0) = 1/2 halves y exactly
    got = oracle.f16_to_float(oracle.shared_gate_f16(y, x, oracle.bf16_bits(np.zeros(4))))
    assert list(got) == [0.5, -1.5, 0.25, 500.0]
    # logit 4 * 32 = 128: sigmoid = 1 in fp32, y unchanged
    got = oracle.shared_gate_f16(y, x, oracle.bf16_bits(np.full(4, 32.0)))
    assert np.array_equal(got, y)
    # logit -128: sigmoid ~ 2.6e-56 -> 0, so y becomes +-0
    got = oracle.f16_to_float(oracle.shared_gate_f16(y, x, oracle.bf16_bits(np.full(4, -32.0))))
    assert np.all(got == 0.0)


def _one_hot_rows(rows, n, cols, group):
    """Sym int4 rows with q = 9 (value +1 * scale 1.0) at column cols[r], zero
    (q = 8) elsewhere: row r . v = v[cols[r]] exactly."""
    w = np.zeros((rows, n), np.float32)
    w[np.arange(rows), cols] = 1.0
    packed = np.full((rows, n // 2), 0x88, np.uint8)
    for r, c in enumerate(cols):
        b = packed[r, c // 2]
        packed[r, c // 2] = (b & 0xF0) | 9 if c % 2 == 0 else (b & 0x0F) | (9 << 4)
    scales = np.full((rows, n // group), oracle.bf16_bits(np.array([1.0]))[0], np.uint16)
    return packed, scales, scales


def test_shared_expert_composition():
    d, f, group = 64, 32, 32
    rng = np.random.default_rng(7)
    cg = rng.permutation(d)[:f]
    cu = rng.permutation(d)[:f]
    cd = rng.integers(0, f, d)
    parts = [_one_hot_rows(f, d, cg, group), _one_hot_rows(f, d, cu, group),
             _one_hot_rows(d, f, cd, group)]
    blob, offs = kc.pack_blob(parts, symmetric=True, keep_biases=False)
    x = h(rng.uniform(-2, 2, d))
    gw = oracle.bf16_bits(np.zeros(d))  # gate 1/2
    got = oracle.shared_expert(blob, offs, x, gw, d, f, group, True)
    act = oracle.silu_mul_f16(x[cg], x[cu])          # the gate/up rows pick x exactly
    want = oracle.f16_bits(oracle.f16_to_float(act[cd]) * np.float32(0.5))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("symmetric", [True, False])
def test_shared_expert_matches_dense_gemv_steps(symmetric):
    """The composition equals the pinned dense GEMV reference step by step."""
    c = kc.shared_expert_case(128, 64, 32, 0x5E, symmetric)
    (gp, gs, gb), (up, us, ub), (dp, ds, db) = c["parts"]
    x = oracle.f16_to_float(c["x_bits"])
    g16 = oracle.f16_bits(oracle.dequant_int4_gemv_ref(gp, gs, None if symmetric else gb, x, 128, 32))
    u16 = oracle.f16_bits(oracle.dequant_int4_gemv_ref(up, us, None if symmetric else ub, x, 128, 32))
    a16 = oracle.silu_mul_f16(g16, u16)
    dn = oracle.f16_bits(oracle.dequant_int4_gemv_ref(dp, ds, None if symmetric else db,
                                                      oracle.f16_to_float(a16), 64, 32))
    assert np.array_equal(c["ref"], oracle.shared_gate_f16(dn, c["x_bits"], c["gate_w"]))


# ------------------------------------------------ Gemma dense MLP pieces

def test_gelu_mul_known_points():
    """gelu_mul_fp16 (utility.metal:7-18) at the reference's literal GELU
    points (MoEReferenceTests.swift:7-17): gelu(0) = 0,
    gelu(1) = 0.5 (1 + tanh(0.7978845608028654 * 1.044715)), gelu(-1) < 0,
    gelu(2) > gelu(1); with up = 1 the product rounds once to fp16."""
    g = oracle.f16_bits(np.array([0.0, 1.0, -1.0, 2.0], np.float32))
    one = oracle.f16_bits(np.ones(4, np.float32))
    out = oracle.f16_to_float(oracle.gelu_mul_f16(g, one))
    at1 = np.float16(0.5 * (1.0 + math.tanh(0.7978845608028654 * (1.0 + 0.044715))))
    assert out[0] == 0.0
    assert out[1] == np.float32(at1)
    assert out[2] < 0 < out[1] < out[3]


def test_gelu_mul_odd_symmetry():
    """0.5 x (1 + tanh(u(x))) - 0.5 (-x) (1 + tanh(u(-x))) = x, u odd: with
    up = 1, gelu(g) - gelu(-g) recovers g within two fp16 roundings."""
    rng = np.random.default_rng(3)
    g = rng.uniform(-6, 6, 512).astype(np.float16)
    gb = g.view(np.uint16)
    one = np.full(512, np.float16(1.0)).view(np.uint16)
    pos = oracle.f16_to_float(oracle.gelu_mul_f16(gb, one)).astype(np.float64)
    neg = oracle.f16_to_float(oracle.gelu_mul_f16((-g).view(np.uint16), one)).astype(np.float64)
    err = np.abs(pos - neg - g.astype(np.float64))
    assert np.all(err <= 2 * np.abs(g.astype(np.float64)) * 2.0 ** -11 + 2.0 ** -24)


def test_dense_mlp_is_the_gemv_steps():
    """SharedExpertInt4's composition over the oracle's pinned steps: GEMV gate
    and up, fp16 rounding, gelu_mul, GEMV down, fp16 rounding."""
    d, f, group = 128, 64, 32
    for symmetric in (True, False):
        rng = oracle.seed_tree_key(0x6E + int(symmetric), "dense-mlp")
        gate = kc.quantized_rows(rng, f, d, group, symmetric)
        up = kc.quantized_rows(rng, f, d, group, symmetric)
        down = kc.quantized_rows(rng, d, f, group, symmetric)
        x = rng.uniforms_f16(-1.0, 1.0, d)
        got = oracle.dense_mlp_int4(gate, up, down, x, d, f, group, symmetric)
        xf = oracle.f16_to_float(x)
        b = lambda t: None if symmetric else t[2]
        g16 = oracle.f16_bits(oracle.dequant_int4_gemv_ref(gate[0], gate[1], b(gate), xf, d, group))
        u16 = oracle.f16_bits(oracle.dequant_int4_gemv_ref(up[0], up[1], b(up), xf, d, group))
        a = oracle.f16_to_float(oracle.gelu_mul_f16(g16, u16))
        want = oracle.f16_bits(oracle.dequant_int4_gemv_ref(down[0], down[1], b(down), a, f, group))
        assert np.array_equal(got, want)
