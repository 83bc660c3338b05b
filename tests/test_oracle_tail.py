"""CPU: the layer-tail oracle (prefill_layer_tail_block, prefill.metal:319-397)
pinned by closed forms, the scale invariance of RMSNorm, a float64 statement
of the formula with a large eps, and row/stride independence."""
import numpy as np

import oracle

D = 2816  # Gemma 4 26B-A4B hidden size


def f16(x):
    return oracle.f16_bits(np.asarray(x, np.float32))


def bf16(x):
    return oracle.bf16_bits(np.asarray(x, np.float32))


def test_constant_rows_closed_form():
    # h2 = 2, eps = 0: rms(h2) = 2, so h2 * inv * 1 = 1; h12 = 0 + 1 has rms 1;
    # hidden = (0.5 + 1 * 0.25) * 2 = 1.5, every step exact.
    d = 96
    h2 = f16(np.full(d, 2.0))
    h1 = f16(np.zeros(d))
    hidden = f16(np.full(d, 0.5))
    out = oracle.layer_tail(h2, h1, hidden, bf16(np.ones(d)), bf16(np.full(d, 0.25)), 1, d,
                            d, d, d, 0.0, 2.0)
    assert np.all(oracle.f16_to_float(out) == 1.5)


def test_layer_scalar_is_rounded_to_fp16_first():
    # layer_scalar 1 + 2^-12 rounds to 1.0 in fp16 (half(layer_scalar), fused.metal:366).
    d = 64
    rng = oracle.SplitMix64(11)
    h2, h1, hid = (rng.uniforms_f16(-1, 1, d) for _ in range(3))
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    a = oracle.layer_tail(h2, h1, hid, w2, w1, 1, d, d, d, d, 1e-6, 1.0 + 2.0 ** -12)
    b = oracle.layer_tail(h2, h1, hid, w2, w1, 1, d, d, d, d, 1e-6, 1.0)
    assert np.array_equal(a, b)


def test_rmsnorm_scale_invariance():
    # Scaling h2 by 2^k (exact in fp16) leaves every output bit unchanged at eps = 0.
    d = D
    rng = oracle.SplitMix64(0x7A11)
    h2 = rng.uniforms_f16(-1, 1, d)
    h1, hid = rng.uniforms_f16(-1, 1, d), rng.uniforms_f16(-1, 1, d)
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    base = oracle.layer_tail(h2, h1, hid, w2, w1, 1, d, d, d, d, 0.0, 1.0)
    for k in (-3, 4):
        scaled = f16(oracle.f16_to_float(h2) * np.float32(2.0 ** k))
        assert np.array_equal(oracle.layer_tail(scaled, h1, hid, w2, w1, 1, d, d, d, d, 0.0, 1.0),
                              base)


def _tail_f64(h2, h1, hid, w2, w1, d, eps, s):
    x2 = oracle.f16_to_float(h2).astype(np.float64)
    x1 = oracle.f16_to_float(h1).astype(np.float64)
    xh = oracle.f16_to_float(hid).astype(np.float64)
    a = oracle.bf16_to_float(w2).astype(np.float64)
    b = oracle.bf16_to_float(w1).astype(np.float64)
    h12 = x1 + x2 / np.sqrt(np.mean(x2 * x2) + eps) * a
    return (xh + h12 / np.sqrt(np.mean(h12 * h12) + eps) * b) * s


def test_matches_float64_formula_with_large_eps():
    # eps = 0.5 against mean squares near 1/3 makes eps placement, the 1/D mean
    # and each weight visible; fp16 staging bounds the gap to a few ulp.
    rng = oracle.SplitMix64(0x7A11_B10C)
    for d in (D, 100, 1):
        h2, h1, hid = (rng.uniforms_f16(-1, 1, d) for _ in range(3))
        w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
        out = oracle.f16_to_float(oracle.layer_tail(h2, h1, hid, w2, w1, 1, d, d, d, d, 0.5, 0.875))
        ref = _tail_f64(h2, h1, hid, w2, w1, d, 0.5, 0.875)
        assert np.max(np.abs(out - ref)) <= 4 * 2.0 ** -11 * max(1.0, np.max(np.abs(ref)))
        if d > 1:  # one element near cancellation has no meaningful relative error
            assert oracle.relative_error(out, ref.astype(np.float32)) <= 1e-3


def test_rows_and_strides_are_independent():
    rows, d = 3, 200
    s2, s1, sh = d + 9, d + 13, d + 17
    rng = oracle.SplitMix64(5)
    h2, h1, hid = (rng.uniforms_f16(-1, 1, rows * s) for s in (s2, s1, sh))
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    out = oracle.layer_tail(h2, h1, hid, w2, w1, rows, d, s2, s1, sh, 1e-6, 1.1)
    for r in range(rows):
        one = oracle.layer_tail(h2[r * s2:r * s2 + d], h1[r * s1:r * s1 + d],
                                hid[r * sh:r * sh + d], w2, w1, 1, d, d, d, d, 1e-6, 1.1)
        assert np.array_equal(out[r * sh:r * sh + d], one)
        assert np.array_equal(out[r * sh + d:(r + 1) * sh], hid[r * sh + d:(r + 1) * sh])
