"""CPU: the dense int4 QMM oracle (PrefillInt4QMM's tiled path, fp16-staged
weights) pinned by a closed form, by the fp32-weight GEMV restatement
(DequantInt4GemvRef, Reference/Quant/DequantInt4Gemv.swift:12-44) row by row,
and by a non-square shape that a transposed operand would break."""
import numpy as np

import oracle


def test_closed_form_sym():
    # sym: w = (q - 8) * s. q = 9 everywhere, s = 1/64, x = 1: y = k / 64 exactly.
    t, n, k, g = 3, 64, 256, 32
    packed = np.full((n, k // 2), 0x99, np.uint8)
    scales = np.full((n, k // g), oracle.bf16_bits(np.float32(1 / 64)), np.uint16)
    x = oracle.f16_bits(np.ones(t * k, np.float32))
    y = oracle.f16_to_float(oracle.int4_qmm(packed, scales, None, x, t, n, k, g, True))
    assert np.all(y == k / 64)


def test_rows_match_fp32_weight_gemv():
    t, n, k = 5, 192, 512
    rng = np.random.default_rng(3)
    for g, sym in ((32, False), (64, True)):
        w = rng.normal(0, 0.05, (n, k)).astype(np.float32)
        packed, scales, biases = oracle.quantize_int4(w, g, sym)
        xb = oracle.f16_bits(rng.normal(0, 1, t * k).astype(np.float32))
        y = oracle.f16_to_float(oracle.int4_qmm(packed, scales, None if sym else biases, xb,
                                                t, n, k, g, sym))
        assert y.shape == (t, n)
        xf = oracle.f16_to_float(xb).reshape(t, k)
        for r in range(t):
            ref = oracle.dequant_int4_gemv_ref(packed, scales, None if sym else biases, xf[r],
                                               k, g)
            assert oracle.relative_error(y[r], ref) <= 1e-3
