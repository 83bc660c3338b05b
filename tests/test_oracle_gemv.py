"""Pins the oracle's GEMV, GELU and MoE FFN against fp64 brute force and the
reference's known GELU points (Tests/.../MoEReferenceTests.swift:7-17)."""
import math

import numpy as np


def test_gelu_known_points(oracle):
    assert oracle.gelu_tanh(0.0) == 0.0
    want = 0.5 * (1 + math.tanh(0.79788456 * 1.044715))
    assert abs(oracle.gelu_tanh(1.0) - want) < 1e-6
    # saturation: the kernel clamps the tanh argument at +/-20, the oracle
    # relies on tanh itself; both give x (large x) and 0 (large -x)
    assert oracle.gelu_tanh(30.0) == 30.0
    assert oracle.gelu_tanh(-30.0) == 0.0


def test_silu_closed_form(oracle):
    for x in (-8.0, -1.0, 0.0, 0.5, 3.0):
        assert abs(oracle.silu(x) - x / (1 + math.exp(-x))) < 1e-6


def test_gemv_matches_fp64_brute_force(oracle):
    rng = oracle.SplitMix64(21)
    for (m, n, group, symmetric) in [(64, 2816, 32, True), (33, 704, 32, False),
                                      (16, 4096, 64, True), (7, 128, 64, False)]:
        w = rng.uniforms(-0.5, 0.5, m * n).reshape(m, n)
        packed, scales, biases = oracle.quantize_int4(w, group, symmetric)
        x = oracle.f16_to_float(rng.uniforms_f16(-1.0, 1.0, n))
        y = oracle.dequant_int4_gemv_ref(packed, scales, None if symmetric else biases,
                                         x, n, group)
        wd = oracle.dequantize_int4(packed, scales, None if symmetric else biases, n, group)
        exact = wd.astype(np.float64) @ x.astype(np.float64)
        # sequential fp32 summation: error <= n * eps * sum|w x|
        bound = n * 2.0**-24 * (np.abs(wd).astype(np.float64) @ np.abs(x).astype(np.float64))
        assert np.all(np.abs(y - exact) <= bound)


def _blob(gate, up, down, symmetric):
    """One expert blob in the packer's order gate(W,S,[B]), up, down
    (RepackPlanner.swift:442-520); returns bytes + the 9 MoEExpertOffsets."""
    parts, offs = [], []
    cur = 0
    for (p, s, b) in (gate, up, down):
        for arr, is_bias in ((p, False), (s, False), (b, True)):
            if is_bias and symmetric:
                offs.append(offs[-1])  # bias offset aliases the scales
                continue
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            offs.append(cur)
            parts.append(raw)
            cur += raw.size
    return np.concatenate(parts), np.array(offs, np.uint32)


def test_routed_ffn_matches_fp64(oracle):
    rng = oracle.SplitMix64(22)
    d, f, k, group = 256, 96, 3, 32
    for symmetric in (True, False):
        blobs, deq = [], []
        for _ in range(k):
            mats = []
            dq = []
            for rows, cols in ((f, d), (f, d), (d, f)):
                w = rng.uniforms(-0.4, 0.4, rows * cols).reshape(rows, cols)
                p, s, b = oracle.quantize_int4(w, group, symmetric)
                mats.append((p, s, b))
                dq.append(oracle.dequantize_int4(p, s, b, cols, group).astype(np.float64))
            blob, offs = _blob(*mats, symmetric)
            blobs.append(blob)
            deq.append(dq)
        x = oracle.f16_to_float(rng.uniforms_f16(-0.5, 0.5, d))
        res = oracle.f16_to_float(rng.uniforms_f16(-0.5, 0.5, d))
        wts = oracle.f16_to_float(oracle.f16_bits(0.04 + np.arange(k, dtype=np.float32) * 0.015))
        y = oracle.moe_apply_streamed_routed(blobs, offs, x, res, wts, d, f, group, symmetric)
        want = res.astype(np.float64).copy()
        for e in range(k):
            g, u, dn = deq[e]
            gx = g @ x
            gelu = 0.5 * gx * (1 + np.tanh(0.7978845608028654 * (gx + 0.044715 * gx ** 3)))
            want += wts[e] * (dn @ (gelu * (u @ x)))
        assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 1e-5
