"""GPU: the decoder-layer tail (PrefillLayerTail / FusedLayerTail) through the
C-ABI. Mirrors PrefillLayerTailTests.blockLayerTailMatchesRepeatedFusedRows:
three rows at strides d+9, d+13, d+17 with sentinel padding, the block form
bit-identical to the fused form row by row, padding and inputs untouched.
Against the oracle (prefill.metal:319-397) within 2^-8 * max(1, |y|) per element
and 1e-3 relative: the two sums of squares run in another order. The reduce-fused form equals
the token-major reduce followed by the tail, bit for bit."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

SENTINEL = 0x7BFF  # fp16 65504
EPS = 1e-6


@pytest.fixture(scope="module")
def tsg():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import tsugumi_amd
    return tsugumi_amd


@pytest.fixture(scope="module")
def ctx(tsg):
    return tsg.Context(0)


def make_block(rng, rows, d, stride, lo, hi):
    v = np.full(rows * stride, SENTINEL, np.uint16)
    for r in range(rows):
        v[r * stride:r * stride + d] = rng.uniforms_f16(lo, hi, d)
    return v


def check_vs_oracle(got, want, d, rows, stride):
    """|got - want| <= 2^-8 * max(1, |want|) per element: one fp16 ulp of an
    intermediate of magnitude < 4 (the sums of squares run in another order, so
    an intermediate may round the other way) and the 1e-3 relative bound."""
    g = oracle.f16_to_float(np.concatenate([got[r * stride:r * stride + d] for r in range(rows)]))
    w = oracle.f16_to_float(np.concatenate([want[r * stride:r * stride + d] for r in range(rows)]))
    assert np.all(np.abs(g - w) <= 2.0 ** -8 * np.maximum(1.0, np.abs(w)))
    assert oracle.relative_error(g, w) <= 1e-3


@pytest.mark.parametrize("d", [2816, 4096, 100, 1])
def test_block_tail_matches_repeated_fused_rows(tsg, ctx, d):
    print(f"layer tail block vs fused d={d}", flush=True)
    rows = 3
    s2, s1, sh = d + 9, d + 13, d + 17
    rng = oracle.SplitMix64(0x7A11_B10C + d)
    h2 = make_block(rng, rows, d, s2, -1, 1)
    h1 = make_block(rng, rows, d, s1, -1, 1)
    hid = make_block(rng, rows, d, sh, -1, 1)
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    scalar = float(rng.uniform(0.75, 1.25))

    dh2, dh1, dhid, dw2, dw1 = dev(h2), dev(h1), dev(hid), dev(w2), dev(w1)
    tsg.PrefillLayerTail(ctx).encode(dh2, dh1, dhid, dw2, dw1, rows, d, s2, s1, sh, EPS, scalar)
    block = host(dhid, np.uint16)
    assert np.array_equal(host(dh2, np.uint16), h2)
    assert np.array_equal(host(dh1, np.uint16), h1)

    fused = hid.copy()
    tail = tsg.FusedLayerTail(ctx)
    for r in range(rows):
        rh = dev(hid[r * sh:r * sh + d])
        tail.encode(dev(h2[r * s2:r * s2 + d]), dev(h1[r * s1:r * s1 + d]), rh, dw2, dw1, d,
                    EPS, scalar)
        fused[r * sh:r * sh + d] = host(rh, np.uint16)
    assert np.array_equal(block, fused)
    for r in range(rows):
        assert np.all(block[r * sh + d:(r + 1) * sh] == SENTINEL)
    check_vs_oracle(block, oracle.layer_tail(h2, h1, hid, w2, w1, rows, d, s2, s1, sh, EPS,
                                             scalar), d, rows, sh)


def test_vector_and_scalar_forms_agree(tsg, ctx):
    """d % 8 == 0 and aligned rows take 16-byte loads; an odd element offset
    takes 2-byte loads. Same chunk ownership and sum order: same bits."""
    import torch
    t, d = 64, 2816
    rng = oracle.SplitMix64(0x5CA1)
    h2, h1, hid = (rng.uniforms_f16(-2, 2, t * d) for _ in range(3))
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    tail = tsg.PrefillLayerTail(ctx)
    a = dev(hid)
    tail.encode(dev(h2), dev(h1), a, dev(w2), dev(w1), t, d, d, d, d, EPS, 1.0625)
    shifted = torch.zeros(t * d + 1, dtype=torch.int16, device="cuda")
    shifted[1:] = dev(hid)
    tail.encode(dev(h2), dev(h1), shifted[1:], dev(w2), dev(w1), t, d, d, d, d, EPS, 1.0625)
    assert np.array_equal(host(a, np.uint16), host(shifted[1:], np.uint16))
    check_vs_oracle(host(a, np.uint16),
                    oracle.layer_tail(h2, h1, hid, w2, w1, t, d, d, d, d, EPS, 1.0625), d, t, d)


@pytest.mark.parametrize("t,k,d", [(2048, 8, 2816), (37, 8, 2816), (5, 3, 104), (7, 8, 100)])
def test_reduce_fused_tail_equals_reduce_then_tail(tsg, ctx, t, k, d):
    print(f"reduce+tail t={t} k={k} d={d}", flush=True)
    rng = oracle.SplitMix64(0x7E11 + d + t)
    P = rng.uniforms_f16(-1, 1, t * k * d)
    w = rng.uniforms_f16(0, 0.3, t * k)
    sh = d + 5
    h1 = rng.uniforms_f16(-1, 1, t * d)
    hid = make_block(rng, t, d, sh, -1, 1)
    w2, w1 = rng.uniforms_bf16(0.5, 1.5, d), rng.uniforms_bf16(0.5, 1.5, d)
    dP, dw, dh1, dw2, dw1 = dev(P), dev(w), dev(h1), dev(w2), dev(w1)

    h2 = empty(t * d)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(dP, dw, h2, t, k, d)
    two = dev(hid)
    tsg.PrefillLayerTail(ctx).encode(h2, dh1, two, dw2, dw1, t, d, d, d, sh, EPS, 0.9)

    one, h2_out = dev(hid), empty(t * d)
    tsg.PrefillMoE(ctx).encode_reduce_layer_tail(dP, dw, dh1, one, dw2, dw1, t, k, d, d, sh,
                                                 EPS, 0.9, h2=h2_out)
    assert np.array_equal(host(h2_out, np.uint16), host(h2, np.uint16))
    assert np.array_equal(host(one, np.uint16), host(two, np.uint16))
    bare = dev(hid)
    tsg.PrefillMoE(ctx).encode_reduce_layer_tail(dP, dw, dh1, bare, dw2, dw1, t, k, d, d, sh,
                                                 EPS, 0.9)
    assert np.array_equal(host(bare, np.uint16), host(two, np.uint16))
    if t <= 64:
        ref_h2 = oracle.reduce_token_major(P, w, t, k, d).ravel()
        assert np.array_equal(host(h2, np.uint16), ref_h2)
        check_vs_oracle(host(one, np.uint16),
                        oracle.layer_tail(ref_h2, h1, hid, w2, w1, t, d, d, d, sh, EPS, 0.9),
                        d, t, sh)


def test_tail_errors(tsg, ctx):
    d = 64
    buf = [empty(4 * d, fill=0) for _ in range(5)]
    tail = tsg.PrefillLayerTail(ctx)
    cases = [((0, d, d, d, d), "queryCount must be positive"),
             ((1, 0, d, d, d), "D must be in 1...4096"),
             ((1, 4097, 4097, 4097, 4097), "D must be in 1...4096"),
             ((2, d, d - 1, d, d), "h2 stride is too small"),
             ((2, d, d, d - 1, d), "h1 stride is too small"),
             ((2, d, d, d, d - 1), "hidden stride is too small")]
    for (t, dd, s2, s1, sh), msg in cases:
        with pytest.raises(tsg.TsgError) as e:
            tail.encode(*buf, t, dd, s2, s1, sh, EPS, 1.0)
        assert msg in str(e.value)
    with pytest.raises(tsg.TsgError) as e:
        tsg.FusedLayerTail(ctx).encode(*buf, 4097, EPS, 1.0)
    assert "kFusedMaxD" in str(e.value)
    before = host(buf[2], np.uint16).copy()
    tsg.FusedLayerTail(ctx).encode(*buf, 0, EPS, 1.0)  # D == 0: nothing to do
    assert np.array_equal(host(buf[2], np.uint16), before)
