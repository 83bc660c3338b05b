"""GPU: PrefillInt4QMM (dense int4 projection over t tokens) through the C-ABI,
against the oracle (fp16-staged weights, exact sums) within the north-star
1e-3 relative bound, at the Gemma projection shapes and ragged token counts.
Output rows past t stay untouched. Declines and errors as documented."""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tsg():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import tsugumi_amd
    return tsugumi_amd


def operands(rng, n, k, g):
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = oracle.bf16_bits((np.abs(rng.normal(0, 0.02, n * (k // g))) / 7).astype(np.float32))
    biases = oracle.bf16_bits(rng.normal(0, 0.01, n * (k // g)).astype(np.float32))
    return packed, scales, biases


@pytest.mark.parametrize("t,n,k,g,scheme", [
    (1, 2816, 2816, 64, "affine"), (37, 4096, 2816, 32, "sym"), (300, 2816, 4096, 64, "sym"),
    (2048, 2816, 2816, 32, "affine"), (129, 704, 2816, 32, "sym"), (255, 8192, 2816, 64, "affine"),
    (2048, 4096, 2816, 32, "sym"),
])
def test_qmm_matches_oracle(tsg, t, n, k, g, scheme):
    print(f"qmm t={t} n={n} k={k} g{g} {scheme}", flush=True)
    sym = scheme == "sym"
    ctx = tsg.Context(0, group_size=g)
    ctx.set_affine_scheme(scheme)
    rng = np.random.default_rng(t * 7 + n)
    packed, scales, biases = operands(rng, n, k, g)
    xb = oracle.f16_bits(rng.normal(0, 1, t * k).astype(np.float32))
    y = empty(t * n + 64, fill=0x1234)
    tsg.PrefillInt4QMM(ctx).encode(dev(packed), dev(scales), None if sym else dev(biases),
                                   dev(xb), y, t, n, k)
    got = host(y, np.uint16)
    assert np.all(got[t * n:] == 0x1234)
    ref = oracle.int4_qmm(packed, scales, None if sym else biases, xb, t, n, k, g, sym)
    rel = oracle.relative_error(oracle.f16_to_float(got[:t * n]),
                                oracle.f16_to_float(ref.ravel()))
    print(f"  rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR
    ctx.close()


@pytest.mark.parametrize("scheme", ["sym", "affine"])
def test_qmm_narrow_tiles_equal_wide_tiles_bitwise(tsg, scheme):
    """Below 256 workgroups of 256 columns the QMM runs 128-column tiles (one
    weight tile per wave); each column keeps the same MFMA sequence, so the
    results are the wide tiles' bit for bit. T = 2048: N = 4096 runs 256 wide
    workgroups, its first 2816 weight rows as N = 2816 176 -> 352 narrow ones;
    the shared 2816 columns must agree exactly."""
    t, k, g, n_wide, n_narrow = 2048, 2816, 32, 4096, 2816
    print(f"qmm narrow vs wide {scheme}", flush=True)
    sym = scheme == "sym"
    ctx = tsg.Context(0, group_size=g)
    ctx.set_affine_scheme(scheme)
    rng = np.random.default_rng(4242 + sym)
    packed, scales, biases = operands(rng, n_wide, k, g)
    xb = oracle.f16_bits(rng.normal(0, 1, t * k).astype(np.float32))
    q = tsg.PrefillInt4QMM(ctx)
    y_wide, y_narrow = empty(t * n_wide), empty(t * n_narrow)
    sg = n_narrow * (k // g)
    q.encode(dev(packed), dev(scales), None if sym else dev(biases), dev(xb), y_wide, t, n_wide, k)
    q.encode(dev(np.ascontiguousarray(packed[:n_narrow])), dev(scales[:sg].copy()),
             None if sym else dev(biases[:sg].copy()), dev(xb), y_narrow, t, n_narrow, k)
    wide = host(y_wide, np.uint16).reshape(t, n_wide)[:, :n_narrow]
    narrow = host(y_narrow, np.uint16).reshape(t, n_narrow)
    assert np.array_equal(wide, narrow)
    ctx.close()


def test_qmm_errors(tsg):
    ctx = tsg.Context(0, group_size=32)
    q = tsg.PrefillInt4QMM(ctx)
    w, s, x, y = empty(64 * 64), empty(64 * 8), empty(4 * 256), empty(4 * 64)
    with pytest.raises(tsg.TsgError) as e:
        q.encode(w, s, s, x, y, 4, 64, 100)          # K % group
    assert e.value.status == 1 and "multiple of 32" in str(e.value)
    with pytest.raises(tsg.TsgError) as e:
        q.encode(w, s, s, x, y, 4, 48, 256)          # N % 64: the tiled path declines
    assert e.value.status == 3
    with pytest.raises(tsg.TsgError) as e:
        q.encode(w, s, s, x[1:], y, 4, 64, 256)      # x misaligned
    assert e.value.status == 2
    with pytest.raises(tsg.TsgError) as e:
        q.encode(w, s, s, x, y, 0, 64, 256)
    assert e.value.status == 1
    ctx.close()
