"""Pins the oracle's PRNG against published vectors.

SplitMix64 (TsugumiValidation/Support/PRNG/SplitMix64.swift:11-24) from seed 0
must give the published first outputs; FNV-1a-64 (SeedTree.swift:12-19) must
give its published offset basis and the value for "a".
"""
import numpy as np


def test_splitmix64_published_vector(oracle):
    rng = oracle.SplitMix64(0)
    assert [rng.next() for _ in range(3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_fnv1a64_published_vectors(oracle):
    assert oracle.fnv1a64("") == 0xCBF29CE484222325
    assert oracle.fnv1a64("a") == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64("foobar") == 0x85944171F73967E8


def test_seed_tree_mixes_root_with_label_hash(oracle):
    root = 0xA1
    label = "int4-gemv-m128-n2816-g32"
    expected = root ^ oracle.fnv1a64(label)
    rng = oracle.seed_tree_key(root, label)
    assert rng.state.value == expected


def test_uniform_is_top24_bits_scaled(oracle):
    # uniform = lo + (hi - lo) * Float(next() >> 40) / 2^24, one rounding per op.
    a = oracle.SplitMix64(12345)
    b = oracle.SplitMix64(12345)
    for _ in range(1000):
        raw = b.next()
        u = np.float32(raw >> 40) / np.float32(1 << 24)
        expected = np.float32(-0.5) + np.float32(np.float32(1.0) * u)
        assert np.float32(a.uniform(-0.5, 0.5)) == expected
    vals = oracle.SplitMix64(7).uniforms(-1.0, 1.0, 100000)
    assert vals.min() >= -1.0 and vals.max() < 1.0
    assert abs(float(vals.mean())) < 0.01
