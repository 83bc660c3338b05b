"""Pins the oracle's router and prefill restatements.

Router (TsugumiKernelCheck/main.swift:384-402, moe.metal:281-329): on draws
whose 8th/9th logit margin is far above fp32 noise the top-k must equal the
fp64 brute-force top-k; explicit ties must resolve to the lower index; -inf
and NaN never enter; softmax weights match fp64 closed form.

Prefill reference (PrefillMoEGEMMCheck.swift:138-173): every partial must be
within the fp16 roundings of the fp64 brute force; the token-major reduce
(prefill.metal:796-817) is checked against its closed form.
"""
import numpy as np


def test_router_reference_matches_fp64_topk(oracle):
    rng = oracle.SplitMix64(31)
    checked = 0
    for draw in range(6):
        w = oracle.bf16_to_float(rng.uniforms_bf16(-0.2, 0.2, 128 * 256)).reshape(128, 256)
        x = oracle.f16_to_float(rng.uniforms_f16(-1.0, 1.0, 256))
        pes = rng.uniforms(0.8, 1.2, 128)
        idx, wts = oracle.router_reference(w, x, 8, pes)
        logits = w.astype(np.float64) @ x.astype(np.float64)
        order = np.lexsort((np.arange(128), -logits))
        if logits[order[7]] - logits[order[8]] < 1e-4:
            continue
        checked += 1
        assert list(idx) == list(order[:8])
        top = logits[order[:8]]
        e = np.exp(top - top.max())
        assert np.allclose(wts, e / e.sum() * pes[order[:8]], rtol=1e-5)
    assert checked >= 4


def test_topk_ties_go_to_lower_index_and_nonfinite_never_enter(oracle):
    logits = np.zeros(16, np.float32)
    logits[[3, 9, 12]] = 2.0      # three-way tie above the rest
    logits[5] = np.nan
    logits[6] = -np.inf
    logits[[1, 2, 4, 7, 8]] = 1.0  # five-way tie for the remaining slots
    pes = np.ones(16, np.float32)
    idx, w = oracle.topk_softmax(logits, 8, pes)
    assert list(idx) == [3, 9, 12, 1, 2, 4, 7, 8]
    wf = oracle.f16_to_float(w)
    assert wf[0] == wf[1] == wf[2] and wf[3] == wf[7]
    # all -inf: nothing enters, slots keep (0, -inf) exactly like the kernel
    idx2, _ = oracle.topk_softmax(np.full(16, -np.inf, np.float32), 8, pes)
    assert list(idx2) == [0] * 8


def test_topk_softmax_matches_router_reference_order(oracle):
    rng = oracle.SplitMix64(32)
    for _ in range(20):
        logits = rng.uniforms(-3, 3, 128)
        pes = rng.uniforms(0.8, 1.2, 128)
        i1, w1 = oracle.topk_softmax(logits, 8, pes)
        order = np.lexsort((np.arange(128), -logits.astype(np.float64)))
        assert list(i1) == list(order[:8])


def _expert_blob(oracle, rng, d, f, group, symmetric, lo=-0.125, hi=0.125):
    parts, offs, deq, cur = [], [], [], 0
    for rows, cols in ((f, d), (f, d), (d, f)):
        w = rng.uniforms(lo, hi, rows * cols).reshape(rows, cols)
        p, s, b = oracle.quantize_int4(w, group, symmetric)
        deq.append(oracle.dequantize_int4(p, s, b, cols, group).astype(np.float64))
        for arr, is_bias in ((p, False), (s, False), (b, True)):
            if is_bias and symmetric:
                offs.append(offs[-1])
                continue
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            offs.append(cur)
            parts.append(raw)
            cur += raw.size
    return np.concatenate(parts), np.array(offs, np.uint32), deq


def test_prefill_reference_within_fp16_roundings_of_fp64(oracle):
    rng = oracle.SplitMix64(33)
    d, f, group, topk, t, ne = 128, 64, 32, 2, 6, 3
    for symmetric in (True, False):
        blobs, deqs = [], []
        offs = None
        for _ in range(ne):
            b, offs, dq = _expert_blob(oracle, rng, d, f, group, symmetric)
            blobs.append(b)
            deqs.append(dq)
        hidden = rng.uniforms_f16(-1.0, 1.0, t * d)
        idx = np.array([[tok % ne, (tok + 1) % ne] for tok in range(t)], np.uint32)
        pairs = oracle.make_token_expert_pairs(idx, np.zeros(t * topk, np.uint16), t, topk)
        g = oracle.group_pairs(pairs, t, topk, ne)
        P = oracle.prefill_moe_ref(blobs, offs, hidden, d, g["sorted_pairs"], topk, d, f,
                                   group, symmetric)
        x = oracle.f16_to_float(hidden).reshape(t, d).astype(np.float64)
        for p in g["sorted_pairs"]:
            gd, ud, dd = deqs[int(p["expert"])]
            gx = gd @ x[p["token"]]
            ux = ud @ x[p["token"]]
            act = 0.5 * gx * (1 + np.tanh(0.7978845608028654 * (gx + 0.044715 * gx ** 3))) * ux
            want = dd @ act
            got = oracle.f16_to_float(P[p["token"] * topk + p["rank"]]).astype(np.float64)
            # three fp16 roundings upstream (g, u, act) and one on the output
            assert np.max(np.abs(got - want)) <= 4e-3 * np.max(np.abs(want)) + 1e-3


def test_reduce_token_major_closed_form(oracle):
    rng = oracle.SplitMix64(34)
    t, k, d = 5, 8, 64
    P = rng.uniforms_f16(-1, 1, t * k * d)
    w = rng.uniforms_f16(0, 0.3, t * k)
    h2 = oracle.reduce_token_major(P, w, t, k, d)
    Pf = oracle.f16_to_float(P).reshape(t, k, d).astype(np.float64)
    wf = oracle.f16_to_float(w).reshape(t, k).astype(np.float64)
    want = np.einsum("tk,tkd->td", wf, Pf)
    got = oracle.f16_to_float(h2)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0**-10 + 1e-6)


def _bf16(oracle, a):
    return oracle.bf16_bits(np.asarray(a, np.float32))


def test_router_canonical_order_is_exact_on_exact_inputs(oracle):
    """router_logits_canonical restates the kernels' summation order. On inputs
    whose products and partial sums are all exactly representable (small
    integers times powers of two), every order gives the fp64 sum exactly, and
    a dropped term, a wrong element or a missing effective scale shows up."""
    rng = np.random.default_rng(5)
    ne, d, rows, stride = 16, 2816, 3, 2816 + 16
    w = rng.integers(-8, 8, size=(ne, d)).astype(np.float32) * np.float32(0.25)
    x = rng.integers(-4, 5, size=(rows, stride)).astype(np.float32) * np.float32(0.5)
    es = rng.choice([0.5, 1.0, 2.0], size=d).astype(np.float32)
    got = oracle.router_logits_canonical(_bf16(oracle, w.ravel()), oracle.f16_bits(x.ravel()),
                                         stride, _bf16(oracle, es), rows, ne, d)
    want = (x[:, :d].astype(np.float64) * es) @ w.T.astype(np.float64)
    assert np.array_equal(got.astype(np.float64), want)


def test_router_canonical_within_fp32_bound(oracle):
    rng = oracle.SplitMix64(77)
    ne, d = 32, 2816
    w = rng.uniforms_bf16(-0.2, 0.2, ne * d)
    h = rng.uniforms_f16(-1.0, 1.0, d)
    es = oracle.bf16_bits(rng.uniforms(0.5, 1.5, d))
    got = oracle.router_logits_canonical(w, h, d, es, 1, ne, d)[0]
    wf = oracle.bf16_to_float(w).reshape(ne, d).astype(np.float64)
    xe = (oracle.f16_to_float(h).astype(np.float32) * oracle.bf16_to_float(es)).astype(np.float64)
    want = wf @ xe
    bound = (d + 8) * 2.0 ** -24 * (np.abs(wf) @ np.abs(xe))
    assert np.all(np.abs(got - want) <= bound)
    # and it is not the naive sequential order (the restated order matters)
    seq = np.zeros(ne, np.float32)
    for i in range(d):
        seq = (seq + wf[:, i].astype(np.float32) * xe[i].astype(np.float32)).astype(np.float32)
    assert not np.array_equal(seq, got)


def test_prefill_ref_rows_path_rounding_exact(oracle):
    """The two rounding modes of the prefill reference, pinned by exact values.
    One sym g32 expert with every scale 1.0: gate row 0 and up row 0 have
    weight 1 at k = 0, 1 (q = 9) and 0 elsewhere; down row 0 has weight 1 at
    k = 0. With x0 = 8, x1 = 2^-8: g = u = 8 + 2^-8 exactly. The tiled GEMM
    rounds both to fp16 first (8 + 2^-8 is half an ulp above 8: a tie, to
    even, 8.0), so act = 8 * 8 = 64 (tanh-GELU(8) = 8 in fp32); the rows path
    keeps them in fp32, so act = half((8 + 2^-8)^2) = 64.0625, one fp16 ulp
    above 64 (prefill.metal:1621-1628). The down row copies act."""
    d = f = 32
    q = np.full((f, d), 8, np.int64)
    q[0, 0] = q[0, 1] = 9
    qd = np.full((d, f), 8, np.int64)
    qd[0, 0] = 9

    def pack(qm):
        return (qm[:, 0::2] | (qm[:, 1::2] << 4)).astype(np.uint8)

    ones = lambda rows: np.full((rows, 1), 0x3F80, np.uint16)  # bf16 1.0
    parts = [(pack(q), ones(f), ones(f)), (pack(q), ones(f), ones(f)), (pack(qd), ones(d), ones(d))]
    from tests import kernelcheck as kc
    blob, offs = kc.pack_blob(parts, True, keep_biases=False)
    x = np.zeros(d, np.float32)
    x[0], x[1] = 8.0, 2.0 ** -8
    hidden = oracle.f16_bits(x)
    pairs = np.array([(0, 0, 0, 0x3C00)], dtype=oracle.PAIR_DTYPE)
    gemm = oracle.prefill_moe_ref([blob], offs, hidden, d, pairs, 1, d, f, 32, True)
    rows = oracle.prefill_moe_ref([blob], offs, hidden, d, pairs, 1, d, f, 32, True,
                                  rows_path=True)
    assert oracle.f16_to_float(gemm)[0, 0] == 64.0
    assert oracle.f16_to_float(rows)[0, 0] == 64.0625
    assert np.all(oracle.f16_to_float(rows)[0, 1:] == 0.0)
