"""GPU parity: int4 QMV, dequantisation, router and decode MoE phases against
the oracle, on the reference KernelCheck fixtures (main.swift:2426-2443)
regenerated bit for bit, plus the bitwise self-consistency invariants of the
reference's own tests (rows == per-row, subset == full)."""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

SCHEMES = ["affine", "sym"]
GROUPS = [64, 32]


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


def configure(ctx, group, scheme):
    ctx.set_affine_group_size(group)
    ctx.set_affine_scheme(scheme)


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,seed", [(128, 2816, 0xA1), (64, 4096, 0xA2), (128, 2112, 0xA3),
                                      (128, 704, 0xA4)])
def test_qmv_kernelcheck_cases(tsg, ctx, group, scheme, m, n, seed):
    sym = scheme == "sym"
    if n % group:
        pytest.skip("shape not a multiple of the group")
    configure(ctx, group, scheme)
    c = kc.int4_gemv_case(m, n, group, seed, sym)
    y = empty(m)
    tsg.DequantInt4GEMV(ctx).encode(dev(c["packed"]), dev(c["scales"]),
                                    dev(c["scales"] if sym else c["biases"]), dev(c["x_bits"]),
                                    y, m, n)
    got = oracle.f16_to_float(host(y, np.uint16))
    rel = oracle.relative_error(got, c["ref"])
    print(f"int4-gemv m={m} n={n} g={group} {scheme}: rel={rel:.3e}")
    assert rel <= kc.FP16_REDUCTION
    assert rel <= kc.NORTH_STAR


def test_qmv_rows_bit_identical_to_single_row(tsg, ctx):
    configure(ctx, 32, "sym")
    m, n, t = 128, 2816, 5
    c = kc.int4_gemv_case(m, n, 32, 0xA1, True)
    rng = oracle.SplitMix64(77)
    xs = rng.uniforms_f16(-1, 1, t * (n + 8)).reshape(t, n + 8)
    q = tsg.DequantInt4GEMV(ctx)
    W, S = dev(c["packed"]), dev(c["scales"])
    yr = empty(t * m)
    q.encode_rows(W, S, S, dev(xs), n + 8, yr, m, t, m, n)
    rows = host(yr, np.uint16).reshape(t, m)
    for r in range(t):
        y1 = empty(m)
        q.encode(W, S, S, dev(np.ascontiguousarray(xs[r, :n])), y1, m, n)
        assert np.array_equal(rows[r], host(y1, np.uint16)), f"row {r} differs"


@pytest.mark.parametrize("offset", [2, 4, 6, 10, 14])
@pytest.mark.parametrize("group,scheme", [(32, "sym"), (64, "affine")])
def test_qmv_weights_at_2_aligned_offset(tsg, ctx, offset, group, scheme):
    """gemv_weightsAt2AlignedNot4AlignedOffset (DequantInt4GEMVTests.swift:
    114-121): the packed weights bound at a 2-aligned but not 16-aligned byte
    offset (the resident layout, whose bf16 scale regions leave weights only
    2-aligned, DequantInt4GEMV.swift:93-96); N = 2816 so every lane loads
    whole 16-byte chunks. The result is the aligned call's bit for bit and
    within the north-star bound of the oracle, for one row and for rows."""
    import torch
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    m, n = 128, 2816
    c = kc.int4_gemv_case(m, n, group, 0xC4, sym)
    q = tsg.DequantInt4GEMV(ctx)
    S, B, X = dev(c["scales"]), dev(c["scales"] if sym else c["biases"]), dev(c["x_bits"])
    W = dev(c["packed"]).reshape(-1)
    # the same bytes at byte `offset` of a 16-byte aligned allocation, with
    # nothing past their end: the first and last chunks touch the buffer's ends
    raw = torch.zeros(offset + c["packed"].size, dtype=torch.uint8, device="cuda")
    raw[offset:] = W.view(torch.uint8)
    Wo = raw[offset:]
    y_al, y_off = empty(m), empty(m)
    q.encode(W, S, B, X, y_al, m, n)
    q.encode(Wo, S, B, X, y_off, m, n)
    a, b = host(y_al, np.uint16), host(y_off, np.uint16)
    assert np.array_equal(a, b)
    rel = oracle.relative_error(oracle.f16_to_float(b), c["ref"])
    assert rel <= kc.NORTH_STAR
    t = 3
    xs = oracle.SplitMix64(0xC4 + offset).uniforms_f16(-1, 1, t * n)
    yr_al, yr_off = empty(t * m), empty(t * m)
    q.encode_rows(W, S, B, dev(xs), n, yr_al, m, t, m, n)
    q.encode_rows(Wo, S, B, dev(xs), n, yr_off, m, t, m, n)
    assert np.array_equal(host(yr_al, np.uint16), host(yr_off, np.uint16))
    print(f"qmv weights at +{offset} g{group} {scheme}: rel={rel:.3e}")


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("scheme", SCHEMES)
def test_dequant_f16_is_bit_exact(tsg, ctx, group, scheme):
    """Dequantised weights, bit for bit: the GEMM's staging routine (fp16 fast
    path and fp32 route) and the direct kernel against the oracle's
    half(fma(q, s, b)) (prefill.metal:1021-1026). Scales span tiny (fp16
    subnormal products, scales not exact in fp16) to large."""
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    rows, n = 96, 1024
    rng = oracle.SplitMix64(0xDE)
    w = rng.uniforms(-0.5, 0.5, rows * n).reshape(rows, n)
    w *= np.exp2(np.linspace(-22, 6, rows, dtype=np.float32))[:, None]
    packed, scales, biases = oracle.quantize_int4(w, group, sym)
    want = oracle.dequantize_int4_f16(packed, scales, biases, n, group, sym)
    q = tsg.DequantInt4GEMV(ctx)
    for gemm_path in (False, True):
        out = empty(rows * n)
        q.debug_dequant_f16(dev(packed), dev(scales), dev(scales if sym else biases), out, rows,
                            n, gemm_path=gemm_path)
        got = host(out, np.uint16).reshape(rows, n)
        bad = np.argwhere(got != want)
        assert bad.size == 0, f"gemm_path={gemm_path}: {len(bad)} mismatches, first {bad[:3]}"


@pytest.mark.parametrize("group", GROUPS)
def test_affine_dequant_rounds_through_fp32(tsg, ctx, group):
    """half(fma(q, s, b)) rounds twice, to fp32 then to fp16. With s of an odd
    8-bit significand (e.g. 1.9921875) and q = 15, q * s needs 12 bits and
    sits on an fp16 midpoint; a bias of +-2^-30 moves the exact sum off the
    midpoint but not its fp32 rounding, so the fp16 tie breaks to even, where
    a single rounding of the exact sum would not."""
    configure(ctx, group, "affine")
    rows, n = 16, 256
    rng = np.random.default_rng(0xDF)
    packed = rng.integers(0, 256, (rows, n // 2), dtype=np.uint8)
    packed[:, ::4] = 0xFF  # q = 15 in both nibbles
    odd = np.array([0x3FFF, 0x3F81, 0x3FC1, 0x4081, 0xBFFF, 0x3E7F], np.uint16)
    tiny = np.array([0x3080, 0xB080, 0x2F80, 0x0001], np.uint16)  # +-2^-30, 2^-32, bf16 subnormal
    scales = odd[rng.integers(0, odd.size, (rows, n // group))]
    biases = tiny[rng.integers(0, tiny.size, (rows, n // group))]
    want = oracle.dequantize_int4_f16(packed, scales, biases, n, group, False)
    # the constructed ties: the oracle's value differs from a single rounding
    q4 = np.stack([packed & 15, packed >> 4], axis=-1).reshape(rows, n).astype(np.float64)
    exact = (q4 * np.repeat(oracle.bf16_to_float(scales).astype(np.float64), group, axis=1) +
             np.repeat(oracle.bf16_to_float(biases).astype(np.float64), group, axis=1))
    single = exact.astype(np.float16).view(np.uint16)  # one rounding of the exact sum
    assert 0 < (single != want).sum() < want.size // 8
    q = tsg.DequantInt4GEMV(ctx)
    for gemm_path in (False, True):
        out = empty(rows * n)
        q.debug_dequant_f16(dev(packed), dev(scales), dev(biases), out, rows, n,
                            gemm_path=gemm_path)
        got = host(out, np.uint16).reshape(rows, n)
        bad = np.argwhere(got != want)
        assert bad.size == 0, f"gemm_path={gemm_path}: {len(bad)} mismatches, first {bad[:3]}"


@pytest.mark.parametrize("group", GROUPS)
def test_router_kernelcheck_and_canonical_order(tsg, ctx, group):
    """checkRouter(16) cases (main.swift:409-517, seed 0xD2, 4 draws): indices
    equal routerReference's; weights within fp16Reduction; logits bit-equal to
    the oracle's restatement of the kernel order, and the selection bit-equal
    to the kernel rule applied to those logits."""
    configure(ctx, group, "sym")
    d, ne = 2816, 128
    moe = tsg.MoE(ctx)
    for draw in range(4):
        c = kc.router_case(d, ne, group, 0xD2, draw)
        W, H, ES, PES = dev(c["w_bits"]), dev(c["hidden"]), dev(c["es_bits"]), dev(c["pes_bits"])
        idx, wts = empty(8, np.uint32), empty(8)
        moe.encode_router_gemma4_bf16(W, H, ES, PES, idx, wts, ne, d)
        gi = host(idx, np.uint32)
        gw = oracle.f16_to_float(host(wts, np.uint16))
        assert list(gi) == list(c["idx"]), f"draw {draw}: gpu={gi} cpu={c['idx']}"
        assert oracle.relative_error(gw, c["wts"]) <= kc.FP16_REDUCTION
        logits = empty(ne, np.float32)
        moe.encode_router_logits_bf16(W, H, ES, logits, ne, d)
        canon = oracle.router_logits_canonical(c["w_bits"], c["hidden"], d, c["es_bits"], 1, ne, d)
        assert np.array_equal(host(logits, np.uint32), canon.view(np.uint32).ravel())
        ci, cw = oracle.topk_softmax(canon[0], 8, oracle.bf16_to_float(c["pes_bits"]))
        assert list(gi) == list(ci)
        assert np.max(np.abs(host(wts, np.uint16).astype(np.int32) - cw.astype(np.int32))) <= 1


def test_router_rows_bit_identical_to_single(tsg, ctx):
    configure(ctx, 32, "sym")
    d, ne, rows = 2816, 128, 5
    moe = tsg.MoE(ctx)
    c = kc.router_case(d, ne, 32, 0xD2, 0)
    rng = oracle.SplitMix64(5)
    stride = d + 16
    hid = rng.uniforms_f16(-1, 1, rows * stride)
    W, ES, PES = dev(c["w_bits"]), dev(c["es_bits"]), dev(c["pes_bits"])
    idx, wts = empty(8 * rows, np.uint32), empty(8 * rows)
    moe.encode_router_gemma4_bf16_rows(W, dev(hid), stride, ES, PES, idx, wts, rows, ne, d)
    gi, gw = host(idx, np.uint32).reshape(rows, 8), host(wts, np.uint16).reshape(rows, 8)
    for r in range(rows):
        i1, w1 = empty(8, np.uint32), empty(8)
        moe.encode_router_gemma4_bf16(W, dev(np.ascontiguousarray(hid[r * stride:r * stride + d])),
                                      ES, PES, i1, w1, ne, d)
        assert np.array_equal(gi[r], host(i1, np.uint32))
        assert np.array_equal(gw[r], host(w1, np.uint16))
    with pytest.raises(tsg.TsgError) as e:
        moe.encode_router_gemma4_bf16_rows(W, dev(hid), stride, ES, PES, idx, wts, 9, ne, d)
    assert e.value.status == 4  # declined, like the reference's `false`


def _tie_router(kind):
    """Router rows for the tie cases at the reference's shape (16 experts,
    D = 128; RouterTopKTests.swift:46-68): row e = pattern * gain_e in bf16,
    hidden uniform(0.5, 1.5), effective and per-expert scales 1.
    'exact': the reference's gains 0.5 and 0.5 * (1 + 1e-4) for experts 7
    and 8, their bf16 rows made identical (the two gains' rows round to bf16
    differently in a few places), so 7 and 8 tie exactly and the lower index
    wins.
    'near': expert 8 = expert 7 with one element one bf16 ulp larger, where
    hidden is smallest: the logits differ by about 1e-5 relative.
    'all': every row identical, so the top 8 are experts 0..7."""
    ne, d = 16, 128
    rng = oracle.SplitMix64(0x71E0F4A)
    pattern = rng.uniforms(0.2, 1.0, d)
    hidden = rng.uniforms_f16(0.5, 1.5, d)
    gains = np.zeros(ne, np.float32)
    for e in range(7):
        gains[e] = 1.0 - e * 0.05
    gains[7] = 0.5
    gains[8] = 0.5 * (1.0 + 1e-4)
    for e in range(9, ne):
        gains[e] = 0.4 - (e - 9) * 0.02
    if kind == "all":
        gains[:] = 0.7
    w = oracle.bf16_bits((pattern[None, :] * gains[:, None]).astype(np.float32))
    if kind in ("exact", "near"):
        w[8] = w[7]  # bf16 rounding of the two gains' rows can differ in places
    if kind == "near":
        w[8, int(np.argmin(oracle.f16_to_float(hidden)))] += 1
    return w.ravel(), hidden, ne, d


@pytest.mark.parametrize("kind", ["exact", "near", "all"])
def test_router_ties_on_gpu(tsg, ctx, kind):
    """Exact and near ties in bf16 router logits (RouterTopKTests.swift:46-68,
    the bf16 form of its int8 case): the router kernel and the one-launch
    decode layer's top-8 both select what the kernel rule (descending, ties
    to the lower index) gives on the canonical-order logits, and on an exact
    tie that is the lower expert. Reported: the fp64 8th/9th margin."""
    configure(ctx, 32, "sym")
    w_bits, hidden, ne, d = _tie_router(kind)
    es = oracle.bf16_bits(np.ones(d, np.float32))
    pes = oracle.bf16_bits(np.ones(ne, np.float32))
    canon = oracle.router_logits_canonical(w_bits, hidden, d, es, 1, ne, d)
    ci, cw = oracle.topk_softmax(canon[0], 8, np.ones(ne, np.float32))
    if kind == "exact":
        assert canon[0][7] == canon[0][8]
        assert list(ci) == list(range(8))
    if kind == "all":
        assert list(ci) == list(range(8))
    l64 = oracle.bf16_to_float(w_bits).reshape(ne, d).astype(np.float64) @ \
        oracle.f16_to_float(hidden).astype(np.float64)
    srt = np.sort(l64)[::-1]
    print(f"router tie '{kind}': fp64 8th/9th margin {srt[7] - srt[8]:.3e}, selected {list(ci)}")
    moe = tsg.MoE(ctx)
    W, X, ES, PES = dev(w_bits), dev(hidden), dev(es), dev(pes)
    idx, wts = empty(8, np.uint32), empty(8)
    moe.encode_router_gemma4_bf16(W, X, ES, PES, idx, wts, ne, d)
    assert list(host(idx, np.uint32)) == list(ci)
    # the staged rows router and its grouped form (candidate top-8 per row):
    # three copies of the row give the one-row call's indices and weights
    m = 3
    Xr = dev(np.tile(hidden, m))
    ri, rw_ = empty(8 * m, np.uint32), empty(8 * m)
    moe.encode_router_gemma4_bf16_rows(W, Xr, d, ES, PES, ri, rw_, m, ne, d)
    gi, gw = empty(8 * m, np.uint32), empty(8 * m)
    sp, off, cnt = empty(8 * m * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    bl, nb = empty(8 * m * 4, np.uint32), empty(1, np.uint32)
    moe.encode_router_gemma4_bf16_rows_grouped(W, Xr, d, ES, PES, gi, gw, m, ne, d, sp, off,
                                               cnt, bl, 8 * m, nb)
    ctx.synchronize()
    for got_i, got_w in ((ri, rw_), (gi, gw)):
        assert list(host(got_i, np.uint32)) == list(ci) * m
        assert np.array_equal(host(got_w, np.uint16), np.tile(host(wts, np.uint16), m))
    assert int(host(nb, np.uint32)[0]) == 8
    assert list(host(cnt, np.uint32)[list(ci)]) == [m] * 8
    # the one-launch layer's own top-8 (random experts of d = 128, f = 64)
    f = 64
    rng = oracle.SplitMix64(0x7E)
    parts = [[oracle.quantize_int4(rng.uniforms(-0.3, 0.3, r * c_).reshape(r, c_), 32, True)
              for (r, c_) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
    image, stride, offs, _ = kc.layer_image(parts, True, keep_biases=False)
    layer = tsg.ResidentLayer(ctx, ne, stride, offs)
    layer.upload(image)
    for fused in (True, False):
        moe.set_fused_decode(fused)
        y, li, lw, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
        moe.encode_decode_layer(layer, W, X, ES, PES, X, X, y, li, lw, acts, ne, d, f)
        ctx.synchronize()
        assert list(host(li, np.uint32)) == list(ci), f"fused={fused}"
        assert np.array_equal(host(lw, np.uint16), host(wts, np.uint16))
    moe.set_fused_decode(True)


def _routed_blobs(case):
    return [dev(b) for b in case["blobs"]]


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("scheme", SCHEMES)
def test_routed_moe_kernelcheck(tsg, ctx, group, scheme):
    """checkRoutedMoE (main.swift:194-303, seed 0xB1): phase 1 + phase 2 at the
    production decode shapes against MoeRef.applyStreamedRouted."""
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    d, f = 2816, 704
    c = kc.routed_moe_case(d, f, group, 0xB1, sym)
    moe = tsg.MoE(ctx)
    blobs = _routed_blobs(c)
    acts, y = empty(8 * f), empty(d)
    moe.encode_routed_phase1(blobs, c["offsets"], dev(c["x_bits"]), acts, d, f)
    moe.encode_routed_phase2(blobs, c["offsets"], acts, dev(c["w_bits"]), dev(c["res_bits"]), y,
                             d, f)
    got = oracle.f16_to_float(host(y, np.uint16))
    rel = oracle.relative_error(got, c["ref"])
    print(f"routed-moe d={d} f={f} g={group} {scheme}: rel={rel:.3e}")
    assert rel <= kc.FP16_CHAINED
    assert rel <= kc.NORTH_STAR


def test_phase1_subset_matches_full_bitwise(tsg, ctx):
    """MoEFusedFFNTests.swift: hit/miss-subset phase 1 == full phase 1."""
    configure(ctx, 32, "sym")
    d, f = 2816, 704
    c = kc.routed_moe_case(d, f, 32, 0xB1, True)
    moe = tsg.MoE(ctx)
    blobs = _routed_blobs(c)
    full = empty(8 * f)
    moe.encode_routed_phase1(blobs, c["offsets"], dev(c["x_bits"]), full, d, f)
    sub = empty(8 * f, fill=0)
    active = np.array([6, 1, 3], np.uint32)
    moe.encode_routed_phase1_subset(blobs, c["offsets"], dev(c["x_bits"]), sub, dev(active), 3,
                                    d, f)
    a, b = host(full, np.uint16).reshape(8, f), host(sub, np.uint16).reshape(8, f)
    for s in active:
        assert np.array_equal(a[s], b[s])
    for s in set(range(8)) - set(active.tolist()):
        assert np.all(b[s] == 0)


def test_decode_preconditions_fail_loudly(tsg, ctx):
    configure(ctx, 32, "sym")
    moe = tsg.MoE(ctx)
    c = kc.routed_moe_case(256, 64, 32, 0x1, True)
    blobs = _routed_blobs(c)
    with pytest.raises(tsg.TsgError) as e:
        moe.encode_routed_phase1(blobs, c["offsets"], dev(c["x_bits"]), empty(8 * 64), 256, 64,
                                 top_k=4)
    assert e.value.status == 1
    with pytest.raises(tsg.TsgError) as e:
        moe.encode_routed_phase1(blobs, c["offsets"], dev(c["x_bits"]), empty(8 * 64), 250, 64)
    assert e.value.status == 1


# ---------------------------------------------------------------- config 2

GEMMA = dict(d=2816, f=704, ne=128, group=32)


def gemma_offsets(d=2816, f=704, group=32):
    """Sym g32 expert blob: gate W, gate S, up W, up S, down W, down S; the
    bias offsets alias the scales (ModelExpertIO.swift:69-84)."""
    gw = f * d // 2
    gs = f * (d // group) * 2
    dw = d * f // 2
    ds = d * (f // group) * 2
    o_gw, o_gs = 0, gw
    o_uw, o_us = gw + gs, 2 * gw + gs
    o_dw, o_ds = 2 * (gw + gs), 2 * (gw + gs) + dw
    payload = o_ds + ds
    stride = (payload + 16383) // 16384 * 16384
    return [o_gw, o_gs, o_gs, o_uw, o_us, o_us, o_dw, o_ds, o_ds], payload, stride


def make_gemma_layer(tsg, ctx, seed, ne=128, d=2816, f=704):
    """Nibbles uniform in [0, 15]; scales bf16(|N(0, 0.02)| / 7)."""
    import torch
    offs, payload, stride = gemma_offsets(d, f)
    buf = torch.empty(ne * stride, dtype=torch.uint8, device="cuda")
    tsg.generators.bytes(buf, seed)
    scale_regions = [(offs[1], f * (d // 32)), (offs[4], f * (d // 32)), (offs[7], d * (f // 32))]
    for e in range(ne):
        for j, (o, n) in enumerate(scale_regions):
            region = buf[e * stride + o:e * stride + o + 2 * n].view(torch.int16)
            tsg.generators.bf16_normal(region, seed * 1000 + e * 3 + j + 1, 0.02, True, 7.0)
    layer = tsg.ResidentLayer(ctx, ne, stride, offs, device_tensor=buf)
    return layer, buf, offs, stride


def test_fresh_context_ignores_earlier_contexts_handoff_words(tsg):
    """A context's first one-launch layers must not take hand-off words left in
    recycled device memory by an earlier context (their tags repeat: every
    context's epoch starts at 0). Contexts are made and dropped in turn, each
    running the fused layer on different inputs, and every launch must equal
    the three-launch form bit for bit."""
    import torch
    d, f, ne = 1024, 512, 64
    outs = []
    for round_ in range(3):
        c = tsg.Context(0, group_size=32, scheme="sym")
        layer, _, _, _ = make_gemma_layer(tsg, c, 0x5EED, ne=ne, d=d, f=f)
        rw = torch.empty(ne * d, dtype=torch.int16, device="cuda")
        tsg.generators.bf16_normal(rw, 0xB00 + round_, 1.0 / np.sqrt(d))
        ones_d = dev(np.full(d, 0x3F80, np.uint16))
        ones_e = dev(np.full(ne, 0x3F80, np.uint16))
        for k in range(3):
            x = torch.empty(d, dtype=torch.int16, device="cuda")
            tsg.generators.f16_normal(x, 0xC00 + 16 * round_ + k, 1.0)
            ys = []
            for fused in (True, False):
                moe = tsg.MoE(c)
                moe.set_fused_decode(fused)
                y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
                moe.encode_decode_layer(layer, rw, x, ones_d, ones_e, x, x, y, idx, wts, acts, ne,
                                        d, f)
                c.synchronize()
                ys.append(host(y, np.uint16))
            assert np.array_equal(ys[0], ys[1]), f"context {round_}, launch {k}"
            outs.append(ys[0])
        layer.close()
        c.close()
    assert len({o.tobytes() for o in outs}) == len(outs)


def test_resident_decode_layer_gemma_shape(tsg, ctx):
    """One Gemma-4-26B-A4B-shaped decode MoE layer (config 2): router over
    128 bf16 rows -> top-8 -> gate/up + GeGLU -> down + combine, all device
    side. Routing bit-exact against the oracle (kernel-order logits + the
    kernel's top-k rule); y within 1e-3 of MoeRef.applyStreamedRouted over the
    chosen experts."""
    import torch
    configure(ctx, 32, "sym")
    d, f, ne = GEMMA["d"], GEMMA["f"], GEMMA["ne"]
    layer, buf, offs, stride = make_gemma_layer(tsg, ctx, 0x5EED)
    rw = torch.empty(ne * d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(rw, 0xA11, 1.0 / np.sqrt(d))
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0xA12, 1.0)
    ones_d = dev(np.full(d, 0x3F80, np.uint16))
    ones_e = dev(np.full(ne, 0x3F80, np.uint16))
    moe = tsg.MoE(ctx)
    y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
    moe.encode_decode_layer(layer, rw, x, ones_d, ones_e, x, x, y, idx, wts, acts, ne, d, f)
    ctx.synchronize()  # reports a one-launch hand-off timeout
    gi, gw = host(idx, np.uint32), host(wts, np.uint16)
    xb, rwb = host(x, np.uint16), host(rw, np.uint16)
    canon = oracle.router_logits_canonical(rwb, xb, d, np.full(d, 0x3F80, np.uint16), 1, ne, d)
    ci, cw = oracle.topk_softmax(canon[0], 8, np.ones(ne, np.float32))
    assert list(gi) == list(ci)
    assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1
    image = host(buf, np.uint8)
    blobs = [np.ascontiguousarray(image[e * stride:(e + 1) * stride]) for e in gi]
    xf = oracle.f16_to_float(xb)
    ref = oracle.moe_apply_streamed_routed(blobs, np.array(offs, np.uint32), xf, xf,
                                           oracle.f16_to_float(gw), d, f, 32, symmetric=True)
    rel = oracle.relative_error(oracle.f16_to_float(host(y, np.uint16)), ref)
    print(f"decode layer gemma: experts={list(gi)} rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


def layer_offsets(d, f, group, symmetric):
    """Expert blob gate(W,S,[B]), up(W,S,[B]), down(W,S,[B]) at a 16 KiB
    stride; without biases the bias offsets alias the scales."""
    regions = []
    cur = 0
    for rows, k in ((f, d), (f, d), (d, f)):
        w = cur
        cur += rows * k // 2
        s = cur
        cur += rows * (k // group) * 2
        if symmetric:
            b = s
        else:
            b = cur
            cur += rows * (k // group) * 2
        regions += [w, s, b]
    stride = (cur + 16383) // 16384 * 16384
    return regions, stride


def make_layer(tsg, ctx, seed, ne, d, f, group, symmetric):
    import torch
    offs, stride = layer_offsets(d, f, group, symmetric)
    buf = torch.empty(ne * stride, dtype=torch.uint8, device="cuda")
    tsg.generators.bytes(buf, seed)
    dims = ((f, d), (f, d), (d, f))
    for e in range(ne):
        for m, (rows, k) in enumerate(dims):
            n = rows * (k // group)
            s_off, b_off = offs[3 * m + 1], offs[3 * m + 2]
            sreg = buf[e * stride + s_off:e * stride + s_off + 2 * n].view(torch.int16)
            tsg.generators.bf16_normal(sreg, seed * 1000 + e * 7 + 2 * m + 1, 0.02, True, 7.0)
            if not symmetric:
                breg = buf[e * stride + b_off:e * stride + b_off + 2 * n].view(torch.int16)
                tsg.generators.bf16_normal(breg, seed * 1000 + e * 7 + 2 * m + 2, 0.01)
    layer = tsg.ResidentLayer(ctx, ne, stride, offs, device_tensor=buf)
    return layer, buf, offs, stride


@pytest.mark.gpu
@pytest.mark.parametrize("d,f,ne,group,scheme,act", [
    (2816, 704, 128, 32, "sym", "gelu"),
    (2048, 512, 256, 32, "sym", "silu"),
    (2048, 512, 256, 64, "affine", "silu"),
    (1024, 512, 64, 64, "affine", "silu"),
    (768, 256, 32, 32, "affine", "gelu"),
])
def test_fused_decode_layer_matches_three_launches(tsg, ctx, d, f, ne, group, scheme, act):
    """The one-launch decode layer (router, top-8, gate/up, down and combine
    separated by in-kernel grid barriers) gives the same bits as the
    three-launch sequence, and both match the oracle (routing bit-exact on the
    kernel's logit order, y within 1e-3 of MoeRef.applyStreamedRouted)."""
    import torch
    configure(ctx, group, scheme)
    sym = scheme == "sym"
    layer, buf, offs, stride = make_layer(tsg, ctx, 0x1234 + d, ne, d, f, group, sym)
    rw = torch.empty(ne * d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(rw, 0xB11 + d, 1.0 / np.sqrt(d))
    es = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(es, 0xB13, 0.1)
    es_h = (host(es, np.uint16).astype(np.uint32) << 16).view(np.float32)
    es_bits = oracle.bf16_bits(np.float32(1.0) + np.abs(es_h))
    pes_bits = oracle.bf16_bits(np.linspace(0.8, 1.2, ne).astype(np.float32))
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0xB12 + d, 1.0)
    res = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(res, 0xB14 + d, 0.5)
    moe = tsg.MoE(ctx, gate_activation=act)
    outs = {}
    for fused in (True, False):
        moe.set_fused_decode(fused)
        y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
        moe.encode_decode_layer(layer, rw, x, dev(es_bits), dev(pes_bits), x, res, y, idx, wts,
                                acts, ne, d, f)
        ctx.synchronize()  # raises if the fused launch's grid barrier timed out
        outs[fused] = [host(t, np.uint16 if t is not idx else np.uint32)
                       for t in (y, idx, wts, acts)]
    for a, b in zip(outs[True], outs[False]):
        assert np.array_equal(a, b)
    y, gi, gw, _ = outs[True]
    xb, rwb = host(x, np.uint16), host(rw, np.uint16)
    canon = oracle.router_logits_canonical(rwb, xb, d, es_bits, 1, ne, d)
    ci, cw = oracle.topk_softmax(canon[0], 8, oracle.bf16_to_float(pes_bits))
    assert list(gi) == list(ci)
    assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1
    image = host(buf, np.uint8)
    blobs = [np.ascontiguousarray(image[e * stride:(e + 1) * stride]) for e in gi]
    ref = oracle.moe_apply_streamed_routed(
        blobs, np.array(offs, np.uint32), oracle.f16_to_float(xb),
        oracle.f16_to_float(host(res, np.uint16)), oracle.f16_to_float(gw), d, f, group,
        symmetric=sym, act=1 if act == "silu" else 0)
    rel = oracle.relative_error(oracle.f16_to_float(y), ref)
    print(f"fused decode d={d} f={f} ne={ne} g{group} {scheme} {act}: rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


@pytest.mark.gpu
@pytest.mark.parametrize("d,f,ne,sf,group,scheme", [
    (2048, 512, 256, 512, 32, "sym"),     # the Qwen3.5-MoE-35B-A3B shape
    (1024, 512, 64, 256, 64, "affine"),
    (1024, 256, 64, 1024, 32, "sym"),     # shared_f > 512: the two-step form
    (2816, 704, 128, 512, 32, "sym"),     # d > 2048: the default chunk batches
])
def test_decode_layer_shared_expert(tsg, ctx, d, f, ne, sf, group, scheme):
    """The Qwen-family layer (QwenForwardRunner.swift:1548-1608): one call gives
    the same bits as tsg_moe_shared_expert followed by the decode layer with
    residual = the shared output, in the one-launch and three-launch forms,
    and y is within 1e-3 of the oracle's shared branch + MoeRef."""
    import torch
    configure(ctx, group, scheme)
    sym = scheme == "sym"
    layer, buf, offs, stride = make_layer(tsg, ctx, 0x5A5 + d, ne, d, f, group, sym)
    rw = torch.empty(ne * d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(rw, 0xC11 + d, 1.0 / np.sqrt(d))
    ones_d = dev(oracle.bf16_bits(np.ones(d, np.float32)))
    pes_bits = oracle.bf16_bits(np.ones(ne, np.float32))
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0xC12 + d, 1.0)
    c = kc.shared_expert_case(d, sf, group, 0xC13 + d, sym)
    sblob, sgw = dev(c["blob"]), dev(c["gate_w"])
    moe = tsg.MoE(ctx, gate_activation="silu")
    outs = {}
    for fused in (True, False):
        moe.set_fused_decode(fused)
        y, idx, wts, acts, sacts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f), empty(sf)
        print(f"shared decode d={d} f={f} ne={ne} sf={sf} fused={fused}", flush=True)
        moe.encode_decode_layer_shared(layer, rw, x, ones_d, dev(pes_bits), x, y, idx, wts, acts,
                                       sblob, c["offsets"], sgw, sacts, ne, d, f, sf)
        ctx.synchronize()
        outs[fused] = [host(t, np.uint16 if t is not idx else np.uint32)
                       for t in (y, idx, wts, acts, sacts)]
    # the explicit two-call sequence
    so, sa2 = empty(d), empty(sf)
    tsg.encode_shared_expert(moe, sblob, c["offsets"], x, sgw, sa2, so, d, sf)
    moe.set_fused_decode(True)
    y2, idx2, wts2, acts2 = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
    moe.encode_decode_layer(layer, rw, x, ones_d, dev(pes_bits), x, so, y2, idx2, wts2, acts2,
                            ne, d, f)
    seq = [host(t, np.uint16 if t is not idx2 else np.uint32) for t in (y2, idx2, wts2, acts2, sa2)]
    for a_, b_, c_ in zip(outs[True], outs[False], seq):
        assert np.array_equal(a_, b_)
        assert np.array_equal(a_, c_)
    y, gi, gw, _, _ = outs[True]
    image = host(buf, np.uint8)
    blobs = [np.ascontiguousarray(image[e * stride:(e + 1) * stride]) for e in gi]
    xb = host(x, np.uint16)
    shared_ref = oracle.shared_expert(c["blob"], c["offsets"], xb, c["gate_w"], d, sf, group, sym)
    ref = oracle.moe_apply_streamed_routed(
        blobs, np.array(offs, np.uint32), oracle.f16_to_float(xb),
        oracle.f16_to_float(shared_ref), oracle.f16_to_float(gw), d, f, group, symmetric=sym, act=1)
    rel = oracle.relative_error(oracle.f16_to_float(y), ref)
    print(f"  rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


@pytest.mark.gpu
@pytest.mark.parametrize("m,n", [(704, 2816), (4096, 2816), (2048, 2816), (2816, 4096),
                                 (8192, 2816), (1024, 2816), (2816, 8192)])
def test_qmv_projection_shapes(tsg, ctx, m, n):
    """DequantInt4GEMV's decode projection shapes (DequantInt4GEMV.swift:13-20)
    and the single QMV of the benchmark's first configuration (W[704 x 2816],
    symmetric group 32, scales |N(0, 0.02)| / 7, x ~ N(0, 1)): encode against
    DequantInt4GemvRef within the north star's 1e-3, and 8 rows
    through encodeRows / encodeRowsWide (split into launches that fit the LDS
    at n = 8192) bit-equal to 8 single-row calls."""
    configure(ctx, 32, "sym")
    rng = np.random.default_rng(m * 7 + n)
    packed = rng.integers(0, 256, (m, n // 2), dtype=np.uint8)
    scales = oracle.bf16_bits((np.abs(rng.normal(0, 0.02, m * (n // 32))) / 7).astype(np.float32))
    xs = oracle.f16_bits(rng.normal(0, 1.0, 8 * n).astype(np.float32)).reshape(8, n)
    W, S = dev(packed), dev(scales)
    q = tsg.DequantInt4GEMV(ctx)
    y = empty(m)
    print(f"qmv shape m={m} n={n}", flush=True)
    q.encode(W, S, S, dev(np.ascontiguousarray(xs[0])), y, m, n)
    ref = oracle.dequant_int4_gemv_ref(packed, scales, None, oracle.f16_to_float(xs[0]), n, 32)
    rel = oracle.relative_error(oracle.f16_to_float(host(y, np.uint16)), ref)
    print(f"  rel={rel:.3e}", flush=True)
    assert rel <= kc.NORTH_STAR
    yr = empty(8 * m)
    q.encode_rows_wide(W, S, S, dev(xs), n, yr, m, 8, m, n)
    rows = host(yr, np.uint16).reshape(8, m)
    for r in (0, 3, 7):
        y1 = empty(m)
        q.encode(W, S, S, dev(np.ascontiguousarray(xs[r])), y1, m, n)
        assert np.array_equal(rows[r], host(y1, np.uint16)), f"row {r}"
