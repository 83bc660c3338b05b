"""GPU parity: prompt router, device grouping, grouped int4 GEMMs (gate/up +
GeGLU, down + scatter), verify rows path and the token-major reduce, against
the oracle on the reference KernelCheck fixtures and bitwise invariants."""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests import workloads as wl
from tests.gpu_util import dev, empty, f16_fill_bits, host

NAN16 = f16_fill_bits(float("nan"))

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("t,kind,seed", [(131, "row", 0xD3), (131, "gemm", 0xD3),
                                         (32, "gemm", 0xD4), (7, "gemm", 0xD5)])
def test_prefill_router_kernelcheck(tsg, ctx, t, kind, seed):
    """checkPrefillRouterBF16 (main.swift:525-612): every row's top-8 equals
    routerReference; weights within fp16Reduction; logits in the decode
    kernel's order (one row == the decode router on that row)."""
    configure(ctx, 32, "sym")
    d, ne = 2816, 128
    c = kc.prefill_router_case(t, d, ne, kind, 32, seed)
    moe = tsg.MoE(ctx)
    idx, w = empty(t * 8, np.uint32), empty(t * 8)
    tsg.PrefillRouter(moe).encode_gemma4_bf16(dev(c["w_bits"]), dev(c["hidden"]), c["stride"],
                                              dev(c["es_bits"]), dev(c["pes_bits"]), idx, w, t,
                                              ne, d)
    gi = host(idx, np.uint32).reshape(t, 8)
    gw = oracle.f16_to_float(host(w, np.uint16)).reshape(t, 8)
    canon = oracle.router_logits_canonical(c["w_bits"], c["hidden"], c["stride"], c["es_bits"],
                                           t, ne, d)
    pes = oracle.bf16_to_float(c["pes_bits"])
    worst = 0.0
    for row in range(t):
        ri, rw = c["refs"][row]
        assert list(gi[row]) == list(ri), f"row {row}: gpu={gi[row]} cpu={ri}"
        ci, _ = oracle.topk_softmax(canon[row], 8, pes)
        assert list(gi[row]) == list(ci)
        worst = max(worst, oracle.relative_error(gw[row], rw))
    assert worst <= kc.FP16_REDUCTION


def _upload_layer(tsg, ctx, expert_parts, symmetric):
    image, stride, offs, blobs = kc.layer_image(expert_parts, symmetric, keep_biases=not symmetric)
    layer = tsg.ResidentLayer(ctx, len(expert_parts), stride, offs)
    layer.upload(image)
    return layer, offs, blobs


@pytest.mark.parametrize("group", [64, 32])
@pytest.mark.parametrize("scheme", ["affine", "sym"])
def test_prefill_moe_gemm_kernelcheck(tsg, ctx, group, scheme):
    """checkPrefillRoutedMoEGEMM (PrefillMoEGEMMCheck.swift:92-353, seed 0xF7):
    gate/up GEMM + GeGLU then down GEMM scattered to route_partials, against
    the expert-major CPU reference with the GPU's fp16 roundings. Partials
    start as NaN (the reference uses -7.0, PrefillMoEGEMMCheck.swift:234-235,
    which is a reachable fp16 output here) so a skipped store scores inf."""
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    c = kc.prefill_moe_gemm_case(group, 0xF7, sym)
    d, f, T, K = c["d"], c["f"], c["tokens"], c["top_k"]
    layer, offs, blobs = _upload_layer(tsg, ctx, c["experts"], sym)
    expected = oracle.prefill_moe_ref(blobs, offs, c["hidden"], d, c["pairs"], K, d, f, group,
                                      sym)
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    rows = c["pairs"].size
    act = empty(rows * f)
    partials = empty(T * K * d, fill=f16_fill_bits(float("nan")))
    P, B = dev(c["pairs"]), dev(c["blocks"])
    g.encode_gate_up(layer, dev(c["hidden"]), d, P, B, c["blocks"].size, act, d, f)
    g.encode_down(layer, act, P, B, c["blocks"].size, partials, K, d, f)
    # the fused persistent launch gives the two launches' bits
    act1 = empty(rows * f)
    partials1 = empty(T * K * d, fill=f16_fill_bits(float("nan")))
    g.encode_gate_up_down(layer, dev(c["hidden"]), d, P, B, c["blocks"].size, act1, partials1, K,
                          d, f)
    ctx.synchronize()
    assert np.array_equal(host(act1, np.uint16), host(act, np.uint16))
    assert np.array_equal(host(partials1, np.uint16), host(partials, np.uint16))
    got = oracle.f16_to_float(host(partials, np.uint16))
    exp = oracle.f16_to_float(expected).ravel()
    assert not np.any(np.isnan(got)), "a route partial was never written"
    rel = oracle.relative_error(got, exp)
    print(f"prefill-moe-gemm g={group} {scheme}: rel={rel:.3e} rows={rows} "
          f"blocks={c['blocks'].size}")
    assert rel <= kc.FP16_CHAINED
    assert rel <= kc.NORTH_STAR


def _zipf_routing(rng, t, ne, k, s):
    """Gumbel-top-k over log p_e, p ~ rank^-s on a permutation of the ids."""
    perm = rng.permutation(ne)
    logp = -s * np.log(np.arange(1, ne + 1, dtype=np.float64))
    logp = logp[np.argsort(perm)]
    g = -np.log(-np.log(rng.random((t, ne))))
    scores = logp[None, :] + g
    idx = np.argsort(-scores, axis=1, kind="stable")[:, :k].astype(np.uint32)
    top = np.take_along_axis(scores, idx.astype(np.int64), axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, oracle.f16_bits(w).reshape(t, k)


@pytest.mark.parametrize("t,ne,k,s,tile", [(2048, 128, 8, 1.1, 64), (2048, 128, 8, 1.1, 128),
                                           (2048, 128, 8, 1.1, 256),
                                           (301, 256, 8, 1.0, 64), (5, 128, 8, 1.1, 128),
                                           (64, 16, 4, 0.5, 32), (4096, 256, 8, 1.0, 128),
                                           (3001, 128, 3, 1.1, 256)])
def test_device_grouping_matches_host_sort(tsg, ctx, t, ne, k, s, tile):
    """The on-device counting sort yields exactly groupTokenExpertPairs'
    permutation (PrefillMoEGrouping.swift:141-150), offsets and counts; the
    block list covers every pair once in <= tile-row slices of one expert."""
    rng = np.random.default_rng(t * 7 + ne)
    idx, w = _zipf_routing(rng, t, ne, k, s)
    pairs = oracle.make_token_expert_pairs(idx, w, t, k)
    want = oracle.group_pairs(pairs, t, k, ne)
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    max_blocks = t * k // tile + ne + 1
    sp, off, cnt = empty(t * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(dev(idx), dev(w), t, k, ne, sp, off, cnt, blocks, max_blocks, nb, scratch,
                         tile_rows=tile)
    got = host(sp, np.uint32).view(oracle.PAIR_DTYPE)
    assert np.array_equal(got, want["sorted_pairs"])
    assert np.array_equal(host(off, np.uint32), want["offsets"])
    assert np.array_equal(host(cnt, np.uint32), want["counts"])
    n = int(host(nb, np.uint32)[0])
    bl = host(blocks, np.uint32).view(oracle.BLOCK_DTYPE)[:n]
    covered = np.zeros(t * k, np.int32)
    for b in bl:
        assert 1 <= b["row_count"] <= tile and b["local_row"] == b["pair_start"]
        sl = got[b["pair_start"]:b["pair_start"] + b["row_count"]]
        assert np.all(sl["expert"] == b["local_slot"])
        covered[b["pair_start"]:b["pair_start"] + b["row_count"]] += 1
    assert np.all(covered == 1)


def test_rows_path_matches_decode_bitwise(tsg, ctx):
    """PrefillRoutedMoERowsVsDecodeTests.swift:23-166: one token routed to all
    eight experts; rows-path activations equal decode phase 1's bit for bit,
    and with weight 1 on one slot and residual 0 the decode output equals the
    rows path's route partial for that slot."""
    configure(ctx, 32, "sym")
    d, f = 576, 384
    rng = oracle.SplitMix64(0x4D5)
    parts = [[oracle.quantize_int4(rng.uniforms(-0.3, 0.3, r * c_).reshape(r, c_), 32, True)
              for (r, c_) in ((f, d), (f, d), (d, f))] for _ in range(8)]
    layer, offs, blobs = _upload_layer(tsg, ctx, parts, True)
    x = oracle.seed_tree_key(0x4D5, "rows-vs-decode").uniforms_f16(-0.8, 0.8, d)
    moe = tsg.MoE(ctx)
    idx = dev(np.arange(8, dtype=np.uint32))
    acts = empty(8 * f)
    moe.encode_phase1_resident(layer, idx, dev(x), acts, d, f)
    pairs = np.array([(0, e, e, 0x3C00) for e in range(8)], dtype=oracle.PAIR_DTYPE)
    blocks = np.array([(e, e, 1, e) for e in range(8)], dtype=oracle.BLOCK_DTYPE)
    ract, parts_out = empty(8 * f), empty(8 * d)
    tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(layer, dev(x), d, dev(pairs), blocks,
                                                          ract, parts_out, 8, d, f)
    assert np.array_equal(host(acts, np.uint16), host(ract, np.uint16))
    po = host(parts_out, np.uint16).reshape(8, d)
    zero = dev(np.zeros(d, np.uint16))
    for slot in (0, 5):
        w = np.zeros(8, np.float32)
        w[slot] = 1.0
        y = empty(d)
        moe.encode_phase2_resident(layer, idx, acts, dev(oracle.f16_bits(w)), zero, y, d, f)
        assert np.array_equal(host(y, np.uint16), po[slot]), f"slot {slot}"
    # more than 8 rows in a block: declined
    with pytest.raises(tsg.TsgError) as e:
        bad = np.array([(0, 0, 9, 0)], dtype=oracle.BLOCK_DTYPE)
        tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(layer, dev(x), d, dev(pairs), bad,
                                                              ract, parts_out, 8, d, f)
    assert e.value.status == 4


def test_rows_path_declines_tile_past_scratch(tsg, ctx):
    """encodeStreamedRows returns 0 when the tile's activation rows exceed
    the scratch it was sized for (PrefillGroupedRoutedMoE.swift:830, `guard
    rows <= maxRows`): the host form declines before any launch and leaves
    the outputs untouched; the device form skips the block and reports it at
    synchronisation; a tile that fits exactly runs."""
    configure(ctx, 32, "sym")
    d, f = 576, 384
    rng = oracle.SplitMix64(0x4D7)
    parts = [[oracle.quantize_int4(rng.uniforms(-0.3, 0.3, r * c_).reshape(r, c_), 32, True)
              for (r, c_) in ((f, d), (f, d), (d, f))] for _ in range(2)]
    layer, offs, blobs = _upload_layer(tsg, ctx, parts, True)
    x = oracle.seed_tree_key(0x4D7, "rows-max-rows").uniforms_f16(-0.8, 0.8, 3 * d)
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    # expert 0 takes tokens 0..2, expert 1 tokens 0..1: 5 activation rows
    pairs = np.array([(0, 0, 0, 0x3C00), (1, 0, 0, 0x3C00), (2, 0, 0, 0x3C00),
                      (0, 1, 1, 0x3C00), (1, 1, 1, 0x3C00)], dtype=oracle.PAIR_DTYPE)
    blocks = np.array([(0, 0, 3, 0), (1, 3, 2, 3)], dtype=oracle.BLOCK_DTYPE)
    act, part = empty(5 * f, fill=NAN16), empty(3 * 2 * d, fill=NAN16)
    for max_rows in (0, 3, 4):
        with pytest.raises(tsg.TsgError) as e:
            g.encode_streamed_rows(layer, dev(x), d, dev(pairs), blocks, act, part, 2, d, f,
                                   max_rows=max_rows)
        assert e.value.status == 4, max_rows
    ctx.synchronize()
    assert np.all(host(act, np.uint16) == np.uint16(NAN16 & 0xFFFF))
    assert np.all(host(part, np.uint16) == np.uint16(NAN16 & 0xFFFF))
    # the device form: block 1 reaches past 4 rows, so it is skipped and reported
    g.encode_streamed_rows_device(layer, dev(x), d, dev(pairs), dev(blocks), 2,
                                  dev(np.array([2], np.uint32)), act, part, 2, d, f, max_rows=4)
    with pytest.raises(tsg.TsgError) as e:
        ctx.synchronize()
    assert e.value.status == 1
    got = host(part, np.uint16).reshape(3, 2, d)
    assert not np.any(np.isnan(oracle.f16_to_float(got[:, 0])))
    assert np.all(got[:2, 1] == np.uint16(NAN16 & 0xFFFF))
    # exactly 5 rows: both forms run and agree bit for bit
    act2, part2 = empty(5 * f), empty(3 * 2 * d, fill=NAN16)
    g.encode_streamed_rows(layer, dev(x), d, dev(pairs), blocks, act2, part2, 2, d, f, max_rows=5)
    act3, part3 = empty(5 * f), empty(3 * 2 * d, fill=NAN16)
    g.encode_streamed_rows_device(layer, dev(x), d, dev(pairs), dev(blocks), 2,
                                  dev(np.array([2], np.uint32)), act3, part3, 2, d, f, max_rows=5)
    ctx.synchronize()
    p2 = host(part2, np.uint16).reshape(3, 2, d)
    assert np.array_equal(p2, host(part3, np.uint16).reshape(3, 2, d))
    assert not np.any(np.isnan(oracle.f16_to_float(p2[:, 0])))
    assert not np.any(np.isnan(oracle.f16_to_float(p2[:2, 1])))


@pytest.mark.parametrize("form", ["host", "device"])
def test_rows_path_many_blocks_matches_decode_bitwise(tsg, ctx, form):
    """A launch with more rows blocks than the device holds at once (24 x 64
    gate/up workgroups): every row still equals decode phase 1 bit for bit
    (PrefillRoutedMoERowsVsDecodeTests.swift:23-166). 8 tokens, each routed to
    all 8 experts, one row per block, through the host and device block
    lists."""
    configure(ctx, 32, "sym")
    d, f, nt = 576, 384, 8
    rng = oracle.SplitMix64(0x4D6)
    parts = [[oracle.quantize_int4(rng.uniforms(-0.3, 0.3, r * c_).reshape(r, c_), 32, True)
              for (r, c_) in ((f, d), (f, d), (d, f))] for _ in range(8)]
    layer, offs, blobs = _upload_layer(tsg, ctx, parts, True)
    x = oracle.seed_tree_key(0x4D6, "rows-many-blocks").uniforms_f16(-0.8, 0.8, nt * d)
    moe = tsg.MoE(ctx)
    idx = dev(np.arange(8, dtype=np.uint32))
    want = np.empty((nt, 8, f), np.uint16)
    for t in range(nt):
        acts = empty(8 * f)
        moe.encode_phase1_resident(layer, idx, dev(x[t * d:(t + 1) * d]), acts, d, f)
        want[t] = host(acts, np.uint16).reshape(8, f)
    n = nt * 8
    pairs = np.array([(i // 8, i % 8, i % 8, 0x3C00) for i in range(n)], dtype=oracle.PAIR_DTYPE)
    blocks = np.array([(i % 8, i, 1, i) for i in range(n)], dtype=oracle.BLOCK_DTYPE)
    ract, parts_out = empty(n * f), empty(nt * 8 * d)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    if form == "host":
        g.encode_streamed_rows(layer, dev(x), d, dev(pairs), blocks, ract, parts_out, 8, d, f)
    else:
        g.encode_streamed_rows_device(layer, dev(x), d, dev(pairs), dev(blocks),
                                      n, dev(np.array([n], np.uint32)), ract, parts_out, 8, d, f)
    ctx.synchronize()
    got = host(ract, np.uint16).reshape(nt, 8, f)
    for t in range(nt):
        assert np.array_equal(got[t], want[t]), f"token {t}"


@pytest.mark.parametrize("t,k,d", [(37, 8, 2816), (5, 4, 104), (5, 3, 104), (7, 8, 100)])
def test_reduce_token_major_bit_exact(tsg, ctx, t, k, d):
    """16-byte vector form (d % 8 == 0, k in 1, 2, 4, 8) and the scalar form
    (k = 3, d = 100)."""
    rng = oracle.SplitMix64(0x7E + d)
    P = rng.uniforms_f16(-1, 1, t * k * d)
    w = rng.uniforms_f16(0, 0.3, t * k)
    h2 = empty(t * d)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(dev(P), dev(w), h2, t, k, d)
    assert np.array_equal(host(h2, np.uint16), oracle.reduce_token_major(P, w, t, k, d).ravel())


@pytest.mark.parametrize("tile", [64, 128, 256])
def test_prefill_pipeline_zipf_end_to_end(tsg, ctx, tile):
    """A Gemma-shaped prefill chunk (T=256, top-8, Zipf(1.1) over 128 experts):
    device grouping -> gate/up -> down -> token-major reduce, against the
    oracle's grouping + expert-major reference + reduce; GEMM blocks of the
    reference's 64 rows, the kernel's widest pass of 128, and 256-row blocks
    that the kernel runs as two passes."""
    configure(ctx, 32, "sym")
    t, ne, k, d, f = 256, 128, 8, 2816, 704
    rng = np.random.default_rng(11)
    idx, w = _zipf_routing(rng, t, ne, k, 1.1)
    orng = oracle.SplitMix64(0xC4)
    parts = []
    for _ in range(ne):
        parts.append([quant(orng, r, c_) for (r, c_) in ((f, d), (f, d), (d, f))])
    layer, offs, blobs = _upload_layer(tsg, ctx, parts, True)
    hidden = orng.uniforms_f16(-1, 1, t * d)
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    max_blocks = t * k // tile + ne
    sp, off, cnt = empty(t * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(dev(idx), dev(w), t, k, ne, sp, off, cnt, blocks, max_blocks, nb, scratch,
                         tile_rows=tile)
    act, partials, h2 = empty(t * k * f), empty(t * k * d), empty(t * d)
    H = dev(hidden)
    g.encode_gate_up(layer, H, d, sp, blocks, max_blocks, act, d, f, n_blocks_device=nb)
    g.encode_down(layer, act, sp, blocks, max_blocks, partials, k, d, f, n_blocks_device=nb)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(partials, dev(w), h2, t, k, d)
    pairs = oracle.make_token_expert_pairs(idx, w, t, k)
    want = oracle.group_pairs(pairs, t, k, ne)
    oracle.set_threads(8)
    P = oracle.prefill_moe_ref(blobs, offs, hidden, d, want["sorted_pairs"], k, d, f, 32, True)
    ref = oracle.reduce_token_major(P, w, t, k, d)
    rel_p = oracle.relative_error(oracle.f16_to_float(host(partials, np.uint16)),
                                  oracle.f16_to_float(P).ravel())
    rel = oracle.relative_error(oracle.f16_to_float(host(h2, np.uint16)),
                                oracle.f16_to_float(ref).ravel())
    print(f"prefill T={t}: partials rel={rel_p:.3e} h2 rel={rel:.3e}")
    assert rel_p <= kc.NORTH_STAR and rel <= kc.NORTH_STAR


def quant(rng, rows, cols):
    return oracle.quantize_int4(rng.uniforms(-0.125, 0.125, rows * cols).reshape(rows, cols),
                                32, True)


def test_device_grouping_reports_expert_out_of_range(tsg, ctx):
    """PrefillMoEGrouping.swift:52-88 throws expertOutOfRange for an expert id
    past numExperts; the device grouping leaves that pair out and the error
    reaches the caller at tsg_ctx_synchronize (status 107). A max_blocks too
    small for the work list is refused before anything is enqueued."""
    t, k, ne, tile = 16, 2, 8, 32
    idx = np.tile(np.arange(k, dtype=np.uint32), (t, 1))
    idx[5, 1] = ne + 3
    w = np.full((t, k), 0x3800, np.uint16)
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    max_blocks = t * k // tile + ne + 1
    sp, off, cnt = empty(t * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(dev(idx), dev(w), t, k, ne, sp, off, cnt, blocks, max_blocks, nb, scratch,
                         tile_rows=tile)
    with pytest.raises(tsg.TsgError) as e:
        ctx.synchronize()
    assert e.value.status == 107
    ctx.synchronize()  # reading the error cleared it
    assert int(host(cnt, np.uint32).sum()) == t * k - 1
    with pytest.raises(tsg.TsgError) as e:
        g.group_pairs_device(dev(idx % ne), dev(w), t, k, ne, sp, off, cnt, blocks, 1, nb,
                             scratch, tile_rows=tile)
    assert e.value.status == 1


@pytest.mark.parametrize("group,scheme", [(32, "sym"), (64, "affine")])
def test_gate_up_half_tile_equals_full_tile(tsg, ctx, group, scheme):
    """F = 704 ends in a 64-column tile, which runs gate and up on separate
    waves; F = 768 covers the same columns with full tiles. A layer whose
    first 704 gate/up rows are the F = 768 layer's gives the same activations
    there, bit for bit, at every block height (1-128 rows)."""
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    d, ne, t, k = 512, 4, 96, 2
    rng = oracle.SplitMix64(0x4A1F)
    g = rng.uniforms(-0.125, 0.125, 768 * d).reshape(768, d)
    u = rng.uniforms(-0.125, 0.125, 768 * d).reshape(768, d)
    layers = {}
    for f in (704, 768):
        parts = []
        for e in range(ne):
            ge, ue = g * (1.0 + 0.1 * e), u * (1.0 - 0.05 * e)
            dn = rng.uniforms(-0.125, 0.125, d * f).reshape(d, f)
            parts.append([oracle.quantize_int4(m, group, sym) for m in (ge[:f], ue[:f], dn)])
        layers[f] = _upload_layer(tsg, ctx, parts, sym)[0]
    # expert e gets 1, 31, 64 and 96 rows: every slice count
    idx = np.zeros((t, k), np.uint32)
    for tok in range(t):
        idx[tok] = (3, 2) if tok < 64 else (3, 1) if tok < 95 else (3, 0)
    w = np.full((t, k), 0x3800, np.uint16)
    grouped = oracle.group_pairs(oracle.make_token_expert_pairs(idx, w, t, k), t, k, ne)
    blocks = wl.rows_blocks(grouped)  # one block per expert
    hidden = dev(rng.uniforms_f16(-1, 1, t * d))
    g_moe = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    P, B = dev(grouped["sorted_pairs"]), dev(blocks)
    out = {}
    for f in (704, 768):
        act = empty(t * k * f, fill=f16_fill_bits(float("nan")))
        g_moe.encode_gate_up(layers[f], hidden, d, P, B, blocks.size, act, d, f)
        out[f] = host(act, np.uint16).reshape(t * k, f)
    assert sorted(blocks["row_count"].tolist()) == [1, 31, 64, 96]
    assert np.array_equal(out[704], out[768][:, :704])
