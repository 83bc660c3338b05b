"""The one-launch verify layer (tsg_moe_verify_layer) against the separate
launches it fuses — the rows router with the device grouping
(tsg_moe_router_bf16_rows_grouped), the device-list rows path and the
token-major reduce, each checked against the oracle elsewhere — bit for bit,
and its outputs against the oracle (the rows path's expert-major reference and
its reduce, PrefillGroupedRoutedMoETests+Execution.swift:213-310):

- configs[2] (Gemma, M = 5, union about 16) and 1 and 8 rows; configs[4]
  decode M = 3 (Qwen shape, 256 experts, SiLU);
- padded rows (hidden stride > d) and a router input distinct from the
  experts' input;
- a small affine g64 layer of 8 experts, where every token takes all eight
  (every slot holds every row);
- calls in a row with fewer rows, and HIP-graph replays of one capture with
  new inputs between them (the launch epoch advances on the device);
- the shapes the one launch declines;
- the shared form (tsg_moe_verify_layer_shared, the Qwen family's shared
  expert in the same launch) against tsg_moe_verify_layer +
  tsg_moe_shared_expert_rows, bit for bit, and the oracle's shared expert,
  also replayed from a HIP graph.
"""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests import workloads as wl
from tests.gpu_util import dev, empty, f16_fill_bits, host

pytestmark = pytest.mark.gpu

NAN16 = f16_fill_bits(float("nan"))
K = 8


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


def upload(tsg, ctx, image, ne, stride, offs):
    layer = tsg.ResidentLayer(ctx, ne, stride, offs)
    layer.upload(image)
    return layer


@pytest.fixture(scope="module")
def gemma_layer(tsg, ctx):
    configure(ctx, 32, "sym")
    image, stride, offs, blobs = wl.random_sym_layer(np.random.default_rng(0x6E3B), 128, 2816, 704)
    return upload(tsg, ctx, image, 128, stride, offs), offs, blobs


@pytest.fixture(scope="module")
def qwen_layer(tsg, ctx):
    configure(ctx, 32, "sym")
    image, stride, offs, blobs = wl.random_sym_layer(np.random.default_rng(0x9E36), 256, 2048, 512)
    return upload(tsg, ctx, image, 256, stride, offs), offs, blobs


def router_inputs(rng, m, d, ne, stride, spread=0.35):
    """M hidden rows sharing a common part (overlapping top-8 sets), stored
    `stride` elements apart (the padding NaN), a N(0, 1/sqrt(d)) bf16 router,
    effective scales near 1 and per-expert gains in [0.5, ...)."""
    x0 = rng.normal(0.0, 1.0, d)
    rows = oracle.f16_bits((x0[None, :] + spread * rng.normal(0.0, 1.0, (m, d))).astype(np.float32))
    hidden = np.full((m, stride), 0x7E00, np.uint16)
    hidden[:, :d] = rows.reshape(m, d)
    rw = oracle.bf16_bits(rng.normal(0.0, 1.0 / np.sqrt(d), ne * d).astype(np.float32))
    es = oracle.bf16_bits((1.0 + 0.1 * rng.normal(0.0, 1.0, d)).astype(np.float32))
    pes = oracle.bf16_bits((0.5 + np.abs(rng.normal(0.0, 1.0, ne))).astype(np.float32))
    return hidden.ravel(), rw, es, pes


def separate(tsg, ctx, moe, layer, RW, RH, X, ES, PES, m, d, f, ne, stride):
    """The three launches the one-launch layer replaces."""
    g = tsg.PrefillGroupedRoutedMoE(moe)
    mb = m * K
    idx, w = empty(m * K, np.uint32, fill=-1), empty(m * K, fill=-1)
    sp, off, cnt = empty(m * K * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    bl, nb = empty(mb * 4, np.uint32), empty(1, np.uint32)
    moe.encode_router_gemma4_bf16_rows_grouped(RW, RH, stride, ES, PES, idx, w, m, ne, d, sp, off,
                                               cnt, bl, mb, nb)
    act, part, h2 = empty(m * K * f), empty(m * K * d, fill=NAN16), empty(m * d, fill=NAN16)
    g.encode_streamed_rows_device(layer, X, stride, sp, bl, mb, nb, act, part, K, d, f)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(part, w, h2, m, K, d)
    ctx.synchronize()
    return (host(idx, np.uint32).copy(), host(w, np.uint16).copy(), host(h2, np.uint16).copy(),
            int(host(nb, np.uint32)[0]))


def fused_outs(m, d):
    return empty(m * K, np.uint32, fill=-1), empty(m * K, fill=-1), empty(m * d, fill=NAN16)


def oracle_h2(blobs, offs, x_rows, idx, w, m, d, f, ne, group, sym, act):
    grouped = oracle.group_pairs(oracle.make_token_expert_pairs(idx, w, m, K), m, K, ne)
    sp = grouped["sorted_pairs"]
    P = oracle.prefill_moe_ref(blobs, offs, x_rows, d, sp, K, d, f, group, sym, act=act,
                               rows_path=True)
    return oracle.reduce_token_major(P, w, m, K, d), len(grouped["groups"])


@pytest.mark.parametrize("shape,m,pad,distinct", [
    ("gemma", 5, 0, False), ("gemma", 1, 0, False), ("gemma", 8, 0, False),
    ("gemma", 5, 64, True), ("qwen", 3, 0, False), ("qwen", 3, 32, True)])
def test_verify_layer_matches_separate_launches(tsg, ctx, gemma_layer, qwen_layer, shape, m, pad,
                                                distinct):
    configure(ctx, 32, "sym")
    if shape == "gemma":
        (layer, offs, blobs), d, f, ne, act = gemma_layer, 2816, 704, 128, "gelu"
    else:
        (layer, offs, blobs), d, f, ne, act = qwen_layer, 2048, 512, 256, "silu"
    stride = d + pad
    rng = np.random.default_rng(0x7E1F + 17 * m + pad + ne)
    hidden, rw, es, pes = router_inputs(rng, m, d, ne, stride)
    xin = router_inputs(rng, m, d, ne, stride)[0] if distinct else hidden
    RW, RH, ES, PES = dev(rw), dev(hidden), dev(es), dev(pes)
    X = dev(xin) if distinct else RH
    moe = tsg.MoE(ctx, gate_activation=act)
    idx0, w0, h20, u = separate(tsg, ctx, moe, layer, RW, RH, X, ES, PES, m, d, f, ne, stride)
    idx, w, h2 = fused_outs(m, d)
    moe.encode_verify_layer(layer, RW, RH, ES, PES, X, stride, h2, idx, w, m, ne, d, f)
    ctx.synchronize()
    got_idx, got_w, got_h2 = host(idx, np.uint32), host(w, np.uint16), host(h2, np.uint16)
    assert np.array_equal(got_idx, idx0) and np.array_equal(got_w, w0)
    assert np.array_equal(got_h2, h20)
    x_rows = xin.reshape(m, stride)[:, :d].ravel().copy()
    ref, u_ref = oracle_h2(blobs, offs, x_rows, idx0.reshape(m, K), w0.reshape(m, K), m, d, f,
                           ne, 32, True, 1 if act == "silu" else 0)
    rel = oracle.relative_error(oracle.f16_to_float(got_h2), oracle.f16_to_float(ref).ravel())
    print(f"{shape} M={m} pad={pad} distinct={distinct}: union={u} h2 rel={rel:.3e}")
    assert u == u_ref and rel <= kc.NORTH_STAR


def test_verify_layer_affine_every_expert(tsg, ctx):
    """A small affine g64 layer of 8 experts (d = f = 320): every token takes
    all eight, so every slot holds every row; GeGLU."""
    configure(ctx, 64, "affine")
    try:
        d = f = 320
        ne, m = 8, 6
        rng = oracle.seed_tree_key(0xAF, "verify-affine")
        experts = [[kc.quantized_rows(rng, r, c, 64, False, -0.3, 0.3)
                    for (r, c) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
        image, stride, offs, blobs = kc.layer_image(experts, False, keep_biases=True)
        layer = upload(tsg, ctx, image, ne, stride, offs)
        nrng = np.random.default_rng(0xAF)
        hidden, rw, es, pes = router_inputs(nrng, m, d, ne, d)
        RW, X, ES, PES = dev(rw), dev(hidden), dev(es), dev(pes)
        moe = tsg.MoE(ctx)
        idx0, w0, h20, u = separate(tsg, ctx, moe, layer, RW, X, X, ES, PES, m, d, f, ne, d)
        assert u == ne
        idx, w, h2 = fused_outs(m, d)
        moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h2, idx, w, m, ne, d, f)
        ctx.synchronize()
        got_h2 = host(h2, np.uint16)
        assert np.array_equal(host(idx, np.uint32), idx0) and np.array_equal(host(w, np.uint16), w0)
        assert np.array_equal(got_h2, h20)
        ref, _ = oracle_h2(blobs, offs, hidden, idx0.reshape(m, K), w0.reshape(m, K), m, d, f, ne,
                           64, False, 0)
        rel = oracle.relative_error(oracle.f16_to_float(got_h2), oracle.f16_to_float(ref).ravel())
        print(f"affine g64, 8 experts, M={m}: h2 rel={rel:.3e}")
        assert rel <= kc.NORTH_STAR
    finally:
        configure(ctx, 32, "sym")


def test_verify_layer_calls_in_a_row_and_graph_replays(tsg, ctx, gemma_layer):
    """Calls in a row (the second with fewer rows), then one capture replayed
    with new inputs copied in between: every result equals the separate
    launches' on the same inputs."""
    import torch
    configure(ctx, 32, "sym")
    layer, offs, blobs = gemma_layer
    d, f, ne = 2816, 704, 128
    moe = tsg.MoE(ctx)
    rng = np.random.default_rng(0x6A7)
    _, rw, es, pes = router_inputs(rng, 1, d, ne, d)
    RW, ES, PES = dev(rw), dev(es), dev(pes)
    for m in (6, 2):
        hidden = router_inputs(rng, m, d, ne, d)[0]
        X = dev(hidden)
        want = separate(tsg, ctx, moe, layer, RW, X, X, ES, PES, m, d, f, ne, d)
        idx, w, h2 = fused_outs(m, d)
        moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h2, idx, w, m, ne, d, f)
        ctx.synchronize()
        assert np.array_equal(host(idx, np.uint32), want[0])
        assert np.array_equal(host(h2, np.uint16), want[2]), m
    m = 5
    X = empty(m * d)
    idx, w, h2 = fused_outs(m, d)
    stream = torch.cuda.Stream()
    X.copy_(dev(router_inputs(rng, m, d, ne, d)[0]))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h2, idx, w, m, ne, d, f,
                                stream=stream)
    torch.cuda.synchronize()
    for rep in range(3):
        X.copy_(dev(router_inputs(rng, m, d, ne, d)[0]))
        h2.fill_(NAN16)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        ctx.synchronize()
        want = separate(tsg, ctx, moe, layer, RW, X, X, ES, PES, m, d, f, ne, d)
        assert np.array_equal(host(idx, np.uint32), want[0]), rep
        assert np.array_equal(host(h2, np.uint16), want[2]), rep


def test_verify_layer_declines(tsg, ctx, gemma_layer):
    configure(ctx, 32, "sym")
    layer, _, _ = gemma_layer
    d, f, ne = 2816, 704, 128
    moe = tsg.MoE(ctx)
    x, rw = empty(9 * d), empty(ne * d)
    es, pes = empty(d), empty(ne)
    idx, w, h2 = fused_outs(9, d)
    for m, nexp in ((0, ne), (9, ne), (5, 7)):
        with pytest.raises(tsg._abi.TsgError) as e:
            moe.encode_verify_layer(layer, rw, x, es, pes, x, d, h2, idx, w, m, nexp, d, f)
        assert e.value.status == tsg._abi.TSG_ERR_DECLINED
    with pytest.raises(tsg._abi.TsgError) as e:  # the layer holds 128 experts
        moe.encode_verify_layer(layer, rw, x, es, pes, x, d, h2, idx, w, 5, 129, d, f)
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT


def test_verify_layer_reports_unroutable_token(tsg, ctx, gemma_layer):
    """A token whose router logits are all NaN leaves its top-8 unfilled: the
    one launch writes NaN outputs, still writes the routing (expert 0 in the
    unfilled slots), every block exits, and tsg_ctx_synchronize reports the
    error; the next call on the context is correct again."""
    configure(ctx, 32, "sym")
    layer, _, _ = gemma_layer
    d, f, ne, m = 2816, 704, 128, 3
    moe = tsg.MoE(ctx)
    rng = np.random.default_rng(0xBAD)
    hidden, rw, es, pes = router_inputs(rng, m, d, ne, d)
    bad = hidden.reshape(m, d).copy()
    bad[1, :] = 0x7E00  # token 1: NaN hidden state, NaN logits
    RW, ES, PES = dev(rw), dev(es), dev(pes)
    idx, w, h2 = fused_outs(m, d)
    moe.encode_verify_layer(layer, RW, dev(bad.ravel()), ES, PES, dev(bad.ravel()), d, h2, idx, w,
                            m, ne, d, f)
    with pytest.raises(tsg._abi.TsgError) as e:
        ctx.synchronize()
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT
    assert np.isnan(oracle.f16_to_float(host(h2, np.uint16))).all()
    assert (host(idx, np.uint32).reshape(m, K)[1] == 0).all()
    X = dev(hidden)
    want = separate(tsg, ctx, moe, layer, RW, X, X, ES, PES, m, d, f, ne, d)
    idx, w, h2 = fused_outs(m, d)
    moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h2, idx, w, m, ne, d, f)
    ctx.synchronize()
    assert np.array_equal(host(h2, np.uint16), want[2])


def shared_expert_inputs(rng, d, f, scheme, group):
    """One shared expert (gate/up [f, d], down [d, f]) and its bf16 gate row."""
    if scheme == "sym":
        image, _, soffs, sblobs = wl.random_sym_layer(rng, 1, d, f)
    else:
        krng = oracle.seed_tree_key(0x5B, f"verify-shared-{d}-{f}")
        experts = [[kc.quantized_rows(krng, r, c, group, False, -0.3, 0.3)
                    for (r, c) in ((f, d), (f, d), (d, f))]]
        image, _, soffs, sblobs = kc.layer_image(experts, False, keep_biases=True)
    gate_w = oracle.bf16_bits((rng.normal(0.0, 1.0 / np.sqrt(d), d)).astype(np.float32))
    return image, soffs, sblobs[0], gate_w


@pytest.mark.parametrize("m,pad,distinct", [(3, 0, False), (3, 32, True), (1, 0, False),
                                            (8, 0, False)])
def test_verify_layer_shared_matches_separate_launches(tsg, ctx, qwen_layer, m, pad, distinct):
    """tsg_moe_verify_layer_shared at configs[4]'s shape (256 experts, d=2048,
    f=512, shared expert f=512): h2 and the routing equal
    tsg_moe_verify_layer's, the shared output tsg_moe_shared_expert_rows' on
    the experts' rows, bit for bit, then calls in a row with fewer rows; the
    shared rows against the oracle's shared expert."""
    configure(ctx, 32, "sym")
    (layer, offs, blobs), d, f, ne = qwen_layer, 2048, 512, 256
    stride = d + pad
    rng = np.random.default_rng(0x5E1 + 13 * m + pad)
    image, soffs, sblob, gate_w = shared_expert_inputs(rng, d, f, "sym", 32)
    SB, G = dev(image), dev(gate_w)
    moe = tsg.MoE(ctx, gate_activation="silu")
    _, rw, es, pes = router_inputs(rng, m, d, ne, stride)
    RW, ES, PES = dev(rw), dev(es), dev(pes)
    for mm in (m, max(1, m - 1)):
        hidden = router_inputs(rng, mm, d, ne, stride)[0]
        xin = router_inputs(rng, mm, d, ne, stride)[0] if distinct else hidden
        RH = dev(hidden)
        X = dev(xin) if distinct else RH
        idx0, w0, h20 = fused_outs(mm, d)
        moe.encode_verify_layer(layer, RW, RH, ES, PES, X, stride, h20, idx0, w0, mm, ne, d, f)
        sact, sout0 = empty(mm * f), empty(mm * d, fill=NAN16)
        tsg.encode_shared_expert_rows(moe, SB, soffs, X, stride, G, sact, sout0, mm, d, f)
        idx, w, h2 = fused_outs(mm, d)
        sout = empty(mm * d, fill=NAN16)
        moe.encode_verify_layer_shared(layer, RW, RH, ES, PES, X, stride, h2, idx, w, SB, soffs,
                                       G, sout, mm, ne, d, f)
        ctx.synchronize()
        assert np.array_equal(host(idx, np.uint32), host(idx0, np.uint32))
        assert np.array_equal(host(w, np.uint16), host(w0, np.uint16))
        assert np.array_equal(host(h2, np.uint16), host(h20, np.uint16)), mm
        got = host(sout, np.uint16).reshape(mm, d).copy()
        assert np.array_equal(got, host(sout0, np.uint16).reshape(mm, d)), mm
        x_rows = xin.reshape(mm, stride)[:, :d]
        for r in (0, mm - 1):
            ref = oracle.shared_expert(sblob, soffs, x_rows[r].copy(), gate_w, d, f, 32, True)
            rel = oracle.relative_error(oracle.f16_to_float(got[r]), oracle.f16_to_float(ref))
            print(f"shared M={mm} pad={pad} distinct={distinct} row {r}: rel={rel:.3e}")
            assert rel <= kc.NORTH_STAR, (mm, r, rel)


def test_verify_layer_shared_wide_shape(tsg, ctx, gemma_layer):
    """The shared form at a shape past the compact batches (d = 2816, f = 704,
    a shared expert of f = 704, SiLU, M = 5): the same bits as
    tsg_moe_verify_layer + tsg_moe_shared_expert_rows."""
    configure(ctx, 32, "sym")
    (layer, offs, blobs), d, f, ne, m = gemma_layer, 2816, 704, 128, 5
    rng = np.random.default_rng(0x5EB)
    image, soffs, sblob, gate_w = shared_expert_inputs(rng, d, f, "sym", 32)
    SB, G = dev(image), dev(gate_w)
    hidden, rw, es, pes = router_inputs(rng, m, d, ne, d)
    RW, X, ES, PES = dev(rw), dev(hidden), dev(es), dev(pes)
    moe = tsg.MoE(ctx, gate_activation="silu")
    idx0, w0, h20 = fused_outs(m, d)
    moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h20, idx0, w0, m, ne, d, f)
    sact, sout0 = empty(m * f), empty(m * d, fill=NAN16)
    tsg.encode_shared_expert_rows(moe, SB, soffs, X, d, G, sact, sout0, m, d, f)
    idx, w, h2 = fused_outs(m, d)
    sout = empty(m * d, fill=NAN16)
    moe.encode_verify_layer_shared(layer, RW, X, ES, PES, X, d, h2, idx, w, SB, soffs, G, sout,
                                   m, ne, d, f)
    ctx.synchronize()
    assert np.array_equal(host(idx, np.uint32), host(idx0, np.uint32))
    assert np.array_equal(host(h2, np.uint16), host(h20, np.uint16))
    assert np.array_equal(host(sout, np.uint16), host(sout0, np.uint16))


def test_verify_layer_shared_affine_every_expert(tsg, ctx):
    """The shared form on a small affine g64 layer of 8 experts (d = f = 320,
    every slot holds every row) with an affine shared expert: the same bits
    as tsg_moe_verify_layer + tsg_moe_shared_expert_rows."""
    configure(ctx, 64, "affine")
    try:
        d = f = 320
        ne, m = 8, 6
        rng = oracle.seed_tree_key(0xB0, "verify-shared-affine")
        experts = [[kc.quantized_rows(rng, r, c, 64, False, -0.3, 0.3)
                    for (r, c) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
        image, stride, offs, _ = kc.layer_image(experts, False, keep_biases=True)
        layer = upload(tsg, ctx, image, ne, stride, offs)
        nrng = np.random.default_rng(0xB0)
        simage, soffs, sblob, gate_w = shared_expert_inputs(nrng, d, f, "affine", 64)
        SB, G = dev(simage), dev(gate_w)
        hidden, rw, es, pes = router_inputs(nrng, m, d, ne, d)
        RW, X, ES, PES = dev(rw), dev(hidden), dev(es), dev(pes)
        moe = tsg.MoE(ctx, gate_activation="silu")
        idx0, w0, h20 = fused_outs(m, d)
        moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h20, idx0, w0, m, ne, d, f)
        sact, sout0 = empty(m * f), empty(m * d, fill=NAN16)
        tsg.encode_shared_expert_rows(moe, SB, soffs, X, d, G, sact, sout0, m, d, f)
        idx, w, h2 = fused_outs(m, d)
        sout = empty(m * d, fill=NAN16)
        moe.encode_verify_layer_shared(layer, RW, X, ES, PES, X, d, h2, idx, w, SB, soffs, G,
                                       sout, m, ne, d, f)
        ctx.synchronize()
        assert np.array_equal(host(idx, np.uint32), host(idx0, np.uint32))
        assert np.array_equal(host(h2, np.uint16), host(h20, np.uint16))
        got = host(sout, np.uint16).reshape(m, d).copy()
        assert np.array_equal(got, host(sout0, np.uint16).reshape(m, d))
        ref = oracle.shared_expert(sblob, soffs, hidden.reshape(m, d)[2].copy(), gate_w, d, f, 64,
                                   False)
        rel = oracle.relative_error(oracle.f16_to_float(got[2]), oracle.f16_to_float(ref))
        print(f"shared affine g64 M={m}: row 2 rel={rel:.3e}")
        assert rel <= kc.NORTH_STAR
    finally:
        configure(ctx, 32, "sym")


def test_verify_layer_shared_declines_and_unroutable(tsg, ctx, qwen_layer):
    """The shared form declines a GeGLU MoE; an unroutable token makes its
    shared output NaN too, and the next call is correct."""
    configure(ctx, 32, "sym")
    (layer, offs, blobs), d, f, ne, m = qwen_layer, 2048, 512, 256, 3
    rng = np.random.default_rng(0x5ED)
    image, soffs, sblob, gate_w = shared_expert_inputs(rng, d, f, "sym", 32)
    SB, G = dev(image), dev(gate_w)
    hidden, rw, es, pes = router_inputs(rng, m, d, ne, d)
    RW, ES, PES = dev(rw), dev(es), dev(pes)
    idx, w, h2 = fused_outs(m, d)
    sout = empty(m * d, fill=0)
    with pytest.raises(tsg._abi.TsgError) as e:
        tsg.MoE(ctx).encode_verify_layer_shared(layer, RW, dev(hidden), ES, PES, dev(hidden), d,
                                                h2, idx, w, SB, soffs, G, sout, m, ne, d, f)
    assert e.value.status == tsg._abi.TSG_ERR_DECLINED
    moe = tsg.MoE(ctx, gate_activation="silu")
    bad = hidden.reshape(m, d).copy()
    bad[2, :] = 0x7E00
    B = dev(bad.ravel())
    moe.encode_verify_layer_shared(layer, RW, B, ES, PES, B, d, h2, idx, w, SB, soffs, G, sout, m,
                                   ne, d, f)
    with pytest.raises(tsg._abi.TsgError) as e:
        ctx.synchronize()
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT
    assert np.isnan(oracle.f16_to_float(host(sout, np.uint16))).all()
    X = dev(hidden)
    sact, sout0 = empty(m * f), empty(m * d)
    tsg.encode_shared_expert_rows(moe, SB, soffs, X, d, G, sact, sout0, m, d, f)
    moe.encode_verify_layer_shared(layer, RW, X, ES, PES, X, d, h2, idx, w, SB, soffs, G, sout, m,
                                   ne, d, f)
    ctx.synchronize()
    assert np.array_equal(host(sout, np.uint16), host(sout0, np.uint16))


def test_verify_layer_shared_graph_replays(tsg, ctx, qwen_layer):
    """The shared form captured once in a HIP graph and replayed with new token
    rows copied in between: each replay equals tsg_moe_verify_layer +
    tsg_moe_shared_expert_rows on the same rows."""
    import torch
    configure(ctx, 32, "sym")
    (layer, offs, blobs), d, f, ne, m = qwen_layer, 2048, 512, 256, 3
    rng = np.random.default_rng(0x5EA)
    image, soffs, sblob, gate_w = shared_expert_inputs(rng, d, f, "sym", 32)
    SB, G = dev(image), dev(gate_w)
    _, rw, es, pes = router_inputs(rng, m, d, ne, d)
    RW, ES, PES = dev(rw), dev(es), dev(pes)
    moe = tsg.MoE(ctx, gate_activation="silu")
    X = empty(m * d)
    X.copy_(dev(router_inputs(rng, m, d, ne, d)[0]))
    idx, w, h2 = fused_outs(m, d)
    sout = empty(m * d, fill=NAN16)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        moe.encode_verify_layer_shared(layer, RW, X, ES, PES, X, d, h2, idx, w, SB, soffs, G,
                                       sout, m, ne, d, f, stream=stream)
    torch.cuda.synchronize()
    for rep in range(3):
        X.copy_(dev(router_inputs(rng, m, d, ne, d)[0]))
        h2.fill_(NAN16)
        sout.fill_(NAN16)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        ctx.synchronize()
        idx0, w0, h20 = fused_outs(m, d)
        moe.encode_verify_layer(layer, RW, X, ES, PES, X, d, h20, idx0, w0, m, ne, d, f)
        sact, sout0 = empty(m * f), empty(m * d)
        tsg.encode_shared_expert_rows(moe, SB, soffs, X, d, G, sact, sout0, m, d, f)
        ctx.synchronize()
        assert np.array_equal(host(idx, np.uint32), host(idx0, np.uint32)), rep
        assert np.array_equal(host(h2, np.uint16), host(h20, np.uint16)), rep
        assert np.array_equal(host(sout, np.uint16), host(sout0, np.uint16)), rep
