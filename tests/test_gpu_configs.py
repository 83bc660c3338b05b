"""GPU parity at BASELINE.json's configuration shapes, against the oracle:

- the verify rows path with 1, 2, 4 and 8 rows per expert
  (PrefillGroupedRoutedMoETests+Execution.swift:213-310), GeGLU and SiLU,
  and no looser than the tiled GEMM at the production shape (:322-431);
- Gemma verify, M = 5 tokens over a union of about 16 experts,
  rows path + token-major reduce;
- configs[4] decode M = 3: Qwen-shaped rows path + shared branch;
- configs[3] at its real size (T = 2048, Zipf(1.1), Gemma) and configs[4]
  prefill (T = 4096, Zipf(1.0), Qwen-shaped, SiLU): device grouping ->
  gate/up GEMM -> down GEMM -> reduce, every pair of the head expert and
  every pair of every 16th token and the edge rows of every routed block
  recomputed on the CPU.
"""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests import workloads as wl
from tests.gpu_util import dev, empty, f16_fill_bits, host

pytestmark = pytest.mark.gpu

NAN16 = f16_fill_bits(float("nan"))


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


def rows_fixture(rows, group, sym, d=320, f=320, ne=8, seed=0x5E):
    """streamedRowsMatchesReference's route set: token t routes to experts
    t % 3 (rank 0) and t % 2 + 3 (rank 1); hidden (i % 17 - 8) * 0.01."""
    pairs = []
    for t in range(rows):
        pairs.append((t, t % 3, 0, 0x3C00))
        pairs.append((t, t % 2 + 3, 1, 0x3C00))
    pairs = np.array(pairs, dtype=oracle.PAIR_DTYPE)
    grouped = oracle.group_pairs(pairs, rows, 2, ne)
    rng = oracle.seed_tree_key(seed, f"rows-{rows}-g{group}")
    experts = [[kc.quantized_rows(rng, r, c, group, sym, -0.3, 0.3)
                for (r, c) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
    hidden = oracle.f16_bits(((np.arange(rows * d) % 17) - 8).astype(np.float32) * np.float32(0.01))
    return grouped, experts, hidden


@pytest.mark.parametrize("rows", [1, 2, 4, 8])
@pytest.mark.parametrize("group,scheme", [(32, "sym"), (64, "affine")])
@pytest.mark.parametrize("act", ["gelu", "silu"])
def test_rows_path_matches_reference(tsg, ctx, rows, group, scheme, act):
    """The verify rows path (encodeStreamedRows) with experts holding 1..rows
    route rows, against the expert-major CPU reference; route partials start
    as NaN so a skipped store fails."""
    sym = scheme == "sym"
    configure(ctx, group, scheme)
    d = f = 320
    top_k = 2
    grouped, experts, hidden = rows_fixture(rows, group, sym)
    image, stride, offs, blobs = kc.layer_image(experts, sym, keep_biases=not sym)
    layer = upload(tsg, ctx, image, len(experts), stride, offs)
    sp = grouped["sorted_pairs"]
    assert int(grouped["counts"].max()) == (rows + 1) // 2  # the widest expert holds ceil(rows/2)
    act_id = 1 if act == "silu" else 0
    ref = oracle.prefill_moe_ref(blobs, offs, hidden, d, sp, top_k, d, f, group, sym, act=act_id,
                                 rows_path=True)
    moe = tsg.MoE(ctx, gate_activation=act)
    act_buf = empty(sp.size * f)
    part = empty(rows * top_k * d, fill=NAN16)
    tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(
        layer, dev(hidden), d, dev(sp), wl.rows_blocks(grouped), act_buf, part, top_k, d, f)
    got = oracle.f16_to_float(host(part, np.uint16))
    rel = oracle.relative_error(got, oracle.f16_to_float(ref).ravel())
    print(f"rows={rows} g{group} {scheme} {act}: rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


def test_rows_no_looser_than_tiled_at_production_shape(tsg, ctx):
    """streamedRowsIsNoLooserThanTiledAtProductionShape (:322-431): D = 2816,
    F = 704, 4 tokens x top-2 over 4 experts; the rows path (decode's
    arithmetic) must be at least as close to the CPU reference as the tiled
    GEMM (fp16-staged weights), and within the north-star bound."""
    configure(ctx, 32, "sym")
    d, f, rows, top_k, ne = 2816, 704, 4, 2, 4
    pairs = []
    for t in range(rows):
        pairs.append((t, t % 2, 0, 0x3C00))
        pairs.append((t, t % 2 + 2, 1, 0x3C00))
    grouped = oracle.group_pairs(np.array(pairs, dtype=oracle.PAIR_DTYPE), rows, top_k, ne)
    rng = oracle.seed_tree_key(0x6E, "rows-vs-tiled")
    experts = [[kc.quantized_rows(rng, r, c, 32, True, -0.125, 0.125)
                for (r, c) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
    hidden = oracle.f16_bits(((np.arange(rows * d) % 23) - 11).astype(np.float32) * np.float32(0.01))
    image, stride, offs, blobs = kc.layer_image(experts, True, keep_biases=False)
    layer = upload(tsg, ctx, image, ne, stride, offs)
    sp = grouped["sorted_pairs"]
    ref = oracle.f16_to_float(
        oracle.prefill_moe_ref(blobs, offs, hidden, d, sp, top_k, d, f, 32, True)).ravel()
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    blocks = wl.rows_blocks(grouped)
    H, P = dev(hidden), dev(sp)
    act_buf = empty(sp.size * f)
    rows_out = empty(rows * top_k * d, fill=NAN16)
    g.encode_streamed_rows(layer, H, d, P, blocks, act_buf, rows_out, top_k, d, f)
    tiled_out = empty(rows * top_k * d, fill=NAN16)
    act2 = empty(sp.size * f)
    B = dev(blocks)
    g.encode_gate_up(layer, H, d, P, B, blocks.size, act2, d, f)
    g.encode_down(layer, act2, P, B, blocks.size, tiled_out, top_k, d, f)
    rel_rows = oracle.relative_error(oracle.f16_to_float(host(rows_out, np.uint16)), ref)
    rel_tiled = oracle.relative_error(oracle.f16_to_float(host(tiled_out, np.uint16)), ref)
    print(f"rows rel={rel_rows:.3e} tiled rel={rel_tiled:.3e}")
    assert rel_rows <= rel_tiled
    assert rel_rows <= kc.NORTH_STAR and rel_tiled <= kc.NORTH_STAR


@pytest.fixture(scope="module")
def gemma_layer(tsg, ctx):
    configure(ctx, 32, "sym")
    image, stride, offs, blobs = wl.random_sym_layer(np.random.default_rng(0x6E3A), 128, 2816, 704)
    return upload(tsg, ctx, image, 128, stride, offs), offs, blobs


@pytest.fixture(scope="module")
def qwen_layer(tsg, ctx):
    configure(ctx, 32, "sym")
    image, stride, offs, blobs = wl.random_sym_layer(np.random.default_rng(0x9E35), 256, 2048, 512)
    return upload(tsg, ctx, image, 256, stride, offs), offs, blobs


def host_grouping(idx, w, m, ne):
    """A verify step's host grouping (PrefillMoEGrouping.groupTokenExpertPairs
    over makeTokenExpertPairs), as the runner does per block."""
    grouped = oracle.group_pairs(oracle.make_token_expert_pairs(idx, w, m, 8), m, 8, ne)
    return grouped["sorted_pairs"], grouped


@pytest.mark.parametrize("seed", [0x5E5E, 0x5E5F])
def test_verify_m5_gemma_rows_path(tsg, ctx, gemma_layer, seed):
    """five tokens whose top-8 sets overlap (union about 16) through
    the rows path and the token-major reduce, against the expert-major CPU
    reference and its reduce."""
    configure(ctx, 32, "sym")
    layer, offs, blobs = gemma_layer
    m, d, f, ne, k = 5, 2816, 704, 128, 8
    rng = np.random.default_rng(seed)
    idx, w, u = wl.verify_routing(rng, m, ne, k)
    assert 12 <= u <= 20
    hidden = wl.f16_normal(rng, m * d)
    sp, grouped = host_grouping(idx, w, m, ne)
    moe = tsg.MoE(ctx)
    blocks = wl.rows_blocks(grouped)
    assert blocks.size == u and int(blocks["row_count"].max()) >= 2
    act_buf, part, h2 = empty(m * k * f), empty(m * k * d, fill=NAN16), empty(m * d)
    tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(layer, dev(hidden), d, dev(sp), blocks,
                                                          act_buf, part, k, d, f)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(part, dev(w), h2, m, k, d)
    P = oracle.prefill_moe_ref(blobs, offs, hidden, d, sp, k, d, f, 32, True, rows_path=True)
    ref_h2 = oracle.reduce_token_major(P, w, m, k, d)
    rel_p = oracle.relative_error(oracle.f16_to_float(host(part, np.uint16)),
                                  oracle.f16_to_float(P).ravel())
    rel = oracle.relative_error(oracle.f16_to_float(host(h2, np.uint16)),
                                oracle.f16_to_float(ref_h2).ravel())
    print(f"verify M=5 union={u} rows/expert max={int(blocks['row_count'].max())}: "
          f"partials rel={rel_p:.3e} h2 rel={rel:.3e}")
    assert rel_p <= kc.NORTH_STAR and rel <= kc.NORTH_STAR


def test_qwen_decode_m3_rows_and_shared(tsg, ctx, qwen_layer):
    """configs[4] decode at M = 3 (MTP width 2 + 1): the routed experts on the
    rows path (SiLU) + reduce, and the shared expert with its sigmoid gate per
    token (QwenForwardRunner.swift:1548-1578), each against the oracle."""
    configure(ctx, 32, "sym")
    layer, offs, blobs = qwen_layer
    m, d, f, ne, k = 3, 2048, 512, 256, 8
    rng = np.random.default_rng(0x3333)
    idx, w, u = wl.verify_routing(rng, m, ne, k, target=12)
    hidden = wl.f16_normal(rng, m * d)
    sp, grouped = host_grouping(idx, w, m, ne)
    moe = tsg.MoE(ctx, gate_activation="silu")
    blocks = wl.rows_blocks(grouped)
    act_buf, part, h2 = empty(m * k * f), empty(m * k * d, fill=NAN16), empty(m * d)
    X = dev(hidden)
    tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(layer, X, d, dev(sp), blocks, act_buf,
                                                          part, k, d, f)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(part, dev(w), h2, m, k, d)
    P = oracle.prefill_moe_ref(blobs, offs, hidden, d, sp, k, d, f, 32, True, act=1,
                               rows_path=True)
    ref_h2 = oracle.reduce_token_major(P, w, m, k, d)
    rel = oracle.relative_error(oracle.f16_to_float(host(h2, np.uint16)),
                                oracle.f16_to_float(ref_h2).ravel())
    # the shared expert (one more sym blob) and its bf16 gate row
    srng = np.random.default_rng(0x51AE)
    simage, _, soffs, sblobs = wl.random_sym_layer(srng, 1, d, f)
    gate_w = oracle.bf16_bits((srng.normal(0.0, 1.0 / np.sqrt(d), d)).astype(np.float32))
    sblob = dev(simage)
    q, qk = tsg.DequantInt4GEMV(ctx), tsg.QwenKernels(ctx)
    sg, su, sa, sout = empty(m * f), empty(m * f), empty(m * f), empty(m * d)
    o = [int(v) for v in soffs]
    q.encode_rows(sblob[o[0]:], sblob[o[1]:], sblob[o[2]:], X, d, sg, f, m, f, d)
    q.encode_rows(sblob[o[3]:], sblob[o[4]:], sblob[o[5]:], X, d, su, f, m, f, d)
    qk.encode_silu_mul(sg, su, sa, m * f)
    q.encode_rows(sblob[o[6]:], sblob[o[7]:], sblob[o[8]:], sa, f, sout, d, m, d, f)
    G = dev(gate_w)
    for t in range(m):
        qk.encode_moe_shared_gate(sout[t * d:(t + 1) * d], X[t * d:(t + 1) * d], G, d)
    got_s = host(sout, np.uint16).reshape(m, d)
    rel_s = 0.0
    for t in range(m):
        ref_s = oracle.shared_expert(sblobs[0], soffs, hidden[t * d:(t + 1) * d], gate_w, d, f,
                                     32, True)
        rel_s = max(rel_s, oracle.relative_error(oracle.f16_to_float(got_s[t]),
                                                 oracle.f16_to_float(ref_s)))
    print(f"qwen M=3 union={u}: routed h2 rel={rel:.3e} shared rel={rel_s:.3e}")
    assert rel <= kc.NORTH_STAR and rel_s <= kc.NORTH_STAR


def device_verify_layer(tsg, ctx, moe, layer, rng, m, d, f, ne, spread=0.35):
    """A verify step's routed MoE with nothing on the host: the router rows
    (M tokens whose hidden states share a common part, so their top-8 sets
    overlap), the device grouping, the device-list rows path and the
    token-major reduce. Returns the device buffers and the inputs."""
    k = 8
    x0 = rng.normal(0.0, 1.0, d)
    hidden = oracle.f16_bits((x0[None, :] + spread * rng.normal(0.0, 1.0, (m, d)))
                             .astype(np.float32)).ravel()
    rw = oracle.bf16_bits(rng.normal(0.0, 1.0 / np.sqrt(d), ne * d).astype(np.float32))
    ones_d = np.full(d, 0x3F80, np.uint16)
    ones_e = np.full(ne, 0x3F80, np.uint16)
    X = dev(hidden)
    idx, wts = empty(m * k, np.uint32), empty(m * k)
    moe.encode_router_gemma4_bf16_rows(dev(rw), X, d, dev(ones_d), dev(ones_e), idx, wts, m, ne,
                                       d)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    max_blocks = m * k
    sp, off, cnt = empty(m * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    g.group_pairs_device_noalloc(idx, wts, m, k, ne, sp, off, cnt, blocks, max_blocks, nb,
                                 tile_rows=32)
    act_buf, part, h2 = empty(m * k * f), empty(m * k * d, fill=NAN16), empty(m * d)
    g.encode_streamed_rows_device(layer, X, d, sp, blocks, max_blocks, nb, act_buf, part, k, d, f)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(part, wts, h2, m, k, d)
    ctx.synchronize()
    return dict(hidden=hidden, X=X, idx=host(idx, np.uint32).reshape(m, k).copy(),
                w=host(wts, np.uint16).reshape(m, k).copy(), sp=sp, part=part, h2=h2,
                n=int(host(nb, np.uint32)[0]))


@pytest.mark.parametrize("shape", ["gemma-m5", "qwen-m3"])
def test_verify_whole_layer_on_device(tsg, ctx, gemma_layer, qwen_layer, shape):
    """configs[2] and configs[4] M=3 as whole layers on the device (router
    rows, device grouping, device-list rows path, reduce): the same partials
    and outputs, bit for bit, as the host-list path run on the routing the
    device chose, which the oracle checks."""
    configure(ctx, 32, "sym")
    if shape == "gemma-m5":
        (layer, offs, blobs), m, d, f, ne, act = gemma_layer, 5, 2816, 704, 128, "gelu"
    else:
        (layer, offs, blobs), m, d, f, ne, act = qwen_layer, 3, 2048, 512, 256, "silu"
    k = 8
    moe = tsg.MoE(ctx, gate_activation=act)
    r = device_verify_layer(tsg, ctx, moe, layer, np.random.default_rng(0xD1CE + m), m, d, f, ne)
    sp_h, grouped = host_grouping(r["idx"], r["w"], m, ne)
    assert np.array_equal(host(r["sp"], np.uint32)[:m * k * 4].view(oracle.PAIR_DTYPE), sp_h)
    blocks = wl.rows_blocks(grouped)
    assert r["n"] == blocks.size and 8 < blocks.size < m * k  # the top-8 sets overlap
    act2, part2, h22 = empty(m * k * f), empty(m * k * d, fill=NAN16), empty(m * d)
    tsg.PrefillGroupedRoutedMoE(moe).encode_streamed_rows(layer, r["X"], d, dev(sp_h), blocks,
                                                          act2, part2, k, d, f)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(part2, dev(r["w"]), h22, m, k, d)
    assert np.array_equal(host(r["part"], np.uint16), host(part2, np.uint16))
    assert np.array_equal(host(r["h2"], np.uint16), host(h22, np.uint16))
    P = oracle.prefill_moe_ref(blobs, offs, r["hidden"], d, sp_h, k, d, f, 32, True,
                               act=1 if act == "silu" else 0, rows_path=True)
    ref_h2 = oracle.reduce_token_major(P, r["w"], m, k, d)
    rel = oracle.relative_error(oracle.f16_to_float(host(r["h2"], np.uint16)),
                                oracle.f16_to_float(ref_h2).ravel())
    print(f"{shape}: union={blocks.size} h2 rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


@pytest.mark.parametrize("m,ne,d", [(5, 128, 2816), (3, 256, 2048), (1, 128, 2816),
                                    (8, 128, 2816)])
def test_router_rows_grouped_matches_router_then_grouping(tsg, ctx, m, ne, d):
    """tsg_moe_router_bf16_rows_grouped gives the rows router's indices and
    weights and the device grouping's sorted pairs, offsets, counts and block
    list, bit for bit (random effective and per-expert scales)."""
    k = 8
    rng = np.random.default_rng(0x6A0 + m * 7 + ne)
    x0 = rng.normal(0.0, 1.0, d)
    hidden = oracle.f16_bits((x0[None, :] + 0.35 * rng.normal(0.0, 1.0, (m, d)))
                             .astype(np.float32)).ravel()
    rw = oracle.bf16_bits(rng.normal(0.0, 1.0 / np.sqrt(d), ne * d).astype(np.float32))
    es = oracle.bf16_bits((1.0 + 0.1 * rng.normal(0.0, 1.0, d)).astype(np.float32))
    pes = oracle.bf16_bits((0.5 + np.abs(rng.normal(0.0, 1.0, ne))).astype(np.float32))
    RW, X, ES, PES = dev(rw), dev(hidden), dev(es), dev(pes)
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    max_blocks = m * k

    def outs():
        return dict(idx=empty(m * k, np.uint32, fill=-1), w=empty(m * k, fill=-1),
                    sp=empty(m * k * 4, np.uint32, fill=-1), off=empty(ne, np.uint32, fill=-1),
                    cnt=empty(ne, np.uint32, fill=-1), bl=empty(max_blocks * 4, np.uint32, fill=-1),
                    nb=empty(1, np.uint32, fill=-1))

    a = outs()
    moe.encode_router_gemma4_bf16_rows(RW, X, d, ES, PES, a["idx"], a["w"], m, ne, d)
    scratch = empty(g.scratch_bytes(m, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(a["idx"], a["w"], m, k, ne, a["sp"], a["off"], a["cnt"], a["bl"],
                         max_blocks, a["nb"], scratch, tile_rows=32)
    b = outs()
    moe.encode_router_gemma4_bf16_rows_grouped(RW, X, d, ES, PES, b["idx"], b["w"], m, ne, d,
                                               b["sp"], b["off"], b["cnt"], b["bl"], max_blocks,
                                               b["nb"])
    ctx.synchronize()
    n = int(host(a["nb"], np.uint32)[0])
    assert n == int(host(b["nb"], np.uint32)[0]) and 8 <= n <= m * k
    for key in ("idx", "w", "sp", "off", "cnt"):
        dt = np.uint16 if key == "w" else np.uint32
        assert np.array_equal(host(a[key], dt), host(b[key], dt)), key
    assert np.array_equal(host(a["bl"], np.uint32)[:4 * n], host(b["bl"], np.uint32)[:4 * n])
    # the one-row router on each row gives the same indices
    for r in range(m):
        i1, w1 = empty(k, np.uint32), empty(k)
        moe.encode_router_gemma4_bf16(RW, X[r * d:], ES, PES, i1, w1, ne, d)
        assert np.array_equal(host(i1, np.uint32), host(b["idx"], np.uint32)[r * k:(r + 1) * k])
        assert np.array_equal(host(w1, np.uint16), host(b["w"], np.uint16)[r * k:(r + 1) * k])


def test_verify_entry_points_reject_bad_arguments(tsg, ctx, gemma_layer):
    """Host-side checks of the verify entry points, before any launch: the
    grouped router declines 0 or more than 8 rows and refuses a block list too
    short for min(rows * 8, experts); the device-list rows path refuses an empty
    or oversized capacity and a missing count."""
    configure(ctx, 32, "sym")
    layer, _, _ = gemma_layer
    d, f, ne, k = 2816, 704, 128, 8
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    rw, x = empty(ne * d), empty(8 * d)
    es, pes = empty(d, fill=0x3F80), empty(ne, fill=0x3F80)
    idx, w = empty(9 * k, np.uint32), empty(9 * k)
    sp, off, cnt = empty(9 * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    bl, nb = empty(9 * k * 4, np.uint32), empty(1, np.uint32)
    for rows, max_blocks, status in ((0, 8, 4), (9, 72, 4), (5, 39, 1)):
        with pytest.raises(tsg.TsgError) as e:
            moe.encode_router_gemma4_bf16_rows_grouped(rw, x, d, es, pes, idx, w, rows, ne, d,
                                                       sp, off, cnt, bl, max_blocks, nb)
        assert e.value.status == status, (rows, max_blocks)
    act, part = empty(8 * k * f), empty(8 * k * d)
    for max_blocks, count in ((0, nb), (65536, nb), (8, None)):
        with pytest.raises(tsg.TsgError) as e:
            g.encode_streamed_rows_device(layer, x, d, sp, bl, max_blocks, count, act, part, k,
                                          d, f)
        assert e.value.status == 1, max_blocks
    ctx.synchronize()


def test_rows_device_list_skips_and_reports(tsg, ctx, gemma_layer):
    """Blocks past the device count are not run; a live block the rows path
    cannot take (9 rows) is skipped and reported at synchronisation."""
    configure(ctx, 32, "sym")
    layer, offs, blobs = gemma_layer
    d, f, k = 2816, 704, 8
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    pairs = np.zeros(16, oracle.PAIR_DTYPE)
    pairs["token"] = np.arange(16) // 8
    pairs["rank"] = np.arange(16) % 8
    pairs["expert"] = 3
    bl = np.zeros(2, oracle.BLOCK_DTYPE)
    bl["local_slot"] = 3
    bl["pair_start"] = bl["local_row"] = [0, 2]
    bl["row_count"] = [2, 9]
    X = dev(wl.f16_normal(np.random.default_rng(1), 16 * d))
    act_buf, part = empty(16 * f), empty(16 * d, fill=NAN16)
    # count 0: nothing runs
    g.encode_streamed_rows_device(layer, X, d, dev(pairs), dev(bl), 2, dev(np.zeros(1, np.uint32)),
                                  act_buf, part, k, d, f)
    ctx.synchronize()
    assert np.all(host(part, np.uint16) == np.uint16(NAN16 & 0xFFFF))
    # count 2: block 0 runs, block 1 (9 rows) is skipped and reported
    g.encode_streamed_rows_device(layer, X, d, dev(pairs), dev(bl), 2, dev(np.full(1, 2, np.uint32)),
                                  act_buf, part, k, d, f)
    with pytest.raises(tsg.TsgError) as e:
        ctx.synchronize()
    assert e.value.status == 1
    got = host(part, np.uint16).reshape(16, d)
    assert np.all(got[2:] == np.uint16(NAN16 & 0xFFFF))
    assert not np.any(np.isnan(oracle.f16_to_float(got[:2])))


@pytest.mark.parametrize("rows,scheme", [(3, "sym"), (8, "sym"), (5, "affine")])
def test_shared_expert_rows_matches_one_row_form(tsg, ctx, rows, scheme):
    """tsg_moe_shared_expert_rows: row r equals tsg_moe_shared_expert on x_r
    bit for bit (configs[4]'s shared expert, d=2048, f=512), and the oracle."""
    configure(ctx, 32, scheme)
    d, f = 2048, 512
    rng = np.random.default_rng(0x5A + rows)
    if scheme == "sym":
        image, _, soffs, sblobs = wl.random_sym_layer(rng, 1, d, f)
    else:
        krng = oracle.seed_tree_key(0x5A, f"shared-rows-{rows}")
        experts = [[kc.quantized_rows(krng, r, c, 32, False, -0.3, 0.3)
                    for (r, c) in ((f, d), (f, d), (d, f))]]
        image, _, soffs, sblobs = kc.layer_image(experts, False, keep_biases=True)
    gate_w = oracle.bf16_bits((rng.normal(0.0, 1.0 / np.sqrt(d), d)).astype(np.float32))
    stride = d + 8  # a token stride other than d
    xs = np.zeros(rows * stride, np.uint16)
    for r in range(rows):
        xs[r * stride:r * stride + d] = wl.f16_normal(rng, d)
    moe = tsg.MoE(ctx, gate_activation="silu")
    blob, X, G = dev(image), dev(xs), dev(gate_w)
    sact, sout = empty(rows * f), empty(rows * d)
    tsg.encode_shared_expert_rows(moe, blob, soffs, X, stride, G, sact, sout, rows, d, f)
    got = host(sout, np.uint16).reshape(rows, d).copy()
    for r in range(rows):
        a1, o1 = empty(f), empty(d)
        tsg.encode_shared_expert(moe, blob, soffs, X[r * stride:], G, a1, o1, d, f)
        assert np.array_equal(got[r], host(o1, np.uint16)), r
        ref = oracle.shared_expert(sblobs[0], soffs, xs[r * stride:r * stride + d], gate_w, d, f,
                                   32, scheme == "sym")
        rel = oracle.relative_error(oracle.f16_to_float(got[r]), oracle.f16_to_float(ref))
        assert rel <= kc.NORTH_STAR, (r, rel)
    with pytest.raises(tsg.TsgError) as e:
        tsg.encode_shared_expert_rows(moe, blob, soffs, X, stride, G, sact, sout, 9, d, f)
    assert e.value.status == 4


def run_prefill_full(tsg, ctx, layer, offs, blobs, t, d, f, ne, s, act, seed):
    """Device grouping -> gate/up -> down -> reduce at full size; the head
    expert, every 16th token and the first and last row of every routed
    block recomputed by the oracle."""
    k = 8
    rng = np.random.default_rng(seed)
    idx, w = wl.zipf_routing(rng, t, ne, k, s)
    hidden = wl.f16_normal(rng, t * d)
    moe = tsg.MoE(ctx, gate_activation=act)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    tile = 256  # the routed GEMM's pass
    max_blocks = t * k // tile + ne
    sp, off, cnt = empty(t * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(dev(idx), dev(w), t, k, ne, sp, off, cnt, blocks, max_blocks, nb, scratch,
                         tile_rows=tile)
    act_buf, partials, h2 = empty(t * k * f), empty(t * k * d, fill=NAN16), empty(t * d)
    g.encode_gate_up(layer, dev(hidden), d, sp, blocks, max_blocks, act_buf, d, f,
                     n_blocks_device=nb)
    g.encode_down(layer, act_buf, sp, blocks, max_blocks, partials, k, d, f, n_blocks_device=nb)
    tsg.PrefillMoE(ctx).encode_reduce_token_major(partials, dev(w), h2, t, k, d)
    want = oracle.group_pairs(oracle.make_token_expert_pairs(idx, w, t, k), t, k, ne)
    assert np.array_equal(host(sp, np.uint32).view(oracle.PAIR_DTYPE), want["sorted_pairs"])
    # every routed block's first and last row too: each GEMM work item's edges
    n_blocks = int(host(nb, np.uint32)[0])
    bl = host(blocks, np.uint32).reshape(-1, 4)[:n_blocks]
    edges = np.concatenate([bl[:, 1], bl[:, 1] + bl[:, 2] - 1]).astype(np.int64)
    sub, _, tokens, head, head_rows = wl.sampled_pairs(want["sorted_pairs"], t, extra_pos=edges)
    oracle.set_threads(16)
    P = oracle.prefill_moe_ref(blobs, offs, hidden, d, sub, k, d, f, 32, True,
                               act=1 if act == "silu" else 0)
    gp = host(partials, np.uint16).reshape(t * k, d)
    assert np.all(np.isfinite(oracle.f16_to_float(gp))), "a route partial was never written"
    rows = sub["token"].astype(np.int64) * k + sub["rank"].astype(np.int64)
    rel_p = oracle.relative_error(oracle.f16_to_float(gp[rows]), oracle.f16_to_float(P[rows]))
    Ps = P.reshape(t, k, d)[tokens].reshape(-1, d)
    ref_h2 = oracle.reduce_token_major(Ps, w[tokens], tokens.size, k, d)
    gh = host(h2, np.uint16).reshape(t, d)[tokens]
    rel = oracle.relative_error(oracle.f16_to_float(gh), oracle.f16_to_float(ref_h2))
    print(f"prefill T={t} E={ne} {act}: head expert {head} ({head_rows} rows), "
          f"{n_blocks} routed blocks, {sub.size} pairs checked: partials rel={rel_p:.3e} "
          f"h2 rel={rel:.3e}")
    return rel_p, rel, head_rows


def test_gemma_prefill_t2048_full_size(tsg, ctx, gemma_layer):
    """configs[3] at its real size: T = 2048, top-8 Zipf(1.1) over 128 experts.
    The head expert holds well over 1,000 rows, so it runs as many 256-row work
    items dealt across the XCDs; all of them are checked."""
    configure(ctx, 32, "sym")
    layer, offs, blobs = gemma_layer
    rel_p, rel, head_rows = run_prefill_full(tsg, ctx, layer, offs, blobs, 2048, 2816, 704, 128,
                                             1.1, "gelu", 0x21F)
    assert head_rows > 1000
    assert rel_p <= kc.NORTH_STAR and rel <= kc.NORTH_STAR


def test_qwen_prefill_t4096_silu(tsg, ctx, qwen_layer):
    """configs[4] prefill: T = 4096, top-8 Zipf(1.0) over 256 experts of
    H = 2048, I = 512 with SwiGLU (the routed GEMM's SiLU activation,
    prefill.metal:78-86; QwenPrefill.swift:1020-1300)."""
    configure(ctx, 32, "sym")
    layer, offs, blobs = qwen_layer
    rel_p, rel, _ = run_prefill_full(tsg, ctx, layer, offs, blobs, 4096, 2048, 512, 256, 1.0,
                                     "silu", 0x4096)
    assert rel_p <= kc.NORTH_STAR and rel <= kc.NORTH_STAR


def run_fused_vs_two_launches(tsg, ctx, layer, t, d, f, ne, s, act, seed, tile=256,
                              device_list=True):
    """tsg_prefill_moe_gate_up_down against tsg_prefill_moe_gate_up then
    tsg_prefill_moe_down on the same grouping: act and route partials equal
    bit for bit."""
    k = 8
    rng = np.random.default_rng(seed)
    idx, w = wl.zipf_routing(rng, t, ne, k, s)
    hidden = dev(wl.f16_normal(rng, t * d))
    moe = tsg.MoE(ctx, gate_activation=act)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    max_blocks = -(-t * k // tile) + ne
    sp, off, cnt = empty(t * k * 4, np.uint32), empty(ne, np.uint32), empty(ne, np.uint32)
    blocks, nb = empty(max_blocks * 4, np.uint32), empty(1, np.uint32)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(dev(idx), dev(w), t, k, ne, sp, off, cnt, blocks, max_blocks, nb, scratch,
                         tile_rows=tile)
    n_blocks = int(host(nb, np.uint32)[0])
    kw = dict(n_blocks_device=nb) if device_list else {}
    nlist = max_blocks if device_list else n_blocks
    a2, p2 = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
    g.encode_gate_up(layer, hidden, d, sp, blocks, nlist, a2, d, f, **kw)
    g.encode_down(layer, a2, sp, blocks, nlist, p2, k, d, f, **kw)
    want_a, want_p = host(a2, np.uint16), host(p2, np.uint16)
    for rep in range(2):  # the second launch runs on the schedule the first left
        a1, p1 = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
        g.encode_gate_up_down(layer, hidden, d, sp, blocks, nlist, a1, p1, k, d, f, **kw)
        ctx.synchronize()
        assert np.array_equal(host(a1, np.uint16), want_a), f"act differs (launch {rep})"
        assert np.array_equal(host(p1, np.uint16), want_p), f"partials differ (launch {rep})"
    print(f"fused T={t} E={ne} {act}: {n_blocks} routed blocks, act and partials bitwise equal")
    return n_blocks


@pytest.mark.parametrize("shape", ["gemma-t2048", "gemma-t2048-tile128", "qwen-t4096", "gemma-t5",
                                   "gemma-t301-host"])
def test_fused_gate_up_down_matches_two_launches(tsg, ctx, gemma_layer, qwen_layer, shape):
    """The fused persistent GEMM equals the two grouped GEMMs bit for bit at
    configs[3] and configs[4]'s prefill sizes, at a verify-sized chunk (fewer
    routed blocks than XCDs) and with a host-counted block list; two launches
    in a row check that each leaves its schedule reset."""
    configure(ctx, 32, "sym")
    if shape == "gemma-t2048":
        run_fused_vs_two_launches(tsg, ctx, gemma_layer[0], 2048, 2816, 704, 128, 1.1, "gelu",
                                  0xF05E)
    elif shape == "gemma-t2048-tile128":  # blocks of at most 4 of the pass's 8 slices
        run_fused_vs_two_launches(tsg, ctx, gemma_layer[0], 2048, 2816, 704, 128, 1.1, "gelu",
                                  0xF05F, tile=128)
    elif shape == "qwen-t4096":
        run_fused_vs_two_launches(tsg, ctx, qwen_layer[0], 4096, 2048, 512, 256, 1.0, "silu",
                                  0xF06E)
    elif shape == "gemma-t5":
        nb = run_fused_vs_two_launches(tsg, ctx, gemma_layer[0], 5, 2816, 704, 128, 1.1, "gelu",
                                       0xF07E)
        assert nb < 40
    else:
        run_fused_vs_two_launches(tsg, ctx, gemma_layer[0], 301, 2816, 704, 128, 1.0, "gelu",
                                  0xF08E, tile=64, device_list=False)


def test_fused_gate_up_down_rejects_unaligned_act(tsg, ctx, gemma_layer):
    """The fused launch needs whole cache lines per activation row; an act
    buffer off a 128-byte boundary is refused before anything is enqueued."""
    configure(ctx, 32, "sym")
    layer = gemma_layer[0]
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    d, f, t, k = 2816, 704, 4, 8
    pairs = np.zeros(t * k * 4, np.uint32)
    blocks = np.array([(0, 0, 4, 0)], dtype=oracle.BLOCK_DTYPE).view(np.uint32)
    act = empty(t * k * f + 64)
    with pytest.raises(tsg.TsgError) as e:
        g.encode_gate_up_down(layer, empty(t * d), d, dev(pairs), dev(blocks), 1, act[8:],
                              empty(t * k * d), k, d, f)
    assert e.value.status == 2  # TSG_ERR_ALIGNMENT
    ctx.synchronize()


def test_grouped_gemm_skips_and_reports_expert_past_layer(tsg, ctx, gemma_layer):
    """A block list written on the device is not seen by the host: a block
    naming an expert past the layer is skipped by the grouped GEMM (two-launch
    and fused forms) and tsg_ctx_synchronize reports it; the other blocks'
    rows are written as usual."""
    configure(ctx, 32, "sym")
    layer = gemma_layer[0]
    d, f, k, t = 2816, 704, 8, 4
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    pairs = np.zeros(t * k, oracle.PAIR_DTYPE)
    pairs["token"] = np.repeat(np.arange(t, dtype=np.uint32), k)
    pairs["rank"] = np.tile(np.arange(k, dtype=np.uint32), t)
    blocks = np.array([(3, 0, 16, 0), (500, 16, 16, 16)], dtype=oracle.BLOCK_DTYPE)
    hidden = dev(wl.f16_normal(np.random.default_rng(5), t * d))
    P, B = dev(pairs), dev(blocks.view(np.uint32))
    for fused in (False, True):
        act, part = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
        if fused:
            g.encode_gate_up_down(layer, hidden, d, P, B, 2, act, part, k, d, f)
        else:
            g.encode_gate_up(layer, hidden, d, P, B, 2, act, d, f)
            g.encode_down(layer, act, P, B, 2, part, k, d, f)
        with pytest.raises(tsg.TsgError) as e:
            ctx.synchronize()
        assert "past the layer" in str(e.value)
        a = host(act, np.uint16).reshape(t * k, f)
        assert np.all(np.isfinite(oracle.f16_to_float(a[:16]))), "the valid block's rows"
        assert np.all(a[16:] == NAN16), "the skipped block wrote nothing"
    ctx.synchronize()  # the error word was cleared


def test_fused_gate_up_down_zero_row_blocks(tsg, ctx, gemma_layer):
    """Routed blocks with no rows, between real ones, are no-ops in both
    forms: the fused launch (64 blocks, 1,088 items, so every workgroup takes
    several and meets zero-row items after others) equals the two launches
    bit for bit and drains its schedule, twice in a row."""
    configure(ctx, 32, "sym")
    layer = gemma_layer[0]
    d, f, k, t = 2816, 704, 8, 64
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    pairs = np.zeros(t * k, oracle.PAIR_DTYPE)
    pairs["token"] = np.repeat(np.arange(t, dtype=np.uint32), k)
    pairs["rank"] = np.tile(np.arange(k, dtype=np.uint32), t)
    pairs["weight_bits"] = 0x3C00
    blocks = np.zeros(64, oracle.BLOCK_DTYPE)
    for i in range(64):
        real = i % 2 == 0
        j = i // 2
        blocks[i] = ((7 * i) % 128, 16 * j, 16 if real else 0, 16 * j)
    pairs["expert"] = np.repeat(blocks["local_slot"][::2], 16)
    hidden = dev(wl.f16_normal(np.random.default_rng(11), t * d))
    P, B = dev(pairs), dev(blocks.view(np.uint32))
    a2, p2 = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
    g.encode_gate_up(layer, hidden, d, P, B, 64, a2, d, f)
    g.encode_down(layer, a2, P, B, 64, p2, k, d, f)
    want_a, want_p = host(a2, np.uint16), host(p2, np.uint16)
    assert np.all(np.isfinite(oracle.f16_to_float(want_p)))
    for rep in range(2):
        a1, p1 = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
        g.encode_gate_up_down(layer, hidden, d, P, B, 64, a1, p1, k, d, f)
        ctx.synchronize()
        assert np.array_equal(host(a1, np.uint16), want_a), f"act differs (launch {rep})"
        assert np.array_equal(host(p1, np.uint16), want_p), f"partials differ (launch {rep})"


def test_fused_gate_up_down_empty_device_list(tsg, ctx, gemma_layer):
    """A device count of zero (no routed block) runs the fused launch to its
    end without work, writes nothing and reports nothing; the next launch on
    the same context still runs a real list (the schedule was left reset)."""
    configure(ctx, 32, "sym")
    layer = gemma_layer[0]
    d, f, k, t = 2816, 704, 8, 4
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    pairs = np.zeros(t * k, oracle.PAIR_DTYPE)
    pairs["token"] = np.repeat(np.arange(t, dtype=np.uint32), k)
    pairs["rank"] = np.tile(np.arange(k, dtype=np.uint32), t)
    blocks = np.array([(3, 0, t * k, 0)], dtype=oracle.BLOCK_DTYPE)
    hidden = dev(wl.f16_normal(np.random.default_rng(9), t * d))
    P, B = dev(pairs), dev(blocks.view(np.uint32))
    act, part = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
    g.encode_gate_up_down(layer, hidden, d, P, B, 1, act, part, k, d, f,
                          n_blocks_device=dev(np.zeros(1, np.uint32)))
    ctx.synchronize()
    assert np.all(host(act, np.uint16) == NAN16) and np.all(host(part, np.uint16) == NAN16)
    a2, p2 = empty(t * k * f, fill=NAN16), empty(t * k * d, fill=NAN16)
    g.encode_gate_up(layer, hidden, d, P, B, 1, a2, d, f)
    g.encode_down(layer, a2, P, B, 1, p2, k, d, f)
    g.encode_gate_up_down(layer, hidden, d, P, B, 1, act, part, k, d, f,
                          n_blocks_device=dev(np.ones(1, np.uint32)))
    ctx.synchronize()
    assert np.array_equal(host(act, np.uint16), host(a2, np.uint16))
    assert np.array_equal(host(part, np.uint16), host(p2, np.uint16))
