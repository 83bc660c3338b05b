"""GPU: an installed MoEPack's layer files in HBM. The upload puts every
expert blob at its logical index whatever the file's physical order
(PackedExpertsLayout.swift:98-114, ModelExpertIO.swift:86-88). The bytes in
HBM equal the logical image. A decode layer run on the loaded layer gives the
same bits as one run on the image uploaded by hand, and both match the oracle
(routing bit-exact, y within 1e-3)."""
import numpy as np
import pytest

import oracle
from tests import kernelcheck as kc
from tests import moepack_writer as W
from tests.gpu_util import dev, empty, host

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


def bf16_from(values: np.ndarray) -> np.ndarray:
    return oracle.bf16_bits(np.ascontiguousarray(values, np.float32))


def random_parts(rng, ne, d, f, group):
    """Per expert (W, S, B) for gate, up, down: uniform nibbles, scales
    |N(0, .02)| / 7 and biases N(0, .01) as bf16 (the bench's draw)."""
    experts = []
    for _ in range(ne):
        parts = []
        for rows, k in ((f, d), (f, d), (d, f)):
            g = rows * (k // group)
            packed = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
            scales = bf16_from(np.abs(rng.normal(0, 0.02, g)) / 7).reshape(rows, k // group)
            biases = bf16_from(rng.normal(0, 0.01, g)).reshape(rows, k // group)
            parts.append((packed, scales, biases))
        experts.append(parts)
    return experts


@pytest.mark.parametrize("d,f,ne,group,scheme,act", [
    (768, 256, 32, 32, "affine", "gelu"),
    (1024, 512, 64, 64, "sym", "silu"),
])
def test_loaded_layers_match_the_logical_image(tsg, ctx, tmp_path, d, f, ne, group, scheme,
                                               act):
    import torch
    sym = scheme == "sym"
    print(f"moepack load d={d} f={f} ne={ne} g{group} {scheme} {act}", flush=True)
    rng = np.random.default_rng(0x3E + d)
    layers = [random_parts(rng, ne, d, f, group) for _ in range(2)]
    perms = [rng.permutation(ne), rng.permutation(ne)]
    stride, offs, images = W.write_pack(tmp_path, layers, d=d, f=f, group=group, symmetric=sym,
                                        physical=perms)
    pack = tsg.MoEPack.open(tmp_path)
    pack.configure(ctx)
    assert (ctx.group_size, ctx.scheme) == (group, scheme)

    # Bytes: each layer uploaded into caller-owned HBM equals its logical image.
    for li in range(2):
        buf = torch.zeros(ne * stride, dtype=torch.uint8, device="cuda")
        wrapped = tsg.ResidentLayer(ctx, ne, stride, pack.routed_offsets(li), device_tensor=buf)
        pack.upload_layer(wrapped, li)
        assert np.array_equal(host(buf, np.uint8), images[li]), f"layer {li} bytes differ"
        wrapped.close()

    # Compute: the decode layer on a loaded layer == on the hand-uploaded image.
    loaded = pack.load_layer(ctx, 1)
    by_hand = tsg.ResidentLayer(ctx, ne, stride, offs)
    by_hand.upload(images[1])
    rw_bits = bf16_from(rng.normal(0, 1.0 / np.sqrt(d), ne * d))
    es_bits = bf16_from(1.0 + np.abs(rng.normal(0, 0.1, d)))
    pes_bits = bf16_from(np.linspace(0.8, 1.2, ne))
    x_bits = oracle.f16_bits(rng.normal(0, 1.0, d).astype(np.float32))
    res_bits = oracle.f16_bits(rng.normal(0, 0.5, d).astype(np.float32))
    rw, es, pes, x, res = (dev(a) for a in (rw_bits, es_bits, pes_bits, x_bits, res_bits))
    moe = tsg.MoE(ctx, gate_activation=act)
    outs = []
    for layer in (loaded, by_hand):
        y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
        moe.encode_decode_layer(layer, rw, x, es, pes, x, res, y, idx, wts, acts, ne, d, f)
        ctx.synchronize()
        outs.append([host(y, np.uint16), host(idx, np.uint32), host(wts, np.uint16)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    y, gi, gw = outs[0]
    canon = oracle.router_logits_canonical(rw_bits, x_bits, d, es_bits, 1, ne, d)
    ci, cw = oracle.topk_softmax(canon[0], 8, oracle.bf16_to_float(pes_bits))
    assert list(gi) == list(ci)
    assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1
    blobs = [np.ascontiguousarray(images[1][e * stride:(e + 1) * stride]) for e in gi]
    ref = oracle.moe_apply_streamed_routed(
        blobs, np.array(offs, np.uint32), oracle.f16_to_float(x_bits),
        oracle.f16_to_float(res_bits), oracle.f16_to_float(gw), d, f, group, symmetric=sym,
        act=1 if act == "silu" else 0)
    rel = oracle.relative_error(oracle.f16_to_float(y), ref)
    print(f"  rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR
    loaded.close()
    by_hand.close()


def test_load_errors(tsg, ctx, tmp_path):
    import torch
    rng = np.random.default_rng(7)
    layers = [random_parts(rng, 8, 128, 64, 32)]
    stride, offs, images = W.write_pack(tmp_path, layers, d=128, f=64, group=32,
                                        symmetric=False)
    pack = tsg.MoEPack.open(tmp_path)
    # destination of another geometry: nothing written
    buf = torch.zeros(8 * stride, dtype=torch.uint8, device="cuda")
    other = tsg.ResidentLayer(ctx, 4, stride, offs, device_tensor=buf)
    with pytest.raises(tsg.TsgError) as e:
        pack.upload_layer(other, 0)
    assert e.value.status == 1 and "geometry" in str(e.value)
    assert not host(buf, np.uint8).any()
    # a parsed pack has no layer files
    mem = tsg.MoEPack.parse((tmp_path / "manifest.json").read_bytes(),
                            (tmp_path / "packed_experts" / "layout.json").read_bytes())
    with pytest.raises(tsg.TsgError) as e:
        mem.load_layer(ctx, 0)
    assert e.value.status == 1 and "parsed from memory" in str(e.value)
    # a truncated layer file
    path = tmp_path / "packed_experts" / "layer_00.bin"
    path.write_bytes(path.read_bytes()[:-16384])
    with pytest.raises(tsg.TsgError) as e:
        pack.load_layer(ctx, 0)
    assert e.value.status == 7 and "layout says" in str(e.value)


@pytest.mark.parametrize("scheme,group", [("affine", 64), ("sym", 32)])
def test_two_byte_aligned_install(tsg, ctx, tmp_path, scheme, group):
    """An install whose sub-tensors are only 2-byte aligned (the repacker's
    guarantee, DequantInt4GEMV.swift:93-96): tsg_moepack_load_layer lays the
    HBM image out anew (every sub-tensor on 256 bytes) and the decode layer
    and both prefill GEMMs on it give the bits they give on the same experts
    packed 16-byte aligned; decode matches the oracle. Wrapping caller-owned
    HBM with such offsets is refused."""
    import torch
    sym = scheme == "sym"
    d, f, ne = 512, 256, 16
    rng = np.random.default_rng(0x2A11)
    parts = random_parts(rng, ne, d, f, group)
    stride2, offs2, images2 = W.write_pack(tmp_path / "a2", [parts], d=d, f=f, group=group,
                                           symmetric=sym, align=2, lead=2)
    assert all(int(o) % 16 == 2 for o in offs2), offs2
    stride16, offs16, images16 = W.write_pack(tmp_path / "a16", [parts], d=d, f=f, group=group,
                                              symmetric=sym)
    pack = tsg.MoEPack.open(tmp_path / "a2")
    pack.configure(ctx)
    loaded = pack.load_layer(ctx, 0)
    dstride, doffs = loaded.device_geometry()
    assert dstride % 16384 == 0 and all(o % 256 == 0 for o in doffs)
    aligned = tsg.ResidentLayer(ctx, ne, stride16, offs16)
    aligned.upload(images16[0])
    with pytest.raises(tsg.TsgError) as e:
        buf = torch.zeros(ne * stride2, dtype=torch.uint8, device="cuda")
        tsg.ResidentLayer(ctx, ne, stride2, offs2, device_tensor=buf)
    assert e.value.status == 2
    # decode layer
    rw_bits = bf16_from(rng.normal(0, 1.0 / np.sqrt(d), ne * d))
    es_bits = bf16_from(np.ones(d))
    pes_bits = bf16_from(np.ones(ne))
    x_bits = oracle.f16_bits(rng.normal(0, 1.0, d).astype(np.float32))
    res_bits = oracle.f16_bits(rng.normal(0, 0.5, d).astype(np.float32))
    rw, es, pes, x, res = (dev(a) for a in (rw_bits, es_bits, pes_bits, x_bits, res_bits))
    moe = tsg.MoE(ctx)
    outs = []
    for layer in (loaded, aligned):
        y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
        moe.encode_decode_layer(layer, rw, x, es, pes, x, res, y, idx, wts, acts, ne, d, f)
        ctx.synchronize()
        outs.append([host(y, np.uint16), host(idx, np.uint32), host(wts, np.uint16)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    y, gi, gw = outs[0]
    blobs = [np.ascontiguousarray(images16[0][e * stride16:(e + 1) * stride16]) for e in gi]
    ref = oracle.moe_apply_streamed_routed(
        blobs, np.array(offs16, np.uint32), oracle.f16_to_float(x_bits),
        oracle.f16_to_float(res_bits), oracle.f16_to_float(gw), d, f, group, symmetric=sym)
    rel = oracle.relative_error(oracle.f16_to_float(y), ref)
    assert rel <= kc.NORTH_STAR
    # prefill GEMMs: 24 tokens x top-8 over the 16 experts
    t, k = 24, 8
    idx_np = np.stack([rng.permutation(ne)[:k] for _ in range(t)]).astype(np.uint32)
    w_np = np.full((t, k), 0x3000, np.uint16)
    grouped = oracle.group_pairs(oracle.make_token_expert_pairs(idx_np, w_np, t, k), t, k, ne)
    sp = grouped["sorted_pairs"]
    blocks = np.array([(int(g_["expert"]), int(g_["pair_start"]), int(g_["pair_count"]),
                        int(g_["pair_start"])) for g_ in grouped["groups"]],
                      dtype=oracle.BLOCK_DTYPE)
    hid = dev(oracle.f16_bits(rng.normal(0, 1.0, t * d).astype(np.float32)))
    g = tsg.PrefillGroupedRoutedMoE(moe)
    P, B = dev(sp), dev(blocks)
    parts_out = []
    for layer in (loaded, aligned):
        act, partials = empty(t * k * f), empty(t * k * d)
        g.encode_gate_up(layer, hid, d, P, B, blocks.size, act, d, f)
        g.encode_down(layer, act, P, B, blocks.size, partials, k, d, f)
        parts_out.append(host(partials, np.uint16))
    assert np.array_equal(parts_out[0], parts_out[1])
    print(f"2-byte aligned install {scheme} g{group}: decode rel={rel:.3e}, "
          f"device stride {dstride} (file {stride2})")
    loaded.close()
    aligned.close()
