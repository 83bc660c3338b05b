"""GPU parity: the INT8-affine router (tsg_moe_router_int8, encodeRouterGemma4,
MoE.swift:201-257) on the reference's KernelCheck fixture (checkRouter(weightBits:
8), main.swift:409-520, seed 0xD1) and its RouterTopKTests cases, against the
oracle's routerReference and its restatement of the kernel's summation order."""
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


@pytest.fixture(scope="module")
def ctx(tsg):
    return tsg.Context(0)


def run_int8_router(moe, c, ne, d):
    idx, wts = empty(8, np.uint32), empty(8)
    moe.encode_router_gemma4(dev(c["packed"]), dev(c["scales"]), dev(c["biases"]),
                             dev(c["hidden"]), dev(c["es_bits"]), dev(c["pes_bits"]), idx, wts,
                             ne, d)
    return host(idx, np.uint32), host(wts, np.uint16)


def kernel_order_selection(c, ne, d, group):
    logits = oracle.router_logits_int8_canonical(c["packed"], c["scales"], c["biases"],
                                                 c["hidden"], c["es_bits"], ne, d, group)
    return oracle.topk_softmax(logits, 8, oracle.bf16_to_float(c["pes_bits"]))


@pytest.mark.parametrize("group", [64, 32])
def test_router_int8_kernelcheck(tsg, ctx, group):
    """checkRouter(weightBits: 8, d: 2816, experts: 128, draws: 4, seed: 0xD1):
    indices equal routerReference's over the dequantised rows, weights within
    Tolerance.fp16Reduction; indices equal, and weights within one fp16 ulp of,
    the kernel rule applied to the oracle's kernel-order logits."""
    ctx.set_affine_group_size(group)
    d, ne = 2816, 128
    moe = tsg.MoE(ctx, router_weight_bits=8)
    for draw in range(4):
        c = kc.router_int8_case(d, ne, group, 0xD1, draw)
        gi, gw = run_int8_router(moe, c, ne, d)
        assert list(gi) == list(c["idx"]), f"g{group} draw {draw}: gpu={gi} cpu={c['idx']}"
        assert oracle.relative_error(oracle.f16_to_float(gw), c["wts"]) <= kc.FP16_REDUCTION
        ci, cw = kernel_order_selection(c, ne, d, group)
        assert list(gi) == list(ci)
        assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1


@pytest.mark.parametrize("kind", ["spread", "near_tie"])
def test_router_int8_reference_router_tests(tsg, ctx, kind):
    """RouterTopKTests.productionRouterMatchesReference and
    productionRouterResolvesNearTieLikeReference (RouterTopKTests.swift:17-69):
    16 experts, d = 128, group 64; same indices, weights within 5e-3."""
    ctx.set_affine_group_size(64)
    c = kc.router_topk_test_case(kind)
    moe = tsg.MoE(ctx, router_weight_bits=8)
    gi, gw = run_int8_router(moe, c, c["ne"], c["d"])
    assert list(gi) == list(c["idx"]), f"{kind}: gpu={gi} cpu={c['idx']}"
    assert np.abs(oracle.f16_to_float(gw) - c["wts"]).max() < 5e-3
    ci, _ = kernel_order_selection(c, c["ne"], c["d"], 64)
    assert list(gi) == list(ci)


def test_router_int8_small_and_ragged_expert_counts(tsg, ctx):
    """Expert counts that leave waves of the last block without a row, and
    fewer experts than top-8 (the unfilled slots keep expert 0, weight 0)."""
    ctx.set_affine_group_size(32)
    d = 2048
    moe = tsg.MoE(ctx, router_weight_bits=8)
    for ne in (5, 37, 256):
        c = kc.router_int8_case(d, ne, 32, 0xD1, 7)
        gi, gw = run_int8_router(moe, c, ne, d)
        ci, cw = kernel_order_selection(c, ne, d, 32)
        assert list(gi) == list(ci), f"ne={ne}: gpu={gi} oracle={ci}"
        assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1


def test_router_formats_are_checked(tsg, ctx):
    """Each router entry point takes only its own weight format (the
    reference's preconditions, MoE.swift:213-214, 269-270), and the INT8
    router's row geometry (d a multiple of 64 and of the group size)."""
    ctx.set_affine_group_size(64)
    d, ne = 2816, 128
    c = kc.router_int8_case(d, ne, 64, 0xD1, 0)
    m8 = tsg.MoE(ctx, router_weight_bits=8)
    m16 = tsg.MoE(ctx, router_weight_bits=16)
    idx, wts = empty(8, np.uint32), empty(8)
    with pytest.raises(tsg.TsgError) as e:
        run_int8_router(m16, c, ne, d)
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT
    w16 = dev(np.zeros(ne * d, np.uint16))
    with pytest.raises(tsg.TsgError) as e:
        m8.encode_router_gemma4_bf16(w16, dev(c["hidden"]), dev(c["es_bits"]),
                                     dev(c["pes_bits"]), idx, wts, ne, d)
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT
    with pytest.raises(tsg.TsgError) as e:
        run_int8_router(m8, c, ne, d - 32)
    assert e.value.status == tsg._abi.TSG_ERR_INVALID_ARGUMENT
    with pytest.raises(tsg.TsgError):
        tsg.MoE(ctx, router_weight_bits=4)


def test_int8_router_decode_layer_gemma_shape(tsg, ctx):
    """The decode layer of a MoE with the INT8-affine router (MoE.init's
    default): encodeRouterGemma4, then phase 1 and phase 2 on the
    HBM-resident Gemma-shaped layer with the expert ids read on the device
    (RealForwardRunner's per-layer sequence, RealForwardRunner.swift:3104-3330).
    Routing bit-exact against the oracle's kernel-order logits and top-k rule;
    y within 1e-3 of MoeRef.applyStreamedRouted over the chosen experts; the
    one-launch INT8 layer (and its three-launch form) equal to that sequence
    bit for bit."""
    import torch
    from tests.test_gpu_qmv_decode import make_gemma_layer
    ctx.set_affine_group_size(32)
    ctx.set_affine_scheme("sym")
    d, f, ne = 2816, 704, 128
    layer, buf, offs, stride = make_gemma_layer(tsg, ctx, 0x5EE8)
    rng = np.random.default_rng(0x1D8)
    raw = rng.normal(0.0, 1.0 / np.sqrt(d), (ne, d)).astype(np.float32)
    packed, scales, biases = oracle.quantize_int8_affine(raw, 32)
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0xA18, 1.0)
    es = np.full(d, 0x3F80, np.uint16)
    pes = oracle.bf16_bits(rng.uniform(0.8, 1.2, ne).astype(np.float32))
    moe = tsg.MoE(ctx, router_weight_bits=8)
    idx, wts = empty(8, np.uint32), empty(8)
    acts, y = empty(8 * f), empty(d)
    moe.encode_router_gemma4(dev(packed), dev(scales), dev(biases), x, dev(es), dev(pes), idx,
                             wts, ne, d)
    moe.encode_phase1_resident(layer, idx, x, acts, d, f)
    moe.encode_phase2_resident(layer, idx, acts, wts, x, y, d, f)
    gi, gw = host(idx, np.uint32), host(wts, np.uint16)
    xb = host(x, np.uint16)
    logits = oracle.router_logits_int8_canonical(packed, scales, biases, xb, es, ne, d, 32)
    ci, cw = oracle.topk_softmax(logits, 8, oracle.bf16_to_float(pes))
    assert list(gi) == list(ci)
    assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1
    image = host(buf, np.uint8)
    blobs = [np.ascontiguousarray(image[e * stride:(e + 1) * stride]) for e in gi]
    xf = oracle.f16_to_float(xb)
    ref = oracle.moe_apply_streamed_routed(blobs, np.array(offs, np.uint32), xf, xf,
                                           oracle.f16_to_float(gw), d, f, 32, symmetric=True)
    rel = oracle.relative_error(oracle.f16_to_float(host(y, np.uint16)), ref)
    print(f"int8-router decode layer: experts={list(gi)} rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR
    # tsg_moe_decode_layer_int8: one launch, and forced to three launches,
    # both the bits of the sequence above
    for fused in (True, False):
        moe.set_fused_decode(fused)
        idx2, wts2, acts2, y2 = empty(8, np.uint32), empty(8), empty(8 * f), empty(d)
        moe.encode_decode_layer_int8(layer, dev(packed), dev(scales), dev(biases), x, dev(es),
                                     dev(pes), x, x, y2, idx2, wts2, acts2, ne, d, f)
        ctx.synchronize()  # reports a one-launch hand-off timeout
        assert np.array_equal(host(idx2, np.uint32), gi), f"fused={fused}"
        assert np.array_equal(host(wts2, np.uint16), gw), f"fused={fused}"
        assert np.array_equal(host(y2, np.uint16), host(y, np.uint16)), f"fused={fused}"
    moe.set_fused_decode(True)
    # each decode-layer entry takes only its own router format
    with pytest.raises(tsg.TsgError):
        moe.encode_decode_layer(layer, dev(np.zeros(ne * d, np.uint16)), x, dev(es), dev(pes),
                                x, x, y, idx, wts, acts, ne, d, f)
    m16 = tsg.MoE(ctx, router_weight_bits=16)
    with pytest.raises(tsg.TsgError):
        m16.encode_decode_layer_int8(layer, dev(packed), dev(scales), dev(biases), x, dev(es),
                                     dev(pes), x, x, y, idx, wts, acts, ne, d, f)


@pytest.mark.parametrize("d,f,ne,group,scheme,act", [
    (2816, 704, 128, 32, "sym", "gelu"),
    (2048, 512, 256, 64, "affine", "silu"),
    (768, 256, 32, 32, "affine", "gelu"),
])
def test_int8_decode_layer_one_launch_matches_three(tsg, ctx, d, f, ne, group, scheme, act):
    """tsg_moe_decode_layer_int8 in one launch and as router + phase 1 + phase
    2 give the same bits; routing bit-exact against the oracle's kernel-order
    INT8 logits, y within 1e-3 of MoeRef.applyStreamedRouted."""
    import torch
    from tests.test_gpu_qmv_decode import make_layer
    ctx.set_affine_group_size(group)
    ctx.set_affine_scheme(scheme)
    sym = scheme == "sym"
    layer, buf, offs, stride = make_layer(tsg, ctx, 0x4321 + d, ne, d, f, group, sym)
    rng = np.random.default_rng(d + ne)
    raw = rng.normal(0.0, 1.0 / np.sqrt(d), (ne, d)).astype(np.float32)
    packed, scales, biases = oracle.quantize_int8_affine(raw, group)
    es_bits = oracle.bf16_bits(rng.uniform(0.5, 1.5, d).astype(np.float32))
    pes_bits = oracle.bf16_bits(np.linspace(0.8, 1.2, ne).astype(np.float32))
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0xC12 + d, 1.0)
    res = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(res, 0xC14 + d, 0.5)
    moe = tsg.MoE(ctx, router_weight_bits=8, gate_activation=act)
    outs = {}
    for fused in (True, False):
        moe.set_fused_decode(fused)
        y, idx, wts, acts = empty(d), empty(8, np.uint32), empty(8), empty(8 * f)
        moe.encode_decode_layer_int8(layer, dev(packed), dev(scales), dev(biases), x,
                                     dev(es_bits), dev(pes_bits), x, res, y, idx, wts, acts,
                                     ne, d, f)
        ctx.synchronize()  # raises if the one-launch hand-off timed out
        outs[fused] = [host(t, np.uint16 if t is not idx else np.uint32)
                       for t in (y, idx, wts, acts)]
    for a, b in zip(outs[True], outs[False]):
        assert np.array_equal(a, b)
    y, gi, gw, _ = outs[True]
    xb = host(x, np.uint16)
    logits = oracle.router_logits_int8_canonical(packed, scales, biases, xb, es_bits, ne, d,
                                                 group)
    ci, cw = oracle.topk_softmax(logits, 8, oracle.bf16_to_float(pes_bits))
    assert list(gi) == list(ci)
    assert np.max(np.abs(gw.astype(np.int32) - cw.astype(np.int32))) <= 1
    image = host(buf, np.uint8)
    blobs = [np.ascontiguousarray(image[e * stride:(e + 1) * stride]) for e in gi]
    ref = oracle.moe_apply_streamed_routed(
        blobs, np.array(offs, np.uint32), oracle.f16_to_float(xb),
        oracle.f16_to_float(host(res, np.uint16)), oracle.f16_to_float(gw), d, f, group,
        symmetric=sym, act=1 if act == "silu" else 0)
    rel = oracle.relative_error(oracle.f16_to_float(y), ref)
    print(f"int8 decode layer d={d} f={f} ne={ne} g{group} {scheme} {act}: rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR
