"""GPU parity: the Qwen shared expert and its sigmoid gate (qwen.metal:33-34,
432-455, 466, 1038-1046; QwenForwardRunner.swift:1548-1578) against the
oracle within the north-star bound, the two-launch fused form bit-identical
to the reference's step-by-step sequence, and the entry points' errors."""
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


def configure(ctx, group, symmetric):
    ctx.set_affine_group_size(group)
    ctx.set_affine_scheme("sym" if symmetric else "affine")


def test_silu_mul(tsg, ctx):
    rng = oracle.seed_tree_key(0x51, "silu-mul")
    n = 4099
    g = rng.uniforms_f16(-8.0, 8.0, n)
    u = rng.uniforms_f16(-2.0, 2.0, n)
    out = empty(n)
    tsg.QwenKernels(ctx).encode_silu_mul(dev(g), dev(u), out, n)
    got = oracle.f16_to_float(host(out, np.uint16))
    want = oracle.f16_to_float(oracle.silu_mul_f16(g, u))
    rel = oracle.relative_error(got, want)
    print(f"silu_mul n={n}: rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


@pytest.mark.parametrize("d", [2048, 2816, 96])
def test_shared_gate(tsg, ctx, d):
    rng = oracle.seed_tree_key(0x52 + d, "shared-gate")
    y = rng.uniforms_f16(-1.0, 1.0, d)
    x = rng.uniforms_f16(-1.0, 1.0, d)
    w = rng.uniforms_bf16(-0.1, 0.1, d)
    yt = dev(y)
    tsg.QwenKernels(ctx).encode_moe_shared_gate(yt, dev(x), dev(w), d)
    got = oracle.f16_to_float(host(yt, np.uint16))
    want = oracle.f16_to_float(oracle.shared_gate_f16(y, x, w))
    rel = oracle.relative_error(got, want)
    print(f"shared_gate d={d}: rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


def test_shared_gate_logit(tsg, ctx):
    d = 2048
    rng = oracle.seed_tree_key(0x53, "shared-gate-logit")
    y = rng.uniforms_f16(-1.0, 1.0, d)
    logit = oracle.f16_bits(np.array([0.8125], np.float32))
    yt = dev(y)
    tsg.QwenKernels(ctx).encode_moe_shared_gate_logit(yt, dev(logit), d)
    # the same gate as a one-term dot product: x = (logit, 0, ...), w = (1, 0, ...)
    x1 = np.zeros(d, np.uint16)
    x1[0] = logit[0]
    w1 = np.zeros(d, np.uint16)
    w1[0] = oracle.bf16_bits(np.array([1.0], np.float32))[0]
    want = oracle.f16_to_float(oracle.shared_gate_f16(y, x1, w1))
    rel = oracle.relative_error(oracle.f16_to_float(host(yt, np.uint16)), want)
    assert rel <= kc.NORTH_STAR


@pytest.mark.parametrize("d,f,group,symmetric", [(2048, 512, 32, True), (2048, 512, 64, False),
                                                 (2816, 704, 32, True), (256, 64, 32, False)])
def test_shared_expert_fused_vs_steps_and_oracle(tsg, ctx, d, f, group, symmetric):
    configure(ctx, group, symmetric)
    c = kc.shared_expert_case(d, f, group, 0x5E + d + f, symmetric)
    moe = tsg.MoE(ctx, gate_activation="silu")
    blob, x, gw = dev(c["blob"]), dev(c["x_bits"]), dev(c["gate_w"])
    act = empty(f)
    out = empty(d)
    print(f"shared expert d={d} f={f} g={group} sym={symmetric}", flush=True)
    tsg.encode_shared_expert(moe, blob, c["offsets"], x, gw, act, out, d, f)
    fused = host(out, np.uint16)
    # the reference's sequence: GEMV gate, GEMV up, silu_mul, GEMV down, gate
    q = tsg.DequantInt4GEMV(ctx)
    o = c["offsets"]
    import torch
    bb = blob.view(torch.uint8)
    g_out, u_out, a_out, d_out = empty(f), empty(f), empty(f), empty(d)
    q.encode(bb[o[0]:], bb[o[1]:], bb[o[2]:], x, g_out, f, d)
    q.encode(bb[o[3]:], bb[o[4]:], bb[o[5]:], x, u_out, f, d)
    tsg.QwenKernels(ctx).encode_silu_mul(g_out, u_out, a_out, f)
    q.encode(bb[o[6]:], bb[o[7]:], bb[o[8]:], a_out, d_out, d, f)
    tsg.QwenKernels(ctx).encode_moe_shared_gate(d_out, x, gw, d)
    steps = host(d_out, np.uint16)
    assert np.array_equal(host(act, np.uint16), host(a_out, np.uint16))
    assert np.array_equal(fused, steps)
    rel = oracle.relative_error(oracle.f16_to_float(fused), oracle.f16_to_float(c["ref"]))
    print(f"  rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


def test_shared_expert_errors(tsg, ctx):
    configure(ctx, 32, True)
    moe = tsg.MoE(ctx, gate_activation="silu")
    c = kc.shared_expert_case(64, 32, 32, 0x5F, True)
    blob, x, gw = dev(c["blob"]), dev(c["x_bits"]), dev(c["gate_w"])
    act, out = empty(32), empty(64)
    with pytest.raises(tsg.TsgError) as e:
        tsg.encode_shared_expert(moe, blob, c["offsets"], x, gw, act, out, 48, 32)
    assert e.value.status == 1  # d not a multiple of the group size
    bad = np.array(c["offsets"], np.uint32)
    bad[0] += 8  # gate weights off the 16-byte grid
    with pytest.raises(tsg.TsgError) as e:
        tsg.encode_shared_expert(moe, blob, bad, x, gw, act, out, 64, 32)
    assert e.value.status == 2
    with pytest.raises(tsg.TsgError) as e:
        tsg.QwenKernels(ctx).encode_silu_mul(act, act, act, 0)
    assert e.value.status == 4  # nothing to encode: the reference returns false


# ------------------------------------------- Gemma dense MLP (SharedExpertInt4)

def test_gelu_mul(tsg, ctx):
    rng = oracle.seed_tree_key(0x61, "gelu-mul")
    n = 4099
    g = rng.uniforms_f16(-8.0, 8.0, n)
    u = rng.uniforms_f16(-2.0, 2.0, n)
    out = empty(n)
    tsg.SharedExpertInt4(ctx).encode_gelu_mul(dev(g), dev(u), out, n)
    got = host(out, np.uint16)
    want = oracle.gelu_mul_f16(g, u)
    # The kernel computes 0.5 x (1 + tanh(u)) as x / (1 + exp(-2u)), the oracle
    # with tanhf. For u below about -3.8, 1 + tanhf(u) has lost more than an fp16
    # ulp to cancellation in fp32, so the exact function decides: GELU in
    # float64, rounded once to fp16, is within one ulp of the kernel wherever it
    # is a normal fp16 value; against the oracle the vector bound applies.
    g64 = oracle.f16_to_float(g).astype(np.float64)
    u64 = np.clip(0.7978845608028654 * (g64 + 0.044715 * g64 ** 3), -20.0, 20.0)
    exact = (0.5 * g64 * (1.0 + np.tanh(u64)) * oracle.f16_to_float(u).astype(np.float64))
    exact16 = exact.astype(np.float16)
    normal = np.abs(exact16) >= np.float16(2.0 ** -14)
    diff = np.abs(got.astype(np.int32) - exact16.view(np.uint16).astype(np.int32))[normal]
    assert diff.max() <= 1, f"max ulp {diff.max()}"
    assert oracle.relative_error(oracle.f16_to_float(got), oracle.f16_to_float(want)) <= kc.NORTH_STAR


def _dense_parts(d, f, group, seed, symmetric):
    rng = oracle.seed_tree_key(seed, f"dense-mlp-d{d}-f{f}")
    gate = kc.quantized_rows(rng, f, d, group, symmetric, -0.3, 0.3)
    up = kc.quantized_rows(rng, f, d, group, symmetric, -0.3, 0.3)
    down = kc.quantized_rows(rng, d, f, group, symmetric, -0.3, 0.3)
    x = rng.uniforms_f16(-1.0, 1.0, d)
    return gate, up, down, x


@pytest.mark.parametrize("d,f,group,symmetric", [(2816, 2112, 32, True), (2816, 2112, 64, False),
                                                 (256, 128, 32, False)])
def test_shared_expert_int4_matches_steps_and_oracle(tsg, ctx, d, f, group, symmetric):
    """Gemma's dense MLP (F = 2112, SharedExpertInt4.swift:30-93): the one call
    equals QMV gate, QMV up, gelu_mul, QMV down bit for bit, and the oracle's
    DequantInt4GemvRef composition within 1e-3."""
    configure(ctx, group, symmetric)
    gate, up, down, x = _dense_parts(d, f, group, 0x6F + f, symmetric)
    S = tsg.SharedExpertInt4(ctx)
    dv = [tuple(dev(a) for a in t) for t in (gate, up, down)]
    proj = [S.projection(w, s, None if symmetric else b, r, c)
            for (w, s, b), (r, c) in zip(dv, ((f, d), (f, d), (d, f)))]
    xd = dev(x)
    y, sg, su, sa = empty(d), empty(f), empty(f), empty(f)
    print(f"dense mlp d={d} f={f} g{group} sym={symmetric}", flush=True)
    S.encode(xd, *proj, y, sg, su, sa)
    fused = host(y, np.uint16)
    q = tsg.DequantInt4GEMV(ctx)
    g1, u1, a1, y1 = empty(f), empty(f), empty(f), empty(d)
    bias = lambda t: t[1] if symmetric else t[2]
    q.encode(dv[0][0], dv[0][1], bias(dv[0]), xd, g1, f, d)
    q.encode(dv[1][0], dv[1][1], bias(dv[1]), xd, u1, f, d)
    S.encode_gelu_mul(g1, u1, a1, f)
    q.encode(dv[2][0], dv[2][1], bias(dv[2]), a1, y1, d, f)
    assert np.array_equal(fused, host(y1, np.uint16))
    want = oracle.dense_mlp_int4(gate, up, down, x, d, f, group, symmetric)
    rel = oracle.relative_error(oracle.f16_to_float(fused), oracle.f16_to_float(want))
    print(f"  rel={rel:.3e}")
    assert rel <= kc.NORTH_STAR


def test_shared_expert_int4_errors(tsg, ctx):
    """SharedExpertError.dimensionMismatch / .scratchTooSmall."""
    configure(ctx, 32, True)
    d, f = 64, 32
    gate, up, down, x = _dense_parts(d, f, 32, 0x70, True)
    S = tsg.SharedExpertInt4(ctx)
    dv = [tuple(dev(a) for a in t) for t in (gate, up, down)]
    pg = S.projection(dv[0][0], dv[0][1], None, f, d)
    pu = S.projection(dv[1][0], dv[1][1], None, f, d)
    pd = S.projection(dv[2][0], dv[2][1], None, d, f)
    bad = S.projection(dv[2][0], dv[2][1], None, d, f + 32)
    y, sg, su, sa = empty(d), empty(f), empty(f), empty(f)
    with pytest.raises(tsg.TsgError) as e:
        S.encode(dev(x), pg, pu, bad, y, sg, su, sa)
    assert e.value.status == 1 and "dimensionMismatch" in str(e.value)
    with pytest.raises(tsg.TsgError) as e:
        S.encode(dev(x), pg, pu, pd, y, sg, su, empty(f - 8))
    assert e.value.status == 1 and "scratchTooSmall" in str(e.value)
    with pytest.raises(tsg.TsgError) as e:
        S.encode(dev(x), pg, pu, pd, empty(d - 8), sg, su, sa)
    assert e.value.status == 1 and "output range exceeds y buffer" in str(e.value)
    with pytest.raises(tsg.TsgError) as e:
        S.encode_gelu_mul(sg, su, sa, 0)
    assert e.value.status == 4
