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
