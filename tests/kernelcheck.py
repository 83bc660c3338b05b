"""Fixtures of the reference's TsugumiKernelCheck harness, regenerated bit for
bit from SplitMix64/SeedTree through the oracle, plus helpers shared by the
GPU parity tests.

Each builder cites the harness function whose fixture it reproduces
(Sources/TsugumiKernelCheck/main.swift, PrefillMoEGEMMCheck.swift).
"""
from __future__ import annotations

import numpy as np

import oracle

# Tolerance.swift:4-21 and the north-star bound.
FP16_REDUCTION = 5e-3
FP16_CHAINED = 1e-2
NORTH_STAR = 1e-3


def quantized_rows(rng, count, n, group, symmetric, lo=-0.5, hi=0.5):
    """quantizedRows (main.swift:120-131): row-major uniform draws, quantised."""
    raw = rng.uniforms(lo, hi, count * n).reshape(count, n)
    return oracle.quantize_int4(raw, group, symmetric)


def int4_gemv_case(m, n, group, seed, symmetric):
    """checkInt4GEMV fixture (main.swift:145-151)."""
    rng = oracle.seed_tree_key(seed, f"int4-gemv-m{m}-n{n}-g{group}")
    packed, scales, biases = quantized_rows(rng, m, n, group, symmetric)
    x_bits = rng.uniforms_f16(-1.0, 1.0, n)
    ref = oracle.dequant_int4_gemv_ref(packed, scales, biases, oracle.f16_to_float(x_bits), n,
                                       group)
    return dict(packed=packed, scales=scales, biases=biases, x_bits=x_bits, ref=ref)


def pack_blob(parts, symmetric, keep_biases=True, align=16, lead=0):
    """Expert blob in the packer's order gate(W,S,[B]), up, down
    (RepackPlanner.swift:442-520). Returns bytes and the 9 MoEExpertOffsets
    (bias offsets alias the scales when the bias is left out). Sub-tensors are
    placed at `align`-byte boundaries after `lead` leading zero bytes (lead=2,
    align=2 gives the 2-byte aligned sub-tensors the repacker allows,
    DequantInt4GEMV.swift:93-96)."""
    chunks, offs, cur = [], [], 0
    if lead:
        chunks.append(np.zeros(lead, np.uint8))
        cur = lead
    for (p, s, b) in parts:
        for arr, is_bias in ((p, False), (s, False), (b, True)):
            if is_bias and not keep_biases:
                offs.append(offs[-1])
                continue
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            pad = (-cur) % align
            if pad:
                chunks.append(np.zeros(pad, np.uint8))
                cur += pad
            offs.append(cur)
            chunks.append(raw)
            cur += raw.size
    return np.concatenate(chunks), np.array(offs, np.uint32)


def routed_moe_case(d, f, group, seed, symmetric):
    """checkRoutedMoE fixture (main.swift:194-231)."""
    top_k = 8
    rng = oracle.seed_tree_key(seed, f"routed-moe-d{d}-f{f}-g{group}")
    mats = []
    for _ in range(top_k):
        g = rng.uniforms(-0.4, 0.4, f * d).reshape(f, d)
        u = rng.uniforms(-0.4, 0.4, f * d).reshape(f, d)
        dn = rng.uniforms(-0.4, 0.4, d * f).reshape(d, f)
        mats.append((g, u, dn))
    x_bits = oracle.f16_bits(rng.uniforms(-0.5, 0.5, d))
    res_bits = oracle.f16_bits(rng.uniforms(-0.5, 0.5, d))
    w = (np.float32(0.04) + np.arange(top_k, dtype=np.float32) * np.float32(0.015)).astype(np.float32)
    w_bits = oracle.f16_bits(w)
    blobs, offs = [], None
    for (g, u, dn) in mats:
        parts = [oracle.quantize_int4(g, group, symmetric),
                 oracle.quantize_int4(u, group, symmetric),
                 oracle.quantize_int4(dn, group, symmetric)]
        blob, offs = pack_blob(parts, symmetric, keep_biases=True)
        blobs.append(blob)
    ref = oracle.moe_apply_streamed_routed(blobs, offs, oracle.f16_to_float(x_bits),
                                           oracle.f16_to_float(res_bits),
                                           oracle.f16_to_float(w_bits), d, f, group,
                                           symmetric=False)
    return dict(blobs=blobs, offsets=offs, x_bits=x_bits, res_bits=res_bits, w_bits=w_bits,
                ref=ref)


def router_case(d, ne, group, seed, draw):
    """checkRouter(weightBits: 16) fixture (main.swift:419-458)."""
    label = f"router-bf16 d={d} experts={ne}"
    rng = oracle.seed_tree_key(seed + draw, f"{label}-g{group}")
    w_bits = rng.uniforms_bf16(-0.2, 0.2, ne * d)
    hidden = rng.uniforms_f16(-1.0, 1.0, d)
    es_bits = oracle.bf16_bits(rng.uniforms(0.5, 1.5, d))
    pes_bits = oracle.bf16_bits(rng.uniforms(0.8, 1.2, ne))
    x = oracle.f16_to_float(hidden) * oracle.bf16_to_float(es_bits)
    idx, wts = oracle.router_reference(oracle.bf16_to_float(w_bits).reshape(ne, d), x, 8,
                                       oracle.bf16_to_float(pes_bits))
    return dict(w_bits=w_bits, hidden=hidden, es_bits=es_bits, pes_bits=pes_bits, idx=idx,
                wts=wts)


def router_int8_case(d, ne, group, seed, draw):
    """checkRouter(weightBits: 8) fixture (main.swift:409-520): uniform rows
    quantised by quantizeInt8Affine at the context's group size; the expected
    top-8 is routerReference over the dequantised rows."""
    label = f"router-int8 d={d} experts={ne}"
    rng = oracle.seed_tree_key(seed + draw, f"{label}-g{group}")
    raw = rng.uniforms(-0.2, 0.2, ne * d).reshape(ne, d)
    packed, scales, biases = oracle.quantize_int8_affine(raw, group)
    wf = oracle.dequantize_int8_affine(packed, scales, biases, group)
    hidden = rng.uniforms_f16(-1.0, 1.0, d)
    es_bits = oracle.bf16_bits(rng.uniforms(0.5, 1.5, d))
    pes_bits = oracle.bf16_bits(rng.uniforms(0.8, 1.2, ne))
    x = oracle.f16_to_float(hidden) * oracle.bf16_to_float(es_bits)
    # routerReference ranks at least top-k experts
    idx, wts = oracle.router_reference(wf, x, 8, oracle.bf16_to_float(pes_bits)) \
        if ne >= 8 else (None, None)
    return dict(packed=packed, scales=scales, biases=biases, hidden=hidden, es_bits=es_bits,
                pes_bits=pes_bits, idx=idx, wts=wts)


def router_topk_test_case(kind):
    """The two cases of RouterTopKTests (Tests/Tsugumi/Core/Kernels/MoE/
    RouterTopKTests.swift:17-69): 16 experts, d = 128, INT8 rows at group 64.
    "spread": rows offset by 0.01 per expert (seed 0xA5B61234); "near_tie":
    one pattern scaled per expert, experts 7 and 8 at gains 0.5 and
    0.5 * (1 + 1e-4) (seed 0x71E0F4A). The expected result is the test's own:
    hidden and scales unrounded, top-8 of the dequantised rows' logits."""
    ne, d = 16, 128
    if kind == "spread":
        rng = oracle.SplitMix64(0xA5B61234)
        w = np.empty((ne, d), np.float32)
        for e in range(ne):
            w[e] = rng.uniforms(-0.05, 0.05, d) + np.float32(e) * np.float32(0.01)
        hidden = rng.uniforms(-1.0, 1.0, d)
        inv_sqrt_d = np.float32(1.0) / np.sqrt(np.float32(d))
        es = rng.uniforms(0.5, 1.5, d) * inv_sqrt_d
        pes = rng.uniforms(0.6, 1.4, ne)
    else:
        rng = oracle.SplitMix64(0x71E0F4A)
        pattern = rng.uniforms(0.2, 1.0, d)
        hidden = rng.uniforms(0.5, 1.5, d)
        gains = np.zeros(ne, np.float32)
        for e in range(7):
            gains[e] = np.float32(1.0) - np.float32(e) * np.float32(0.05)
        gains[7] = np.float32(0.5)
        gains[8] = np.float32(0.5) * (np.float32(1.0) + np.float32(1e-4))
        for e in range(9, ne):
            gains[e] = np.float32(0.4) - np.float32(e - 9) * np.float32(0.02)
        w = (gains[:, None] * pattern[None, :]).astype(np.float32)
        es = np.ones(d, np.float32)
        pes = np.ones(ne, np.float32)
    packed, scales, biases = oracle.quantize_int8_affine(w, 64)
    wf = oracle.dequantize_int8_affine(packed, scales, biases, 64)
    idx, wts = oracle.router_reference(wf, (hidden * es).astype(np.float32), 8, pes)
    return dict(ne=ne, d=d, packed=packed, scales=scales, biases=biases,
                hidden=oracle.f16_bits(hidden), es_bits=oracle.bf16_bits(es),
                pes_bits=oracle.bf16_bits(pes), idx=idx, wts=wts)


def prefill_router_case(t, d, ne, kind, group, seed):
    """checkPrefillRouterBF16 fixture (main.swift:525-548); stride d + 16."""
    stride = d + 16
    label = f"prefill-router-bf16-{kind} t={t} d={d} experts={ne}"
    rng = oracle.seed_tree_key(seed, label.replace("-nax ", "-gemm "))
    w_bits = rng.uniforms_bf16(-0.2, 0.2, ne * d)
    hidden = rng.uniforms_f16(-1.0, 1.0, t * stride)
    es_bits = oracle.bf16_bits(rng.uniforms(0.5, 1.5, d))
    pes_bits = oracle.bf16_bits(rng.uniforms(0.8, 1.2, ne))
    refs = []
    wf = oracle.bf16_to_float(w_bits).reshape(ne, d)
    for row in range(t):
        x = oracle.f16_to_float(hidden[row * stride:row * stride + d]) * oracle.bf16_to_float(es_bits)
        refs.append(oracle.router_reference(wf, x, 8, oracle.bf16_to_float(pes_bits)))
    return dict(stride=stride, w_bits=w_bits, hidden=hidden, es_bits=es_bits,
                pes_bits=pes_bits, refs=refs)


def prefill_moe_gemm_case(group, seed, symmetric, d=2816, f=704, tokens=72, top_k=4,
                          n_experts=16):
    """checkPrefillRoutedMoEGEMM fixture (PrefillMoEGEMMCheck.swift:92-136):
    16 experts, rank 0 always expert 0 (72 rows: a full block + a partial
    one), the other ranks spread over experts 1..15."""
    rng = oracle.seed_tree_key(seed, f"prefill-moe-gemm-g{group}")
    experts = []
    for _ in range(n_experts):
        parts = [quantized_rows(rng, f, d, group, symmetric, -0.125, 0.125),
                 quantized_rows(rng, f, d, group, symmetric, -0.125, 0.125),
                 quantized_rows(rng, d, f, group, symmetric, -0.125, 0.125)]
        experts.append(parts)
    hidden = rng.uniforms_f16(-1.0, 1.0, tokens * d)
    by_expert = [[] for _ in range(n_experts)]
    for token in range(tokens):
        picks = [0, 1 + token % 5, 6 + token % 4, 10 + token % 6]
        for rank, e in enumerate(picks):
            by_expert[e].append((token, e, rank, 0))
    pairs, blocks = [], []
    for e in range(n_experts):
        start = 0
        while start < len(by_expert[e]):
            cnt = min(64, len(by_expert[e]) - start)
            blocks.append((e, len(pairs) + start, cnt, len(pairs) + start))
            start += cnt
        pairs.extend(by_expert[e])
    pairs = np.array(pairs, dtype=oracle.PAIR_DTYPE)
    blocks = np.array(blocks, dtype=oracle.BLOCK_DTYPE)
    return dict(experts=experts, hidden=hidden, pairs=pairs, blocks=blocks, tokens=tokens,
                top_k=top_k, d=d, f=f)


def layer_image(expert_parts, symmetric, keep_biases, stride_align=16384):
    """A MoEPack layer file image: expert blobs at a common stride rounded up to
    16 KiB (RepackPlanner.swift:514-516). Returns (bytes, stride, offsets9)."""
    blobs, offs = [], None
    for parts in expert_parts:
        blob, offs = pack_blob(parts, symmetric, keep_biases=keep_biases)
        blobs.append(blob)
    size = max(b.size for b in blobs)
    stride = (size + stride_align - 1) // stride_align * stride_align
    image = np.zeros(stride * len(blobs), np.uint8)
    for i, b in enumerate(blobs):
        image[i * stride:i * stride + b.size] = b
    return image, stride, offs, blobs


def shared_expert_case(d, f, group, seed, symmetric):
    """A Qwen shared-expert case (QwenForwardRunner.swift:1548-1578): this
    build's own seeded draw with the harness generators (the reference's
    harness has no shared-expert check). gate/up [f, d], down [d, f] in the
    blob layout, x fp16, the bf16 gate row [d]."""
    rng = oracle.seed_tree_key(seed, f"shared-expert-d{d}-f{f}-g{group}")
    g = rng.uniforms(-0.4, 0.4, f * d).reshape(f, d)
    u = rng.uniforms(-0.4, 0.4, f * d).reshape(f, d)
    dn = rng.uniforms(-0.4, 0.4, d * f).reshape(d, f)
    x_bits = oracle.f16_bits(rng.uniforms(-0.5, 0.5, d))
    gate_w = rng.uniforms_bf16(-0.05, 0.05, d)
    parts = [oracle.quantize_int4(m, group, symmetric) for m in (g, u, dn)]
    blob, offs = pack_blob(parts, symmetric, keep_biases=not symmetric)
    ref = oracle.shared_expert(blob, offs, x_bits, gate_w, d, f, group, symmetric)
    return dict(blob=blob, offsets=offs, x_bits=x_bits, gate_w=gate_w, parts=parts, ref=ref)
