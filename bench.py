#!/usr/bin/env python3
"""Benchmark of the int4 MoE expert-matmul path on one MI355X.

Workload (BASELINE.json configs[1] and [3]):
  decode  Gemma-4-26B-A4B-shaped MoE layer, 1 token: H=2816, 128 experts of
          gate/up [2x704, 2816] + down [2816, 704], int4 sym group-32 with bf16
          scales, bf16 router [128, 2816] -> top-8 -> GeGLU. 30 layers
          (12.9 GB of experts) resident in HBM, run back to back on one stream
          with a fresh N(0,1) hidden state per (token, layer), so every layer
          routes fresh experts. One step = one token through the 30 layers;
          8 tokens are captured once in a HIP graph (6.6 GB of expert reads
          per replay: nothing is served from cache across replays).
  prefill the same layer shape, T=2048 tokens, top-8 Zipf(1.1) routing:
          device grouping -> gate/up GEMM + GeGLU -> down GEMM -> token-major
          reduce.

Also reported, under "other_configs" (skipped with --no-extra-configs):
  qmv        configs[0]: one int4 QMV, K=2816, N=704 (sym group 32), as
             back-to-back launches in a HIP graph (launch-bound).
  verify_m5  configs[2]: Gemma speculative verify, M=5 tokens whose top-8
             sets overlap (union about 16), 30 layers, rows path + reduce.
  qwen35     configs[4]: Qwen3.5-MoE-35B-A3B-shaped layer (H=2048, 256
             experts of I=512, SwiGLU, shared expert I=512 with a sigmoid
             gate), 40 layers: decode M=1 and M=3, prefill T=4096 Zipf(1.0).

`value` is the decode layer's algorithmic HBM throughput (GB/s): 27,506,944
bytes per layer / measured time per layer (one token through the 30
layers). The roofline object is for the dominant (and
only) decode kernel, decode_layer_kernel, which runs the whole layer in one
launch; its 27,506,944 algorithmic bytes per launch / its average launch
duration, timed with HIP events on the stream it runs on over a graph of
launches alone. `traffic` is the HBM bytes per launch that rocprofv3's
FETCH_SIZE + WRITE_SIZE counters report, scaled by the factor a plain copy
kernel of known size reads on the same counters (constant TRAFFIC_BYTES,
measured with `--traffic-probe` under rocprofv3). cpu_baseline times the oracle's restatement of the
reference's CPU path (DequantInt4GemvRef + MoeRef + routerReference) on the
host cores, on a bounded sample of the same layers.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

H, F, E, TOPK, GROUP = 2816, 704, 128, 8, 32
LAYERS = 30
# bytes per expert sub-tensor (sym g32: no bias arrays)
W_GU = F * H // 2          # 991,232
S_GU = F * (H // GROUP) * 2  # 123,904
W_D = H * F // 2           # 991,232
S_D = H * (F // GROUP) * 2   # 123,904
EXPERT_BYTES = 2 * (W_GU + S_GU) + W_D + S_D  # 3,345,408
ROUTER_BYTES = E * H * 2   # 720,896
LAYER_BYTES = TOPK * EXPERT_BYTES + ROUTER_BYTES + H * 2 + E * 2 + 3 * H * 2  # 27,506,944
PREFILL_T = 2048
PREFILL_FLOP = 2 * PREFILL_T * TOPK * 3 * F * H  # 194,884,141,056
HBM_PEAK_GBS = 8000.0
# HBM bytes per decode_layer_kernel launch: rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over `bench.py --traffic-probe` (16,415.92 KiB fetched, 320.09 KiB
# written per dispatch), scaled by the counters of a plain 64 MiB device copy in
# the same runs (fetch x 1.9990, write x 1.000).
TRAFFIC_BYTES = 33931486
MFMA_F16_PEAK_TFLOPS = 2500.0


def gemma_offsets():
    offs, stride, _ = shape_offsets(H, F)
    return offs, stride


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def shape_offsets(h, f, group=GROUP):
    """MoEExpertOffsets of a sym expert blob of shape (h, f) and its stride
    (RepackPlanner.swift:442-520: gate W, S, up W, S, down W, S; stride
    rounded up to 16,384; the bias offsets alias the scales)."""
    w_gu, s_gu = f * h // 2, f * (h // group) * 2
    w_d, s_d = h * f // 2, h * (f // group) * 2
    o_gs, o_uw = w_gu, w_gu + s_gu
    o_us, o_dw = 2 * w_gu + s_gu, 2 * (w_gu + s_gu)
    o_ds = o_dw + w_d
    payload = o_ds + s_d
    return [0, o_gs, o_gs, o_uw, o_us, o_us, o_dw, o_ds, o_ds], (payload + 16383) // 16384 * 16384, payload


def make_layers(tsg, ctx, torch, n_layers, seed=0x7E57, h=H, f=F, e=E):
    """n_layers resident layers of e experts of shape (h, f): nibbles uniform in
    [0,15], scales bf16(|N(0,0.02)|/7), router bf16 N(0, 1/sqrt(h))."""
    offs, stride, _ = shape_offsets(h, f)
    layers, bufs, routers = [], [], []
    regions = [(offs[1], f * (h // GROUP)), (offs[4], f * (h // GROUP)), (offs[7], h * (f // GROUP))]
    for l in range(n_layers):
        buf = torch.empty(e * stride, dtype=torch.uint8, device="cuda")
        tsg.generators.bytes(buf, seed + l)
        for x in range(e):
            for j, (o, n) in enumerate(regions):
                reg = buf[x * stride + o:x * stride + o + 2 * n].view(torch.int16)
                tsg.generators.bf16_normal(reg, (seed + l) * 4096 + x * 3 + j + 1, 0.02, True, 7.0)
        rw = torch.empty(e * h, dtype=torch.int16, device="cuda")
        tsg.generators.bf16_normal(rw, (seed + l) * 4096 + 4000, 1.0 / np.sqrt(h))
        layers.append(tsg.ResidentLayer(ctx, e, stride, offs, device_tensor=buf))
        bufs.append(buf)
        routers.append(rw)
    torch.cuda.synchronize()
    return layers, bufs, routers, offs, stride


def run_decode(tsg, torch, ctx, args, layers, routers):
    moe = tsg.MoE(ctx)
    ones_h = torch.full((H,), 0x3F80, dtype=torch.int16, device="cuda")
    ones_e = torch.full((E,), 0x3F80, dtype=torch.int16, device="cuda")
    n_inputs = 8
    # a fresh N(0,1) hidden state per (token, layer): fresh routing everywhere
    # (chaining raw layer outputs without the model's norms overflows fp16
    # within a few layers and would collapse the routing)
    inputs = torch.empty(n_inputs * LAYERS * H, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(inputs, 0x1A2B, 1.0)
    ys = torch.empty(LAYERS * H, dtype=torch.int16, device="cuda")
    idx = torch.empty(LAYERS * TOPK, dtype=torch.int32, device="cuda")
    wts = torch.empty(LAYERS * TOPK, dtype=torch.int16, device="cuda")
    acts = torch.empty(LAYERS * TOPK * F, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()

    def x_of(k, l):
        return inputs[(k * LAYERS + l) * H:(k * LAYERS + l + 1) * H]

    def layer(k, l):
        moe.encode_decode_layer(layers[l], routers[l], x_of(k, l), ones_h, ones_e, x_of(k, l),
                                x_of(k, l), ys[l * H:(l + 1) * H], idx[l * TOPK:(l + 1) * TOPK],
                                wts[l * TOPK:(l + 1) * TOPK],
                                acts[l * TOPK * F:(l + 1) * TOPK * F], E, H, F, stream=stream)

    def one_token(k):
        for l in range(LAYERS):
            layer(k, l)

    # one graph = n_inputs tokens (each a 30-layer pass from its own input)
    with torch.cuda.stream(stream):
        for k in range(n_inputs):
            one_token(k)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for k in range(n_inputs):
            one_token(k)
    torch.cuda.synchronize()
    replays_w = max(1, (args.warmup + n_inputs - 1) // n_inputs)
    replays = max(1, (args.steps + n_inputs - 1) // n_inputs)
    # CUDAGraph.replay() launches on the current stream: make it `stream`, the
    # stream the events are recorded on.
    with torch.cuda.stream(stream):
        for _ in range(replays_w):
            graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop)
    tokens = replays * n_inputs
    us_per_layer = ms * 1000.0 / (tokens * LAYERS)
    log(f"decode: {tokens} tokens x {LAYERS} layers in {ms:.3f} ms (wall {wall*1e3:.1f} ms): "
        f"{us_per_layer:.3f} us/layer")
    check_decode_outputs(torch, ys, idx)
    # dominant kernel: the one-launch decode layer alone, 4 tokens x 30 layers
    # per graph, timed on the stream the launches go to.
    g2 = torch.cuda.CUDAGraph()
    k_reps = 4
    with torch.cuda.graph(g2, stream=stream):
        for k in range(k_reps):
            one_token(k)
    with torch.cuda.stream(stream):
        g2.replay()
    torch.cuda.synchronize()
    reps = max(2, replays // 2)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            g2.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    k_us = start.elapsed_time(stop) * 1000.0 / (reps * k_reps * LAYERS)
    log(f"decode_layer_kernel alone: {k_us:.3f} us/launch")
    check_decode_outputs(torch, ys, idx)
    # the graph's last token is the last one executed: its inputs and routing
    last = [x_of(n_inputs - 1, l) for l in range(LAYERS)]
    with torch.cuda.stream(stream):
        one_token(n_inputs - 1)
    torch.cuda.synchronize()
    return dict(ms_per_step=ms / tokens, us_per_layer=us_per_layer, tokens=tokens,
                kernel_us=k_us, idx=idx, xs=last, wts=wts)


def check_decode_outputs(torch, ys, idx):
    """The measured work must be the claimed work: finite outputs and routing
    that spreads over many experts (a collapsed routing reads one expert)."""
    y = ys.view(torch.float16).float()
    if not bool(torch.isfinite(y).all()):
        raise RuntimeError("decode produced non-finite outputs: the benchmark would not "
                           "measure the claimed work")
    per_layer = idx.view(LAYERS, TOPK).cpu().numpy()
    distinct = min(len(set(row.tolist())) for row in per_layer)
    if distinct != TOPK:
        raise RuntimeError(f"a decode layer routed to only {distinct} distinct experts")


def zipf_routing(t, ne, k, s, seed):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(ne)
    logp = (-s * np.log(np.arange(1, ne + 1, dtype=np.float64)))[np.argsort(perm)]
    scores = logp[None, :] - np.log(-np.log(rng.random((t, ne))))
    idx = np.argsort(-scores, axis=1, kind="stable")[:, :k].astype(np.int32)
    top = np.take_along_axis(scores, idx.astype(np.int64), axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float16)
    return idx, w


def run_prefill(tsg, torch, ctx, args, layer):
    return run_prefill_shape(tsg, torch, ctx, args, layer, PREFILL_T, H, F, E, 1.1, "gelu")


def run_prefill_shape(tsg, torch, ctx, args, layer, t, h, f, e, zipf_s, act):
    """One prefill MoE layer of t tokens, top-8 Zipf(zipf_s) routing over e
    experts of shape (h, f): device grouping -> gate/up GEMM + activation ->
    down GEMM -> token-major reduce."""
    moe = tsg.MoE(ctx, gate_activation=act)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    red = tsg.PrefillMoE(ctx)
    k = TOPK
    flop = 2 * t * k * 3 * f * h
    idx_np, w_np = zipf_routing(t, e, k, zipf_s, 0x21F)
    idx = torch.from_numpy(idx_np.ravel()).cuda()
    w = torch.from_numpy(w_np.ravel().view(np.int16)).cuda()
    hidden = torch.empty(t * h, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(hidden, 0x33, 1.0)
    tile_rows = 128  # the grouped GEMM's widest pass
    max_blocks = t * k // tile_rows + e
    sp = torch.empty(t * k * 4, dtype=torch.int32, device="cuda")
    off = torch.empty(e, dtype=torch.int32, device="cuda")
    cnt = torch.empty(e, dtype=torch.int32, device="cuda")
    blocks = torch.empty(max_blocks * 4, dtype=torch.int32, device="cuda")
    nb = torch.empty(1, dtype=torch.int32, device="cuda")
    scratch = torch.empty(g.scratch_bytes(t, k, e) // 4 + 1, dtype=torch.int32, device="cuda")
    act_buf = torch.empty(t * k * f, dtype=torch.int16, device="cuda")
    partials = torch.empty(t * k * h, dtype=torch.int16, device="cuda")
    h2 = torch.empty(t * h, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]

    def chunk(record=False):
        if record:
            ev[0].record(stream)
        g.group_pairs_device(idx, w, t, k, e, sp, off, cnt, blocks, max_blocks, nb, scratch,
                             tile_rows=tile_rows, stream=stream)
        if record:
            ev[1].record(stream)
        g.encode_gate_up(layer, hidden, h, sp, blocks, max_blocks, act_buf, h, f,
                         n_blocks_device=nb, stream=stream)
        if record:
            ev[2].record(stream)
        g.encode_down(layer, act_buf, sp, blocks, max_blocks, partials, k, h, f,
                      n_blocks_device=nb, stream=stream)
        if record:
            ev[3].record(stream)
        red.encode_reduce_token_major(partials, w, h2, t, k, h, stream=stream)
        if record:
            ev[4].record(stream)

    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup // 4)):
            chunk()
    torch.cuda.synchronize()
    reps = max(2, args.steps // 4)
    totals = np.zeros(4)
    for _ in range(reps):
        with torch.cuda.stream(stream):
            chunk(record=True)
        torch.cuda.synchronize()
        totals += [ev[i].elapsed_time(ev[i + 1]) for i in range(4)]
    per = totals / reps  # ms
    total_ms = float(per.sum())
    gemm_ms = float(per[1] + per[2])
    log(f"prefill T={t}: group {per[0]*1e3:.1f} us, gate/up {per[1]*1e3:.1f} us, down "
        f"{per[2]*1e3:.1f} us, reduce {per[3]*1e3:.1f} us")
    nblocks = int(nb.cpu()[0])
    return dict(us_per_layer=total_ms * 1e3, gemm_us=gemm_ms * 1e3,
                gate_up_us=float(per[1]) * 1e3, down_us=float(per[2]) * 1e3,
                group_us=float(per[0]) * 1e3, reduce_us=float(per[3]) * 1e3,
                gemm_tflops=flop / (gemm_ms * 1e-3) / 1e12,
                layer_tflops=flop / (total_ms * 1e-3) / 1e12, blocks=nblocks, flop=flop)


# ------------------------------------------------- the other BASELINE configs
# Gemma speculative verify, M=5 tokens over an expert union of
# about 12-20, 30 layers. configs[4]: a Qwen3.5-MoE-35B-A3B-shaped layer
# (H=2048, 256 experts of I=512, SwiGLU, one shared expert of I=512 with a
# sigmoid(bf16 [1, 2048]) gate): decode at M=1 and M=3, prefill T=4096
# Zipf(1.0), 40 layers. Reported beside the headline, not as `value`.
QW_H, QW_F, QW_E, QW_LAYERS, QW_T = 2048, 512, 256, 40, 4096


def verify_routing(m, ne, k, seed, target=16):
    """Routing of M tokens whose top-k sets overlap: a shared random logit
    prefix plus a per-token perturbation, its scale picked from a fixed grid so
    the union of the sets is nearest `target` (configs[2]: about 12-20)."""
    rng = np.random.default_rng(seed)
    base = rng.normal(0.0, 1.0, ne)
    noise = rng.normal(0.0, 1.0, (m, ne))
    best = None
    for sigma in np.linspace(0.02, 2.0, 100):
        scores = base[None, :] + sigma * noise
        idx = np.argsort(-scores, axis=1, kind="stable")[:, :k]
        u = len(set(idx.ravel().tolist()))
        if best is None or abs(u - target) < abs(best[2] - target):
            best = (scores, idx, u)
    scores, idx, u = best
    top = np.take_along_axis(scores, idx, axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float16)
    return idx.astype(np.int32), w, u


def rows_plan(tsg, idx, w, m, k, ne):
    """Host grouping of one verify step (PrefillMoEGrouping.groupTokenExpertPairs)
    and its rows-path blocks: one block per routed expert, <= M rows."""
    pairs = tsg.PrefillRouter.make_token_expert_pairs(idx.ravel().astype(np.uint32),
                                                      w.ravel().view(np.uint16), m, k)
    g = tsg.PrefillMoEGrouping.group_token_expert_pairs(pairs, m, k, ne)
    blocks = np.array([(int(x["expert"]), int(x["pair_start"]), int(x["pair_count"]),
                        int(x["pair_start"])) for x in g["groups"]], dtype=tsg.BLOCK_DTYPE)
    return g["sorted_pairs"], blocks


def time_graph(torch, stream, body, reps, warm=2):
    """Captures `body` once into a HIP graph and times `reps` replays with HIP
    events on `stream`; returns ms per replay."""
    with torch.cuda.stream(stream):
        body()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        body()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(warm):
            graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        for _ in range(reps):
            graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def run_rows_path(tsg, torch, ctx, moe, layers, n_layers, m, h, f, ne, seed, shared=None):
    """M tokens through n_layers layers on the rows path (encodeStreamedRows)
    plus the token-major reduce, routing precomputed per layer (a verify step's
    routing is known before its MoE runs). `shared` (Qwen) adds the shared
    branch for the M tokens: GEMV rows for gate/up/down, SiLU-mul and the gate
    per token. Returns us per layer and the mean expert union."""
    k = TOPK
    g = tsg.PrefillGroupedRoutedMoE(moe)
    red = tsg.PrefillMoE(ctx)
    q = tsg.DequantInt4GEMV(ctx)
    qk = tsg.QwenKernels(ctx)
    plans, unions = [], []
    for l in range(n_layers):
        idx, w, u = verify_routing(m, ne, k, seed + l)
        sp, blocks = rows_plan(tsg, idx, w, m, k, ne)
        plans.append((torch.from_numpy(sp.view(np.int32).ravel().copy()).cuda(), blocks,
                      torch.from_numpy(w.ravel().view(np.int16).copy()).cuda()))
        unions.append(u)
    hidden = torch.empty(n_layers * m * h, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(hidden, seed ^ 0x5A5A, 1.0)
    act = torch.empty(m * k * f, dtype=torch.int16, device="cuda")
    part = torch.empty(m * k * h, dtype=torch.int16, device="cuda")
    h2 = torch.empty(n_layers * m * h, dtype=torch.int16, device="cuda")
    if shared is not None:
        sg, su, sa = (torch.empty(m * f, dtype=torch.int16, device="cuda") for _ in range(3))
        sout = torch.empty(n_layers * m * h, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()

    def body():
        for l in range(n_layers):
            x = hidden[l * m * h:(l + 1) * m * h]
            sp, blocks, wd = plans[l]
            g.encode_streamed_rows(layers[l], x, h, sp, blocks, act, part, k, h, f, stream=stream)
            red.encode_reduce_token_major(part, wd, h2[l * m * h:(l + 1) * m * h], m, k, h,
                                          stream=stream)
            if shared is not None:
                blob, o, gw = shared[l]
                bb = blob
                q.encode_rows(bb[o[0]:], bb[o[1]:], bb[o[2]:], x, h, sg, f, m, f, h, stream=stream)
                q.encode_rows(bb[o[3]:], bb[o[4]:], bb[o[5]:], x, h, su, f, m, f, h, stream=stream)
                qk.encode_silu_mul(sg, su, sa, m * f, stream=stream)
                y = sout[l * m * h:(l + 1) * m * h]
                q.encode_rows(bb[o[6]:], bb[o[7]:], bb[o[8]:], sa, f, y, h, m, h, f, stream=stream)
                for t in range(m):
                    qk.encode_moe_shared_gate(y[t * h:(t + 1) * h], x[t * h:(t + 1) * h], gw, h,
                                              stream=stream)

    ms = time_graph(torch, stream, body, reps=8)
    out = h2.view(torch.float16).float()
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError("rows path produced non-finite outputs")
    return ms * 1000.0 / n_layers, float(np.mean(unions))


def make_shared_experts(tsg, torch, n_layers, h, f, seed):
    """One shared expert (sym g32, the routed experts' generators) and a bf16
    gate row N(0, 1/sqrt(h)) per layer."""
    offs, stride, _ = shape_offsets(h, f)
    regions = [(offs[1], f * (h // GROUP)), (offs[4], f * (h // GROUP)), (offs[7], h * (f // GROUP))]
    out = []
    for l in range(n_layers):
        blob = torch.empty(stride, dtype=torch.uint8, device="cuda")
        tsg.generators.bytes(blob, seed + l)
        for j, (o, n) in enumerate(regions):
            tsg.generators.bf16_normal(blob[o:o + 2 * n].view(torch.int16), (seed + l) * 16 + j,
                                       0.02, True, 7.0)
        gw = torch.empty(h, dtype=torch.int16, device="cuda")
        tsg.generators.bf16_normal(gw, (seed + l) * 16 + 9, 1.0 / np.sqrt(h))
        out.append((blob, offs, gw))
    torch.cuda.synchronize()
    return out


def run_qwen(tsg, torch, args):
    """decode M=1 (the shared branch and the routed experts on top
    of it, QwenForwardRunner.swift:1548-1608, in one launch), decode M=3 (rows
    path + shared branch), prefill T=4096 Zipf(1.0) (grouped GEMM)."""
    h, f, e, nl = QW_H, QW_F, QW_E, QW_LAYERS
    ctx = tsg.Context(0, group_size=GROUP, scheme="sym")
    _, stride, payload = shape_offsets(h, f)
    log(f"qwen-shaped: building {nl} resident layers ({nl * e * stride / 1e9:.2f} GB)")
    layers, bufs, routers, offs, _ = make_layers(tsg, ctx, torch, nl, seed=0x9E37, h=h, f=f, e=e)
    shared = make_shared_experts(tsg, torch, nl, h, f, 0x51AE)
    moe = tsg.MoE(ctx, gate_activation="silu")
    ones_h = torch.full((h,), 0x3F80, dtype=torch.int16, device="cuda")
    ones_e = torch.full((e,), 0x3F80, dtype=torch.int16, device="cuda")
    n_tok = 4
    xs = torch.empty(n_tok * nl * h, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(xs, 0x7777, 1.0)
    ys = torch.empty(nl * h, dtype=torch.int16, device="cuda")
    sact = torch.empty(f, dtype=torch.int16, device="cuda")
    idx = torch.empty(nl * TOPK, dtype=torch.int32, device="cuda")
    wts = torch.empty(nl * TOPK, dtype=torch.int16, device="cuda")
    acts = torch.empty(nl * TOPK * f, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()

    def decode():
        for k in range(n_tok):
            for l in range(nl):
                x = xs[(k * nl + l) * h:(k * nl + l + 1) * h]
                blob, o, gw = shared[l]
                moe.encode_decode_layer_shared(layers[l], routers[l], x, ones_h, ones_e, x,
                                               ys[l * h:(l + 1) * h], idx[l * TOPK:(l + 1) * TOPK],
                                               wts[l * TOPK:(l + 1) * TOPK],
                                               acts[l * TOPK * f:(l + 1) * TOPK * f], blob, o, gw,
                                               sact, e, h, f, f, stream=stream)

    ms = time_graph(torch, stream, decode, reps=max(2, args.steps // 8))
    us1 = ms * 1000.0 / (n_tok * nl)
    y = ys.view(torch.float16).float()
    if not bool(torch.isfinite(y).all()):
        raise RuntimeError("qwen decode produced non-finite outputs")
    distinct = min(len(set(r.tolist())) for r in idx.view(nl, TOPK).cpu().numpy())
    if distinct != TOPK:
        raise RuntimeError("qwen decode routing collapsed")
    bytes1 = TOPK * payload + payload + e * h * 2 + h * 2 + 6 * h * 2
    log(f"qwen decode M=1: {us1:.3f} us/layer ({bytes1 / (us1 * 1e-6) / 1e9:.1f} GB/s)")
    us3, u3 = run_rows_path(tsg, torch, ctx, moe, layers, nl, 3, h, f, e, 0x3333, shared=shared)
    bytes3 = u3 * payload + payload
    log(f"qwen decode M=3: {us3:.3f} us/layer over a mean union of {u3:.1f} experts")
    pre = run_prefill_shape(tsg, torch, ctx, args, layers[0], QW_T, h, f, e, 1.0, "silu")
    return {"workload": "qwen3.5-moe-35b-a3b-shaped layer (configs[4]): H=2048, 256 experts "
                        "I=512 top-8 SwiGLU + shared expert I=512 with sigmoid gate, 40 layers",
            "decode_m1": {"us_per_layer": round(us1, 3),
                          "GBps": round(bytes1 / (us1 * 1e-6) / 1e9, 2),
                          "bytes_per_layer": bytes1,
                          "launches_per_layer": 1},
            "decode_m3": {"us_per_layer": round(us3, 3), "mean_union": round(u3, 2),
                          "GBps": round(bytes3 / (us3 * 1e-6) / 1e9, 2),
                          "path": "rows path + token-major reduce + shared branch (GEMV rows, "
                                  "SiLU-mul, 3 gates)"},
            "prefill_t4096": prefill_summary(pre)}


def run_qmv(tsg, torch, ctx):
    """DequantInt4GEMV.encode, K=2816, N=704: 1,122,176 B per call
    (int4 weights + bf16 scales + fp16 x and y). 256 calls per graph replay."""
    n, m = H, F
    w = torch.empty(m * n // 2, dtype=torch.uint8, device="cuda")
    tsg.generators.bytes(w, 0x9A1)
    sc = torch.empty(m * (n // GROUP), dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(sc, 0x9A2, 0.02, True, 7.0)
    x = torch.empty(n, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0x9A3, 1.0)
    y = torch.empty(m, dtype=torch.int16, device="cuda")
    q = tsg.DequantInt4GEMV(ctx)
    stream = torch.cuda.Stream()
    calls = 256

    def body():
        for _ in range(calls):
            q.encode(w, sc, sc, x, y, m, n, stream=stream)

    ms = time_graph(torch, stream, body, reps=8)
    us = ms * 1000.0 / calls
    nbytes = m * n // 2 + m * (n // GROUP) * 2 + n * 2 + m * 2
    if not bool(torch.isfinite(y.view(torch.float16).float()).all()):
        raise RuntimeError("qmv produced non-finite outputs")
    log(f"qmv K={n} N={m}: {us:.3f} us/call ({nbytes / (us * 1e-6) / 1e9:.1f} GB/s)")
    return {"workload": "int4 QMV K=2816 N=704 sym g32 (configs[0]), back-to-back launches",
            "us_per_call": round(us, 3), "bytes_per_call": nbytes,
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 2),
            "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def run_tail(tsg, torch, ctx):
    """Layer tail after the prefill MoE, T=2048, top-8, D=2816: the token-major
    reduce then PrefillLayerTail (two launches), and the reduce-fused tail (one
    launch, h2 kept in registers). Algorithmic bytes of the fused launch:
    partials T*8*D*2 + route weights + h1 T*D*2 + hidden read and written
    T*D*4 + two bf16 weight rows."""
    t, k, d = 2048, 8, H
    P = torch.empty(t * k * d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(P, 0x7A1, 0.5)
    w = torch.empty(t * k, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(w, 0x7A2, 0.1)
    h1 = torch.empty(t * d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(h1, 0x7A3, 1.0)
    hid = torch.empty(t * d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(hid, 0x7A4, 1.0)
    w2 = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(w2, 0x7A5, 0.1, True, 1.0)
    w1 = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(w1, 0x7A6, 0.1, True, 1.0)
    h2 = torch.empty(t * d, dtype=torch.int16, device="cuda")
    pm, tail = tsg.PrefillMoE(ctx), tsg.PrefillLayerTail(ctx)
    stream = torch.cuda.Stream()
    calls = 16

    def two():
        for _ in range(calls):
            pm.encode_reduce_token_major(P, w, h2, t, k, d, stream=stream)
            tail.encode(h2, h1, hid, w2, w1, t, d, d, d, d, 1e-6, 1.0, stream=stream)

    def one():
        for _ in range(calls):
            pm.encode_reduce_layer_tail(P, w, h1, hid, w2, w1, t, k, d, d, d, 1e-6, 1.0,
                                        stream=stream)

    ft = tsg.FusedLayerTail(ctx)

    def decode_tail():  # FusedLayerTail: one row per call, as each decode step
        for _ in range(256):
            ft.encode(h2, h1, hid, w2, w1, d, 1e-6, 1.0, stream=stream)

    us_two = time_graph(torch, stream, two, reps=4) * 1000.0 / calls
    us_one = time_graph(torch, stream, one, reps=4) * 1000.0 / calls
    us_dec = time_graph(torch, stream, decode_tail, reps=4) * 1000.0 / 256
    nbytes = t * k * d * 2 + t * k * 2 + t * d * 2 + t * d * 4 + 2 * d * 2
    log(f"reduce+tail T={t}: fused {us_one:.2f} us, reduce then tail {us_two:.2f} us; "
        f"decode tail (one row) {us_dec:.2f} us")
    return {"workload": "prefill reduce + layer tail, T=2048 top-8 D=2816 (Gemma)",
            "us_fused": round(us_one, 3), "us_reduce_then_tail": round(us_two, 3),
            "us_decode_tail_one_row": round(us_dec, 3),
            "bytes_fused": nbytes, "GBps_fused": round(nbytes / (us_one * 1e-6) / 1e9, 2),
            "frac_hbm_peak_fused": round(nbytes / (us_one * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def run_dense_qmm(tsg, torch, ctx):
    """PrefillInt4QMM at T=2048 on two Gemma projection shapes (N x K =
    2816 x 2816 and 4096 x 2816), sym g32 as the bench's experts: 2*T*N*K FLOP
    per call on the dequant-to-LDS MFMA GEMM."""
    t = 2048
    out = {}
    for n, k in ((2816, 2816), (4096, 2816)):
        w = torch.empty(n * k // 2, dtype=torch.uint8, device="cuda")
        tsg.generators.bytes(w, 0xD1 + n)
        sc = torch.empty(n * (k // GROUP), dtype=torch.int16, device="cuda")
        tsg.generators.bf16_normal(sc, 0xD2 + n, 0.02, True, 7.0)
        x = torch.empty(t * k, dtype=torch.int16, device="cuda")
        tsg.generators.f16_normal(x, 0xD3 + n, 1.0)
        y = torch.empty(t * n, dtype=torch.int16, device="cuda")
        q = tsg.PrefillInt4QMM(ctx)
        stream = torch.cuda.Stream()
        calls = 16

        def body():
            for _ in range(calls):
                q.encode(w, sc, sc, x, y, t, n, k, stream=stream)

        us = time_graph(torch, stream, body, reps=4) * 1000.0 / calls
        if not bool(torch.isfinite(y.view(torch.float16).float()).all()):
            raise RuntimeError("qmm produced non-finite outputs")
        tf = 2.0 * t * n * k / (us * 1e-6) / 1e12
        log(f"dense qmm T={t} N={n} K={k}: {us:.2f} us ({tf:.0f} TFLOP/s)")
        out[f"{n}x{k}"] = {"us_per_call": round(us, 3), "TFLOPs": round(tf, 1),
                           "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    return {"workload": "dense int4 projection QMM, T=2048, sym g32 (PrefillInt4QMM)", **out}


def run_verify(tsg, torch, ctx, args, layers):
    """Gemma verify, M=5 over a union of about 12-20 experts, 30
    layers on the rows path."""
    moe = tsg.MoE(ctx)
    us, u = run_rows_path(tsg, torch, ctx, moe, layers, LAYERS, 5, H, F, E, 0x5E5E)
    _, _, payload = shape_offsets(H, F)
    b = u * payload
    log(f"verify M=5: {us:.3f} us/layer over a mean union of {u:.1f} experts "
        f"({b / (us * 1e-6) / 1e9:.1f} GB/s)")
    return {"workload": "gemma4-26b-a4b verify, M=5 (draft 4 + 1), union ~12-20, 30 layers "
                        "(configs[2])",
            "us_per_layer": round(us, 3), "mean_union": round(u, 2),
            "GBps": round(b / (us * 1e-6) / 1e9, 2),
            "frac_hbm_peak": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "path": "rows path (encodeStreamedRows) + token-major reduce, routing precomputed"}


def prefill_summary(pre):
    return {"us_per_layer": round(pre["us_per_layer"], 2),
            "gemm_us": round(pre["gemm_us"], 2), "gate_up_us": round(pre["gate_up_us"], 2),
            "down_us": round(pre["down_us"], 2), "group_us": round(pre["group_us"], 2),
            "reduce_us": round(pre["reduce_us"], 2),
            "gemm_TFLOPs": round(pre["gemm_tflops"], 2),
            "frac_mfma_peak": round(pre["gemm_tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "layer_TFLOPs": round(pre["layer_tflops"], 2),
            "flop_per_layer": pre["flop"], "routed_blocks": pre["blocks"]}


def cpu_baseline(torch, dec, bufs, routers, offs, stride, budget_s=12.0):
    """The reference's CPU path for the same math, restated in C (oracle):
    routerReference + MoeRef.applyStreamedRouted per layer, on the host cores,
    over the first layers of the decode chain with their real inputs."""
    import oracle
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(threads, 16))
    oracle.set_threads(threads)
    idx = dec["idx"].cpu().numpy().reshape(LAYERS, TOPK)
    done, elapsed = 0, 0.0
    es = np.ones(H, np.float32)
    pes = np.ones(E, np.float32)
    for l in range(LAYERS):
        x_bits = dec["xs"][l].cpu().numpy().view(np.uint16)
        rw = oracle.bf16_to_float(routers[l].cpu().numpy().view(np.uint16)).reshape(E, H)
        experts = idx[l]
        blobs = [bufs[l][int(e) * stride:(int(e) + 1) * stride].cpu().numpy() for e in experts]
        x = oracle.f16_to_float(x_bits)
        t0 = time.perf_counter()
        ri, rwts = oracle.router_reference(rw, x * es, TOPK, pes)
        oracle.moe_apply_streamed_routed(blobs, np.array(offs, np.uint32), x, x, rwts, H, F,
                                         GROUP, True)
        elapsed += time.perf_counter() - t0
        done += 1
        if elapsed > budget_s:
            break
    us = elapsed * 1e6 / done
    return dict(value=round(LAYER_BYTES / (us * 1e-6) / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=f"{done} decode layers (router + 8 experts, H=2816 F=704 sym g32) "
                       f"through the C restatement of routerReference + MoeRef, "
                       f"{us:.0f} us/layer on {threads} threads")


COPY_BYTES = 64 << 20


def traffic_probe(tsg, torch, ctx, layers, routers):
    """For rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE: a plain device copy of
    COPY_BYTES (three dispatches; its counters give the factor between counter
    KiB and bytes moved) and one token through the layers (one
    decode_layer_kernel dispatch per layer)."""
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    moe = tsg.MoE(ctx)
    ones_h = torch.full((H,), 0x3F80, dtype=torch.int16, device="cuda")
    ones_e = torch.full((E,), 0x3F80, dtype=torch.int16, device="cuda")
    xs = torch.empty(LAYERS * H, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(xs, 0x1A2B, 1.0)
    ys = torch.empty(LAYERS * H, dtype=torch.int16, device="cuda")
    idx = torch.empty(LAYERS * TOPK, dtype=torch.int32, device="cuda")
    wts = torch.empty(TOPK, dtype=torch.int16, device="cuda")
    acts = torch.empty(TOPK * F, dtype=torch.int16, device="cuda")
    for l in range(LAYERS):
        x = xs[l * H:(l + 1) * H]
        moe.encode_decode_layer(layers[l], routers[l], x, ones_h, ones_e, x, x,
                                ys[l * H:(l + 1) * H], idx[l * TOPK:(l + 1) * TOPK], wts, acts,
                                E, H, F)
    ctx.synchronize()
    torch.cuda.synchronize()
    check_decode_outputs(torch, ys, idx)
    log(f"traffic probe: 3 copies of {COPY_BYTES} bytes, {LAYERS} decode layers")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the verify (configs[2]) and Qwen-shaped (configs[4]) figures")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the prefill layer (for profiling) and print its figures")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the copy + one-token dispatches for rocprofv3 --pmc and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch
    import tsugumi_amd as tsg
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        sys.exit(1)
    ctx = tsg.Context(0, group_size=GROUP, scheme="sym")
    log(f"building {LAYERS} resident layers ({LAYERS * E * gemma_offsets()[1] / 1e9:.2f} GB)")
    layers, bufs, routers, offs, stride = make_layers(tsg, ctx, torch, LAYERS)
    if args.traffic_probe:
        traffic_probe(tsg, torch, ctx, layers, routers)
        return
    if args.prefill_only:
        pre = run_prefill(tsg, torch, ctx, args, layers[0])
        print(json.dumps({"prefill_gemm_us": round(pre["gemm_us"], 2),
                          "gemm_TFLOPs": round(pre["gemm_tflops"], 2)}), flush=True)
        return
    dec = run_decode(tsg, torch, ctx, args, layers, routers)
    pre = None if args.no_prefill else run_prefill(tsg, torch, ctx, args, layers[0])
    gbs = LAYER_BYTES / (dec["us_per_layer"] * 1e-6) / 1e9
    k_gbs = LAYER_BYTES / (dec["kernel_us"] * 1e-6) / 1e9
    out = {
        "metric": "MoE-FFN decode µs/layer + HBM GB/s (%peak); prefill grouped-GEMM "
                  "TFLOP/s (%MFMA)",
        "value": round(gbs, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["tokens"],
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xfp16->fp32",
        "data": "synthetic (seeded device generators; nibbles U{0..15}, scales bf16(|N(0,.02)|/7), "
                "x fp16 N(0,1))",
        "config": {"workload": "gemma4-26b-a4b decode MoE layer, 1 token, 30 "
                               "HBM-resident layers (config 2); prefill T=2048 top-8 "
                               "Zipf(1.1) (config 4)",
                   "hidden": H, "intermediate": F, "experts": E, "top_k": TOPK,
                   "group": GROUP, "scheme": "sym", "layers": LAYERS,
                   "bytes_per_layer": LAYER_BYTES},
        "decode": {"us_per_layer": round(dec["us_per_layer"], 3), "GBps": round(gbs, 2),
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm",
                     "kernel": "decode_layer_kernel (router, top-8, gate/up+GeGLU, "
                               "down+combine in one launch)",
                     "achieved": round(k_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_BYTES,
                     "bytes_per_launch": LAYER_BYTES,
                     "avg_launch_us": round(dec["kernel_us"], 3)},
    }
    if pre is not None:
        out["prefill"] = prefill_summary(pre)
    if not args.no_extra_configs:
        # the other BASELINE configs, after the headline figures (a failure here
        # is reported in its entry and does not void the headline)
        extra = {}
        for name, fn in (("qmv", lambda: run_qmv(tsg, torch, ctx)),
                         ("layer_tail", lambda: run_tail(tsg, torch, ctx)),
                         ("dense_qmm", lambda: run_dense_qmm(tsg, torch, ctx)),
                         ("verify_m5", lambda: run_verify(tsg, torch, ctx, args, layers)),
                         ("qwen35", lambda: run_qwen(tsg, torch, args))):
            try:
                extra[name] = fn()
            except Exception as exc:  # noqa: BLE001 - reported, not hidden
                log(f"{name} failed: {exc}")
                extra[name] = {"error": str(exc)}
        out["other_configs"] = extra
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, dec, bufs, routers, offs, stride)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
