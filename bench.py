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
  router_int8  the INT8-affine router (MoE.init's default router format) at
             the Gemma router shape, back-to-back launches.
  decode_int8_router  the headline decode layer with that router, one launch.
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
SUSTAIN_LAYERS = 10  # prefill layers back to back in the sustained graph
PREFILL_FLOP = 2 * PREFILL_T * TOPK * 3 * F * H  # 194,884,141,056
HBM_PEAK_GBS = 8000.0
# HBM bytes per decode_layer_kernel launch: rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over `bench.py --traffic-probe` (13,973.6 KiB fetched, 320.09 KiB
# written per dispatch), scaled by the counters of a plain 64 MiB device copy in
# the same runs (fetch x 1.9992, write x 1.000).
TRAFFIC_BYTES = 28934411
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

    # one graph = n_inputs tokens (each a 30-layer pass from its own input);
    # a second graph holds the steps % n_inputs tokens left over, so exactly
    # `steps` tokens are timed
    def capture(n_tok):
        with torch.cuda.stream(stream):
            for k in range(n_tok):
                one_token(k)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for k in range(n_tok):
                one_token(k)
        torch.cuda.synchronize()
        return g

    graph = capture(n_inputs)
    full, rem = divmod(args.steps, n_inputs)
    graph_rem = capture(rem) if rem else None
    replays_w = max(1, (args.warmup + n_inputs - 1) // n_inputs)
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
        for _ in range(full):
            graph.replay()
        if graph_rem is not None:
            graph_rem.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop)
    tokens = args.steps
    replays = max(1, full)
    us_per_layer = ms * 1000.0 / (tokens * LAYERS)
    log(f"decode: {tokens} tokens x {LAYERS} layers in {ms:.3f} ms (wall {wall*1e3:.1f} ms): "
        f"{us_per_layer:.3f} us/layer")
    ctx.synchronize()  # raises if a launch's hand-off wait timed out (its outputs are invalid)
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
    ctx.synchronize()
    check_decode_outputs(torch, ys, idx)
    # the graph's last token is the last one executed: its inputs and routing
    last = [x_of(n_inputs - 1, l) for l in range(LAYERS)]
    with torch.cuda.stream(stream):
        one_token(n_inputs - 1)
    torch.cuda.synchronize()
    return dict(ms_per_step=ms / tokens, us_per_layer=us_per_layer, tokens=tokens,
                kernel_us=k_us, idx=idx, xs=last, wts=wts)


def routing_margins(torch, dec, routers):
    """The fp64 margin between the 8th and 9th router logits of the last timed
    token of every layer (RouterTopKTests.swift:46-68 pins ties; this shows
    how far the measured routing is from one): logits W x in fp64 from the
    same bf16 weights and fp16 inputs (effective scale 1), the fp32
    accumulation's worst-case error n u sum|w x| beside it, and whether the
    GPU's top-8 set is the fp64 one."""
    idx = dec["idx"].view(LAYERS, TOPK).cpu().numpy()
    margins, ratios, same = [], [], 0
    for l in range(LAYERS):
        w = routers[l].cpu().numpy().view(np.uint16).astype(np.uint32) << 16
        w = w.view(np.float32).astype(np.float64).reshape(E, H)
        x = dec["xs"][l].cpu().numpy().view(np.float16).astype(np.float64)
        logits = w @ x
        order = np.argsort(-logits, kind="stable")
        m = float(logits[order[7]] - logits[order[8]])
        bound = H * 2.0 ** -24 * float(np.max(np.abs(w) @ np.abs(x)))
        margins.append(m)
        ratios.append(m / bound)
        same += int(set(order[:TOPK].tolist()) == set(idx[l].tolist()))
    out = {"min_margin": round(min(margins), 6), "median_margin": round(float(np.median(margins)), 6),
           "min_margin_over_fp32_bound": round(min(ratios), 2), "layers": LAYERS,
           "gpu_top8_equals_fp64_top8": same,
           "note": "8th minus 9th logit in fp64 for the last timed token of each layer; the "
                   "bound is n * 2^-24 * max_e sum_i |w_ei x_i| (n = 2816)"}
    log(f"routing margins: min {out['min_margin']:.4g} (x{out['min_margin_over_fp32_bound']} "
        f"the fp32 bound), fp64 top-8 = GPU top-8 on {same}/{LAYERS} layers")
    return out


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


def run_prefill(tsg, torch, ctx, args, layers):
    return run_prefill_shape(tsg, torch, ctx, args, layers[0], PREFILL_T, H, F, E, 1.1, "gelu",
                             layers=layers)


def run_prefill_shape(tsg, torch, ctx, args, layer, t, h, f, e, zipf_s, act, layers=None):
    """One prefill MoE layer of t tokens, top-8 Zipf(zipf_s) routing over e
    experts of shape (h, f): device grouping -> gate/up GEMM + activation ->
    down GEMM -> token-major reduce. The per-kernel split comes from HIP
    events around each kernel of single layers run as two GEMM launches; the
    sustained figures from a HIP graph of SUSTAIN_LAYERS layers back to back
    (each with its own weights from `layers` when given), replayed: the GEMMs
    as one fused persistent launch (and, for comparison, as two launches),
    and the whole layer with the fused launch."""
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
    nblocks = int(nb.cpu()[0])
    # MFMA work issued: each routed block runs ceil(rows / 32) 32-row slices
    # (PrefillMoEGEMMBench.swift:141-143 pads rows to the tier's block rows)
    row_counts = blocks.view(-1, 4)[:nblocks, 2].cpu().numpy().astype(np.int64)
    padded_rows = int(((row_counts + 31) // 32 * 32).sum())
    if int(row_counts.sum()) != t * k:
        raise RuntimeError(f"prefill T={t}: routed blocks hold {row_counts.sum()} rows, not {t * k}")
    padded_flop = 2 * padded_rows * 3 * f * h
    # outputs of the measured work: every routed row written, finite
    out_ok = bool(torch.isfinite(h2.view(torch.float16).float()).all()) and \
        bool(torch.isfinite(partials.view(torch.float16).float()).all())
    if not out_ok:
        raise RuntimeError(f"prefill T={t} produced non-finite outputs")
    # the fused persistent launch (tsg_prefill_moe_gate_up_down) gives the two
    # GEMMs' bits: checked here on the measured inputs
    # the copy, the clearing and the fused launch all on the launch's stream,
    # in that order (torch's current stream is another one)
    with torch.cuda.stream(stream):
        want = partials.clone()
        partials.fill_(0)
        g.encode_gate_up_down(layer, hidden, h, sp, blocks, max_blocks, act_buf, partials, k, h, f,
                              n_blocks_device=nb, stream=stream)
    ctx.synchronize(stream)
    if not torch.equal(want, partials):
        raise RuntimeError(f"prefill T={t}: the fused GEMM differs from the two GEMMs")
    # sustained: SUSTAIN_LAYERS layers back to back in one graph
    lays = [layer] * SUSTAIN_LAYERS if not layers else \
        [layers[i % len(layers)] for i in range(SUSTAIN_LAYERS)]

    def gemms_two():
        for L in lays:
            g.encode_gate_up(L, hidden, h, sp, blocks, max_blocks, act_buf, h, f,
                             n_blocks_device=nb, stream=stream)
            g.encode_down(L, act_buf, sp, blocks, max_blocks, partials, k, h, f,
                          n_blocks_device=nb, stream=stream)

    def gemms():
        for L in lays:
            g.encode_gate_up_down(L, hidden, h, sp, blocks, max_blocks, act_buf, partials, k, h,
                                  f, n_blocks_device=nb, stream=stream)

    def whole():
        for L in lays:
            g.group_pairs_device(idx, w, t, k, e, sp, off, cnt, blocks, max_blocks, nb, scratch,
                                 tile_rows=tile_rows, stream=stream)
            g.encode_gate_up_down(L, hidden, h, sp, blocks, max_blocks, act_buf, partials, k, h,
                                  f, n_blocks_device=nb, stream=stream)
            red.encode_reduce_token_major(partials, w, h2, t, k, h, stream=stream)

    # the clock takes a few ms of MFMA work to settle: warm up first, then
    # alternate the three graphs and keep each one's median
    for _ in range(3):
        time_graph(torch, stream, gemms, reps=2)
    runs = {"two": [], "fused": [], "whole": []}
    for _ in range(3):
        runs["two"].append(time_graph(torch, stream, gemms_two, reps=2) / SUSTAIN_LAYERS)
        runs["fused"].append(time_graph(torch, stream, gemms, reps=2) / SUSTAIN_LAYERS)
        runs["whole"].append(time_graph(torch, stream, whole, reps=2) / SUSTAIN_LAYERS)
    two_ms, gemm_ms, total_ms = (float(np.median(runs[k])) for k in ("two", "fused", "whole"))
    ctx.synchronize(stream)  # a fused launch's schedule error would surface here
    if not bool(torch.isfinite(h2.view(torch.float16).float()).all()):
        raise RuntimeError(f"prefill T={t} produced non-finite outputs")
    log(f"prefill T={t}: single layers: group {per[0]*1e3:.1f} us, gate/up {per[1]*1e3:.1f} us, "
        f"down {per[2]*1e3:.1f} us, reduce {per[3]*1e3:.1f} us; sustained over "
        f"{SUSTAIN_LAYERS} layers: fused GEMMs {gemm_ms*1e3:.1f} us (two launches "
        f"{two_ms*1e3:.1f} us), layer {total_ms*1e3:.1f} us")
    return dict(us_per_layer=total_ms * 1e3, gemm_us=gemm_ms * 1e3, two_launch_gemm_us=two_ms * 1e3,
                gate_up_us=float(per[1]) * 1e3, down_us=float(per[2]) * 1e3,
                group_us=float(per[0]) * 1e3, reduce_us=float(per[3]) * 1e3,
                burst_gemm_us=float(per[1] + per[2]) * 1e3,
                gemm_tflops=flop / (gemm_ms * 1e-3) / 1e12,
                padded_tflops=padded_flop / (gemm_ms * 1e-3) / 1e12, padded_flop=padded_flop,
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


def run_verify_layer(tsg, torch, ctx, moe, layers, routers, n_layers, m, h, f, ne, seed,
                     shared=None, fused=True):
    """M tokens through n_layers whole layers with nothing on the host: the
    router rows (RealForwardRunner.swift:1826-1872) and the grouping of their
    pairs (:2116-2151) in one launch, the rows path over the device block
    list and the token-major reduce; `shared` (Qwen) adds the
    shared expert over the M rows. The M hidden states of a layer
    share a common part (x0 + 0.35 N(0,1)), so their top-8 sets overlap (a
    union of about 12-20). `fused`: the whole layer, the shared expert
    included, as one launch (tsg_moe_verify_layer / _shared); otherwise the
    router + grouping launch, the two rows-path launches and the reduce, with
    the shared expert's two launches on a second stream. Returns us per
    layer, the mean union and the launches per layer."""
    k = TOPK
    rng = np.random.default_rng(seed)
    hid = np.empty((n_layers, m, h), np.float32)
    for l in range(n_layers):
        hid[l] = rng.normal(0.0, 1.0, h)[None, :] + 0.35 * rng.normal(0.0, 1.0, (m, h))
    hidden = torch.from_numpy(hid.astype(np.float16).view(np.int16).ravel().copy()).cuda()
    ones_h = torch.full((h,), 0x3F80, dtype=torch.int16, device="cuda")
    ones_e = torch.full((ne,), 0x3F80, dtype=torch.int16, device="cuda")
    g = tsg.PrefillGroupedRoutedMoE(moe)
    red = tsg.PrefillMoE(ctx)
    max_blocks = m * k
    idx = torch.empty(n_layers * m * k, dtype=torch.int32, device="cuda")
    wts = torch.empty(n_layers * m * k, dtype=torch.int16, device="cuda")
    sp = torch.empty(m * k * 4, dtype=torch.int32, device="cuda")
    off = torch.empty(ne, dtype=torch.int32, device="cuda")
    cnt = torch.empty(ne, dtype=torch.int32, device="cuda")
    blocks = torch.empty(max_blocks * 4, dtype=torch.int32, device="cuda")
    nbs = torch.empty(n_layers, dtype=torch.int32, device="cuda")
    act = torch.empty(m * k * f, dtype=torch.int16, device="cuda")
    part = torch.empty(m * k * h, dtype=torch.int16, device="cuda")
    h2 = torch.empty(n_layers * m * h, dtype=torch.int16, device="cuda")
    if shared is not None:
        sact = torch.empty(m * f, dtype=torch.int16, device="cuda")
        sout = torch.empty(n_layers * m * h, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    # the shared branch depends only on the layer's input: it runs on a second
    # stream (default priority) beside the routed path and joins at the
    # layer's end (the shared-expert entry points use no context scratch)
    side = torch.cuda.Stream()

    def body():
        for l in range(n_layers):
            x = hidden[l * m * h:(l + 1) * m * h]
            il, wl = idx[l * m * k:(l + 1) * m * k], wts[l * m * k:(l + 1) * m * k]
            nb = nbs[l:l + 1]
            if shared is not None and not fused:
                # beside the four launches on a second stream
                side.wait_stream(stream)
                blob, o, gw = shared[l]
                tsg.encode_shared_expert_rows(moe, blob, o, x, h, gw, sact,
                                              sout[l * m * h:(l + 1) * m * h], m, h, f,
                                              stream=side)
            if fused and shared is not None:
                blob, o, gw = shared[l]
                moe.encode_verify_layer_shared(layers[l], routers[l], x, ones_h, ones_e, x, h,
                                               h2[l * m * h:(l + 1) * m * h], il, wl, blob, o, gw,
                                               sout[l * m * h:(l + 1) * m * h], m, ne, h, f,
                                               stream=stream)
            elif fused:
                moe.encode_verify_layer(layers[l], routers[l], x, ones_h, ones_e, x, h,
                                        h2[l * m * h:(l + 1) * m * h], il, wl, m, ne, h, f,
                                        stream=stream)
            else:
                moe.encode_router_gemma4_bf16_rows_grouped(routers[l], x, h, ones_h, ones_e, il,
                                                           wl, m, ne, h, sp, off, cnt, blocks,
                                                           max_blocks, nb, stream=stream)
                g.encode_streamed_rows_device(layers[l], x, h, sp, blocks, max_blocks, nb, act,
                                              part, k, h, f, stream=stream)
                red.encode_reduce_token_major(part, wl, h2[l * m * h:(l + 1) * m * h], m, k, h,
                                              stream=stream)
            if shared is not None and not fused:
                stream.wait_stream(side)

    ms = time_graph(torch, stream, body, reps=8)
    ctx.synchronize()
    out = h2.view(torch.float16).float()
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError("verify layer produced non-finite outputs")
    if shared is not None and not bool(torch.isfinite(sout.view(torch.float16).float()).all()):
        raise RuntimeError("shared expert rows produced non-finite outputs")
    ids = idx.view(n_layers, m * k).cpu().numpy()
    unions = [len(set(r.tolist())) for r in ids]
    if not fused and not np.array_equal(nbs.cpu().numpy(), unions):
        raise RuntimeError("device grouping's block count differs from the routing's union")
    launches = 1 if fused else 1 + 2 + 1 + (2 if shared is not None else 0)
    return ms * 1000.0 / n_layers, float(np.mean(unions)), launches


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
    ctx.synchronize()  # raises if a launch's hand-off wait timed out
    us1 = ms * 1000.0 / (n_tok * nl)
    y = ys.view(torch.float16).float()
    if not bool(torch.isfinite(y).all()):
        raise RuntimeError("qwen decode produced non-finite outputs")
    distinct = min(len(set(r.tolist())) for r in idx.view(nl, TOPK).cpu().numpy())
    if distinct != TOPK:
        raise RuntimeError("qwen decode routing collapsed")
    bytes1 = TOPK * payload + payload + e * h * 2 + h * 2 + 6 * h * 2
    log(f"qwen decode M=1: {us1:.3f} us/layer ({bytes1 / (us1 * 1e-6) / 1e9:.1f} GB/s)")
    us3, u3, nl3 = run_verify_layer(tsg, torch, ctx, moe, layers, routers, nl, 3, h, f, e,
                                    0x3333, shared=shared)
    us34, u34, nl34 = run_verify_layer(tsg, torch, ctx, moe, layers, routers, nl, 3, h, f, e,
                                       0x3333, shared=shared, fused=False)
    bytes3 = u3 * payload + payload + e * h * 2 + h * 2
    log(f"qwen decode M=3 whole layer: {us3:.3f} us/layer over a mean union of {u3:.1f} "
        f"experts ({bytes3 / (us3 * 1e-6) / 1e9:.1f} GB/s); routed part as four launches "
        f"{us34:.3f} us")
    pre = run_prefill_shape(tsg, torch, ctx, args, layers[0], QW_T, h, f, e, 1.0, "silu",
                            layers=layers)
    return {"workload": "qwen3.5-moe-35b-a3b-shaped layer (configs[4]): H=2048, 256 experts "
                        "I=512 top-8 SwiGLU + shared expert I=512 with sigmoid gate, 40 layers",
            "decode_m1": {"us_per_layer": round(us1, 3),
                          "GBps": round(bytes1 / (us1 * 1e-6) / 1e9, 2),
                          "bytes_per_layer": bytes1,
                          "launches_per_layer": 1},
            "decode_m3": {"us_per_layer": round(us3, 3), "mean_union": round(u3, 2),
                          "GBps": round(bytes3 / (us3 * 1e-6) / 1e9, 2),
                          "bytes_per_layer": int(bytes3), "launches_per_layer": nl3,
                          "path": "one launch (tsg_moe_verify_layer_shared: router rows, "
                                  "top-8, grouping, rows path over the routed experts and the "
                                  "shared expert, shared gate, reduce)",
                          "four_launches": {"us_per_layer": round(us34, 3),
                                            "mean_union": round(u34, 2),
                                            "launches_per_layer": nl34,
                                            "path": "router rows + grouping, two rows-path "
                                                    "launches, reduce; the shared expert beside "
                                                    "them on a second stream"}},
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


def run_router_int8(tsg, torch, ctx):
    """encodeRouterGemma4 (the INT8-affine router, MoE.swift:201-257) at the
    Gemma router shape: 128 experts x 2816 uint8 codes with bf16 scale and
    bias per group of 32, one fp16 row, top-8. 256 calls per graph replay."""
    ne, d, g = E, H, GROUP
    w = torch.empty(ne * d, dtype=torch.uint8, device="cuda")
    tsg.generators.bytes(w, 0x18A1)
    sc = torch.empty(ne * (d // g), dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(sc, 0x18A2, 0.002, True, 1.0)
    bi = torch.empty(ne * (d // g), dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(bi, 0x18A3, 0.1, False, 1.0)
    x = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(x, 0x18A4, 1.0)
    es = torch.empty(d, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(es, 0x18A5, 0.1, True, 1.0)
    pes = torch.empty(ne, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(pes, 0x18A6, 0.1, True, 1.0)
    idx = torch.empty(8, dtype=torch.int32, device="cuda")
    wts = torch.empty(8, dtype=torch.int16, device="cuda")
    ctx.set_affine_group_size(g)
    moe = tsg.MoE(ctx, router_weight_bits=8)
    stream = torch.cuda.Stream()
    calls = 256

    def body():
        for _ in range(calls):
            moe.encode_router_gemma4(w, sc, bi, x, es, pes, idx, wts, ne, d, stream=stream)

    us = time_graph(torch, stream, body, reps=8) * 1000.0 / calls
    nbytes = ne * d + 2 * ne * (d // g) * 2 + 2 * d * 2 + ne * 2 + 8 * 4 + 8 * 2
    ids = idx.cpu().numpy()
    if len(set(ids.tolist())) != 8 or ids.min() < 0 or ids.max() >= ne:
        raise RuntimeError(f"router_int8 selected {ids}")
    log(f"router int8 {ne}x{d} g{g}: {us:.3f} us/call ({nbytes / (us * 1e-6) / 1e9:.1f} GB/s)")
    return {"workload": f"INT8-affine router, {ne} experts x {d}, group {g}, top-8, "
                        "back-to-back launches", "us_per_call": round(us, 3),
            "bytes_per_call": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 2)}


def run_decode_int8(tsg, torch, ctx, layers):
    """The headline decode layer with the INT8-affine router (MoE.init's
    default router format, tsg_moe_decode_layer_int8) over the same 30
    resident layers: 8 tokens x 30 layers per graph replay, a fresh N(0,1)
    input per (token, layer). Algorithmic bytes per layer: the 8 experts, the
    router's 128 x 2816 codes and its group-32 scales and biases, x / es /
    residual / y rows and the gains."""
    n_in, ng = 8, H // GROUP
    rw = torch.empty(LAYERS * E * H, dtype=torch.uint8, device="cuda")
    tsg.generators.bytes(rw, 0x8A1)
    rs = torch.empty(LAYERS * E * ng, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(rs, 0x8A2, 0.0002, True, 1.0)
    rb = torch.empty(LAYERS * E * ng, dtype=torch.int16, device="cuda")
    tsg.generators.bf16_normal(rb, 0x8A3, 0.02, False, 1.0)
    ones_h = torch.full((H,), 0x3F80, dtype=torch.int16, device="cuda")
    ones_e = torch.full((E,), 0x3F80, dtype=torch.int16, device="cuda")
    inputs = torch.empty(n_in * LAYERS * H, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(inputs, 0x8A4, 1.0)
    ys = torch.empty(LAYERS * H, dtype=torch.int16, device="cuda")
    idx = torch.empty(LAYERS * TOPK, dtype=torch.int32, device="cuda")
    wts = torch.empty(LAYERS * TOPK, dtype=torch.int16, device="cuda")
    acts = torch.empty(TOPK * F, dtype=torch.int16, device="cuda")
    ctx.set_affine_group_size(GROUP)
    moe = tsg.MoE(ctx, router_weight_bits=8)
    stream = torch.cuda.Stream()

    def body():
        for k in range(n_in):
            for l in range(LAYERS):
                x = inputs[(k * LAYERS + l) * H:(k * LAYERS + l + 1) * H]
                moe.encode_decode_layer_int8(
                    layers[l], rw[l * E * H:(l + 1) * E * H], rs[l * E * ng:(l + 1) * E * ng],
                    rb[l * E * ng:(l + 1) * E * ng], x, ones_h, ones_e, x, x,
                    ys[l * H:(l + 1) * H], idx[l * TOPK:(l + 1) * TOPK],
                    wts[l * TOPK:(l + 1) * TOPK], acts, E, H, F, stream=stream)

    us = time_graph(torch, stream, body, reps=4) * 1000.0 / (n_in * LAYERS)
    ctx.synchronize()
    ids = idx.view(LAYERS, TOPK).cpu().numpy()
    if any(len(set(r.tolist())) != TOPK for r in ids) or ids.min() < 0 or ids.max() >= E:
        raise RuntimeError("decode_int8: a layer's top-8 is not 8 distinct experts")
    if not bool(torch.isfinite(ys.view(torch.float16).float()).all()):
        raise RuntimeError("decode_int8 produced non-finite outputs")
    nbytes = TOPK * shape_offsets(H, F)[2] + E * H + 2 * E * ng * 2 + 5 * H * 2 + E * 2
    log(f"decode layer, INT8 router: {us:.3f} us/layer ({nbytes / (us * 1e-6) / 1e9:.1f} GB/s)")
    return {"workload": "gemma4-26b-a4b decode MoE layer with the INT8-affine router (group 32), "
                        "one launch, 30 resident layers",
            "us_per_layer": round(us, 3), "bytes_per_layer": nbytes,
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


def run_verify(tsg, torch, ctx, args, layers, routers):
    """Gemma verify, M=5 over a union of about 12-20 experts, 30
    layers: the whole layer (router rows, top-8, grouping, rows path, reduce)
    in one launch, the same as four launches, and the rows path alone with
    the routing precomputed."""
    moe = tsg.MoE(ctx)
    us, u, nl = run_verify_layer(tsg, torch, ctx, moe, layers, routers, LAYERS, 5, H, F, E,
                                 0x5E5E)
    us4, u4, nl4 = run_verify_layer(tsg, torch, ctx, moe, layers, routers, LAYERS, 5, H, F, E,
                                    0x5E5E, fused=False)
    us0, u0 = run_rows_path(tsg, torch, ctx, moe, layers, LAYERS, 5, H, F, E, 0x5E5E)
    _, _, payload = shape_offsets(H, F)
    b = u * payload + ROUTER_BYTES
    log(f"verify M=5 whole layer, one launch: {us:.3f} us/layer over a mean union of {u:.1f} "
        f"experts ({b / (us * 1e-6) / 1e9:.1f} GB/s); four launches {us4:.3f} us; rows path "
        f"alone {us0:.3f} us")
    return {"workload": "gemma4-26b-a4b verify, M=5 (draft 4 + 1), union ~12-20, 30 layers "
                        "(configs[2])",
            "us_per_layer": round(us, 3), "mean_union": round(u, 2),
            "bytes_per_layer": int(b),
            "GBps": round(b / (us * 1e-6) / 1e9, 2),
            "frac_hbm_peak": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "launches_per_layer": nl,
            "path": "whole layer in one launch (tsg_moe_verify_layer): router rows, top-8, "
                    "grouping, rows path over the routed experts, token-major reduce",
            "four_launches": {"us_per_layer": round(us4, 3), "mean_union": round(u4, 2),
                              "launches_per_layer": nl4,
                              "path": "router rows + grouping (one launch), rows path over the "
                                      "device block list (two), token-major reduce"},
            "rows_path_only": {"us_per_layer": round(us0, 3), "mean_union": round(u0, 2),
                               "path": "rows path + reduce, routing precomputed on the host"}}


def attainable_gemm(torch):
    """The attainable dense fp16 GEMM rate on this GPU (torch.matmul ->
    hipBLASLt, fp16 in, fp32 accumulate): a square 8192^3 GEMM, and the
    prefill layer's two GEMMs as dense ones of the same shapes (gate/up:
    16,384 rows x 1,408 columns x K 2,816; down: 16,384 x 2,816 x K 704),
    whose combined rate is the layer-shape denominator of the prefill
    fraction."""
    out = {}
    for name, (m, n, k) in (("square_8192", (8192, 8192, 8192)),
                            ("layer_gate_up_dense", (PREFILL_T * TOPK, 2 * F, H)),
                            ("layer_down_dense", (PREFILL_T * TOPK, H, F))):
        a = torch.randn(m, k, dtype=torch.float16, device="cuda")
        b = torch.randn(k, n, dtype=torch.float16, device="cuda")
        stream = torch.cuda.Stream()
        c = torch.empty(m, n, dtype=torch.float16, device="cuda")

        def body():
            for _ in range(10):
                torch.matmul(a, b, out=c)

        ms = time_graph(torch, stream, body, reps=4) / 10
        out[name] = {"shape_mnk": [m, n, k], "us": round(ms * 1e3, 2),
                     "TFLOPs": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1)}
        del a, b, c
    gu, dn = out["layer_gate_up_dense"], out["layer_down_dense"]
    lf = sum(2.0 * m * n * k for m, n, k in (gu["shape_mnk"], dn["shape_mnk"]))
    out["layer_dense"] = {"us": round(gu["us"] + dn["us"], 2),
                          "TFLOPs": round(lf / ((gu["us"] + dn["us"]) * 1e-6) / 1e12, 1)}
    log(f"attainable fp16 GEMM (torch.matmul): {out}")
    return out


def prefill_summary(pre):
    return {"us_per_layer": round(pre["us_per_layer"], 2),
            "gemm_us": round(pre["gemm_us"], 2),
            "gemm_kernel": "moe_gemm_fused_kernel: gate/up + GeGLU and down in one persistent "
                           "launch (tsg_prefill_moe_gate_up_down)",
            "gemm_measure": f"sustained: {SUSTAIN_LAYERS} layers back to back in a HIP graph, "
                            f"each with its own weights; after a warm-up, the two-launch, "
                            f"fused and whole-layer graphs alternate three times, medians",
            "two_launch_gemm_us": round(pre["two_launch_gemm_us"], 2),
            "burst_gemm_us": round(pre["burst_gemm_us"], 2),
            "gate_up_us": round(pre["gate_up_us"], 2),
            "down_us": round(pre["down_us"], 2), "group_us": round(pre["group_us"], 2),
            "reduce_us": round(pre["reduce_us"], 2),
            "split_measure": "single layers, HIP events around each kernel of the two-launch "
                             "form (moe_gemm_kernel gate/up, then down)",
            "gemm_TFLOPs": round(pre["gemm_tflops"], 2),
            "frac_mfma_peak": round(pre["gemm_tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "padded_TFLOPs": round(pre["padded_tflops"], 2),
            "padded_flop_per_layer": pre["padded_flop"],
            "padded_measure": "MFMA work issued (each routed block's rows rounded up to 32-row "
                              "slices) over the same sustained time",
            "layer_TFLOPs": round(pre["layer_tflops"], 2),
            "flop_per_layer": pre["flop"], "routed_blocks": pre["blocks"]}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# One GPU's share of the box's host cores: worker pools on the GPU box are
# sized to it whatever nproc reports.
CPU_SHARE = 16


def cpu_baseline(torch, dec, bufs, routers, offs, stride, budget_s=6.0):
    """The reference's CPU path for the same math, restated in C (oracle,
    the timed build: -O3 -march=native for this host, vectorizable dot
    products like vDSP_dotpr's):
      decode  routerReference + MoeRef.applyStreamedRouted per layer
              (main.swift:384-402, Reference/MoE/Moe.swift:16-123) over the
              decode chain's layers with their real inputs and routing;
      prefill the expert-major reference of PrefillMoEGEMMCheck.swift:138-173
              on a sample of config 4's tokens (all 8 of each token's pairs,
              its experts dequantised once), in TFLOP/s of the GEMM work.
    Timed on CPU_SHARE threads (one GPU's share of this host) and on one."""
    import oracle
    path = oracle.use_timed_build()
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(nproc, CPU_SHARE))
    idx = dec["idx"].cpu().numpy().reshape(LAYERS, TOPK)
    es = np.ones(H, np.float32)
    pes = np.ones(E, np.float32)
    layer_in = []
    for l in range(LAYERS):
        x_bits = dec["xs"][l].cpu().numpy().view(np.uint16)
        rw = oracle.bf16_to_float(routers[l].cpu().numpy().view(np.uint16)).reshape(E, H)
        blobs = [bufs[l][int(e) * stride:(int(e) + 1) * stride].cpu().numpy() for e in idx[l]]
        layer_in.append((oracle.f16_to_float(x_bits), rw, blobs))

    def decode_us(n_threads, budget):
        oracle.set_threads(n_threads)
        done, elapsed = 0, 0.0
        while elapsed < budget and done < 100 * LAYERS:
            x, rw, blobs = layer_in[done % LAYERS]
            t0 = time.perf_counter()
            _, rwts = oracle.router_reference(rw, x * es, TOPK, pes)
            oracle.moe_apply_streamed_routed(blobs, np.array(offs, np.uint32), x, x, rwts, H, F,
                                             GROUP, True)
            elapsed += time.perf_counter() - t0
            done += 1
        return elapsed * 1e6 / done, done

    us_n, n_n = decode_us(threads, budget_s)
    us_1, n_1 = decode_us(1, budget_s * 5 / 6)
    # prefill: config 4's routing and inputs, every pair of a sample of tokens
    t_all = PREFILL_T
    idx_p, w_p = zipf_routing(t_all, E, TOPK, 1.1, 0x21F)
    image = bufs[0].cpu().numpy()
    blobs_all = [image[e * stride:(e + 1) * stride] for e in range(E)]
    hid = np.random.default_rng(0x33).normal(0, 1, t_all * H).astype(np.float32)
    hid_bits = oracle.f16_bits(hid)

    def prefill_rate(n_threads, tokens):
        oracle.set_threads(n_threads)
        sel = np.arange(tokens, dtype=np.int64)
        pairs = oracle.make_token_expert_pairs(idx_p[sel].astype(np.uint32),
                                               w_p[sel].view(np.uint16), tokens, TOPK)
        sp = oracle.group_pairs(pairs, tokens, TOPK, E)["sorted_pairs"]
        t0 = time.perf_counter()
        oracle.prefill_moe_ref(blobs_all, np.array(offs, np.uint32), hid_bits[:tokens * H], H, sp,
                               TOPK, H, F, GROUP, True)
        el = time.perf_counter() - t0
        flop = 2.0 * sp.size * 3 * F * H
        return flop / el / 1e12, el, sp.size, len(set(sp["expert"].tolist()))

    pre_n = prefill_rate(threads, 512)
    pre_1 = prefill_rate(1, 64)
    return dict(value=round(LAYER_BYTES / (us_n * 1e-6) / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=f"{n_n} decode layers (router + 8 experts, H=2816 F=704 sym g32) through "
                       f"the C restatement of routerReference + MoeRef, {us_n:.0f} us/layer on "
                       f"{threads} threads ({n_1} layers, {us_1:.0f} us/layer on 1 thread)",
                us_per_layer=round(us_n, 1), one_thread_us_per_layer=round(us_1, 1),
                one_thread_value=round(LAYER_BYTES / (us_1 * 1e-6) / 1e9, 3),
                nproc=nproc, cpu_model=_cpu_model(),
                build=os.path.basename(path) + " (gcc -O3 -march=native -ffp-contract=off)",
                prefill={"unit": "TFLOP/s", "value": round(pre_n[0], 5),
                         "one_thread_value": round(pre_1[0], 5),
                         "sample": f"config 4, first 512 tokens: {pre_n[2]} pairs over "
                                   f"{pre_n[3]} experts, {pre_n[1]:.2f} s on {threads} threads; "
                                   f"first 64 tokens ({pre_1[2]} pairs) {pre_1[1]:.2f} s on 1 "
                                   f"thread; expert-major with fp16 roundings "
                                   f"(PrefillMoEGEMMCheck.swift:138-173)"})


def run_floors(tsg, torch, layers, reps=8):
    """Two floors of a one-launch decode layer of this shape (measurement
    kernels of libtsugumi_floors.so), each as 120 launches back to back in a
    HIP graph (4 tokens x 30 layers, fresh random expert ids per launch):
    an empty kernel with the layer's grid, block and LDS (the launch-to-launch
    period), and a kernel of the same grid that only streams the 8 routed
    experts' 26,763,264 payload bytes with 16-byte loads (the time to move the
    expert bytes once the routing is known)."""
    import ctypes as C
    lib = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tsugumi_amd",
                              "libtsugumi_floors.so"))
    lib.tsg_floor_empty.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p]
    lib.tsg_floor_stream.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32,
                                     C.c_uint32, C.c_uint32, C.c_void_p]
    _, stride = gemma_offsets()
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    rng = np.random.default_rng(0xF1)
    ids = [(rng.permutation(E)[:TOPK]).astype(np.uint32) for _ in range(4 * LAYERS)]
    blocks, threads, lds = 256, 768, 20080  # decode_layer_kernel's launch at this shape

    def empty():
        for _ in range(4 * LAYERS):
            if lib.tsg_floor_empty(stream.cuda_stream, blocks, threads, lds, sink.data_ptr()):
                raise RuntimeError("floor_empty launch failed")

    def stream_all():
        for i in range(4 * LAYERS):
            if lib.tsg_floor_stream(stream.cuda_stream, layers[i % LAYERS].device_ptr, stride,
                                    ids[i].ctypes.data, EXPERT_BYTES, blocks, 1024,
                                    sink.data_ptr()):
                raise RuntimeError("floor_stream launch failed")

    us_empty = time_graph(torch, stream, empty, reps=reps) * 1000.0 / (4 * LAYERS)
    us_stream = time_graph(torch, stream, stream_all, reps=reps) * 1000.0 / (4 * LAYERS)
    nbytes = TOPK * EXPERT_BYTES
    log(f"floors: empty launch {us_empty:.3f} us, 8-expert stream {us_stream:.3f} us "
        f"({nbytes / (us_stream * 1e-6) / 1e9:.1f} GB/s)")
    return {"empty_launch_us": round(us_empty, 3), "expert_stream_us": round(us_stream, 3),
            "expert_stream_bytes": nbytes,
            "expert_stream_GBps": round(nbytes / (us_stream * 1e-6) / 1e9, 1),
            "grid": f"{blocks} blocks x {threads} threads, {lds} B dynamic LDS (empty); "
                    f"{blocks} x 1024 (stream)"}


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
    ap.add_argument("--floors", action="store_true",
                    help="time the decode layer's floors (empty launch, expert stream) and exit")
    ap.add_argument("--verify-only", action="store_true",
                    help="run only the verify M=5 figures (configs[2], for profiling) and exit")
    ap.add_argument("--qwen-only", action="store_true",
                    help="run only the Qwen-shaped figures (configs[4], for profiling) and exit")
    ap.add_argument("--qmv-only", action="store_true",
                    help="run only the single QMV figure (configs[0], for profiling) and exit")
    ap.add_argument("--router-int8-only", action="store_true",
                    help="run only the INT8-affine router figure (for profiling) and exit")
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
    if args.qwen_only:
        print(json.dumps({"qwen35": run_qwen(tsg, torch, args)}), flush=True)
        return
    if args.router_int8_only:
        print(json.dumps({"router_int8": run_router_int8(tsg, torch, ctx)}), flush=True)
        return
    if args.qmv_only:
        print(json.dumps({"qmv": run_qmv(tsg, torch, ctx)}), flush=True)
        return
    log(f"building {LAYERS} resident layers ({LAYERS * E * gemma_offsets()[1] / 1e9:.2f} GB)")
    layers, bufs, routers, offs, stride = make_layers(tsg, ctx, torch, LAYERS)
    if args.traffic_probe:
        traffic_probe(tsg, torch, ctx, layers, routers)
        return
    if args.floors:
        print(json.dumps({"floors": run_floors(tsg, torch, layers)}), flush=True)
        return
    if args.verify_only:
        print(json.dumps({"verify_m5": run_verify(tsg, torch, ctx, args, layers, routers)}),
              flush=True)
        return
    if args.prefill_only:
        pre = run_prefill(tsg, torch, ctx, args, layers)
        print(json.dumps({"prefill_gemm_us": round(pre["gemm_us"], 2),
                          "gemm_TFLOPs": round(pre["gemm_tflops"], 2)}), flush=True)
        return
    dec = run_decode(tsg, torch, ctx, args, layers, routers)
    pre = None if args.no_prefill else run_prefill(tsg, torch, ctx, args, layers)
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
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                   "routing_margin": routing_margins(torch, dec, routers)},
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
        try:
            att = attainable_gemm(torch)
            out["prefill"]["attainable_fp16_gemm"] = att
            out["prefill"]["frac_attainable_square"] = round(
                pre["gemm_tflops"] / att["square_8192"]["TFLOPs"], 4)
            out["prefill"]["frac_attainable_layer_shape"] = round(
                pre["gemm_tflops"] / att["layer_dense"]["TFLOPs"], 4)
        except Exception as exc:  # noqa: BLE001 - reported, not hidden
            log(f"attainable GEMM failed: {exc}")
    try:
        out["decode"]["floors"] = run_floors(tsg, torch, layers)
    except Exception as exc:  # noqa: BLE001 - reported, not hidden
        log(f"floors failed: {exc}")
    if not args.no_extra_configs:
        # the other BASELINE configs, after the headline figures (a failure here
        # is reported in its entry and does not void the headline)
        extra = {}
        for name, fn in (("qmv", lambda: run_qmv(tsg, torch, ctx)),
                         ("router_int8", lambda: run_router_int8(tsg, torch, ctx)),
                         ("decode_int8_router", lambda: run_decode_int8(tsg, torch, ctx, layers)),
                         ("layer_tail", lambda: run_tail(tsg, torch, ctx)),
                         ("dense_qmm", lambda: run_dense_qmm(tsg, torch, ctx)),
                         ("verify_m5", lambda: run_verify(tsg, torch, ctx, args, layers, routers)),
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
