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
    o_gw, o_gs = 0, W_GU
    o_uw, o_us = W_GU + S_GU, 2 * W_GU + S_GU
    o_dw, o_ds = 2 * (W_GU + S_GU), 2 * (W_GU + S_GU) + W_D
    stride = (o_ds + S_D + 16383) // 16384 * 16384
    return [o_gw, o_gs, o_gs, o_uw, o_us, o_us, o_dw, o_ds, o_ds], stride


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layers(tsg, ctx, torch, n_layers, seed=0x7E57):
    """n_layers resident Gemma-shaped layers: nibbles uniform in [0,15], scales
    bf16(|N(0,0.02)|/7), router bf16 N(0, 1/sqrt(H))."""
    offs, stride = gemma_offsets()
    layers, bufs, routers = [], [], []
    regions = [(offs[1], F * (H // GROUP)), (offs[4], F * (H // GROUP)), (offs[7], H * (F // GROUP))]
    for l in range(n_layers):
        buf = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
        tsg.generators.bytes(buf, seed + l)
        for e in range(E):
            for j, (o, n) in enumerate(regions):
                reg = buf[e * stride + o:e * stride + o + 2 * n].view(torch.int16)
                tsg.generators.bf16_normal(reg, (seed + l) * 4096 + e * 3 + j + 1, 0.02, True, 7.0)
        rw = torch.empty(E * H, dtype=torch.int16, device="cuda")
        tsg.generators.bf16_normal(rw, (seed + l) * 4096 + 4000, 1.0 / np.sqrt(H))
        layers.append(tsg.ResidentLayer(ctx, E, stride, offs, device_tensor=buf))
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
    moe = tsg.MoE(ctx)
    g = tsg.PrefillGroupedRoutedMoE(moe)
    red = tsg.PrefillMoE(ctx)
    t, k = PREFILL_T, TOPK
    idx_np, w_np = zipf_routing(t, E, k, 1.1, 0x21F)
    idx = torch.from_numpy(idx_np.ravel()).cuda()
    w = torch.from_numpy(w_np.ravel().view(np.int16)).cuda()
    hidden = torch.empty(t * H, dtype=torch.int16, device="cuda")
    tsg.generators.f16_normal(hidden, 0x33, 1.0)
    tile_rows = 128  # the grouped GEMM's widest pass
    max_blocks = t * k // tile_rows + E
    sp = torch.empty(t * k * 4, dtype=torch.int32, device="cuda")
    off = torch.empty(E, dtype=torch.int32, device="cuda")
    cnt = torch.empty(E, dtype=torch.int32, device="cuda")
    blocks = torch.empty(max_blocks * 4, dtype=torch.int32, device="cuda")
    nb = torch.empty(1, dtype=torch.int32, device="cuda")
    scratch = torch.empty(g.scratch_bytes(t, k, E) // 4 + 1, dtype=torch.int32, device="cuda")
    act = torch.empty(t * k * F, dtype=torch.int16, device="cuda")
    partials = torch.empty(t * k * H, dtype=torch.int16, device="cuda")
    h2 = torch.empty(t * H, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]

    def chunk(record=False):
        if record:
            ev[0].record(stream)
        g.group_pairs_device(idx, w, t, k, E, sp, off, cnt, blocks, max_blocks, nb, scratch,
                             tile_rows=tile_rows, stream=stream)
        if record:
            ev[1].record(stream)
        g.encode_gate_up(layer, hidden, H, sp, blocks, max_blocks, act, H, F,
                         n_blocks_device=nb, stream=stream)
        if record:
            ev[2].record(stream)
        g.encode_down(layer, act, sp, blocks, max_blocks, partials, k, H, F,
                      n_blocks_device=nb, stream=stream)
        if record:
            ev[3].record(stream)
        red.encode_reduce_token_major(partials, w, h2, t, k, H, stream=stream)
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
                gemm_tflops=PREFILL_FLOP / (gemm_ms * 1e-3) / 1e12,
                layer_tflops=PREFILL_FLOP / (total_ms * 1e-3) / 1e12, blocks=nblocks)


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
        out["prefill"] = {
            "us_per_layer": round(pre["us_per_layer"], 2),
            "gemm_us": round(pre["gemm_us"], 2), "gate_up_us": round(pre["gate_up_us"], 2),
            "down_us": round(pre["down_us"], 2), "group_us": round(pre["group_us"], 2),
            "reduce_us": round(pre["reduce_us"], 2),
            "gemm_TFLOPs": round(pre["gemm_tflops"], 2),
            "frac_mfma_peak": round(pre["gemm_tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "layer_TFLOPs": round(pre["layer_tflops"], 2),
            "flop_per_layer": PREFILL_FLOP, "routed_blocks": pre["blocks"]}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, dec, bufs, routers, offs, stride)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
