"""Synthetic inputs shaped like BASELINE.json's configurations, for the GPU
parity tests: resident sym-g32 layers with random nibbles and bf16 scales,
Zipf prefill routing, and speculative-verify routing whose top-8 sets overlap.

Everything is drawn with numpy from a fixed seed on the host, so the oracle
and the kernels see the same bytes.
"""
from __future__ import annotations

import numpy as np

import oracle

GROUP = 32


def sym_offsets(h: int, f: int, group: int = GROUP):
    """MoEExpertOffsets of a sym blob of shape (h, f) in the packer's order
    (RepackPlanner.swift:442-520: gate W, S, up W, S, down W, S; the bias
    offsets alias the scales), its payload and its 16 KiB stride."""
    w_gu, s_gu = f * h // 2, f * (h // group) * 2
    w_d = h * f // 2
    s_d = h * (f // group) * 2
    o_gs, o_uw = w_gu, w_gu + s_gu
    o_us, o_dw = 2 * w_gu + s_gu, 2 * (w_gu + s_gu)
    o_ds = o_dw + w_d
    payload = o_ds + s_d
    stride = (payload + 16383) // 16384 * 16384
    return np.array([0, o_gs, o_gs, o_uw, o_us, o_us, o_dw, o_ds, o_ds], np.uint32), payload, stride


def scale_bits(rng, n: int) -> np.ndarray:
    """bf16(|N(0, 0.02)| / 7), the BASELINE scale distribution."""
    return oracle.bf16_bits(np.abs(rng.normal(0.0, 0.02, n)).astype(np.float32) / np.float32(7.0))


def random_sym_layer(rng, ne: int, h: int, f: int):
    """A layer-file image of `ne` sym g32 experts: nibbles uniform in [0, 15],
    scales bf16(|N(0,.02)|/7). Returns (image, stride, offsets, blobs) with
    blobs[e] a view of expert e's bytes."""
    offs, payload, stride = sym_offsets(h, f)
    image = np.zeros(ne * stride, np.uint8)
    for e in range(ne):
        blob = image[e * stride:e * stride + payload]
        blob[:] = rng.integers(0, 256, payload, dtype=np.uint8)
        for o_s, n in ((offs[1], f * (h // GROUP)), (offs[4], f * (h // GROUP)),
                       (offs[7], h * (f // GROUP))):
            blob[o_s:o_s + 2 * n] = scale_bits(rng, n).view(np.uint8)
    blobs = [image[e * stride:(e + 1) * stride] for e in range(ne)]
    return image, stride, offs, blobs


def f16_normal(rng, n: int, sigma: float = 1.0) -> np.ndarray:
    """fp16 bits of sigma * N(0,1), |x| < 2^-17 flushed to zero."""
    x = (rng.normal(0.0, sigma, n)).astype(np.float32)
    x[np.abs(x) < 2.0 ** -17] = 0.0
    return oracle.f16_bits(x)


def zipf_routing(rng, t: int, ne: int, k: int, s: float):
    """Gumbel-top-k over log p_e, p ~ rank^-s on a permutation of the ids;
    weights are the fp16 softmax over the k perturbed scores."""
    perm = rng.permutation(ne)
    logp = -s * np.log(np.arange(1, ne + 1, dtype=np.float64))
    logp = logp[np.argsort(perm)]
    g = -np.log(-np.log(rng.random((t, ne))))
    scores = logp[None, :] + g
    idx = np.argsort(-scores, axis=1, kind="stable")[:, :k].astype(np.uint32)
    top = np.take_along_axis(scores, idx.astype(np.int64), axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, oracle.f16_bits(w).reshape(t, k)


def verify_routing(rng, m: int, ne: int, k: int, target: int = 16):
    """Routing of M tokens whose top-k sets overlap: a shared
    random logit prefix plus a per-token perturbation whose scale, from a fixed
    grid, brings the union of the sets nearest `target`. Returns ids [m, k],
    fp16 weight bits [m, k] and the union size."""
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
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx.astype(np.uint32), oracle.f16_bits(w).reshape(m, k), u


def rows_blocks(grouped) -> np.ndarray:
    """One rows-path block per expert group: (expert, pair_start, rows,
    pair_start), the block list encodeStreamedRows builds from the groups
    (PrefillGroupedRoutedMoE.swift:835-870)."""
    return np.array([(int(g["expert"]), int(g["pair_start"]), int(g["pair_count"]),
                      int(g["pair_start"])) for g in grouped["groups"]], dtype=oracle.BLOCK_DTYPE)


def sampled_pairs(sorted_pairs: np.ndarray, t: int, every: int = 16, extra_pos=None):
    """The pairs a full-size check recomputes on the CPU: every pair of the
    largest expert (the one split over the most GEMM work items), every pair
    of every `every`-th token, and the positions `extra_pos` (e.g. the first
    and last row of every routed block). Returns (subset in sorted order, its
    positions in sorted_pairs, the sampled tokens, the head expert, its rows)."""
    experts, counts = np.unique(sorted_pairs["expert"], return_counts=True)
    head = experts[np.argmax(counts)]
    tokens = np.arange(0, t, every)
    keep = (sorted_pairs["expert"] == head) | np.isin(sorted_pairs["token"], tokens)
    if extra_pos is not None:
        keep[np.asarray(extra_pos, np.int64)] = True
    pos = np.nonzero(keep)[0]
    return sorted_pairs[pos], pos, tokens, int(head), int(counts.max())
