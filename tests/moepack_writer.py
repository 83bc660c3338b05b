"""Writes small MoEPack installs for the loader tests: manifest.json,
packed_experts/layout.json and the layer files, shaped as the reference's
writers shape them (MoEPackJSON.encodeManifest / encodeLayout,
MoEPackJSON.swift:252-300; sub-tensor order gate, gate_scales, [gate_biases],
up..., down... from RepackPlanner.swift:442-520; stride rounded up to 16 KiB).

Expert blobs are given in logical order; `physical` (logical -> physical rank)
scatters them in the layer file the way a reordered install does.
"""
from __future__ import annotations

import copy
import hashlib
import json
import os

import numpy as np

from tests import kernelcheck as kc

ZERO_SHA = "0" * 64
ROLES = ("gate", "up", "down")


def toy_manifest(num_layers=1, experts=2, stride=16384, layer_files=None, **top):
    """A valid manifest dict in the shape of the reference's toy installs
    (ManifestReaderTests.swift gemma4Toy; the v1 fixture's field set)."""
    if layer_files is None:
        layer_files = {f"packed_experts/layer_{i:02d}.bin": experts * stride
                       for i in range(num_layers)}
    slot = {"weightBits": 4, "scheme": "affine", "scaleType": "BF16", "biasType": "BF16",
            "groupSize": 64}
    m = {
        "magic": "MOEPACK", "versionMajor": 1, "versionMinor": 0,
        "flags": {"streamingPresent": True, "turboQuantKV": False, "aneSharedExpert": False},
        "modelID": "fixture/model", "sourceSnapshotHash": "fixture-snapshot",
        "arch": {
            "hiddenSize": 64, "ffnIntermediate": 128, "moeIntermediateSize": 32,
            "numHeads": 4, "numKVHeads": 2, "numFullKVHeads": 1, "headDim": 16,
            "fullHeadDim": 32, "vocabSize": 1024, "slidingWindow": 128,
            "finalLogitSoftcap": 30, "ropeTheta": 10000, "fullRopeTheta": 1000000,
            "partialRotaryFactor": 0.25, "numLayers": num_layers, "numExperts": experts,
            "topKExperts": 1, "tieWordEmbeddings": True, "attentionKEqV": True,
            "hiddenActivation": "gelu_pytorch_tanh",
            "fullAttentionLayerMask": [0] * num_layers,
        },
        "quant": {k: dict(slot) for k in ("embedding", "attention", "sharedExpert",
                                          "routedExpert")},
        "files": {"model_weights.bin": {"size": 16416, "sha256": ZERO_SHA},
                  "packed_experts/layout.json": {"size": 1, "sha256": ZERO_SHA}},
        "expertsPerLayer": experts, "numLayers": num_layers, "expertStride": stride,
    }
    m["quant"]["router"] = dict(slot, weightBits=8)
    for path, size in layer_files.items():
        m["files"][path] = {"size": size, "sha256": ZERO_SHA}
    m.update(top)
    return m


def toy_layout(num_layers=1, experts=2, stride=16384, tensors=None, physical=None,
               explicit_ids=True):
    """A valid layout dict; every expert carries `tensors` (default: the v1
    fixture's single `gate`)."""
    if tensors is None:
        tensors = {"gate": {"offset": 0, "size": 32, "dtype": "U32", "shape": [8, 8],
                            "bits": 4}}
    layers = []
    for li in range(num_layers):
        perm = [int(p) for p in physical[li]] if physical is not None else list(range(experts))
        ex = []
        for e in range(experts):
            entry = {"offset": perm[e] * stride, "size": stride,
                     "tensors": copy.deepcopy(tensors)}
            if explicit_ids:
                entry["expert"] = e
            if physical is not None:
                entry["physicalRank"] = perm[e]
            ex.append(entry)
        layers.append({"layer": li, "file": f"layer_{li:02d}.bin", "experts": ex})
    return {"expertStride": stride, "numLayers": num_layers, "expertsPerLayer": experts,
            "layers": layers}


def dumps(doc) -> bytes:
    return json.dumps(doc, indent=2, sort_keys=True).encode()


def expert_tensors(parts, offsets, symmetric):
    """Layout `tensors` of one expert blob made by kernelcheck.pack_blob."""
    out = {}
    for r, (role, (packed, scales, biases)) in enumerate(zip(ROLES, parts)):
        rows, nbytes = packed.shape  # two int4 weights per byte
        out[role] = {"offset": int(offsets[3 * r]), "size": int(packed.nbytes), "dtype": "U32",
                     "shape": [int(rows), int(nbytes) * 2], "bits": 4}
        out[role + "_scales"] = {"offset": int(offsets[3 * r + 1]), "size": int(scales.nbytes),
                                 "dtype": "BF16", "shape": list(map(int, scales.shape))}
        if not symmetric:
            out[role + "_biases"] = {"offset": int(offsets[3 * r + 2]),
                                     "size": int(biases.nbytes), "dtype": "BF16",
                                     "shape": list(map(int, biases.shape))}
    return out


def write_pack(root, layer_parts, *, d, f, group, symmetric, physical=None, top_k=8,
               family=None, align=16, lead=0):
    """Writes an install under `root`. layer_parts[l][e] = ((Wg,Sg,Bg),
    (Wu,Su,Bu), (Wd,Sd,Bd)) of logical expert e in layer l. Returns
    (stride, offsets9, logical images: one uint8 array per layer)."""
    os.makedirs(os.path.join(root, "packed_experts"), exist_ok=True)
    n_layers, n_exp = len(layer_parts), len(layer_parts[0])
    blobs = [[kc.pack_blob(p, symmetric, keep_biases=not symmetric, align=align, lead=lead)
              for p in layer] for layer in layer_parts]
    offs = blobs[0][0][1]
    size = max(b.size for layer in blobs for b, _ in layer)
    stride = int((size + 16383) // 16384 * 16384)
    tensors = expert_tensors(layer_parts[0][0], offs, symmetric)
    images, files = [], {}
    for li, layer in enumerate(blobs):
        perm = physical[li] if physical is not None else list(range(n_exp))
        logical = np.zeros(n_exp * stride, np.uint8)
        phys = np.zeros(n_exp * stride, np.uint8)
        for e, (b, o) in enumerate(layer):
            assert np.array_equal(o, offs)
            logical[e * stride:e * stride + b.size] = b
            phys[perm[e] * stride:perm[e] * stride + b.size] = b
        path = f"packed_experts/layer_{li:02d}.bin"
        with open(os.path.join(root, path), "wb") as fh:
            fh.write(phys.tobytes())
        files[path] = phys
        images.append(logical)
    weights = np.zeros(16384, np.uint8)  # stand-in: the resident weights are not read here
    with open(os.path.join(root, "model_weights.bin"), "wb") as fh:
        fh.write(weights.tobytes())
    layout = toy_layout(n_layers, n_exp, stride, tensors, physical)
    layout_bytes = dumps(layout)
    with open(os.path.join(root, "packed_experts/layout.json"), "wb") as fh:
        fh.write(layout_bytes)
    m = toy_manifest(n_layers, n_exp, stride)
    m["arch"].update(hiddenSize=d, moeIntermediateSize=f, topKExperts=top_k)
    scheme = {"scheme": "sym", "biasType": "none"} if symmetric else {}
    for k in ("embedding", "attention", "sharedExpert", "routedExpert"):
        m["quant"][k].update(groupSize=group, **scheme)
    m["quant"]["router"] = {"weightBits": 16, "scheme": "bf16", "scaleType": "none",
                            "biasType": "none", "groupSize": group}
    if family is not None:
        m["arch"]["family"] = family

    def entry(data: bytes):
        return {"size": len(data), "sha256": hashlib.sha256(data).hexdigest()}
    m["files"] = {"model_weights.bin": entry(weights.tobytes()),
                  "packed_experts/layout.json": entry(layout_bytes)}
    for path, img in files.items():
        m["files"][path] = entry(img.tobytes())
    with open(os.path.join(root, "manifest.json"), "wb") as fh:
        fh.write(dumps(m))
    return stride, offs, images
