"""tsugumi_amd — Tsugumi's int4 MoE expert-matmul path on one MI355X (gfx950).

Python mirror of the reference's Swift encoder classes over the C ABI in
include/tsugumi_hip.h (libtsugumi_hip.so). Names follow the reference:

    MetalContext            -> Context
    MoE                     -> MoE            (Kernels/MoE/MoE.swift:42-662)
    DequantInt4GEMV         -> DequantInt4GEMV (Kernels/Quant/DequantInt4GEMV.swift)
    PrefillRouter           -> PrefillRouter  (Kernels/Prefill/MoE/PrefillRouter.swift)
    PrefillMoEGrouping      -> PrefillMoEGrouping (PrefillMoEGrouping.swift:90-202)
    PrefillRoutedGEMMPlanner-> PrefillRoutedGEMMPlanner (PrefillGroupedRoutedMoE.swift:42-83)
    PrefillGroupedRoutedMoE -> PrefillGroupedRoutedMoE (PrefillGroupedRoutedMoE.swift)
    PrefillMoE              -> PrefillMoE     (PrefillMoE.swift:11-38)
    streamed experts        -> ResidentLayer  (whole layer held in HBM)
    ManifestReader + PackedExpertsLayoutReader -> MoEPack (install reader + layer upload)
    SharedExpertInt4        -> SharedExpertInt4 (Gemma's dense int4 MLP)

Device buffers are torch CUDA tensors (plumbing only); `stream` defaults to
torch's current stream. Every call raises TsgError on a non-OK status; there
is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi
from ._abi import (TSG_ACT_GELU_TANH, TSG_ACT_SILU, TSG_AFFINE, TSG_SYM, ExpertOffsets,
                   RoutedBlock, TokenExpertPair, TsgError, check, load)

__all__ = [
    "Context", "MoE", "DequantInt4GEMV", "QwenKernels", "encode_shared_expert",
    "PrefillRouter", "PrefillMoEGrouping",
    "PrefillRoutedGEMMPlanner", "PrefillGroupedRoutedMoE", "PrefillMoE", "ResidentLayer",
    "MoEPack", "SharedExpertInt4", "PrefillLayerTail", "FusedLayerTail", "PrefillInt4QMM",
    "ExpertOffsets", "TsgError", "PAIR_DTYPE", "BLOCK_DTYPE", "GROUP_DTYPE", "TILE_DTYPE",
    "generators", "load",
]

PAIR_DTYPE = np.dtype([("token", "<u4"), ("expert", "<u4"), ("rank", "<u4"),
                       ("weight_bits", "<u4")])
GROUP_DTYPE = np.dtype([("expert", "<u4"), ("pair_start", "<u4"), ("pair_count", "<u4")])
TILE_DTYPE = np.dtype([("group_start", "<u4"), ("group_count", "<u4"),
                       ("pair_start", "<u4"), ("pair_count", "<u4")])
BLOCK_DTYPE = np.dtype([("local_slot", "<u4"), ("pair_start", "<u4"),
                        ("row_count", "<u4"), ("local_row", "<u4")])


def _ptr(t) -> int | None:
    """Device address of a contiguous torch CUDA tensor (None passes NULL)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    assert t.is_cuda, "device buffers must be CUDA (HIP) tensors"
    assert t.is_contiguous(), "device buffers must be contiguous"
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch
    return torch.cuda.current_stream().cuda_stream


def _np_ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _scratch_rows(scratch, f: int, max_rows) -> int:
    """Rows of f elements a scratch buffer holds: max_rows when given, else
    what the tensor's size allows (an address given as an int needs max_rows)."""
    if max_rows is not None:
        return int(max_rows)
    if scratch is None or isinstance(scratch, int):
        raise ValueError("max_rows is required when the scratch is not a tensor")
    return int(scratch.numel()) // int(f) if f else 0


def offsets_from(seq) -> ExpertOffsets:
    if isinstance(seq, ExpertOffsets):
        return seq
    return ExpertOffsets(*[int(v) for v in seq])


# ------------------------------------------------------------------ context

class Context:
    """MetalContext analogue: device binding, affine group size and scheme
    (MetalContext.swift:79-175). Defaults: group 64, affine."""

    def __init__(self, device: int = 0, group_size: int | None = None,
                 scheme: str | None = None):
        self.lib = load()
        h = C.c_void_p()
        check(self.lib.tsg_ctx_create(device, C.byref(h)))
        self.handle = h
        self.device = device
        if group_size is not None:
            self.set_affine_group_size(group_size)
        if scheme is not None:
            self.set_affine_scheme(scheme)

    def set_affine_group_size(self, g: int) -> None:
        check(self.lib.tsg_ctx_set_affine_group_size(self.handle, g))
        self.group_size = g

    def set_affine_scheme(self, scheme: str) -> None:
        check(self.lib.tsg_ctx_set_affine_scheme(self.handle,
                                                 TSG_SYM if scheme == "sym" else TSG_AFFINE))
        self.scheme = scheme

    def synchronize(self, stream=None) -> None:
        check(self.lib.tsg_ctx_synchronize(self.handle, _stream(stream)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.tsg_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ResidentLayer:
    """One MoEPack layer file held byte-for-byte in HBM (replaces the SSD
    streamer + MTLResidencySet, ModelExpertIO.swift:112-324)."""

    def __init__(self, ctx: Context, num_experts: int, expert_stride: int, offsets,
                 device_tensor=None):
        self.ctx = ctx
        self.lib = ctx.lib
        self.num_experts = num_experts
        self.expert_stride = expert_stride
        self.offsets = offsets_from(offsets)
        self._keep = device_tensor
        h = C.c_void_p()
        if device_tensor is None:
            check(self.lib.tsg_layer_create(ctx.handle, num_experts, expert_stride,
                                            C.byref(self.offsets), C.byref(h)))
        else:
            check(self.lib.tsg_layer_wrap(ctx.handle, _ptr(device_tensor), num_experts,
                                          expert_stride, C.byref(self.offsets), C.byref(h)))
        self.handle = h

    def upload(self, host_bytes: np.ndarray, dst_offset: int = 0, stream=None) -> None:
        a = np.ascontiguousarray(host_bytes).view(np.uint8)
        check(self.lib.tsg_layer_upload(self.handle, _stream(stream), _np_ptr(a), a.nbytes,
                                        dst_offset))
        self.ctx.synchronize(stream)

    @classmethod
    def _adopt(cls, ctx: Context, handle, num_experts: int, expert_stride: int, offsets):
        """Takes ownership of a tsg_layer made by the library (MoEPack.load_layer)."""
        self = cls.__new__(cls)
        self.ctx = ctx
        self.lib = ctx.lib
        self.num_experts = num_experts
        self.expert_stride = expert_stride
        self.offsets = offsets_from(offsets)
        self._keep = None
        self.handle = handle
        return self

    @property
    def device_ptr(self) -> int:
        return int(self.lib.tsg_layer_device_ptr(self.handle))

    def device_geometry(self):
        """(stride, offsets) of the HBM image: the file's, unless the layer was
        laid out anew for 2-byte aligned sub-tensors."""
        stride, offs = C.c_uint64(), ExpertOffsets()
        check(self.lib.tsg_layer_get_geometry(self.handle, C.byref(stride), C.byref(offs)))
        return int(stride.value), [getattr(offs, n) for n, _ in ExpertOffsets._fields_]

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.tsg_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SharedExpertInt4:
    """SharedExpertInt4 (Kernels/MoE/SharedExpertInt4.swift:20-93): Gemma's
    dense int4 MLP y = down(gelu(gate x) * up x), and gelu_mul_fp16
    (utility.metal:7-18). Projections are (weights, scales, biases, rows,
    cols) with torch CUDA tensors."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    @staticmethod
    def projection(weights, scales, biases, rows: int, cols: int) -> "_abi.Int4Projection":
        return _abi.Int4Projection(_ptr(weights), _ptr(scales),
                                   _ptr(biases if biases is not None else scales), rows, cols)

    def encode_gelu_mul(self, gate, up, out, count: int, stream=None) -> None:
        check(self.lib.tsg_gelu_mul_f16(self.ctx.handle, _stream(stream), _ptr(gate), _ptr(up),
                                        _ptr(out), count))

    def encode(self, x, gate, up, down, y, scratch_gate, scratch_up, scratch_act,
               stream=None) -> None:
        nbytes = lambda t: t.numel() * t.element_size()
        check(self.lib.tsg_shared_expert_int4(
            self.ctx.handle, _stream(stream), _ptr(x), nbytes(x), C.byref(gate), C.byref(up),
            C.byref(down), _ptr(y), nbytes(y), _ptr(scratch_gate), nbytes(scratch_gate),
            _ptr(scratch_up), nbytes(scratch_up), _ptr(scratch_act), nbytes(scratch_act)))


class MoEPack:
    """An installed MoEPack's manifest.json + packed_experts/layout.json,
    validated as ManifestReader.load (ManifestReader.swift:169-313) and
    PackedExpertsLayoutReader.load (PackedExpertsLayout.swift:60-115) do.

    `load_layer` replaces the reference's per-expert SSD streamer
    (ModelExpertIO.swift:112-324): the whole layer file goes to HBM, each
    expert blob at its logical index. Errors raise TsgError with status
    TSG_ERR_FORMAT (7) or TSG_ERR_IO (8); the message starts with the
    reference's ModelError case name."""

    def __init__(self, handle, lib):
        self.handle = handle
        self.lib = lib
        info = _abi.MoEPackInfo()
        check(lib.tsg_moepack_get_info(handle, C.byref(info)))
        self.info = {name: (getattr(info, name).decode() if name == "family"
                            else int(getattr(info, name)))
                     for name, _ in _abi.MoEPackInfo._fields_}

    @classmethod
    def open(cls, directory, manifest_max_bytes: int = 0, layout_max_bytes: int = 0):
        lib = load()
        h = C.c_void_p()
        check(lib.tsg_moepack_open(str(directory).encode(), manifest_max_bytes,
                                   layout_max_bytes, C.byref(h)))
        return cls(h, lib)

    @classmethod
    def parse(cls, manifest: bytes, layout: bytes | None = None):
        lib = load()
        h = C.c_void_p()
        check(lib.tsg_moepack_parse(manifest, len(manifest), layout,
                                    0 if layout is None else len(layout), C.byref(h)))
        return cls(h, lib)

    @property
    def num_layers(self) -> int:
        return self.info["num_layers"]

    @property
    def experts_per_layer(self) -> int:
        return self.info["experts_per_layer"]

    @property
    def expert_stride(self) -> int:
        return self.info["expert_stride"]

    def routed_offsets(self, layer: int) -> ExpertOffsets:
        """Model.routedExpertOffsets(layer:) (ModelExpertIO.swift:56-84)."""
        o = ExpertOffsets()
        check(self.lib.tsg_moepack_routed_offsets(self.handle, layer, C.byref(o)))
        return o

    def physical_offsets(self, layer: int) -> np.ndarray:
        """Model.routedExpertPhysicalOffsets(layer:) (ModelExpertIO.swift:86-88)."""
        out = np.zeros(self.experts_per_layer, np.uint64)
        check(self.lib.tsg_moepack_physical_offsets(self.handle, layer, _np_ptr(out),
                                                    out.size))
        return out

    def tensor(self, layer: int, expert: int, name: str) -> dict:
        """expert(layer:expert:).subTensors[name] (PackedExpertsLayout.swift:51-54)."""
        t = _abi.MoEPackSubTensor()
        check(self.lib.tsg_moepack_tensor(self.handle, layer, expert, name.encode(),
                                          C.byref(t)))
        return {"offset": t.offset, "size": t.size, "dtype": ("U32", "BF16")[t.dtype],
                "bits": t.bits or None, "shape": list(t.shape[:min(t.rank, 8)]),
                "physical_rank": t.physical_rank}

    def configure(self, ctx: "Context") -> None:
        """Sets the context's affine group size and scheme from manifest.quant."""
        if self.info["has_quant"]:
            ctx.set_affine_group_size(self.info["affine_group_size"])
            ctx.set_affine_scheme("sym" if self.info["symmetric"] else "affine")

    def load_layer(self, ctx: "Context", layer: int, stream=None) -> ResidentLayer:
        h = C.c_void_p()
        check(self.lib.tsg_moepack_load_layer(self.handle, ctx.handle, _stream(stream), layer,
                                              C.byref(h)))
        return ResidentLayer._adopt(ctx, h, self.experts_per_layer, self.expert_stride,
                                    self.routed_offsets(layer))

    def upload_layer(self, dst: ResidentLayer, layer: int, stream=None) -> None:
        """Uploads layer `layer` into an existing ResidentLayer of the same
        geometry (e.g. one wrapping caller-owned HBM)."""
        check(self.lib.tsg_moepack_upload_layer(self.handle, _stream(stream), layer,
                                                dst.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.tsg_moepack_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------ decode

class MoE:
    """MoE (MoE.swift:42-662): router + top-8, phase 1 gate/up + activation,
    phase 2 down + weighted combine. `router_weight_bits` 16 (bf16 router, the
    QAT checkpoints') is this façade's default; the reference's MoE.init
    defaults to 8 (INT8-affine router, encode_router_gemma4)."""

    def __init__(self, ctx: Context, router_weight_bits: int = 16,
                 gate_activation: str = "gelu"):
        self.ctx = ctx
        self.lib = ctx.lib
        h = C.c_void_p()
        act = TSG_ACT_SILU if gate_activation == "silu" else TSG_ACT_GELU_TANH
        check(self.lib.tsg_moe_create(ctx.handle, router_weight_bits, act, C.byref(h)))
        self.handle = h

    def set_fused_decode(self, enabled: bool) -> None:
        """One-launch decode layer when it fits (default) or the three-launch
        sequence; both give identical bits."""
        check(self.lib.tsg_moe_set_fused_decode(self.handle, int(enabled)))

    def encode_router_gemma4(self, weights, scales, biases, hidden, effective_scale,
                             per_expert_scale, out_indices, out_weights, num_experts, d,
                             top_k=8, stream=None):
        """encodeRouterGemma4 (MoE.swift:201-257): the INT8-affine router
        (router_weight_bits=8)."""
        check(self.lib.tsg_moe_router_int8(
            self.handle, _stream(stream), _ptr(weights), _ptr(scales), _ptr(biases),
            _ptr(hidden), _ptr(effective_scale), _ptr(per_expert_scale), _ptr(out_indices),
            _ptr(out_weights), num_experts, d, top_k))

    def encode_router_gemma4_bf16(self, weights, hidden, effective_scale, per_expert_scale,
                                  out_indices, out_weights, num_experts, d, top_k=8,
                                  stream=None):
        check(self.lib.tsg_moe_router_bf16(
            self.handle, _stream(stream), _ptr(weights), _ptr(hidden), _ptr(effective_scale),
            _ptr(per_expert_scale), _ptr(out_indices), _ptr(out_weights), num_experts, d,
            top_k))

    def encode_router_gemma4_bf16_rows(self, weights, hidden, hidden_stride_elements,
                                       effective_scale, per_expert_scale, out_indices,
                                       out_weights, row_count, num_experts, d, top_k=8,
                                       stream=None):
        check(self.lib.tsg_moe_router_bf16_rows(
            self.handle, _stream(stream), _ptr(weights), _ptr(hidden), hidden_stride_elements,
            _ptr(effective_scale), _ptr(per_expert_scale), _ptr(out_indices),
            _ptr(out_weights), row_count, num_experts, d, top_k))

    def encode_router_gemma4_bf16_rows_grouped(self, weights, hidden, hidden_stride_elements,
                                               effective_scale, per_expert_scale, out_indices,
                                               out_weights, row_count, num_experts, d,
                                               sorted_pairs, offsets, counts, blocks, max_blocks,
                                               n_blocks, top_k=8, stream=None):
        """encode_router_gemma4_bf16_rows + the device grouping of its pairs
        in one launch (the outputs of both, bit for bit)."""
        check(self.lib.tsg_moe_router_bf16_rows_grouped(
            self.handle, _stream(stream), _ptr(weights), _ptr(hidden), hidden_stride_elements,
            _ptr(effective_scale), _ptr(per_expert_scale), _ptr(out_indices), _ptr(out_weights),
            row_count, num_experts, d, top_k, _ptr(sorted_pairs), _ptr(offsets), _ptr(counts),
            _ptr(blocks), max_blocks, _ptr(n_blocks)))

    def encode_router_logits_bf16(self, weights, hidden, effective_scale, out_logits,
                                  num_experts, d, stream=None):
        check(self.lib.tsg_moe_router_logits_bf16(
            self.handle, _stream(stream), _ptr(weights), _ptr(hidden), _ptr(effective_scale),
            _ptr(out_logits), num_experts, d))

    @staticmethod
    def _blobs(blobs):
        arr = (C.c_void_p * len(blobs))()
        for i, b in enumerate(blobs):
            arr[i] = _ptr(b)
        return arr

    def encode_routed_phase1(self, routed_blobs, routed_offsets, x, acts, d, f, top_k=8,
                             stream=None):
        check(self.lib.tsg_moe_phase1(self.handle, _stream(stream), self._blobs(routed_blobs),
                                      C.byref(offsets_from(routed_offsets)), _ptr(x),
                                      _ptr(acts), d, f, top_k))

    def encode_routed_phase1_subset(self, routed_blobs, routed_offsets, x, acts,
                                    active_slots, active_count, d, f, top_k=8, stream=None):
        check(self.lib.tsg_moe_phase1_subset(
            self.handle, _stream(stream), self._blobs(routed_blobs),
            C.byref(offsets_from(routed_offsets)), _ptr(x), _ptr(acts), _ptr(active_slots),
            active_count, d, f, top_k))

    def encode_routed_phase2(self, routed_blobs, routed_offsets, acts, routing_weights,
                             residual, y, d, f, top_k=8, stream=None):
        check(self.lib.tsg_moe_phase2(self.handle, _stream(stream), self._blobs(routed_blobs),
                                      C.byref(offsets_from(routed_offsets)), _ptr(acts),
                                      _ptr(routing_weights), _ptr(residual), _ptr(y), d, f,
                                      top_k))

    def encode_phase1_resident(self, layer: ResidentLayer, indices, x, acts, d, f, top_k=8,
                               stream=None):
        check(self.lib.tsg_moe_phase1_resident(self.handle, _stream(stream), layer.handle,
                                               _ptr(indices), _ptr(x), _ptr(acts), d, f, top_k))

    def encode_phase2_resident(self, layer: ResidentLayer, indices, acts, routing_weights,
                               residual, y, d, f, top_k=8, stream=None):
        check(self.lib.tsg_moe_phase2_resident(self.handle, _stream(stream), layer.handle,
                                               _ptr(indices), _ptr(acts), _ptr(routing_weights),
                                               _ptr(residual), _ptr(y), d, f, top_k))

    def encode_decode_layer(self, layer: ResidentLayer, router_weights, router_hidden,
                            effective_scale, per_expert_scale, x, residual, y, out_indices,
                            out_weights, acts_scratch, num_experts, d, f, top_k=8,
                            stream=None):
        check(self.lib.tsg_moe_decode_layer(
            self.handle, _stream(stream), layer.handle, _ptr(router_weights),
            _ptr(router_hidden), _ptr(effective_scale), _ptr(per_expert_scale), _ptr(x),
            _ptr(residual), _ptr(y), _ptr(out_indices), _ptr(out_weights), _ptr(acts_scratch),
            num_experts, d, f, top_k))

    def encode_verify_layer(self, layer: ResidentLayer, router_weights, router_hidden,
                            effective_scale, per_expert_scale, x, hidden_stride, h2,
                            out_indices, out_weights, row_count, num_experts, d, f, top_k=8,
                            stream=None):
        """One verify layer of row_count <= 8 tokens in one launch: the rows
        router's top-8, the grouping, the rows path over the routed experts and
        the token-major sum (encodeRouterGemma4BF16Rows + grouping +
        encodeStreamedRows + encodeReduceTokenMajor), the same bits. Raises
        TsgError(TSG_ERR_DECLINED) when the one launch does not fit."""
        check(self.lib.tsg_moe_verify_layer(
            self.handle, _stream(stream), layer.handle, _ptr(router_weights),
            _ptr(router_hidden), _ptr(effective_scale), _ptr(per_expert_scale), _ptr(x),
            hidden_stride, _ptr(h2), _ptr(out_indices), _ptr(out_weights), row_count,
            num_experts, d, f, top_k))

    def encode_verify_layer_shared(self, layer: ResidentLayer, router_weights, router_hidden,
                                   effective_scale, per_expert_scale, x, hidden_stride, h2,
                                   out_indices, out_weights, shared_blob, shared_offsets,
                                   shared_gate_weight, shared_out, row_count, num_experts, d, f,
                                   top_k=8, stream=None):
        """encode_verify_layer with the Qwen family's shared expert over the
        same rows in the same launch (its intermediate size f): shared_out
        [row_count, d] gets encode_shared_expert_rows' bits. Raises
        TsgError(TSG_ERR_DECLINED) when the one launch does not fit."""
        o = offsets_from(shared_offsets)
        check(self.lib.tsg_moe_verify_layer_shared(
            self.handle, _stream(stream), layer.handle, _ptr(router_weights),
            _ptr(router_hidden), _ptr(effective_scale), _ptr(per_expert_scale), _ptr(x),
            hidden_stride, _ptr(h2), _ptr(out_indices), _ptr(out_weights), _ptr(shared_blob),
            C.byref(o), _ptr(shared_gate_weight), _ptr(shared_out), row_count, num_experts, d,
            f, top_k))

    def encode_decode_layer_int8(self, layer: ResidentLayer, router_weights, router_scales,
                                 router_biases, router_hidden, effective_scale,
                                 per_expert_scale, x, residual, y, out_indices, out_weights,
                                 acts_scratch, num_experts, d, f, top_k=8, stream=None):
        """The decode layer with the INT8-affine router (router_weight_bits=8)."""
        check(self.lib.tsg_moe_decode_layer_int8(
            self.handle, _stream(stream), layer.handle, _ptr(router_weights),
            _ptr(router_scales), _ptr(router_biases), _ptr(router_hidden),
            _ptr(effective_scale), _ptr(per_expert_scale), _ptr(x), _ptr(residual), _ptr(y),
            _ptr(out_indices), _ptr(out_weights), _ptr(acts_scratch), num_experts, d, f,
            top_k))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.tsg_moe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode_decode_layer_shared(self, layer: ResidentLayer, router_weights, router_hidden,
                                   effective_scale, per_expert_scale, x, y, out_indices,
                                   out_weights, acts_scratch, shared_blob, shared_offsets,
                                   shared_gate_weight, shared_acts, num_experts, d, f, shared_f,
                                   top_k=8, stream=None):
        """The Qwen-family layer: shared branch + routed experts with
        residual = sharedOut (QwenForwardRunner.swift:1548-1608) in one call."""
        o = offsets_from(shared_offsets)
        check(self.lib.tsg_moe_decode_layer_shared(
            self.handle, _stream(stream), layer.handle, _ptr(router_weights),
            _ptr(router_hidden), _ptr(effective_scale), _ptr(per_expert_scale), _ptr(x), _ptr(y),
            _ptr(out_indices), _ptr(out_weights), _ptr(acts_scratch), _ptr(shared_blob),
            C.byref(o), _ptr(shared_gate_weight), _ptr(shared_acts), num_experts, d, f,
            shared_f, top_k))

class QwenKernels:
    """The Qwen-family shared-expert steps of QwenKernels (QwenKernels.swift)
    and QwenForwardRunner.encodeSharedExpert (QwenForwardRunner.swift:1548-1578)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode_silu_mul(self, gate, up, out, count, stream=None):
        check(self.lib.tsg_qwen_silu_mul(self.ctx.handle, _stream(stream), _ptr(gate), _ptr(up),
                                         _ptr(out), count))

    def encode_moe_shared_gate(self, y, x, weight, hidden_size, stream=None):
        check(self.lib.tsg_qwen_moe_shared_gate(self.ctx.handle, _stream(stream), _ptr(y),
                                                _ptr(x), _ptr(weight), hidden_size))

    def encode_moe_shared_gate_logit(self, y, logit, hidden_size, stream=None):
        check(self.lib.tsg_qwen_moe_shared_gate_logit(self.ctx.handle, _stream(stream), _ptr(y),
                                                      _ptr(logit), hidden_size))


def encode_shared_expert(moe: "MoE", blob, offsets, x, gate_weight, act_scratch, out, d, f,
                         stream=None):
    """The shared branch of QwenForwardRunner.encodeSharedExpert in two launches."""
    o = offsets_from(offsets)
    check(moe.lib.tsg_moe_shared_expert(moe.handle, _stream(stream), _ptr(blob), C.byref(o),
                                        _ptr(x), _ptr(gate_weight), _ptr(act_scratch), _ptr(out),
                                        d, f))


def encode_shared_expert_rows(moe: "MoE", blob, offsets, x, x_stride, gate_weight, act_scratch,
                              out, rows, d, f, stream=None):
    """encode_shared_expert for rows <= 8 token rows (x + r * x_stride), each
    weight read once; row r gives encode_shared_expert's bits on x_r."""
    o = offsets_from(offsets)
    check(moe.lib.tsg_moe_shared_expert_rows(moe.handle, _stream(stream), _ptr(blob),
                                             C.byref(o), _ptr(x), x_stride, _ptr(gate_weight),
                                             _ptr(act_scratch), _ptr(out), rows, d, f))


class DequantInt4GEMV:
    """DequantInt4GEMV (DequantInt4GEMV.swift:6-364)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode(self, weights, scales, biases, x, y, m, n, stream=None):
        check(self.lib.tsg_qmv_int4(self.ctx.handle, _stream(stream), _ptr(weights),
                                    _ptr(scales), _ptr(biases), _ptr(x), _ptr(y), m, n))

    def encode_rows(self, weights, scales, biases, x, x_stride, y, y_stride, t, m, n,
                    stream=None):
        check(self.lib.tsg_qmv_int4_rows(self.ctx.handle, _stream(stream), _ptr(weights),
                                         _ptr(scales), _ptr(biases), _ptr(x), x_stride, _ptr(y),
                                         y_stride, t, m, n))

    # encodeRowsWide (DequantInt4GEMV.swift:220-267) gives encodeRows' bits by
    # definition; the same entry point serves both.
    encode_rows_wide = encode_rows

    def debug_dequant_f16(self, weights, scales, biases, out, rows, n, gemm_path=False,
                          stream=None):
        fn = self.lib.tsg_debug_gemm_dequant_f16 if gemm_path else self.lib.tsg_debug_dequant_f16
        check(fn(self.ctx.handle, _stream(stream), _ptr(weights), _ptr(scales), _ptr(biases),
                 _ptr(out), rows, n))


# ----------------------------------------------------------------- prefill

class PrefillRouter:
    """PrefillRouter (PrefillRouter.swift:69-258)."""

    def __init__(self, moe: MoE):
        self.moe = moe
        self.lib = moe.lib

    def encode_gemma4_bf16(self, weights, hidden, hidden_stride_elements, effective_scale,
                           per_expert_scale, out_indices, out_weights, query_count,
                           num_experts, d, top_k=8, stream=None):
        check(self.lib.tsg_prefill_router_bf16(
            self.moe.handle, _stream(stream), _ptr(weights), _ptr(hidden),
            hidden_stride_elements, _ptr(effective_scale), _ptr(per_expert_scale),
            _ptr(out_indices), _ptr(out_weights), query_count, num_experts, d, top_k))

    @staticmethod
    def make_token_expert_pairs(indices, weights_bits, query_count, top_k) -> np.ndarray:
        idx = np.ascontiguousarray(indices, np.uint32).ravel()
        w = np.ascontiguousarray(weights_bits, np.uint16).ravel()
        out = np.empty(query_count * top_k, PAIR_DTYPE)
        check(load().tsg_make_token_expert_pairs(_np_ptr(idx), _np_ptr(w), query_count, top_k,
                                                 _np_ptr(out)))
        return out


class PrefillMoEGrouping:
    """PrefillMoEGrouping.groupTokenExpertPairs (PrefillMoEGrouping.swift:90-202),
    host side, with the reference's error cases (TsgError.case)."""

    @staticmethod
    def group_token_expert_pairs(pairs, query_count, top_k, num_experts,
                                 tile_expert_count=16, expert_sort_keys=None,
                                 tile_break_after_group=None):
        lib = load()
        pairs = np.ascontiguousarray(pairs, PAIR_DTYPE)
        n = pairs.size
        sorted_pairs = np.empty(max(n, 1), PAIR_DTYPE)
        offsets = np.empty(max(num_experts, 1), np.uint32)
        counts = np.empty(max(num_experts, 1), np.uint32)
        groups = np.empty(max(n, 1), GROUP_DTYPE)
        tiles = np.empty(max(n, 1), TILE_DTYPE)
        ng, nt = C.c_uint32(0), C.c_uint32(0)
        keys, nkeys = None, 0
        if expert_sort_keys is not None:
            keys = np.ascontiguousarray(expert_sort_keys, np.uint64)
            nkeys = keys.size
        check(lib.tsg_group_token_expert_pairs(
            _np_ptr(pairs), n, query_count & 0xFFFFFFFF, top_k & 0xFFFFFFFF,
            num_experts & 0xFFFFFFFF, tile_expert_count,
            _np_ptr(keys) if keys is not None else None, nkeys,
            -1 if tile_break_after_group is None else tile_break_after_group,
            _np_ptr(sorted_pairs), _np_ptr(offsets), _np_ptr(counts), _np_ptr(groups),
            C.byref(ng), _np_ptr(tiles), C.byref(nt)))
        return dict(sorted_pairs=sorted_pairs[:n], offsets=offsets[:num_experts],
                    counts=counts[:num_experts], groups=groups[:ng.value],
                    tiles=tiles[:nt.value])


class PrefillRoutedGEMMPlanner:
    """PrefillRoutedGEMMPlanner.plan (PrefillGroupedRoutedMoE.swift:42-83)."""
    tile_rows = 64

    @staticmethod
    def plan(groups, max_rows_per_batch):
        lib = load()
        groups = np.ascontiguousarray(groups, GROUP_DTYPE)
        total = int(groups["pair_count"].sum()) if groups.size else 0
        cap = total + groups.size + 1
        blocks = np.empty(cap, BLOCK_DTYPE)
        rows = np.empty(cap, np.uint32)
        first = np.empty(cap, np.uint32)
        nb, nbatch = C.c_uint32(0), C.c_uint32(0)
        check(lib.tsg_plan_routed_gemm(_np_ptr(groups) if groups.size else None, groups.size,
                                       max_rows_per_batch, _np_ptr(blocks), C.byref(nb),
                                       _np_ptr(rows), _np_ptr(first), C.byref(nbatch)))
        out = []
        for i in range(nbatch.value):
            end = first[i + 1] if i + 1 < nbatch.value else nb.value
            out.append((int(rows[i]), blocks[first[i]:end].copy()))
        return out


class PrefillGroupedRoutedMoE:
    """PrefillGroupedRoutedMoE (PrefillGroupedRoutedMoE.swift:174-1051) on an
    HBM-resident layer: device grouping, tiled gate/up + down GEMMs, rows path."""

    def __init__(self, moe: MoE):
        self.moe = moe
        self.ctx = moe.ctx
        self.lib = moe.lib

    def scratch_bytes(self, query_count, top_k, num_experts) -> int:
        return int(self.lib.tsg_prefill_group_scratch_bytes(query_count, top_k, num_experts))

    def group_pairs_device(self, indices, weights, query_count, top_k, num_experts, sorted_pairs,
                           offsets, counts, blocks, max_blocks, n_blocks, scratch, tile_rows=64,
                           stream=None):
        check(self.lib.tsg_prefill_group_pairs_device(
            self.ctx.handle, _stream(stream), _ptr(indices), _ptr(weights), query_count, top_k,
            num_experts, tile_rows, _ptr(sorted_pairs), _ptr(offsets), _ptr(counts),
            _ptr(blocks), max_blocks, _ptr(n_blocks), _ptr(scratch)))

    def group_pairs_device_noalloc(self, indices, weights, query_count, top_k, num_experts,
                                   sorted_pairs, offsets, counts, blocks, max_blocks, n_blocks,
                                   tile_rows=64, stream=None):
        """group_pairs_device with the library's file-scope rank scratch (no
        workspace, no allocation; at most 65536 pairs; calls on one GPU must
        not overlap)."""
        check(self.lib.tsg_prefill_group_pairs_device_noalloc(
            self.ctx.handle, _stream(stream), _ptr(indices), _ptr(weights), query_count, top_k,
            num_experts, tile_rows, _ptr(sorted_pairs), _ptr(offsets), _ptr(counts),
            _ptr(blocks), max_blocks, _ptr(n_blocks)))

    def encode_gate_up(self, layer, hidden, hidden_stride, sorted_pairs, blocks, n_blocks, act,
                       d, f, n_blocks_device=None, stream=None):
        check(self.lib.tsg_prefill_moe_gate_up(
            self.moe.handle, _stream(stream), layer.handle, _ptr(hidden), hidden_stride,
            _ptr(sorted_pairs), _ptr(blocks), n_blocks, _ptr(n_blocks_device), _ptr(act), d, f))

    def encode_down(self, layer, act, sorted_pairs, blocks, n_blocks, route_partials, top_k, d,
                    f, n_blocks_device=None, stream=None):
        check(self.lib.tsg_prefill_moe_down(
            self.moe.handle, _stream(stream), layer.handle, _ptr(act), _ptr(sorted_pairs),
            _ptr(blocks), n_blocks, _ptr(n_blocks_device), _ptr(route_partials), top_k, d, f))

    def encode_gate_up_down(self, layer, hidden, hidden_stride, sorted_pairs, blocks, n_blocks,
                            act, route_partials, top_k, d, f, n_blocks_device=None,
                            stream=None):
        """encode_gate_up then encode_down in one persistent launch (same
        results; act 128-byte aligned)."""
        check(self.lib.tsg_prefill_moe_gate_up_down(
            self.moe.handle, _stream(stream), layer.handle, _ptr(hidden), hidden_stride,
            _ptr(sorted_pairs), _ptr(blocks), n_blocks, _ptr(n_blocks_device), _ptr(act),
            _ptr(route_partials), top_k, d, f))

    def encode_streamed_rows_device(self, layer, hidden, hidden_stride, sorted_pairs, blocks,
                                    max_blocks, n_blocks_device, act_scratch, route_partials,
                                    top_k, d, f, stream=None, max_rows=None):
        """encode_streamed_rows with the block list (and its count) on the
        device, as group_pairs_device writes them."""
        check(self.lib.tsg_prefill_moe_rows_device(
            self.moe.handle, _stream(stream), layer.handle, _ptr(hidden), hidden_stride,
            _ptr(sorted_pairs), _ptr(blocks), max_blocks, _ptr(n_blocks_device),
            _ptr(act_scratch), _scratch_rows(act_scratch, f, max_rows), _ptr(route_partials),
            top_k, d, f))

    def encode_streamed_rows(self, layer, hidden, hidden_stride, sorted_pairs, host_blocks,
                             act_scratch, route_partials, top_k, d, f, stream=None,
                             max_rows=None):
        """encodeStreamedRows (PrefillGroupedRoutedMoE.swift:793-917). max_rows
        is the activation scratch's capacity in rows of f (the reference's
        maxRows); by default, what act_scratch holds. A tile it cannot take
        raises TsugumiError with TSG_ERR_DECLINED (the reference returns 0)."""
        hb = np.ascontiguousarray(host_blocks, BLOCK_DTYPE)
        check(self.lib.tsg_prefill_moe_rows(
            self.moe.handle, _stream(stream), layer.handle, _ptr(hidden), hidden_stride,
            _ptr(sorted_pairs), _np_ptr(hb) if hb.size else None, hb.size, _ptr(act_scratch),
            _scratch_rows(act_scratch, f, max_rows), _ptr(route_partials), top_k, d, f))


class PrefillMoE:
    """PrefillMoE.encodeReduceTokenMajor (PrefillMoE.swift:11-38)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode_reduce_token_major(self, route_partials, route_weights, h2, query_count, top_k,
                                  d, stream=None):
        check(self.lib.tsg_prefill_moe_reduce_token_major(
            self.ctx.handle, _stream(stream), _ptr(route_partials), _ptr(route_weights),
            _ptr(h2), query_count, top_k, d))

    def encode_reduce_layer_tail(self, route_partials, route_weights, h1, hidden,
                                 post_ffn2_weight, post_ffn_weight, query_count, top_k, d,
                                 h1_stride, hidden_stride, eps, layer_scalar, h2=None,
                                 stream=None):
        """encodeReduceTokenMajor then PrefillLayerTail.encode in one launch;
        h2 is written only when given."""
        check(self.lib.tsg_prefill_moe_reduce_layer_tail(
            self.ctx.handle, _stream(stream), _ptr(route_partials), _ptr(route_weights),
            _ptr(h2) if h2 is not None else None, _ptr(h1), _ptr(hidden),
            _ptr(post_ffn2_weight), _ptr(post_ffn_weight), query_count, top_k, d, h1_stride,
            hidden_stride, eps, layer_scalar))


class PrefillInt4QMM:
    """PrefillInt4QMM.encode (PrefillPrimitives.swift:75-175): the dense int4
    projection y[t, n] over t tokens on the dequant-to-LDS MFMA GEMM."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode(self, weights, scales, biases, x, y, t, n, k, stream=None):
        check(self.lib.tsg_prefill_int4_qmm(
            self.ctx.handle, _stream(stream), _ptr(weights), _ptr(scales), _ptr(biases),
            _ptr(x), _ptr(y), t, n, k))


class PrefillLayerTail:
    """PrefillLayerTail.encode (PrefillLayerTail.swift:11-58): post-FFN RMSNorms,
    residual adds and the layer scalar over query_count strided rows."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode(self, h2, h1, hidden, post_ffn2_weight, post_ffn_weight, query_count, d,
               h2_stride, h1_stride, hidden_stride, eps, layer_scalar, stream=None):
        check(self.lib.tsg_prefill_layer_tail(
            self.ctx.handle, _stream(stream), _ptr(h2), _ptr(h1), _ptr(hidden),
            _ptr(post_ffn2_weight), _ptr(post_ffn_weight), query_count, d, h2_stride, h1_stride,
            hidden_stride, eps, layer_scalar))


class FusedLayerTail:
    """FusedLayerTail.encode (FusedLayerTail.swift:25-56): the decode form, one row."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def encode(self, h2, h1, hidden, post_ffn2_weight, post_ffn_weight, d, eps, layer_scalar,
               stream=None):
        check(self.lib.tsg_fused_layer_tail(
            self.ctx.handle, _stream(stream), _ptr(h2), _ptr(h1), _ptr(hidden),
            _ptr(post_ffn2_weight), _ptr(post_ffn_weight), d, eps, layer_scalar))


class generators:
    """Device-side synthetic fixtures (counter-based SplitMix64)."""

    @staticmethod
    def bytes(out, seed, stream=None):
        check(load().tsg_gen_bytes(_stream(stream), seed, _ptr(out), out.numel() * out.element_size()))

    @staticmethod
    def bf16_normal(out, seed, sigma, abs_value=False, divisor=1.0, stream=None):
        check(load().tsg_gen_bf16_normal(_stream(stream), seed, _ptr(out), out.numel(), sigma,
                                         int(abs_value), divisor))

    @staticmethod
    def f16_normal(out, seed, sigma=1.0, stream=None):
        check(load().tsg_gen_f16_normal(_stream(stream), seed, _ptr(out), out.numel(), sigma))
