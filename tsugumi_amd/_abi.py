"""ctypes declarations of the C ABI in include/tsugumi_hip.h.

Loading fails loudly when libtsugumi_hip.so is missing: there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtsugumi_hip.so")

# tsg_status values (include/tsugumi_hip.h)
TSG_OK = 0
TSG_ERR_INVALID_ARGUMENT = 1
TSG_ERR_ALIGNMENT = 2
TSG_ERR_UNSUPPORTED = 3
TSG_ERR_DECLINED = 4
TSG_ERR_HIP = 5
TSG_ERR_OUT_OF_MEMORY = 6
TSG_ERR_FORMAT = 7
TSG_ERR_IO = 8
GROUPING_ERRORS = {
    100: "invalidQueryCount", 101: "invalidTopK", 102: "invalidNumExperts",
    103: "invalidTileExpertCount", 104: "pairCountMismatch", 105: "tokenOutOfRange",
    106: "rankOutOfRange", 107: "expertOutOfRange", 108: "duplicateTokenRank",
    109: "expertSortKeyCountMismatch",
}

TSG_AFFINE, TSG_SYM = 0, 1
TSG_ACT_GELU_TANH, TSG_ACT_SILU = 0, 1


class ExpertOffsets(C.Structure):
    """MoEExpertOffsets (MoE.swift:4-29), 36 bytes."""
    _fields_ = [(n, C.c_uint32) for n in (
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")]


class TokenExpertPair(C.Structure):
    """PrefillTokenExpertPair (PrefillRouter.swift:4-28), 16 bytes."""
    _fields_ = [("token", C.c_uint32), ("expert", C.c_uint32), ("rank", C.c_uint32),
                ("weight_bits", C.c_uint32)]


class MoEGroup(C.Structure):
    _fields_ = [("expert", C.c_uint32), ("pair_start", C.c_uint32), ("pair_count", C.c_uint32)]


class MoETile(C.Structure):
    _fields_ = [("group_start", C.c_uint32), ("group_count", C.c_uint32),
                ("pair_start", C.c_uint32), ("pair_count", C.c_uint32)]


class RoutedBlock(C.Structure):
    """PrefillRoutedGEMMBlock (PrefillGroupedRoutedMoE.swift:20-25), 16 bytes."""
    _fields_ = [("local_slot", C.c_uint32), ("pair_start", C.c_uint32),
                ("row_count", C.c_uint32), ("local_row", C.c_uint32)]


class MoEPackInfo(C.Structure):
    """tsg_moepack_info: what a validated manifest says about the routed experts."""
    _fields_ = [("num_layers", C.c_uint32), ("experts_per_layer", C.c_uint32),
                ("expert_stride", C.c_uint64), ("hidden_size", C.c_uint32),
                ("moe_intermediate_size", C.c_uint32), ("top_k", C.c_uint32),
                ("version_minor", C.c_uint32), ("legacy_magic", C.c_uint32),
                ("has_quant", C.c_uint32), ("affine_group_size", C.c_uint32),
                ("symmetric", C.c_uint32), ("routed_weight_bits", C.c_uint32),
                ("shared_weight_bits", C.c_uint32), ("router_weight_bits", C.c_uint32),
                ("has_layout", C.c_uint32), ("is_gemma4", C.c_uint32),
                ("family", C.c_char * 32)]


class MoEPackSubTensor(C.Structure):
    """SubTensorEntry (PackedExpertsLayout.swift:4-10) plus the expert's physical rank."""
    _fields_ = [("offset", C.c_uint64), ("size", C.c_uint64), ("dtype", C.c_uint32),
                ("bits", C.c_uint32), ("rank", C.c_uint32), ("shape", C.c_uint32 * 8),
                ("physical_rank", C.c_uint32)]


class Int4Projection(C.Structure):
    """SharedExpertProjection (SharedExpertInt8.swift:9-33): device pointers
    and the [rows, cols] shape of one int4 matrix."""
    _fields_ = [("weights", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("rows", C.c_uint32), ("cols", C.c_uint32)]


P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64

# name -> (restype, argtypes)
SIGNATURES = {
    "tsg_last_error": (C.c_char_p, []),
    "tsg_status_string": (C.c_char_p, [C.c_int]),
    "tsg_version": (C.c_char_p, []),
    "tsg_ctx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "tsg_ctx_destroy": (None, [P]),
    "tsg_ctx_set_affine_group_size": (C.c_int, [P, U32]),
    "tsg_ctx_set_affine_scheme": (C.c_int, [P, C.c_int]),
    "tsg_ctx_synchronize": (C.c_int, [P, P]),
    "tsg_layer_create": (C.c_int, [P, U32, U64, C.POINTER(ExpertOffsets), C.POINTER(P)]),
    "tsg_layer_wrap": (C.c_int, [P, P, U32, U64, C.POINTER(ExpertOffsets), C.POINTER(P)]),
    "tsg_layer_upload": (C.c_int, [P, P, P, U64, U64]),
    "tsg_layer_device_ptr": (P, [P]),
    "tsg_layer_get_geometry": (C.c_int, [P, C.POINTER(U64), C.POINTER(ExpertOffsets)]),
    "tsg_layer_destroy": (None, [P]),
    "tsg_moe_create": (C.c_int, [P, U32, C.c_int, C.POINTER(P)]),
    "tsg_moe_destroy": (None, [P]),
    "tsg_moe_router_bf16": (C.c_int, [P, P, P, P, P, P, P, P, U32, U32, U32]),
    "tsg_moe_router_int8": (C.c_int, [P, P, P, P, P, P, P, P, P, P, U32, U32, U32]),
    "tsg_moe_router_bf16_rows": (C.c_int, [P, P, P, P, U32, P, P, P, P, U32, U32, U32, U32]),
    "tsg_moe_router_bf16_rows_grouped": (C.c_int, [P, P, P, P, U32, P, P, P, P, U32, U32, U32,
                                                   U32, P, P, P, P, U32, P]),
    "tsg_moe_router_logits_bf16": (C.c_int, [P, P, P, P, P, P, U32, U32]),
    "tsg_moe_phase1": (C.c_int, [P, P, P, C.POINTER(ExpertOffsets), P, P, U32, U32, U32]),
    "tsg_moe_phase1_subset": (C.c_int, [P, P, P, C.POINTER(ExpertOffsets), P, P, P, U32,
                                        U32, U32, U32]),
    "tsg_moe_phase2": (C.c_int, [P, P, P, C.POINTER(ExpertOffsets), P, P, P, P, U32, U32,
                                 U32]),
    "tsg_moe_phase1_resident": (C.c_int, [P, P, P, P, P, P, U32, U32, U32]),
    "tsg_moe_phase2_resident": (C.c_int, [P, P, P, P, P, P, P, P, U32, U32, U32]),
    "tsg_moe_decode_layer": (C.c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, U32, U32, U32,
                                       U32]),
    "tsg_moe_verify_layer": (C.c_int, [P, P, P, P, P, P, P, P, U32, P, P, P, U32, U32, U32, U32,
                                       U32]),
    "tsg_moe_verify_layer_shared": (C.c_int, [P, P, P, P, P, P, P, P, U32, P, P, P, P, P, P, P,
                                              U32, U32, U32, U32, U32]),
    "tsg_moe_decode_layer_int8": (C.c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, U32,
                                            U32, U32, U32]),
    "tsg_moe_decode_layer_shared": (C.c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P,
                                              U32, U32, U32, U32, U32]),
    "tsg_moe_set_fused_decode": (C.c_int, [P, C.c_int]),
    "tsg_qmv_int4": (C.c_int, [P, P, P, P, P, P, P, U32, U32]),
    "tsg_qwen_silu_mul": (C.c_int, [P, P, P, P, P, U32]),
    "tsg_gelu_mul_f16": (C.c_int, [P, P, P, P, P, U32]),
    "tsg_shared_expert_int4": (C.c_int, [P, P, P, U64, C.POINTER(Int4Projection),
                                         C.POINTER(Int4Projection), C.POINTER(Int4Projection),
                                         P, U64, P, U64, P, U64, P, U64]),
    "tsg_qwen_moe_shared_gate": (C.c_int, [P, P, P, P, P, U32]),
    "tsg_qwen_moe_shared_gate_logit": (C.c_int, [P, P, P, P, U32]),
    "tsg_moe_shared_expert": (C.c_int, [P, P, P, P, P, P, P, P, U32, U32]),
    "tsg_moe_shared_expert_rows": (C.c_int, [P, P, P, P, P, U32, P, P, P, U32, U32, U32]),
    "tsg_qmv_int4_rows": (C.c_int, [P, P, P, P, P, P, U32, P, U32, U32, U32, U32]),
    "tsg_debug_dequant_f16": (C.c_int, [P, P, P, P, P, P, U32, U32]),
    "tsg_debug_gemm_dequant_f16": (C.c_int, [P, P, P, P, P, P, U32, U32]),
    "tsg_prefill_router_bf16": (C.c_int, [P, P, P, P, U32, P, P, P, P, U32, U32, U32, U32]),
    "tsg_make_token_expert_pairs": (C.c_int, [P, P, U32, U32, P]),
    "tsg_group_token_expert_pairs": (C.c_int, [P, U32, U32, U32, U32, U32, P, U32, C.c_int32,
                                               P, P, P, P, P, P, P]),
    "tsg_plan_routed_gemm": (C.c_int, [P, U32, U32, P, P, P, P, P]),
    "tsg_prefill_group_scratch_bytes": (C.c_size_t, [U32, U32, U32]),
    "tsg_prefill_group_pairs_device": (C.c_int, [P, P, P, P, U32, U32, U32, U32, P, P, P, P,
                                                 U32, P, P]),
    "tsg_prefill_group_pairs_device_noalloc": (C.c_int, [P, P, P, P, U32, U32, U32, U32, P, P,
                                                         P, P, U32, P]),
    "tsg_prefill_moe_gate_up": (C.c_int, [P, P, P, P, U32, P, P, U32, P, P, U32, U32]),
    "tsg_prefill_moe_down": (C.c_int, [P, P, P, P, P, P, U32, P, P, U32, U32, U32]),
    "tsg_prefill_moe_gate_up_down": (C.c_int, [P, P, P, P, U32, P, P, U32, P, P, P, U32, U32,
                                               U32]),
    "tsg_prefill_moe_rows": (C.c_int, [P, P, P, P, U32, P, P, U32, P, U32, P, U32, U32, U32]),
    "tsg_prefill_moe_rows_device": (C.c_int, [P, P, P, P, U32, P, P, U32, P, P, U32, P, U32,
                                              U32, U32]),
    "tsg_prefill_moe_reduce_token_major": (C.c_int, [P, P, P, P, P, U32, U32, U32]),
    "tsg_prefill_int4_qmm": (C.c_int, [P, P, P, P, P, P, P, U32, U32, U32]),
    "tsg_prefill_layer_tail": (C.c_int, [P, P, P, P, P, P, P, U32, U32, U32, U32, U32,
                                         C.c_float, C.c_float]),
    "tsg_fused_layer_tail": (C.c_int, [P, P, P, P, P, P, P, U32, C.c_float, C.c_float]),
    "tsg_prefill_moe_reduce_layer_tail": (C.c_int, [P, P, P, P, P, P, P, P, P, U32, U32, U32,
                                                    U32, U32, C.c_float, C.c_float]),
    "tsg_moepack_open": (C.c_int, [C.c_char_p, U64, U64, C.POINTER(P)]),
    "tsg_moepack_parse": (C.c_int, [C.c_char_p, U64, C.c_char_p, U64, C.POINTER(P)]),
    "tsg_moepack_close": (None, [P]),
    "tsg_moepack_get_info": (C.c_int, [P, C.POINTER(MoEPackInfo)]),
    "tsg_moepack_routed_offsets": (C.c_int, [P, U32, C.POINTER(ExpertOffsets)]),
    "tsg_moepack_physical_offsets": (C.c_int, [P, U32, P, U32]),
    "tsg_moepack_tensor": (C.c_int, [P, U32, U32, C.c_char_p, C.POINTER(MoEPackSubTensor)]),
    "tsg_moepack_load_layer": (C.c_int, [P, P, P, U32, C.POINTER(P)]),
    "tsg_moepack_upload_layer": (C.c_int, [P, P, U32, P]),
    "tsg_gen_bytes": (C.c_int, [P, U64, P, U64]),
    "tsg_gen_bf16_normal": (C.c_int, [P, U64, P, U64, C.c_float, C.c_int, C.c_float]),
    "tsg_gen_f16_normal": (C.c_int, [P, U64, P, U64, C.c_float]),
}

_lib = None


class TsgError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        self.case = GROUPING_ERRORS.get(status)
        super().__init__(f"[{status}] {message}")


def load() -> C.CDLL:
    """Loads the in-tree library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m tsugumi_amd.build` "
                "(there is no CPU fallback)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != TSG_OK:
        msg = load().tsg_last_error().decode(errors="replace")
        raise TsgError(status, msg)


def declared_symbols() -> list[str]:
    """Function names declared in include/tsugumi_hip.h."""
    import re
    hdr = os.path.join(os.path.dirname(HERE), "include", "tsugumi_hip.h")
    text = open(hdr).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsg_[a-z0-9_]+)\s*\(", text)))
