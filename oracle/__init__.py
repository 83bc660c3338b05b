"""ctypes binding of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: the checker that the HIP path is compared against.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package; the product path never does.

Each wrapper names the reference file:line its C function restates (paths are
relative to the he-be/tsugumi checkout).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

PAIR_DTYPE = np.dtype([("token", "<u4"), ("expert", "<u4"), ("rank", "<u4"),
                       ("weight_bits", "<u4")])
GROUP_DTYPE = np.dtype([("expert", "<u4"), ("pair_start", "<u4"), ("pair_count", "<u4")])
TILE_DTYPE = np.dtype([("group_start", "<u4"), ("group_count", "<u4"),
                       ("pair_start", "<u4"), ("pair_count", "<u4")])
BLOCK_DTYPE = np.dtype([("local_slot", "<u4"), ("pair_start", "<u4"),
                        ("row_count", "<u4"), ("local_row", "<u4")])

# PrefillMoEGroupingError cases (PrefillMoEGrouping.swift:52-62), by code.
GROUPING_ERRORS = {
    -1: "invalidQueryCount", -2: "invalidTopK", -3: "invalidNumExperts",
    -4: "invalidTileExpertCount", -5: "pairCountMismatch", -6: "tokenOutOfRange",
    -7: "rankOutOfRange", -8: "expertOutOfRange", -9: "duplicateTokenRank",
    -10: "expertSortKeyCountMismatch",
}


class GroupingError(ValueError):
    def __init__(self, code: int):
        self.code = code
        self.case = GROUPING_ERRORS.get(code, f"error {code}")
        super().__init__(self.case)


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def use_timed_build() -> str:
    """Switches this process to liboracle_timed.so (`make timed`: -O3
    -march=native for the CPU it runs on, dot products in eight interleaved
    partial sums), the copy bench.py times as the CPU baseline. It is never
    used as a checker. Returns its path."""
    global _lib
    subprocess.run(["make", "-s", "-C", _HERE, "timed"], check=True)
    path = os.path.join(_HERE, "liboracle_timed.so")
    _lib = C.CDLL(path)
    _declare(_lib)
    return path


_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_intp = C.POINTER(C.c_int)


def _declare(L):
    L.tsgo_splitmix64_next.argtypes = [_u64p]
    L.tsgo_splitmix64_next.restype = C.c_uint64
    L.tsgo_fnv1a64.argtypes = [C.c_char_p]
    L.tsgo_fnv1a64.restype = C.c_uint64
    L.tsgo_seedtree_key.argtypes = [C.c_uint64, C.c_char_p]
    L.tsgo_seedtree_key.restype = C.c_uint64
    L.tsgo_uniform.argtypes = [_u64p, C.c_float, C.c_float]
    L.tsgo_uniform.restype = C.c_float
    for name in ("tsgo_fill_uniform",):
        getattr(L, name).argtypes = [_u64p, C.c_float, C.c_float, _f32p, C.c_size_t]
    for name in ("tsgo_fill_uniform_f16", "tsgo_fill_uniform_bf16"):
        getattr(L, name).argtypes = [_u64p, C.c_float, C.c_float, _u16p, C.c_size_t]
    L.tsgo_bf16_bits.argtypes = [C.c_float]
    L.tsgo_bf16_bits.restype = C.c_uint16
    L.tsgo_bf16_to_float.argtypes = [C.c_uint16]
    L.tsgo_bf16_to_float.restype = C.c_float
    L.tsgo_f16_bits.argtypes = [C.c_float]
    L.tsgo_f16_bits.restype = C.c_uint16
    L.tsgo_f16_to_float.argtypes = [C.c_uint16]
    L.tsgo_f16_to_float.restype = C.c_float
    L.tsgo_sym_bias_bits.argtypes = [C.c_uint16]
    L.tsgo_sym_bias_bits.restype = C.c_uint16
    L.tsgo_f16_to_float_n.argtypes = [_u16p, _f32p, C.c_size_t]
    L.tsgo_float_to_f16_n.argtypes = [_f32p, _u16p, C.c_size_t]
    L.tsgo_quantize_int4.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                     _u8p, _u16p, _u16p]
    L.tsgo_dequantize_int4.argtypes = [_u8p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, _f32p]
    L.tsgo_dequantize_int4_f16.argtypes = [_u8p, _u16p, _u16p, C.c_int, C.c_int, C.c_int,
                                           C.c_int, _u16p]
    L.tsgo_dequant_int4_gemv_ref.argtypes = [_u8p, _u16p, _u16p, _f32p, C.c_int, C.c_int,
                                             C.c_int, _f32p]
    L.tsgo_layer_tail.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, C.c_int, C.c_int,
                                  C.c_int, C.c_int, C.c_int, C.c_float, C.c_float]
    L.tsgo_layer_tail.restype = None
    L.tsgo_gelu_tanh.argtypes = [C.c_float]
    L.tsgo_gelu_tanh.restype = C.c_float
    L.tsgo_silu.argtypes = [C.c_float]
    L.tsgo_silu.restype = C.c_float
    L.tsgo_sigmoid.argtypes = [C.c_float]
    L.tsgo_sigmoid.restype = C.c_float
    L.tsgo_silu_mul_f16.argtypes = [_u16p, _u16p, _u16p, C.c_int]
    L.tsgo_gelu_mul_f16.argtypes = [_u16p, _u16p, _u16p, C.c_int]
    L.tsgo_dense_mlp_int4.argtypes = [_u8p, _u16p, _u16p, _u8p, _u16p, _u16p, _u8p, _u16p, _u16p,
                                      _u16p, C.c_int, C.c_int, C.c_int, _u16p]
    L.tsgo_shared_gate_f16.argtypes = [_u16p, _u16p, _u16p, C.c_int]
    L.tsgo_shared_expert.argtypes = [_u8p, _u32p, _u16p, _u16p, C.c_int, C.c_int, C.c_int,
                                     C.c_int, _u16p]
    L.tsgo_moe_run_ffn.argtypes = [_u8p, _u16p, _u16p, _u8p, _u16p, _u16p, _u8p, _u16p, _u16p,
                                   _f32p, C.c_int, C.c_int, C.c_int, C.c_int, _f32p]
    L.tsgo_moe_apply_streamed_routed.argtypes = [C.POINTER(_u8p), _u32p, _f32p, _f32p, _f32p,
                                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                                 C.c_int, _f32p]
    L.tsgo_router_reference.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p,
                                        _i32p, _f32p]
    L.tsgo_router_logits_canonical.argtypes = [_u16p, _u16p, C.c_int, _u16p, C.c_int, C.c_int,
                                               C.c_int, _f32p]
    L.tsgo_topk_softmax.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _i32p, _u16p]
    L.tsgo_quantize_int8_affine.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, _u8p, _u16p,
                                            _u16p]
    L.tsgo_dequantize_int8_affine.argtypes = [_u8p, _u16p, _u16p, C.c_int, C.c_int, C.c_int,
                                              _f32p]
    L.tsgo_router_logits_int8_canonical.argtypes = [_u8p, _u16p, _u16p, _u16p, _u16p, C.c_int,
                                                    C.c_int, C.c_int, _f32p]
    L.tsgo_make_token_expert_pairs.argtypes = [_u32p, _u16p, C.c_int, C.c_int, C.c_void_p]
    L.tsgo_group_pairs.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   _u64p, C.c_int, C.c_int, C.c_void_p, _u32p, _u32p,
                                   C.c_void_p, _intp, C.c_void_p, _intp]
    L.tsgo_group_pairs.restype = C.c_int
    L.tsgo_plan_routed_gemm.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, _intp,
                                        _intp, _intp, _intp]
    L.tsgo_plan_routed_gemm.restype = C.c_int
    L.tsgo_prefill_moe_ref.argtypes = [C.POINTER(_u8p), _u32p, _u16p, C.c_int, C.c_void_p,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, _u16p]
    L.tsgo_reduce_token_major.argtypes = [_u16p, _u16p, C.c_int, C.c_int, C.c_int, _u16p]
    L.tsgo_set_threads.argtypes = [C.c_int]
    L.tsgo_get_threads.restype = C.c_int


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.POINTER(ctype))


def set_threads(n: int) -> None:
    lib().tsgo_set_threads(int(n))


# ---------------------------------------------------------------- PRNG ----

class SplitMix64:
    """SplitMix64 (TsugumiValidation/Support/PRNG/SplitMix64.swift:11-24)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next(self) -> int:
        return int(lib().tsgo_splitmix64_next(C.byref(self.state)))

    def uniform(self, lo: float, hi: float) -> float:
        return float(lib().tsgo_uniform(C.byref(self.state), lo, hi))

    def uniforms(self, lo: float, hi: float, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().tsgo_fill_uniform(C.byref(self.state), lo, hi, _p(out, C.c_float), n)
        return out

    def uniforms_f16(self, lo: float, hi: float, n: int) -> np.ndarray:
        """n draws of Float16(uniform(lo, hi)), as uint16 bits."""
        out = np.empty(n, np.uint16)
        lib().tsgo_fill_uniform_f16(C.byref(self.state), lo, hi, _p(out, C.c_uint16), n)
        return out

    def uniforms_bf16(self, lo: float, hi: float, n: int) -> np.ndarray:
        out = np.empty(n, np.uint16)
        lib().tsgo_fill_uniform_bf16(C.byref(self.state), lo, hi, _p(out, C.c_uint16), n)
        return out


def fnv1a64(label: str) -> int:
    return int(lib().tsgo_fnv1a64(label.encode()))


def seed_tree_key(root: int, label: str) -> SplitMix64:
    """SeedTree(root).key(label) (SeedTree.swift:12-19)."""
    return SplitMix64(int(lib().tsgo_seedtree_key(root & 0xFFFFFFFFFFFFFFFF, label.encode())))


# --------------------------------------------------------- conversions ----

def bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return (((u + 0x7FFF + lsb) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_to_float(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().tsgo_float_to_f16_n(_p(x, C.c_float), _p(out, C.c_uint16), x.size)
    return out


def f16_to_float(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, np.uint16)
    flat = b.ravel()
    out = np.empty(flat.size, np.float32)
    lib().tsgo_f16_to_float_n(_p(flat, C.c_uint16), _p(out, C.c_float), flat.size)
    return out.reshape(b.shape)


def sym_bias_bits(scale_bits: int) -> int:
    return int(lib().tsgo_sym_bias_bits(int(scale_bits)))


# -------------------------------------------------------- quantisation ----

def quantize_int4(w: np.ndarray, group: int, symmetric: bool):
    """Quantization.quantizeInt4Affine / quantizeInt4Symmetric over rows."""
    w = np.ascontiguousarray(w, np.float32)
    rows, n = w.shape
    packed = np.empty((rows, n // 2), np.uint8)
    scales = np.empty((rows, n // group), np.uint16)
    biases = np.empty((rows, n // group), np.uint16)
    lib().tsgo_quantize_int4(_p(w, C.c_float), rows, n, group, int(symmetric),
                             _p(packed, C.c_uint8), _p(scales, C.c_uint16),
                             _p(biases, C.c_uint16))
    return packed, scales, biases


def dequantize_int4(packed, scales, biases, n: int, group: int) -> np.ndarray:
    """Quantization.dequantizeInt4Affine; biases=None means sym (-8*scale)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    rows = packed.size // (n // 2)
    out = np.empty((rows, n), np.float32)
    bp = _p(np.ascontiguousarray(biases, np.uint16), C.c_uint16) if biases is not None else None
    lib().tsgo_dequantize_int4(_p(packed, C.c_uint8), _p(scales, C.c_uint16), bp,
                               rows, n, group, _p(out, C.c_float))
    return out


def dequantize_int4_f16(packed, scales, biases, n: int, group: int, symmetric: bool):
    """half(fma(q, s, b)) staging (prefill.metal:1021-1026) as fp16 bits."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    rows = packed.size // (n // 2)
    out = np.empty((rows, n), np.uint16)
    bp = (_p(np.ascontiguousarray(biases, np.uint16), C.c_uint16)
          if (biases is not None and not symmetric) else None)
    lib().tsgo_dequantize_int4_f16(_p(packed, C.c_uint8), _p(scales, C.c_uint16), bp,
                                   rows, n, group, int(symmetric), _p(out, C.c_uint16))
    return out


# ---------------------------------------------------------- GEMV / FFN ----

def dequant_int4_gemv_ref(packed, scales, biases, x, n: int, group: int) -> np.ndarray:
    """DequantInt4GemvRef.apply (Reference/Quant/DequantInt4Gemv.swift:12-44)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    m = packed.size // (n // 2)
    y = np.empty(m, np.float32)
    bp = _p(np.ascontiguousarray(biases, np.uint16), C.c_uint16) if biases is not None else None
    lib().tsgo_dequant_int4_gemv_ref(_p(packed, C.c_uint8), _p(scales, C.c_uint16), bp,
                                     _p(x, C.c_float), m, n, group, _p(y, C.c_float))
    return y


def gelu_tanh(x: float) -> float:
    return float(lib().tsgo_gelu_tanh(float(x)))


def silu(x: float) -> float:
    return float(lib().tsgo_silu(float(x)))


def sigmoid(x: float) -> float:
    """qwen_sigmoid (qwen.metal:33)."""
    return float(lib().tsgo_sigmoid(float(x)))


def silu_mul_f16(gate, up) -> np.ndarray:
    """qwen_silu_mul (qwen.metal:466) on fp16 bits."""
    gate = np.ascontiguousarray(gate, np.uint16)
    up = np.ascontiguousarray(up, np.uint16)
    out = np.empty_like(gate)
    lib().tsgo_silu_mul_f16(_p(gate, C.c_uint16), _p(up, C.c_uint16), _p(out, C.c_uint16),
                            gate.size)
    return out


def gelu_mul_f16(gate, up) -> np.ndarray:
    """gelu_mul_fp16 (utility.metal:7-18) on fp16 bits."""
    gate = np.ascontiguousarray(gate, np.uint16)
    up = np.ascontiguousarray(up, np.uint16)
    out = np.empty_like(gate)
    lib().tsgo_gelu_mul_f16(_p(gate, C.c_uint16), _p(up, C.c_uint16), _p(out, C.c_uint16),
                            gate.size)
    return out


def dense_mlp_int4(gate, up, down, x_bits, d: int, f: int, group: int,
                   symmetric: bool) -> np.ndarray:
    """SharedExpertInt4.encode (SharedExpertInt4.swift:30-93) over
    DequantInt4GemvRef; gate/up/down are (packed, scales, biases) triples
    ([f, d], [f, d], [d, f]). Returns y as fp16 bits."""
    def ptrs(t):
        packed, scales, biases = t
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        b = None if symmetric else _p(np.ascontiguousarray(biases, np.uint16), C.c_uint16)
        return packed, scales, b
    keep = [ptrs(t) for t in (gate, up, down)]
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    out = np.empty(d, np.uint16)
    args = []
    for packed, scales, b in keep:
        args += [_p(packed, C.c_uint8), _p(scales, C.c_uint16), b]
    lib().tsgo_dense_mlp_int4(*args, _p(x_bits, C.c_uint16), d, f, group, _p(out, C.c_uint16))
    return out


def shared_gate_f16(y, x, w_bf16) -> np.ndarray:
    """qwen_moe_shared_gate (qwen.metal:432-455): returns the gated copy of y."""
    y = np.array(y, np.uint16, copy=True)
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w_bf16, np.uint16)
    lib().tsgo_shared_gate_f16(_p(y, C.c_uint16), _p(x, C.c_uint16), _p(w, C.c_uint16), y.size)
    return y


def shared_expert(blob, offsets9, x, gate_w_bf16, d: int, f: int, group: int,
                  symmetric: bool) -> np.ndarray:
    """QwenForwardRunner.encodeSharedExpert (QwenForwardRunner.swift:1548-1578)
    over one expert blob; returns sharedOut as fp16 bits."""
    blob = np.ascontiguousarray(blob, np.uint8)
    o = np.ascontiguousarray(offsets9, np.uint32)
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(gate_w_bf16, np.uint16)
    out = np.empty(d, np.uint16)
    lib().tsgo_shared_expert(_p(blob, C.c_uint8), _p(o, C.c_uint32), _p(x, C.c_uint16),
                             _p(w, C.c_uint16), d, f, group, int(symmetric), _p(out, C.c_uint16))
    return out


def _blob_ptr_array(blobs):
    arr = (_u8p * len(blobs))()
    for i, b in enumerate(blobs):
        assert b.dtype == np.uint8 and b.flags["C_CONTIGUOUS"]
        arr[i] = b.ctypes.data_as(_u8p)
    return arr


def moe_apply_streamed_routed(blobs, offsets9, x, residual, routing_weights, d, f, group,
                              symmetric, act=0) -> np.ndarray:
    """MoeRef.applyStreamedRouted (Reference/MoE/Moe.swift:90-121) over expert
    blobs laid out as MoEExpertOffsets (MoE.swift:4-29)."""
    o = np.ascontiguousarray(offsets9, np.uint32)
    x = np.ascontiguousarray(x, np.float32)
    r = np.ascontiguousarray(residual, np.float32)
    w = np.ascontiguousarray(routing_weights, np.float32)
    y = np.empty(d, np.float32)
    arr = _blob_ptr_array(blobs)
    lib().tsgo_moe_apply_streamed_routed(arr, _p(o, C.c_uint32), _p(x, C.c_float),
                                         _p(r, C.c_float), _p(w, C.c_float), len(blobs),
                                         d, f, group, int(symmetric), act, _p(y, C.c_float))
    return y


# -------------------------------------------------------------- router ----

def router_reference(w_rows, x, top_k, per_expert_scale):
    """routerReference (TsugumiKernelCheck/main.swift:384-402)."""
    w_rows = np.ascontiguousarray(w_rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    pes = np.ascontiguousarray(per_expert_scale, np.float32)
    ne, d = w_rows.shape
    assert ne >= top_k, "routerReference ranks at least top_k experts"
    idx = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    lib().tsgo_router_reference(_p(w_rows, C.c_float), _p(x, C.c_float), ne, d, top_k,
                                _p(pes, C.c_float), _p(idx, C.c_int32), _p(w, C.c_float))
    return idx, w


def router_logits_canonical(w_bf16, hidden_f16, stride, es_bf16, rows, num_experts, d):
    """Router logits in the MI355X kernels' summation order (see tsg_oracle.h)."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    h = np.ascontiguousarray(hidden_f16, np.uint16)
    es = np.ascontiguousarray(es_bf16, np.uint16)
    out = np.empty((rows, num_experts), np.float32)
    lib().tsgo_router_logits_canonical(_p(w, C.c_uint16), _p(h, C.c_uint16), stride,
                                       _p(es, C.c_uint16), rows, num_experts, d,
                                       _p(out, C.c_float))
    return out


def quantize_int8_affine(w: np.ndarray, group: int):
    """Quantization.quantizeInt8Affine (Quantization.swift:243-287) per row of
    `w` [rows, n]: (packed uint8 [rows, n], scale bits, bias bits [rows, n/group])."""
    w = np.ascontiguousarray(np.atleast_2d(w), np.float32)
    rows, n = w.shape
    assert n % group == 0
    packed = np.empty((rows, n), np.uint8)
    scales = np.empty((rows, n // group), np.uint16)
    biases = np.empty((rows, n // group), np.uint16)
    lib().tsgo_quantize_int8_affine(_p(w, C.c_float), rows, n, group, _p(packed, C.c_uint8),
                                    _p(scales, C.c_uint16), _p(biases, C.c_uint16))
    return packed, scales, biases


def dequantize_int8_affine(packed, scales, biases, group: int) -> np.ndarray:
    """Quantization.dequantizeInt8Affine (Quantization.swift:289-303)."""
    packed = np.ascontiguousarray(np.atleast_2d(packed), np.uint8)
    rows, n = packed.shape
    s = np.ascontiguousarray(scales, np.uint16).reshape(rows, n // group)
    b = np.ascontiguousarray(biases, np.uint16).reshape(rows, n // group)
    out = np.empty((rows, n), np.float32)
    lib().tsgo_dequantize_int8_affine(_p(packed, C.c_uint8), _p(s, C.c_uint16),
                                      _p(b, C.c_uint16), rows, n, group, _p(out, C.c_float))
    return out


def router_logits_int8_canonical(packed, scales, biases, hidden_f16, es_bf16, num_experts, d,
                                 group):
    """INT8-affine router logits in the MI355X kernel's summation order (see
    tsg_oracle.h)."""
    w = np.ascontiguousarray(packed, np.uint8).ravel()
    s = np.ascontiguousarray(scales, np.uint16).ravel()
    b = np.ascontiguousarray(biases, np.uint16).ravel()
    h = np.ascontiguousarray(hidden_f16, np.uint16).ravel()
    es = np.ascontiguousarray(es_bf16, np.uint16).ravel()
    assert w.size == num_experts * d and s.size == num_experts * (d // group)
    out = np.empty(num_experts, np.float32)
    lib().tsgo_router_logits_int8_canonical(_p(w, C.c_uint8), _p(s, C.c_uint16),
                                            _p(b, C.c_uint16), _p(h, C.c_uint16),
                                            _p(es, C.c_uint16), num_experts, d, group,
                                            _p(out, C.c_float))
    return out


def topk_softmax(logits, top_k, per_expert_scale):
    """router_topk_select_k8_body rule (moe.metal:281-329) over given logits."""
    logits = np.ascontiguousarray(logits, np.float32)
    pes = np.ascontiguousarray(per_expert_scale, np.float32)
    idx = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.uint16)
    lib().tsgo_topk_softmax(_p(logits, C.c_float), logits.size, top_k, _p(pes, C.c_float),
                            _p(idx, C.c_int32), _p(w, C.c_uint16))
    return idx, w


# -------------------------------------------------------------- prefill ---

def make_token_expert_pairs(idx, w_bits, t, top_k) -> np.ndarray:
    """PrefillRouter.makeTokenExpertPairs (PrefillRouter.swift:238-258)."""
    idx = np.ascontiguousarray(idx, np.uint32).ravel()
    w_bits = np.ascontiguousarray(w_bits, np.uint16).ravel()
    out = np.empty(t * top_k, PAIR_DTYPE)
    lib().tsgo_make_token_expert_pairs(_p(idx, C.c_uint32), _p(w_bits, C.c_uint16), t, top_k,
                                       out.ctypes.data)
    return out


def group_pairs(pairs, query_count, top_k, num_experts, tile_expert_count=16,
                expert_sort_keys=None, tile_break_after_group=None):
    """PrefillMoEGrouping.groupTokenExpertPairs (PrefillMoEGrouping.swift:90-202).
    Raises GroupingError on the reference's error cases."""
    pairs = np.ascontiguousarray(pairs, PAIR_DTYPE)
    n = pairs.size
    sorted_pairs = np.empty(max(n, 1), PAIR_DTYPE)
    offsets = np.empty(max(num_experts, 1), np.uint32)
    counts = np.empty(max(num_experts, 1), np.uint32)
    groups = np.empty(max(n, 1), GROUP_DTYPE)
    tiles = np.empty(max(n, 1), TILE_DTYPE)
    ng, nt = C.c_int(0), C.c_int(0)
    keys = None
    nkeys = 0
    if expert_sort_keys is not None:
        keys = np.ascontiguousarray(expert_sort_keys, np.uint64)
        nkeys = keys.size
    rc = lib().tsgo_group_pairs(pairs.ctypes.data, n, query_count, top_k, num_experts,
                                tile_expert_count,
                                _p(keys, C.c_uint64) if keys is not None else None, nkeys,
                                -1 if tile_break_after_group is None else tile_break_after_group,
                                sorted_pairs.ctypes.data, _p(offsets, C.c_uint32),
                                _p(counts, C.c_uint32), groups.ctypes.data, C.byref(ng),
                                tiles.ctypes.data, C.byref(nt))
    if rc != 0:
        raise GroupingError(rc)
    return dict(sorted_pairs=sorted_pairs[:n], offsets=offsets[:num_experts],
                counts=counts[:num_experts], groups=groups[:ng.value],
                tiles=tiles[:nt.value])


def plan_routed_gemm(groups, max_rows_per_batch):
    """PrefillRoutedGEMMPlanner.plan (PrefillGroupedRoutedMoE.swift:42-83).
    Returns a list of (rows, blocks) batches."""
    groups = np.ascontiguousarray(groups, GROUP_DTYPE)
    total = int(groups["pair_count"].sum()) if groups.size else 0
    cap = total + groups.size + 1
    blocks = np.empty(cap, BLOCK_DTYPE)
    rows = np.empty(cap, np.int32)
    first = np.empty(cap, np.int32)
    nb, nbatch = C.c_int(0), C.c_int(0)
    lib().tsgo_plan_routed_gemm(groups.ctypes.data, groups.size, max_rows_per_batch,
                                blocks.ctypes.data, C.byref(nb), _p(rows, C.c_int32),
                                _p(first, C.c_int32), C.byref(nbatch))
    out = []
    for i in range(nbatch.value):
        end = first[i + 1] if i + 1 < nbatch.value else nb.value
        out.append((int(rows[i]), blocks[first[i]:end].copy()))
    return out


def prefill_moe_ref(expert_blobs, offsets9, hidden_bits, hidden_stride, sorted_pairs,
                    top_k, d, f, group, symmetric, act=0, partials=None, rows_path=False):
    """Expert-major prefill reference with the GPU's fp16 roundings
    (TsugumiKernelCheck/PrefillMoEGEMMCheck.swift:138-173). `expert_blobs` is
    indexed by expert id. Returns fp16 bits [T*top_k, d] (rows never routed keep
    whatever `partials` held). rows_path: the verify rows kernel's roundings
    (gate and up stay fp32 into the activation, prefill.metal:1621-1628)
    instead of the tiled GEMM's (both rounded to fp16)."""
    o = np.ascontiguousarray(offsets9, np.uint32)
    hidden_bits = np.ascontiguousarray(hidden_bits, np.uint16)
    sp = np.ascontiguousarray(sorted_pairs, PAIR_DTYPE)
    t = hidden_bits.size // hidden_stride
    if partials is None:
        partials = np.zeros((t * top_k, d), np.uint16)
    arr = _blob_ptr_array(expert_blobs)
    lib().tsgo_prefill_moe_ref(arr, _p(o, C.c_uint32), _p(hidden_bits, C.c_uint16),
                               hidden_stride, sp.ctypes.data, sp.size, top_k, d, f, group,
                               int(symmetric), act, int(rows_path), _p(partials, C.c_uint16))
    return partials


def reduce_token_major(partials_bits, route_w_bits, t, top_k, d) -> np.ndarray:
    """prefill_moe_reduce_token_major (prefill.metal:796-817)."""
    p = np.ascontiguousarray(partials_bits, np.uint16)
    w = np.ascontiguousarray(route_w_bits, np.uint16)
    h2 = np.empty((t, d), np.uint16)
    lib().tsgo_reduce_token_major(_p(p, C.c_uint16), _p(w, C.c_uint16), t, top_k, d,
                                  _p(h2, C.c_uint16))
    return h2


def int4_qmm(packed, scales, biases, x_bits, t: int, n: int, k: int, group: int,
             symmetric: bool) -> np.ndarray:
    """PrefillInt4QMM's tiled path (prefill_int4_qmm_simdgroup_f16, the default):
    weights staged as half(fma(q, s, b)) (prefill.metal:1021-1026), products
    summed exactly (float64 here, fp32 MMA accumulation there), y rounded to
    fp16. Returns [t, n] fp16 bits."""
    w16 = dequantize_int4_f16(packed, scales, biases, k, group, symmetric).reshape(n, k)
    w = f16_to_float(w16).astype(np.float64)
    x = f16_to_float(np.ascontiguousarray(x_bits, np.uint16)).astype(np.float64).reshape(t, k)
    return f16_bits((x @ w.T).astype(np.float32)).reshape(t, n)


def layer_tail(h2, h1, hidden, w_post2, w_post, t, d, h2_stride, h1_stride, hidden_stride,
               eps, layer_scalar) -> np.ndarray:
    """prefill_layer_tail_block (prefill.metal:319-397) on fp16/bf16 bits;
    returns the updated hidden buffer (a copy, strided like the input)."""
    h2 = np.ascontiguousarray(h2, np.uint16)
    h1 = np.ascontiguousarray(h1, np.uint16)
    out = np.array(hidden, np.uint16, copy=True)
    w2 = np.ascontiguousarray(w_post2, np.uint16)
    w1 = np.ascontiguousarray(w_post, np.uint16)
    lib().tsgo_layer_tail(_p(h2, C.c_uint16), _p(h1, C.c_uint16), _p(out, C.c_uint16),
                          _p(w2, C.c_uint16), _p(w1, C.c_uint16), t, d, h2_stride, h1_stride,
                          hidden_stride, eps, layer_scalar)
    return out


# ------------------------------------------------------------ harness ----

def relative_error(actual, reference) -> float:
    """NaN-safe max-relative error (TsugumiKernelCheck/main.swift:69-86):
    max|a-r| / max|r|; any non-finite actual scores infinity."""
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(reference, np.float64).ravel()
    assert a.shape == r.shape
    assert np.all(np.isfinite(r)), "reference is not finite — harness bug"
    ref_norm = float(np.max(np.abs(r))) if r.size else 0.0
    assert ref_norm > 1e-4, f"reference has no signal (max |ref| = {ref_norm})"
    if not np.all(np.isfinite(a)):
        return float("inf")
    return float(np.max(np.abs(a - r)) / ref_norm)
