// prefill_gemm.hpp — the grouped int4 GEMM's argument block, the fp16
// dequantisation its weight tiles go through (shared with the staging probe
// of prefill.hip) and the launchers of its kernels. The kernels themselves
// (prefill_gemm_impl.hpp) are compiled once per (group size, scheme) in
// gemm_g32_sym.hip, gemm_g32_affine.hip, gemm_g64_sym.hip and
// gemm_g64_affine.hip, so the four build in parallel.
#pragma once

#include "gemv_lane.hpp"

namespace tsg {

// K runs in 64-element chunks: d and f must be multiples of it.
constexpr uint32_t kGemmKC = 64;

struct GemmArgs {
    const uint8_t* layer_base;
    uint64_t expert_stride;
    tsg_expert_offsets o;
    const uint16_t* a;          // hidden (gate/up) or act (down)
    uint32_t a_stride;          // elements
    const tsg_token_expert_pair* pairs;
    const tsg_routed_block* blocks;
    uint32_t n_blocks;
    const uint32_t* n_blocks_device;
    uint16_t* out;              // act (gate/up), route partials (down) or y (dense)
    uint32_t d, f, top_k;
    uint32_t dense_rows;        // MODE 2: rows of x and y
    const uint8_t* dense_s;     // MODE 2: scales (the weights are at layer_base)
    const uint8_t* dense_b;     // MODE 2: biases (the scales again under sym)
    uint32_t ntiles;            // weight-row tiles per routed block
    uint32_t dense_narrow;      // MODE 2: 128-column tiles, one 32-row weight tile per wave
    uint32_t num_experts;       // experts of the layer (device block lists are checked)
    uint32_t max_rows;          // rows path, device list: rows of the activation scratch
    uint32_t* error;            // the context's device error word
};

// The routed GEMMs: mode 0 gate/up + activation, mode 1 down + scatter
// (tsg_prefill_moe_gate_up / tsg_prefill_moe_down); both in one persistent
// launch (tsg_prefill_moe_gate_up_down); the dense projection
// (tsg_prefill_int4_qmm).
template <int G, bool SYM>
tsg_status routed_gemm_launch(const tsg_moe* moe, hipStream_t s, int mode, const GemmArgs& a,
                              uint32_t max_blocks);
template <int G, bool SYM>
tsg_status routed_gemm_fused_launch(const tsg_moe* moe, hipStream_t s, GemmArgs gu, GemmArgs dn,
                                    uint32_t max_blocks);
template <int G, bool SYM>
tsg_status dense_qmm_launch(hipStream_t s, const GemmArgs& a, uint32_t num_cus);

namespace {

// ------------------------------------------------------- fp16 dequant

typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));

// Per (weight row, group) dequantisation parameters. Every weight is staged
// as RNE_f16(fmaf(q, s, b)) with b = -8 s under sym (prefill.metal:1021-1026):
// fmaf rounds q * s + b to fp32, the conversion rounds that to fp16. The
// nibble q is isolated inside a 16-bit half, where as an fp16 bit pattern it
// is the subnormal q * 2^-24 (bits 0..3) or q * 2^-20 (bits 4..7); the scale
// is pre-multiplied by 2^24 or 2^20, so v_fma_mix forms the exact product
// q * s (for |s| < 2^103, where s * 2^24 stays finite), with no per-group test.
//  - sym: q * s - 8 s = (q - 8) * s has at most 12 significant bits, exact in
//    fp32, so v_fma_mix{lo,hi}_f16, which round the exact sum once to fp16,
//    give the reference's bits.
//  - affine: q * s + b can need more than 24 bits (b far smaller or larger
//    than s), and rounding it to fp32 first can land on an fp16 tie that a
//    single rounding would not; the sum is therefore taken to fp32 with
//    v_fma_mix_f32 and converted with its own instruction.
struct GroupScale {
    float s_lo, s_hi, b;  // s * 2^24, s * 2^20, b
};

template <bool SYM>
__device__ __forceinline__ GroupScale group_scale(uint16_t s_bits, uint16_t b_bits) {
    const float s = bf16_to_f32(s_bits);
    GroupScale g;
    g.s_lo = s * 16777216.0f;
    g.s_hi = s * 1048576.0f;
    g.b = SYM ? -8.0f * s : bf16_to_f32(b_bits);
    return g;
}

// Eight weights (one packed u32, elements 0..7 of a K run), in element order.
// Two ANDs of the word and two of the word shifted right by 8 leave every
// nibble alone in a 16-bit half, at bits 0..3 (elements 0, 2 | 4, 6: the low
// nibbles of bytes 0, 1 | 2, 3) or 4..7 (elements 1, 3 | 5, 7); one v_fma_mix
// per element reads its half. 13 VALU per 8 weights under sym (the pair
// packing folds into v_fma_mix{lo,hi}_f16), 17 under affine (fp32 sums, one
// v_cvt_pk_f16_f32 per pair). Split into the extraction and four pairs so the
// GEMM can spread the work between its MFMAs.
struct Nibbles {
    h2_t n0, n1, n2, n3;  // e0|e4, e1|e5, e2|e6, e3|e7
};

__device__ __forceinline__ Nibbles nibbles8(uint32_t w) {
    const uint32_t w8 = w >> 8;
    return Nibbles{__builtin_bit_cast(h2_t, w & 0x000F000Fu), __builtin_bit_cast(h2_t, w & 0x00F000F0u),
                   __builtin_bit_cast(h2_t, w8 & 0x000F000Fu), __builtin_bit_cast(h2_t, w8 & 0x00F000F0u)};
}

// Pair j (elements 2j, 2j+1) of the eight.
template <bool SYM, int J>
__device__ __forceinline__ h2_t dequant_pair(const Nibbles& n, const GroupScale& g) {
    const _Float16 lo_src = J == 0 ? n.n0.x : J == 1 ? n.n2.x : J == 2 ? n.n0.y : n.n2.y;
    const _Float16 hi_src = J == 0 ? n.n1.x : J == 1 ? n.n3.x : J == 2 ? n.n1.y : n.n3.y;
    if constexpr (SYM) {
        // the empty asm makes the low half a value of its own, so the pair
        // becomes v_fma_mixlo_f16 + v_fma_mixhi_f16 rather than two
        // v_fma_mix_f32 and a v_cvt_pk_f16_f32
        _Float16 lo = (_Float16)__builtin_fmaf((float)lo_src, g.s_lo, g.b);
        asm("" : "+v"(lo));
        return h2_t{lo, (_Float16)__builtin_fmaf((float)hi_src, g.s_hi, g.b)};
    } else {
        float lo = __builtin_fmaf((float)lo_src, g.s_lo, g.b);
        float hi = __builtin_fmaf((float)hi_src, g.s_hi, g.b);
        asm("" : "+v"(lo), "+v"(hi));
        return h2_t{(_Float16)lo, (_Float16)hi};
    }
}

__device__ __forceinline__ h8v_t pack_pairs(h2_t p0, h2_t p1, h2_t p2, h2_t p3) {
    return h8v_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

template <bool SYM>
__device__ __forceinline__ h8v_t dequant8(uint32_t w, const GroupScale& g) {
    const Nibbles n = nibbles8(w);
    return pack_pairs(dequant_pair<SYM, 0>(n, g), dequant_pair<SYM, 1>(n, g),
                      dequant_pair<SYM, 2>(n, g), dequant_pair<SYM, 3>(n, g));
}

// Dump of the GEMM's staging (tsg_debug_gemm_dequant_f16): one thread per 8
// weights. The eight values leave as one 16-byte vector: extracting them one
// by one into 16-bit stores made this hipcc fold all eight to the first.
template <int G, bool SYM>
__global__ void gemm_dequant_probe_kernel(const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ scales,
                                          const uint16_t* __restrict__ biases,
                                          uint16_t* __restrict__ out, uint32_t rows,
                                          uint32_t n) {
    const uint64_t pieces = (uint64_t)rows * (n / 8u);
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < pieces;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = p / (n / 8u);
        const uint32_t k0 = (uint32_t)(p - r * (n / 8u)) * 8u;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(w + r * (n / 2u) + k0 / 2u);
        const uint32_t g = k0 / G;
        const GroupScale gs = group_scale<SYM>(scales[r * (n / G) + g],
                                               SYM ? (uint16_t)0 : biases[r * (n / G) + g]);
        *reinterpret_cast<uint4*>(out + r * n + k0) = __builtin_bit_cast(uint4, dequant8<SYM>(v, gs));
    }
}

}  // namespace
}  // namespace tsg
