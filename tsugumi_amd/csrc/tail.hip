// tail.hip — the Gemma decoder-layer tail that follows the MoE FFN, per row:
//
//   h12    = half(h1 + half(h2  * rms_inv(h2)  * post_ffn_2))
//   hidden = half(half(hidden + half(h12 * rms_inv(h12) * post_ffn)) * half(layer_scalar))
//
// rms_inv(x) = 1 / sqrt(sum(x^2) / D + eps). This restates
// prefill_layer_tail_block (prefill.metal:319-397, PrefillLayerTail.swift) and
// fused_layer_tail (fused.metal:271-374, FusedLayerTail.swift), which keep the
// same fp16 stage boundaries. Every fp16 add or multiply of two fp16 values is
// formed in fp32 and rounded once to fp16; fp32 carries 24 bits ≥ 2·11 + 2, so
// this equals the correctly rounded fp16 operation.
//
// One 256-thread block per row. Thread i owns the 8-element chunks i and
// i + 256 (D ≤ 4096), and each sum of squares runs in one fixed order over the
// element index: per thread chunk by chunk and element by element, a 64-lane
// butterfly, then the four waves in order. The order does not depend on the
// strides or on whether a chunk is read with one 16-byte load or eight 2-byte
// loads, so the block form at any strides, the one-row decode form and the
// reduce-fused form give identical bits for a row.
//
// The reduce-fused form computes h2 in registers from the route partials with
// the token-major reduce's per-element fma order (the same bits as
// tsg_prefill_moe_reduce_token_major), so h2 is never written to HBM unless the
// caller asks for it.
#include "tsg_internal.hpp"

namespace tsg {
namespace {

constexpr uint32_t kTailThreads = 256;
constexpr uint32_t kTailMaxD = 4096;  // kPrefillPostMaxD / kFusedMaxD
constexpr uint32_t kTailChunks = kTailMaxD / (8u * kTailThreads);

bool is16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct TailArgs {
    const uint16_t* h2;
    const uint16_t* h1;
    uint16_t* hidden;
    const uint16_t* w_post2;  // post_feedforward_layernorm_2, bf16
    const uint16_t* w_post;   // post_feedforward_layernorm, bf16
    const uint16_t* partials;  // reduce-fused form: [t * top_k, d] fp16
    const uint16_t* route_w;   // reduce-fused form: [t, top_k] fp16
    uint16_t* h2_out;          // reduce-fused form, optional
    uint64_t h2_stride, h1_stride, hidden_stride;
    uint32_t t, d, top_k;
    float eps, layer_scalar;
};

struct Chunk {
    uint16_t h[8];
};

// Elements base..base+7 of a row; those at or past d read as zero (only the
// scalar form has such a chunk). VEC: one 16-byte load.
template <bool VEC>
__device__ __forceinline__ Chunk load_chunk(const uint16_t* __restrict__ row, uint32_t base,
                                            uint32_t d) {
    Chunk c;
    if (VEC) {
        const uint4 q = *reinterpret_cast<const uint4*>(row + base);
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            c.h[2 * e] = (uint16_t)(u[e] & 0xFFFFu);
            c.h[2 * e + 1] = (uint16_t)(u[e] >> 16);
        }
    } else {
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) c.h[e] = base + e < d ? row[base + e] : (uint16_t)0;
    }
    return c;
}

template <bool VEC>
__device__ __forceinline__ void store_chunk(uint16_t* __restrict__ row, uint32_t base, uint32_t d,
                                            const Chunk& c) {
    if (VEC) {
        uint4 q;
        q.x = (uint32_t)c.h[0] | ((uint32_t)c.h[1] << 16);
        q.y = (uint32_t)c.h[2] | ((uint32_t)c.h[3] << 16);
        q.z = (uint32_t)c.h[4] | ((uint32_t)c.h[5] << 16);
        q.w = (uint32_t)c.h[6] | ((uint32_t)c.h[7] << 16);
        *reinterpret_cast<uint4*>(row + base) = q;
    } else {
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e)
            if (base + e < d) row[base + e] = c.h[e];
    }
}

// Sum over the block: butterfly within each wave (every lane ends with the
// same bits, as a + b == b + a), then the four wave sums in wave order.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

__device__ __forceinline__ float rms_inv(float sum_sq, uint32_t d, float eps) {
    return 1.0f / __builtin_sqrtf(sum_sq / (float)d + eps);
}

// One row per block. REDUCE: h2 = half(sum_r fma(w[row, r], P[row*top_k + r], ·))
// in rank order, the token-major reduce's per-element formula.
template <bool VEC, bool REDUCE>
__global__ __launch_bounds__(kTailThreads) void layer_tail_kernel(TailArgs a) {
    __shared__ float red[2][4];
    const uint32_t row = blockIdx.x;
    const uint32_t d = a.d;
    Chunk x[kTailChunks];
    bool live[kTailChunks];
#pragma unroll
    for (uint32_t j = 0; j < kTailChunks; ++j) live[j] = 8u * (threadIdx.x + j * kTailThreads) < d;

    if (REDUCE) {
        const uint32_t k = a.top_k;
        const uint16_t* wrow = a.route_w + (uint64_t)row * k;
#pragma unroll
        for (uint32_t j = 0; j < kTailChunks; ++j) {
            if (!live[j]) continue;
            const uint32_t base = 8u * (threadIdx.x + j * kTailThreads);
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
            for (uint32_t r = 0; r < k; ++r) {
                const float wf = f16_to_f32(wrow[r]);
                const Chunk p = load_chunk<VEC>(a.partials + ((uint64_t)row * k + r) * d, base, d);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(wf, f16_to_f32(p.h[e]), acc[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) x[j].h[e] = base + e < d ? f32_to_f16(acc[e]) : (uint16_t)0;
            if (a.h2_out) store_chunk<VEC>(a.h2_out + (uint64_t)row * d, base, d, x[j]);
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < kTailChunks; ++j)
            if (live[j])
                x[j] = load_chunk<VEC>(a.h2 + row * a.h2_stride, 8u * (threadIdx.x + j * kTailThreads), d);
    }

    // h12 = half(h1 + half(h2 * inv_h2 * w_post2))
    float ss = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kTailChunks; ++j)
        if (live[j])
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = f16_to_f32(x[j].h[e]);
                ss = __builtin_fmaf(v, v, ss);
            }
    const float inv_h2 = rms_inv(block_sum(ss, red[0]), d, a.eps);
    float ss2 = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kTailChunks; ++j) {
        if (!live[j]) continue;
        const uint32_t base = 8u * (threadIdx.x + j * kTailThreads);
        const Chunk h1 = load_chunk<VEC>(a.h1 + row * a.h1_stride, base, d);
        const Chunk w2 = load_chunk<VEC>(a.w_post2, base, d);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t tmp = f32_to_f16((f16_to_f32(x[j].h[e]) * inv_h2) * bf16_to_f32(w2.h[e]));
            x[j].h[e] = f32_to_f16(f16_to_f32(h1.h[e]) + f16_to_f32(tmp));
            const float v = f16_to_f32(x[j].h[e]);
            ss2 = __builtin_fmaf(v, v, ss2);
        }
    }
    const float inv_h12 = rms_inv(block_sum(ss2, red[1]), d, a.eps);

    // hidden = half(half(hidden + half(h12 * inv_h12 * w_post)) * half(layer_scalar))
    const float scale = f16_to_f32(f32_to_f16(a.layer_scalar));
    uint16_t* hrow = a.hidden + row * a.hidden_stride;
#pragma unroll
    for (uint32_t j = 0; j < kTailChunks; ++j) {
        if (!live[j]) continue;
        const uint32_t base = 8u * (threadIdx.x + j * kTailThreads);
        Chunk h = load_chunk<VEC>(hrow, base, d);
        const Chunk w1 = load_chunk<VEC>(a.w_post, base, d);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t tmp = f32_to_f16((f16_to_f32(x[j].h[e]) * inv_h12) * bf16_to_f32(w1.h[e]));
            const uint16_t sum = f32_to_f16(f16_to_f32(h.h[e]) + f16_to_f32(tmp));
            h.h[e] = f32_to_f16(f16_to_f32(sum) * scale);
        }
        store_chunk<VEC>(hrow, base, d, h);
    }
}

template <bool REDUCE>
tsg_status launch_tail(const TailArgs& a, tsg_stream stream) {
    const bool vec = a.d % 8u == 0 && a.h2_stride % 8u == 0 && a.h1_stride % 8u == 0 &&
                     a.hidden_stride % 8u == 0 && is16(a.h1) && is16(a.hidden) &&
                     is16(a.w_post2) && is16(a.w_post) &&
                     (REDUCE ? is16(a.partials) && is16(a.h2_out) : is16(a.h2));
    const dim3 grid(a.t), block(kTailThreads);
    if (vec)
        hipLaunchKernelGGL((layer_tail_kernel<true, REDUCE>), grid, block, 0, as_stream(stream), a);
    else
        hipLaunchKernelGGL((layer_tail_kernel<false, REDUCE>), grid, block, 0, as_stream(stream), a);
    return check_launch(REDUCE ? "reduce_layer_tail" : "layer_tail");
}

}  // namespace
}  // namespace tsg

using namespace tsg;

extern "C" tsg_status tsg_prefill_layer_tail(tsg_ctx* ctx, tsg_stream stream, const uint16_t* h2,
                                             const uint16_t* h1, uint16_t* hidden,
                                             const uint16_t* post_ffn2_weight,
                                             const uint16_t* post_ffn_weight,
                                             uint32_t query_count, uint32_t d,
                                             uint32_t h2_stride_elements,
                                             uint32_t h1_stride_elements,
                                             uint32_t hidden_stride_elements, float eps,
                                             float layer_scalar) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(query_count > 0, TSG_ERR_INVALID_ARGUMENT, "queryCount must be positive");
    TSG_REQUIRE(d > 0 && d <= kTailMaxD, TSG_ERR_INVALID_ARGUMENT, "D must be in 1...4096");
    TSG_REQUIRE(h2_stride_elements >= d, TSG_ERR_INVALID_ARGUMENT, "h2 stride is too small");
    TSG_REQUIRE(h1_stride_elements >= d, TSG_ERR_INVALID_ARGUMENT, "h1 stride is too small");
    TSG_REQUIRE(hidden_stride_elements >= d, TSG_ERR_INVALID_ARGUMENT,
                "hidden stride is too small");
    TSG_REQUIRE(h2 && h1 && hidden && post_ffn2_weight && post_ffn_weight,
                TSG_ERR_INVALID_ARGUMENT, "NULL layer-tail operand");
    TailArgs a{};
    a.h2 = h2;
    a.h1 = h1;
    a.hidden = hidden;
    a.w_post2 = post_ffn2_weight;
    a.w_post = post_ffn_weight;
    a.h2_stride = h2_stride_elements;
    a.h1_stride = h1_stride_elements;
    a.hidden_stride = hidden_stride_elements;
    a.t = query_count;
    a.d = d;
    a.eps = eps;
    a.layer_scalar = layer_scalar;
    return launch_tail<false>(a, stream);
}

extern "C" tsg_status tsg_fused_layer_tail(tsg_ctx* ctx, tsg_stream stream, const uint16_t* h2,
                                           const uint16_t* h1, uint16_t* hidden,
                                           const uint16_t* post_ffn2_weight,
                                           const uint16_t* post_ffn_weight, uint32_t d, float eps,
                                           float layer_scalar) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(d <= kTailMaxD, TSG_ERR_INVALID_ARGUMENT,
                "D > 4096 exceeds the fused-tail threadgroup scratch (kFusedMaxD)");
    if (d == 0) return TSG_OK;  // the reference's loops run zero times
    return tsg_prefill_layer_tail(ctx, stream, h2, h1, hidden, post_ffn2_weight, post_ffn_weight,
                                  1, d, d, d, d, eps, layer_scalar);
}

extern "C" tsg_status tsg_prefill_moe_reduce_layer_tail(
    tsg_ctx* ctx, tsg_stream stream, const uint16_t* route_partials,
    const uint16_t* route_weights, uint16_t* h2_out, const uint16_t* h1, uint16_t* hidden,
    const uint16_t* post_ffn2_weight, const uint16_t* post_ffn_weight, uint32_t query_count,
    uint32_t top_k, uint32_t d, uint32_t h1_stride_elements, uint32_t hidden_stride_elements,
    float eps, float layer_scalar) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(query_count > 0, TSG_ERR_INVALID_ARGUMENT, "queryCount must be positive");
    TSG_REQUIRE(top_k > 0, TSG_ERR_INVALID_ARGUMENT, "topK must be positive");
    TSG_REQUIRE(d > 0 && d <= kTailMaxD, TSG_ERR_INVALID_ARGUMENT, "D must be in 1...4096");
    TSG_REQUIRE(h1_stride_elements >= d, TSG_ERR_INVALID_ARGUMENT, "h1 stride is too small");
    TSG_REQUIRE(hidden_stride_elements >= d, TSG_ERR_INVALID_ARGUMENT,
                "hidden stride is too small");
    TSG_REQUIRE(route_partials && route_weights && h1 && hidden && post_ffn2_weight &&
                    post_ffn_weight,
                TSG_ERR_INVALID_ARGUMENT, "NULL layer-tail operand");
    TailArgs a{};
    a.partials = route_partials;
    a.route_w = route_weights;
    a.h2_out = h2_out;
    a.h1 = h1;
    a.hidden = hidden;
    a.w_post2 = post_ffn2_weight;
    a.w_post = post_ffn_weight;
    a.h2_stride = d;
    a.h1_stride = h1_stride_elements;
    a.hidden_stride = hidden_stride_elements;
    a.t = query_count;
    a.d = d;
    a.top_k = top_k;
    a.eps = eps;
    a.layer_scalar = layer_scalar;
    return launch_tail<true>(a, stream);
}
