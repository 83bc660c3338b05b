// qwen_shared.hpp — the per-element steps of the Qwen-family shared expert
// and its sigmoid gate, shared by the separate kernels (shared.hip) and the
// one-launch decode layer (decode.hip) so every form gives the same bits.
#pragma once

#include "gemv_lane.hpp"

namespace tsg {
namespace {

// qwen.metal:33-34.
__device__ __forceinline__ float qwen_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float qwen_silu(float x) { return x * qwen_sigmoid(x); }

// half(silu(float(g)) * float(u)) (qwen.metal:466).
__device__ __forceinline__ uint16_t silu_mul_h(uint16_t g, uint16_t u) {
    return f32_to_f16(qwen_silu(f16_to_f32(g)) * f16_to_f32(u));
}

// The gate logit sum_i float(x[i]) * float(w[i]) (x fp16, w bf16, d a
// multiple of 8, d <= 4096) on one wave: lane l owns the 8-element units
// l, l + 64, ... (16-byte loads, all issued before any use) and accumulates
// their elements in order with fma; the lanes sum as group16_sum and then the
// four 16-lane rows as (r0 + r1) + (r2 + r3). Every lane returns the same
// value; every form of the gate (separate, fused into the shared branch,
// fused into the decode layer) uses this sum.
constexpr uint32_t kGateUnits = 8;  // units per lane: d <= 64 * 8 * 8

__device__ __forceinline__ float gate_logit_wave(const uint16_t* __restrict__ x,
                                                 const uint16_t* __restrict__ w, uint32_t d) {
    const uint32_t lane = threadIdx.x & 63u, units = d / 8u;
    uint4 xv[kGateUnits], wv[kGateUnits];
#pragma unroll
    for (uint32_t k = 0; k < kGateUnits; ++k) {
        const uint32_t u = min(lane + 64u * k, units - 1u);
        xv[k] = *reinterpret_cast<const uint4*>(x + u * 8u);
        wv[k] = *reinterpret_cast<const uint4*>(w + u * 8u);
    }
    float acc = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kGateUnits; ++k) {
        if (lane + 64u * k >= units) break;
        const uint32_t xa[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
        const uint32_t wa[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc = __builtin_fmaf(f16_to_f32((uint16_t)(xa[e] & 0xFFFFu)),
                                 __uint_as_float(wa[e] << 16), acc);
            acc = __builtin_fmaf(f16_to_f32((uint16_t)(xa[e] >> 16)),
                                 __uint_as_float(wa[e] & 0xFFFF0000u), acc);
        }
    }
    acc = group16_sum(acc);
    return (lane_value(acc, 0) + lane_value(acc, 16)) + (lane_value(acc, 32) + lane_value(acc, 48));
}

}  // namespace
}  // namespace tsg
