// decode.hip — decode MoE for gfx950: router GEMV + top-k, expert gate/up +
// activation (phase 1), down + routing-weighted combine (phase 2).
//
// Reference semantics: moe.metal:136-687, MoE.swift:259-644.
//
// Layout of the work (wave64):
//  * router: a 32-lane half-wave owns one expert row; lane l sums the 8-element
//    chunks c = l, l+32, ... in order with fma, then a xor butterfly over the 32
//    lanes (16, 8, 4, 2, 1). The oracle restates exactly this order, which is
//    what makes the selected experts bit-exact (and identical between decode
//    and the prompt router, which runs the same body per row).
//  * phase 1: 8 lanes own one (slot, f) row pair of gate and up. Lane j streams
//    16-byte chunks j, j+8, ... (one g32 group each) with all of its loads in
//    flight at once, converts nibbles to fp16 with the 0x6400 exponent trick
//    and accumulates with v_dot2_f32_f16 against x staged once per block in
//    LDS; fp32 per-group scale fma; 3-step xor reduction.
//  * phase 2: a wave owns 4 output rows x 8 slots x 2 half-rows; the 8 slot
//    values of a row are combined in slot order in one lane, as the reference
//    does (moe.metal:678-686).
#include "tsg_internal.hpp"

namespace tsg {
namespace {

// ------------------------------------------------------------ blob lookup

// Where each routed slot's expert blob lives: either explicit pointers (the
// reference's argument buffer of 8 MTLBuffers) or base + expert_id * stride
// with the ids read on the device.
struct BlobSource {
    const uint8_t* ptrs[kTopK];
    const uint8_t* base;
    uint64_t stride;
    const uint32_t* indices;      // device, top_k ids (resident mode)
    const uint32_t* active_slots; // device, subset mode
    uint32_t active_count;
    uint32_t resident;            // 0: ptrs, 1: base + indices[slot] * stride
};

__device__ __forceinline__ const uint8_t* blob_for(const BlobSource& src, uint32_t slot) {
    if (src.resident) return src.base + (uint64_t)src.indices[slot] * src.stride;
    return src.ptrs[slot];
}

// ----------------------------------------------------------------- router

// Sum of one expert row against x*es in the canonical order (see file
// comment). `lane` is 0..31 within the half-wave; all 32 lanes return the sum.
__device__ __forceinline__ float router_row_dot(const uint16_t* __restrict__ w_row,
                                                const uint16_t* __restrict__ x,
                                                const uint16_t* __restrict__ es,
                                                uint32_t d, uint32_t lane) {
    const uint32_t nchunks = d / 8u;
    float acc = 0.0f;
    for (uint32_t c = lane; c < nchunks; c += 32u) {
        const uint4 wv = *reinterpret_cast<const uint4*>(w_row + c * 8u);
        const uint4 xv = *reinterpret_cast<const uint4*>(x + c * 8u);
        const uint4 ev = *reinterpret_cast<const uint4*>(es + c * 8u);
        const uint32_t wa[4] = {wv.x, wv.y, wv.z, wv.w};
        const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
        const uint32_t ea[4] = {ev.x, ev.y, ev.z, ev.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float x0 = f16_to_f32((uint16_t)(xa[k] & 0xFFFFu));
            const float x1 = f16_to_f32((uint16_t)(xa[k] >> 16));
            const float e0 = bf16_to_f32((uint16_t)(ea[k] & 0xFFFFu));
            const float e1 = bf16_to_f32((uint16_t)(ea[k] >> 16));
            const float w0 = bf16_to_f32((uint16_t)(wa[k] & 0xFFFFu));
            const float w1 = bf16_to_f32((uint16_t)(wa[k] >> 16));
            acc = __builtin_fmaf(w0, x0 * e0, acc);
            acc = __builtin_fmaf(w1, x1 * e1, acc);
        }
    }
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) acc += shfl_xor(acc, off);
    return acc;
}

// Wave-wide top-k over `ne` logits with the reference's rule
// (moe.metal:281-329): descending score, ties to the lower index, -inf and NaN
// never enter; unfilled slots keep (0, -inf). Softmax over the k with the
// per-expert gain, rounded to fp16. Runs on one full wave.
__device__ void wave_topk_softmax(const float* logits, uint32_t ne, uint32_t top_k,
                                  const uint16_t* __restrict__ per_expert_scale,
                                  uint32_t* __restrict__ out_idx,
                                  uint16_t* __restrict__ out_w) {
    const uint32_t lane = threadIdx.x & 63u;
    // up to kMaxExperts / 64 = 4 candidates per lane: expert lane + 64 * j
    float v[4];
    bool eligible[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        float s = e < ne ? logits[e] : -INFINITY;
        v[j] = s;
        eligible[j] = e < ne && s == s && s != -INFINITY;
    }
    float top_s[kTopK];
    uint32_t top_i[kTopK];
    for (uint32_t r = 0; r < top_k; ++r) {
        float best = -INFINITY;
        uint32_t best_i = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = lane + 64u * j;
            if (eligible[j] && (best_i == 0xFFFFFFFFu || v[j] > best ||
                                (v[j] == best && e < best_i))) {
                best = v[j];
                best_i = e;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = shfl_xor(best, off);
            const uint32_t oi = shfl_xor(best_i, off);
            const bool take = oi != 0xFFFFFFFFu &&
                              (best_i == 0xFFFFFFFFu || ob > best || (ob == best && oi < best_i));
            if (take) { best = ob; best_i = oi; }
        }
        if (best_i == 0xFFFFFFFFu) {
            top_s[r] = -INFINITY;
            top_i[r] = 0u;
        } else {
            top_s[r] = best;
            top_i[r] = best_i;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (lane + 64u * j == best_i) eligible[j] = false;
        }
    }
    if (lane == 0) {
        const float max_s = top_s[0];
        float exps[kTopK];
        float sum_exp = 0.0f;
        for (uint32_t r = 0; r < top_k; ++r) {
            exps[r] = expf(top_s[r] - max_s);
            sum_exp += exps[r];
        }
        for (uint32_t r = 0; r < top_k; ++r) {
            const float weight = exps[r] / sum_exp;
            out_idx[r] = top_i[r];
            out_w[r] = f32_to_f16(weight * bf16_to_f32(per_expert_scale[top_i[r]]));
        }
    }
}

// grid (ceil(ne / 8), rows), block 256: half-wave h of wave w owns expert
// blockIdx.x * 8 + w * 2 + h. With SELECT, the last block to finish a row
// (completion counter) runs the top-k for it and resets the counter.
template <bool SELECT>
__global__ __launch_bounds__(256) void router_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ hidden, uint32_t hidden_stride,
    const uint16_t* __restrict__ es, const uint16_t* __restrict__ pes,
    float* __restrict__ logits, uint32_t logits_stride, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w, uint32_t ne, uint32_t d,
    uint32_t top_k) {
    const uint32_t row = blockIdx.y;
    const uint32_t lane32 = threadIdx.x & 31u;
    const uint32_t e = blockIdx.x * 8u + (threadIdx.x >> 5);
    const uint16_t* x = hidden + (uint64_t)row * hidden_stride;
    float* row_logits = logits + (uint64_t)row * logits_stride;
    if (e < ne) {
        const float s = router_row_dot(w + (uint64_t)e * d, x, es, d, lane32);
        if (lane32 == 0) row_logits[e] = s;
    }
    if constexpr (SELECT) {
        __shared__ uint32_t is_last;
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t done = atomicAdd(&counters[row], 1u);
            is_last = (done == gridDim.x - 1u) ? 1u : 0u;
        }
        __syncthreads();
        if (is_last) {
            __threadfence();
            if (threadIdx.x < 64u) {
                wave_topk_softmax(row_logits, ne, top_k, pes, out_idx + (uint64_t)row * top_k,
                                  out_w + (uint64_t)row * top_k);
            }
            if (threadIdx.x == 0) atomicExch(&counters[row], 0u);
        }
    }
}

// ---------------------------------------------------------------- phase 1

constexpr int kP1Batch = 12;  // chunks per lane in flight per matrix

// grid ceil(rows / 16), block 128: 16 (slot, f) row pairs per block, 8 lanes
// each. rows = top_k * F, or active_count * F for the subset form.
template <int G, bool SYM, int ACT, bool SUBSET>
__global__ __launch_bounds__(128) void phase1_kernel(BlobSource src, tsg_expert_offsets o,
                                                     const uint16_t* __restrict__ x,
                                                     uint16_t* __restrict__ acts, uint32_t d,
                                                     uint32_t f, uint32_t top_k) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + d * 2u);
    stage_x<SYM>(x, d, xs, xsum);
    __syncthreads();

    const uint32_t rows = (SUBSET ? src.active_count : top_k) * f;
    const uint32_t rowg = blockIdx.x * 16u + (threadIdx.x >> 3);
    const uint32_t j = threadIdx.x & 7u;
    if (rowg >= rows) return;
    uint32_t slot = rowg / f;
    const uint32_t fr = rowg - slot * f;
    if constexpr (SUBSET) {
        slot = src.active_slots[slot];
        if (slot >= top_k) return;
    }
    const uint8_t* blob = blob_for(src, slot);
    const uint32_t row_bytes = d / 2u;
    const uint32_t ngroups = d / G;
    const uint8_t* gw = blob + o.gate_w + (uint64_t)fr * row_bytes;
    const uint8_t* uw = blob + o.up_w + (uint64_t)fr * row_bytes;
    const uint16_t* gs = reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (uint64_t)fr * ngroups;
    const uint16_t* us = reinterpret_cast<const uint16_t*>(blob + o.up_s) + (uint64_t)fr * ngroups;
    const uint16_t* gb = reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (uint64_t)fr * ngroups;
    const uint16_t* ub = reinterpret_cast<const uint16_t*>(blob + o.up_b) + (uint64_t)fr * ngroups;

    const uint32_t nchunks = d / 32u;
    const h2_t bias = SYM ? h2_t{(_Float16)1032.0f, (_Float16)1032.0f}
                          : h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
    float g_acc = 0.0f, u_acc = 0.0f;
    for (uint32_t base = 0; base < nchunks; base += 8u * kP1Batch) {
        uint4 gv[kP1Batch], uv[kP1Batch];
        uint16_t gsv[kP1Batch], usv[kP1Batch];
#pragma unroll
        for (int i = 0; i < kP1Batch; ++i) {
            const uint32_t c = base + j + 8u * i;
            if (c < nchunks) {
                gv[i] = load16_nt(reinterpret_cast<const uint4*>(gw) + c);
                uv[i] = load16_nt(reinterpret_cast<const uint4*>(uw) + c);
                gsv[i] = gs[c * 32u / G];
                usv[i] = us[c * 32u / G];
            }
        }
#pragma unroll
        for (int i = 0; i < kP1Batch; ++i) {
            const uint32_t c = base + j + 8u * i;
            if (c < nchunks) {
                const h2_t* xp = reinterpret_cast<const h2_t*>(xs + c * 32u);
                const float gd = chunk_dot(gv[i], xp, bias);
                const float ud = chunk_dot(uv[i], xp, bias);
                const float gsc = bf16_to_f32(gsv[i]);
                const float usc = bf16_to_f32(usv[i]);
                g_acc = __builtin_fmaf(gsc, gd, g_acc);
                u_acc = __builtin_fmaf(usc, ud, u_acc);
                if constexpr (!SYM) {
                    const uint32_t g = c * 32u / G;
                    g_acc = __builtin_fmaf(bf16_to_f32(gb[g]), xsum[c], g_acc);
                    u_acc = __builtin_fmaf(bf16_to_f32(ub[g]), xsum[c], u_acc);
                }
            }
        }
    }
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
        g_acc += shfl_xor(g_acc, off);
        u_acc += shfl_xor(u_acc, off);
    }
    if (j == 0) acts[slot * f + fr] = f32_to_f16(gate_activation<ACT>(g_acc) * u_acc);
}

// ---------------------------------------------------------------- phase 2

constexpr int kP2Batch = 12;

// grid ceil(d / 16), block 256: wave w owns rows blockIdx.x * 16 + w * 4 .. +3;
// lane = row_in_wave * 16 + slot * 2 + half.
template <int G, bool SYM>
__global__ __launch_bounds__(256) void phase2_kernel(BlobSource src, tsg_expert_offsets o,
                                                     const uint16_t* __restrict__ acts,
                                                     const uint16_t* __restrict__ routing_w,
                                                     const uint16_t* __restrict__ residual,
                                                     uint16_t* __restrict__ y, uint32_t d,
                                                     uint32_t f) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);              // 8 * f
    float* asum = reinterpret_cast<float*>(smem + kTopK * f * 2u); // 8 * f / 32
    for (uint32_t s = 0; s < kTopK; ++s) {
        // stage_x works on threadIdx-strided blocks; do each slot in turn
        const uint16_t* a = acts + s * f;
        for (uint32_t b = threadIdx.x; b < f / 8u; b += blockDim.x) {
            const uint4 v = *reinterpret_cast<const uint4*>(a + b * 8u);
            uint4 ov;
            ov.x = (v.x & 0xFFFFu) | (v.z << 16);
            ov.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
            ov.z = (v.y & 0xFFFFu) | (v.w << 16);
            ov.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
            *reinterpret_cast<uint4*>(as + s * f + b * 8u) = ov;
        }
        if constexpr (!SYM) {
            for (uint32_t c = threadIdx.x; c < f / 32u; c += blockDim.x) {
                float sum = 0.0f;
                for (uint32_t k = 0; k < 32u; ++k) sum += f16_to_f32(a[c * 32u + k]);
                asum[s * (f / 32u) + c] = sum;
            }
        }
    }
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t rl = lane >> 4;
    const uint32_t slot = (lane >> 1) & 7u;
    const uint32_t half = lane & 1u;
    const uint32_t row = blockIdx.x * 16u + wave * 4u + rl;
    const bool live = row < d;
    const uint8_t* blob = blob_for(src, slot);
    const uint32_t row_bytes = f / 2u;
    const uint32_t ngroups = f / G;
    const uint32_t nchunks = f / 32u;
    const uint8_t* w = blob + o.down_w + (uint64_t)(live ? row : 0u) * row_bytes;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + o.down_s) + (uint64_t)(live ? row : 0u) * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + o.down_b) + (uint64_t)(live ? row : 0u) * ngroups;
    const h2_t bias = SYM ? h2_t{(_Float16)1032.0f, (_Float16)1032.0f}
                          : h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
    float acc = 0.0f;
    if (live) {
        for (uint32_t base = 0; base < nchunks; base += 2u * kP2Batch) {
            uint4 wv[kP2Batch];
            uint16_t sv[kP2Batch];
#pragma unroll
            for (int i = 0; i < kP2Batch; ++i) {
                const uint32_t c = base + half + 2u * i;
                if (c < nchunks) {
                    wv[i] = load16_nt(reinterpret_cast<const uint4*>(w) + c);
                    sv[i] = sc[c * 32u / G];
                }
            }
#pragma unroll
            for (int i = 0; i < kP2Batch; ++i) {
                const uint32_t c = base + half + 2u * i;
                if (c < nchunks) {
                    const h2_t* xp = reinterpret_cast<const h2_t*>(as + slot * f + c * 32u);
                    acc = __builtin_fmaf(bf16_to_f32(sv[i]), chunk_dot(wv[i], xp, bias), acc);
                    if constexpr (!SYM)
                        acc = __builtin_fmaf(bf16_to_f32(bi[c * 32u / G]),
                                             asum[slot * nchunks + c], acc);
                }
            }
        }
    }
    acc += shfl_xor(acc, 1);
    // slot values of row rl live in lanes rl*16 + 2s; combine in slot order
    float vals[kTopK];
#pragma unroll
    for (int s = 0; s < (int)kTopK; ++s) vals[s] = __shfl(acc, (int)(rl * 16u + 2u * s), 64);
    if ((lane & 15u) == 0 && live) {
        float out = f16_to_f32(residual[row]);
#pragma unroll
        for (int s = 0; s < (int)kTopK; ++s) {
            const float p = f16_to_f32(routing_w[s]) * vals[s];
            out = out + p;
        }
        y[row] = f32_to_f16(out);
    }
}

// ------------------------------------------------------------ host helpers

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

tsg_status check_moe(const tsg_moe* moe) {
    TSG_REQUIRE(moe && moe->ctx, TSG_ERR_INVALID_ARGUMENT, "moe is NULL");
    return TSG_OK;
}

tsg_status check_decode_shape(const tsg_ctx* ctx, uint32_t d, uint32_t f, uint32_t top_k) {
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT,
                "topK must be %u (MoE.maxStreamedExperts), got %u", kTopK, top_k);
    TSG_REQUIRE(d > 0 && f > 0, TSG_ERR_INVALID_ARGUMENT, "empty shape d=%u f=%u", d, f);
    TSG_REQUIRE(d % ctx->group_size == 0 && f % ctx->group_size == 0, TSG_ERR_INVALID_ARGUMENT,
                "d=%u and f=%u must be multiples of the affine group size %u", d, f,
                ctx->group_size);
    return TSG_OK;
}

tsg_status router_launch(tsg_moe* moe, hipStream_t stream, const uint16_t* w,
                         const uint16_t* hidden, uint32_t stride, const uint16_t* es,
                         const uint16_t* pes, uint32_t* out_idx, uint16_t* out_w,
                         float* logits_out, uint32_t rows, uint32_t ne, uint32_t d,
                         uint32_t top_k, bool select) {
    TSG_REQUIRE(ne > 0 && ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "numExperts %u not in 1..%u", ne, kMaxExperts);
    TSG_REQUIRE(d > 0 && d % 8 == 0, TSG_ERR_INVALID_ARGUMENT, "d=%u must be a multiple of 8", d);
    TSG_REQUIRE(stride % 8 == 0, TSG_ERR_ALIGNMENT, "hidden stride %u must be a multiple of 8",
                stride);
    TSG_REQUIRE(w && hidden && es, TSG_ERR_INVALID_ARGUMENT, "NULL router operand");
    TSG_REQUIRE(aligned16(w) && aligned16(hidden) && aligned16(es), TSG_ERR_ALIGNMENT,
                "router weights, hidden and effective_scale must be 16-byte aligned");
    tsg_ctx* ctx = moe->ctx;
    const dim3 grid((ne + 7) / 8, rows);
    if (select) {
        TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK,
                    top_k);
        TSG_REQUIRE(pes && out_idx && out_w, TSG_ERR_INVALID_ARGUMENT, "NULL router output");
        hipLaunchKernelGGL(router_kernel<true>, grid, dim3(256), 0, stream, w, hidden, stride, es,
                           pes, ctx->logits, kMaxExperts, ctx->counters, out_idx, out_w, ne, d,
                           top_k);
    } else {
        TSG_REQUIRE(logits_out, TSG_ERR_INVALID_ARGUMENT, "out_logits is NULL");
        hipLaunchKernelGGL(router_kernel<false>, grid, dim3(256), 0, stream, w, hidden, stride,
                           es, pes, logits_out, ne, ctx->counters, out_idx, out_w, ne, d, top_k);
    }
    return check_launch("router");
}

template <int G, bool SYM>
tsg_status launch_phase1(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                         const tsg_expert_offsets& o, const uint16_t* x, uint16_t* acts,
                         uint32_t d, uint32_t f, uint32_t top_k, bool subset) {
    const uint32_t rows = (subset ? src.active_count : top_k) * f;
    if (rows == 0) return TSG_OK;
    const dim3 grid((rows + 15) / 16);
    const size_t lds = d * 2u + (SYM ? 0u : (d / 32u) * 4u);
    if (moe->activation == TSG_ACT_SILU) {
        if (subset)
            hipLaunchKernelGGL((phase1_kernel<G, SYM, TSG_ACT_SILU, true>), grid, dim3(128), lds,
                               stream, src, o, x, acts, d, f, top_k);
        else
            hipLaunchKernelGGL((phase1_kernel<G, SYM, TSG_ACT_SILU, false>), grid, dim3(128), lds,
                               stream, src, o, x, acts, d, f, top_k);
    } else {
        if (subset)
            hipLaunchKernelGGL((phase1_kernel<G, SYM, TSG_ACT_GELU_TANH, true>), grid, dim3(128),
                               lds, stream, src, o, x, acts, d, f, top_k);
        else
            hipLaunchKernelGGL((phase1_kernel<G, SYM, TSG_ACT_GELU_TANH, false>), grid,
                               dim3(128), lds, stream, src, o, x, acts, d, f, top_k);
    }
    return check_launch("phase1");
}

tsg_status phase1_dispatch(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                           const tsg_expert_offsets& o, const uint16_t* x, uint16_t* acts,
                           uint32_t d, uint32_t f, uint32_t top_k, bool subset) {
    TSG_REQUIRE(x && acts, TSG_ERR_INVALID_ARGUMENT, "NULL x/acts");
    TSG_REQUIRE(aligned16(x), TSG_ERR_ALIGNMENT, "x must be 16-byte aligned");
    TSG_REQUIRE(d * 2u + (d / 32u) * 4u <= 160u * 1024u, TSG_ERR_UNSUPPORTED,
                "d=%u does not fit the LDS staging", d);
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32)
        return sym ? launch_phase1<32, true>(moe, stream, src, o, x, acts, d, f, top_k, subset)
                   : launch_phase1<32, false>(moe, stream, src, o, x, acts, d, f, top_k, subset);
    return sym ? launch_phase1<64, true>(moe, stream, src, o, x, acts, d, f, top_k, subset)
               : launch_phase1<64, false>(moe, stream, src, o, x, acts, d, f, top_k, subset);
}

tsg_status phase2_dispatch(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                           const tsg_expert_offsets& o, const uint16_t* acts,
                           const uint16_t* rw, const uint16_t* residual, uint16_t* y,
                           uint32_t d, uint32_t f) {
    TSG_REQUIRE(acts && rw && residual && y, TSG_ERR_INVALID_ARGUMENT, "NULL phase-2 operand");
    TSG_REQUIRE(aligned16(acts), TSG_ERR_ALIGNMENT, "acts must be 16-byte aligned");
    const size_t lds = kTopK * f * 2u + kTopK * (f / 32u) * 4u;
    TSG_REQUIRE(lds <= 160u * 1024u, TSG_ERR_UNSUPPORTED, "f=%u does not fit the LDS staging", f);
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const dim3 grid((d + 15) / 16);
    if (ctx->group_size == 32) {
        if (sym)
            hipLaunchKernelGGL((phase2_kernel<32, true>), grid, dim3(256), lds, stream, src, o,
                               acts, rw, residual, y, d, f);
        else
            hipLaunchKernelGGL((phase2_kernel<32, false>), grid, dim3(256), lds, stream, src, o,
                               acts, rw, residual, y, d, f);
    } else {
        if (sym)
            hipLaunchKernelGGL((phase2_kernel<64, true>), grid, dim3(256), lds, stream, src, o,
                               acts, rw, residual, y, d, f);
        else
            hipLaunchKernelGGL((phase2_kernel<64, false>), grid, dim3(256), lds, stream, src, o,
                               acts, rw, residual, y, d, f);
    }
    return check_launch("phase2");
}

tsg_status blobs_from_ptrs(const void* const* routed_blobs, const tsg_expert_offsets* offsets,
                           uint32_t top_k, BlobSource* src) {
    TSG_REQUIRE(routed_blobs && offsets, TSG_ERR_INVALID_ARGUMENT, "NULL routed blobs/offsets");
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK, top_k);
    *src = BlobSource{};
    for (uint32_t s = 0; s < top_k; ++s) {
        TSG_REQUIRE(routed_blobs[s], TSG_ERR_INVALID_ARGUMENT, "routed blob %u is NULL", s);
        src->ptrs[s] = static_cast<const uint8_t*>(routed_blobs[s]);
        TSG_REQUIRE(aligned16(src->ptrs[s]), TSG_ERR_ALIGNMENT, "routed blob %u must be 16-byte aligned", s);
    }
    const tsg_expert_offsets& o = *offsets;
    TSG_REQUIRE(o.gate_w % 16 == 0 && o.up_w % 16 == 0 && o.down_w % 16 == 0, TSG_ERR_ALIGNMENT,
                "weight offsets (%u, %u, %u) must be 16-byte aligned", o.gate_w, o.up_w, o.down_w);
    TSG_REQUIRE(o.gate_s % 2 == 0 && o.up_s % 2 == 0 && o.down_s % 2 == 0, TSG_ERR_ALIGNMENT,
                "scale offsets must be 2-byte aligned");
    return TSG_OK;
}

tsg_status blobs_from_layer(const tsg_layer* layer, const uint32_t* indices, BlobSource* src) {
    TSG_REQUIRE(layer && indices, TSG_ERR_INVALID_ARGUMENT, "NULL layer/indices");
    *src = BlobSource{};
    src->resident = 1;
    src->base = layer->base;
    src->stride = layer->expert_stride;
    src->indices = indices;
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

using namespace tsg;

// ------------------------------------------------------------------- ABI

extern "C" tsg_status tsg_moe_create(tsg_ctx* ctx, uint32_t bits, tsg_activation act,
                                     tsg_moe** out) {
    TSG_REQUIRE(ctx && out, TSG_ERR_INVALID_ARGUMENT, "ctx/out is NULL");
    *out = nullptr;
    TSG_REQUIRE(bits == 8 || bits == 16, TSG_ERR_INVALID_ARGUMENT,
                "Unsupported router weight bits: %u (expected 8 or 16)", bits);
    TSG_REQUIRE(bits == 16, TSG_ERR_UNSUPPORTED,
                "the INT8 affine router is not built; QAT checkpoints ship a BF16 router");
    TSG_REQUIRE(act == TSG_ACT_GELU_TANH || act == TSG_ACT_SILU, TSG_ERR_INVALID_ARGUMENT,
                "unknown gate activation %d", (int)act);
    tsg_moe* m = new tsg_moe();
    m->ctx = ctx;
    m->router_weight_bits = bits;
    m->activation = act;
    *out = m;
    return TSG_OK;
}

extern "C" void tsg_moe_destroy(tsg_moe* moe) { delete moe; }

extern "C" tsg_status tsg_moe_router_bf16(tsg_moe* moe, tsg_stream stream, const uint16_t* w,
                                          const uint16_t* hidden, const uint16_t* es,
                                          const uint16_t* pes, uint32_t* out_idx,
                                          uint16_t* out_w, uint32_t ne, uint32_t d,
                                          uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    return router_launch(moe, as_stream(stream), w, hidden, d, es, pes, out_idx, out_w, nullptr,
                         1, ne, d, top_k, true);
}

extern "C" tsg_status tsg_moe_router_bf16_rows(tsg_moe* moe, tsg_stream stream,
                                               const uint16_t* w, const uint16_t* hidden,
                                               uint32_t stride, const uint16_t* es,
                                               const uint16_t* pes, uint32_t* out_idx,
                                               uint16_t* out_w, uint32_t rows, uint32_t ne,
                                               uint32_t d, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK, top_k);
    TSG_REQUIRE(ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT, "numExperts %u > %u", ne, kMaxExperts);
    if (rows == 0 || rows > kMaxRouterRows)
        return fail(TSG_ERR_DECLINED, "rows router takes 1..%u rows, got %u", kMaxRouterRows,
                    rows);
    return router_launch(moe, as_stream(stream), w, hidden, stride, es, pes, out_idx, out_w,
                         nullptr, rows, ne, d, top_k, true);
}

extern "C" tsg_status tsg_moe_router_logits_bf16(tsg_moe* moe, tsg_stream stream,
                                                 const uint16_t* w, const uint16_t* hidden,
                                                 const uint16_t* es, float* out_logits,
                                                 uint32_t ne, uint32_t d) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    return router_launch(moe, as_stream(stream), w, hidden, d, es, nullptr, nullptr, nullptr,
                         out_logits, 1, ne, d, kTopK, false);
}

extern "C" tsg_status tsg_moe_phase1(tsg_moe* moe, tsg_stream stream,
                                     const void* const* routed_blobs,
                                     const tsg_expert_offsets* offsets, const uint16_t* x,
                                     uint16_t* acts, uint32_t d, uint32_t f, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    BlobSource src;
    if ((st = blobs_from_ptrs(routed_blobs, offsets, top_k, &src))) return st;
    return phase1_dispatch(moe, as_stream(stream), src, *offsets, x, acts, d, f, top_k, false);
}

extern "C" tsg_status tsg_moe_phase1_subset(tsg_moe* moe, tsg_stream stream,
                                            const void* const* routed_blobs,
                                            const tsg_expert_offsets* offsets,
                                            const uint16_t* x, uint16_t* acts,
                                            const uint32_t* active_slots, uint32_t active_count,
                                            uint32_t d, uint32_t f, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if (active_count == 0) return TSG_OK;  // MoE.swift:578: nothing to encode
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    TSG_REQUIRE(active_slots, TSG_ERR_INVALID_ARGUMENT, "active_slots is NULL");
    TSG_REQUIRE(active_count <= top_k, TSG_ERR_INVALID_ARGUMENT,
                "active_count %u exceeds topK %u", active_count, top_k);
    BlobSource src;
    if ((st = blobs_from_ptrs(routed_blobs, offsets, top_k, &src))) return st;
    src.active_slots = active_slots;
    src.active_count = active_count;
    return phase1_dispatch(moe, as_stream(stream), src, *offsets, x, acts, d, f, top_k, true);
}

extern "C" tsg_status tsg_moe_phase2(tsg_moe* moe, tsg_stream stream,
                                     const void* const* routed_blobs,
                                     const tsg_expert_offsets* offsets, const uint16_t* acts,
                                     const uint16_t* rw, const uint16_t* residual, uint16_t* y,
                                     uint32_t d, uint32_t f, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    BlobSource src;
    if ((st = blobs_from_ptrs(routed_blobs, offsets, top_k, &src))) return st;
    return phase2_dispatch(moe, as_stream(stream), src, *offsets, acts, rw, residual, y, d, f);
}

extern "C" tsg_status tsg_moe_phase1_resident(tsg_moe* moe, tsg_stream stream,
                                              const tsg_layer* layer, const uint32_t* indices,
                                              const uint16_t* x, uint16_t* acts, uint32_t d,
                                              uint32_t f, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    BlobSource src;
    if ((st = blobs_from_layer(layer, indices, &src))) return st;
    return phase1_dispatch(moe, as_stream(stream), src, layer->offsets, x, acts, d, f, top_k,
                           false);
}

extern "C" tsg_status tsg_moe_phase2_resident(tsg_moe* moe, tsg_stream stream,
                                              const tsg_layer* layer, const uint32_t* indices,
                                              const uint16_t* acts, const uint16_t* rw,
                                              const uint16_t* residual, uint16_t* y, uint32_t d,
                                              uint32_t f, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    BlobSource src;
    if ((st = blobs_from_layer(layer, indices, &src))) return st;
    return phase2_dispatch(moe, as_stream(stream), src, layer->offsets, acts, rw, residual, y, d,
                           f);
}

extern "C" tsg_status tsg_moe_decode_layer(tsg_moe* moe, tsg_stream stream,
                                           const tsg_layer* layer, const uint16_t* router_w,
                                           const uint16_t* router_hidden, const uint16_t* es,
                                           const uint16_t* pes, const uint16_t* x,
                                           const uint16_t* residual, uint16_t* y,
                                           uint32_t* out_idx, uint16_t* out_w,
                                           uint16_t* acts, uint32_t ne, uint32_t d, uint32_t f,
                                           uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    TSG_REQUIRE(layer, TSG_ERR_INVALID_ARGUMENT, "layer is NULL");
    TSG_REQUIRE(ne <= layer->num_experts, TSG_ERR_INVALID_ARGUMENT,
                "router has %u experts but the layer holds %u", ne, layer->num_experts);
    hipStream_t s = as_stream(stream);
    if ((st = router_launch(moe, s, router_w, router_hidden, d, es, pes, out_idx, out_w, nullptr,
                            1, ne, d, top_k, true)))
        return st;
    BlobSource src;
    if ((st = blobs_from_layer(layer, out_idx, &src))) return st;
    if ((st = phase1_dispatch(moe, s, src, layer->offsets, x, acts, d, f, top_k, false)))
        return st;
    return phase2_dispatch(moe, s, src, layer->offsets, acts, out_w, residual, y, d, f);
}

// Prompt router: the decode router body per row (bit-identical per row).
extern "C" tsg_status tsg_prefill_router_bf16(tsg_moe* moe, tsg_stream stream,
                                              const uint16_t* w, const uint16_t* hidden,
                                              uint32_t stride, const uint16_t* es,
                                              const uint16_t* pes, uint32_t* out_idx,
                                              uint16_t* out_w, uint32_t query_count,
                                              uint32_t ne, uint32_t d, uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    TSG_REQUIRE(query_count > 0, TSG_ERR_INVALID_ARGUMENT, "queryCount must be positive");
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_UNSUPPORTED, "topK %u: the prompt router is built for 8",
                top_k);
    hipStream_t s = as_stream(stream);
    // Rows go through in chunks of kMaxRouterRows so the context's logit
    // staging and counters are reused; launches are stream-ordered.
    for (uint32_t r0 = 0; r0 < query_count; r0 += kMaxRouterRows) {
        const uint32_t rows = (query_count - r0 < kMaxRouterRows) ? query_count - r0 : kMaxRouterRows;
        if ((st = router_launch(moe, s, w, hidden + (uint64_t)r0 * stride, stride, es, pes,
                                out_idx + (uint64_t)r0 * top_k, out_w + (uint64_t)r0 * top_k,
                                nullptr, rows, ne, d, top_k, true)))
            return st;
    }
    return TSG_OK;
}
