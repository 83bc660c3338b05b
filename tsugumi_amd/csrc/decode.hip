// decode.hip — decode MoE for gfx950: router GEMV + top-k, expert gate/up +
// activation (phase 1), down + routing-weighted combine (phase 2).
//
// Reference semantics: moe.metal:136-687, MoE.swift:259-644.
//
// Layout of the work (wave64):
//  * router: a wave owns one expert row; lane l sums the 8-element chunks
//    c = l, l+64, ... in order with fma, then a xor butterfly over the 64
//    lanes (32, 16, 8, 4, 2, 1). The oracle restates exactly this order, which is
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
#include "gemv_lane.hpp"

namespace tsg {
namespace {

// ------------------------------------------------------------ blob lookup

// Where each routed slot's expert blob lives: explicit pointers (the
// reference's argument buffer of 8 MTLBuffers), or base + expert_id * stride
// with the ids read from device memory (written by an earlier launch) or from
// LDS (the one-launch layer, which routes in-kernel).
struct BlobSource {
    const uint8_t* ptrs[kTopK];
    const uint8_t* base;
    uint64_t stride;
    const uint32_t* indices;      // device, top_k ids (resident mode)
    const uint32_t* active_slots; // device, subset mode
    uint32_t active_count;
    uint32_t resident;            // 0: ptrs, 1: base + indices[slot] * stride

    __device__ __forceinline__ const uint8_t* blob(uint32_t slot) const {
        if (resident) return base + (uint64_t)indices[slot] * stride;
        return ptrs[slot];
    }
};

// The one-launch layer's lookup: expert ids chosen in-kernel, held in LDS.
struct LdsBlobs {
    const uint8_t* base;
    uint64_t stride;
    const uint32_t* ids;  // LDS

    __device__ __forceinline__ const uint8_t* blob(uint32_t slot) const {
        return base + (uint64_t)ids[slot] * stride;
    }
};

// ----------------------------------------------------------------- router

// Wave-wide top-8 over `ne` logits with the reference's rule
// (moe.metal:281-329): descending score, ties to the lower index, -inf and NaN
// never enter; unfilled slots keep (0, -inf). Softmax over the 8 with the
// per-expert gain, rounded to fp16. Runs on one full wave; lane l holds the
// logits of experts l + 64 j (j < 4). Every lane returns the same result.
//
// Scores become order-preserving 32-bit keys (0 marks "not eligible"; -0 is
// keyed as +0, the two compare equal). Each round takes the wave-wide max key
// on DPP moves inside 16-lane rows and permlane swaps across rows, then the
// lowest expert holding it from per-j ballots (experts l + 64 j ascend with j
// and, within j, with the lane).
struct TopK {
    uint32_t idx[kTopK];
    uint16_t w[kTopK];
};

__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __float_as_uint(v + 0.0f);  // -0 -> +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float order_key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t k) {
    return __builtin_amdgcn_update_dpp(0u, k, CTRL, 0xF, 0xF, false);
}

// Of the two results of a permlane swap each lane finds its partner's value
// in one and its own in the other, so the max of both is the pairwise max
// whichever holds which.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
    k = max(k, dpp_u32<0xB1>(k));   // quad_perm [1,0,3,2]
    k = max(k, dpp_u32<0x4E>(k));   // quad_perm [2,3,0,1]
    k = max(k, dpp_u32<0x141>(k));  // row_half_mirror
    k = max(k, dpp_u32<0x140>(k));  // row_mirror
    const auto a = __builtin_amdgcn_permlane16_swap(k, k, false, false);
    k = max(k, max((uint32_t)a[0], (uint32_t)a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(k, k, false, false);
    k = max(k, max((uint32_t)b[0], (uint32_t)b[1]));
    return k;
}

// Lane l's per-expert gains (bf16 bits) of experts l + 64 j, loaded early so
// their latency is off the top-k's critical path.
__device__ __forceinline__ void load_expert_gains(const uint16_t* __restrict__ per_expert_scale,
                                                  uint32_t ne, uint32_t (&pes)[4]) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        pes[j] = e < ne ? per_expert_scale[e] : 0u;
    }
}

__device__ __forceinline__ TopK wave_topk_softmax_regs(const float (&logit)[4], uint32_t ne,
                                                      const uint32_t (&pes)[4]) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        const float s = logit[j];
        const bool eligible = e < ne && s == s && s != -INFINITY;
        key[j] = eligible ? order_key(s) : 0u;
    }
    TopK t;
    float top_s[kTopK], gain[kTopK];
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r) {
        const uint32_t m = wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
        if (m == 0u) {  // unfilled: (expert 0, -inf)
            top_s[r] = -INFINITY;
            t.idx[r] = 0u;
            gain[r] = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane(pes[0], 0));
        } else {
            const uint64_t b0 = __ballot(key[0] == m), b1 = __ballot(key[1] == m);
            const uint64_t b2 = __ballot(key[2] == m), b3 = __ballot(key[3] == m);
            const uint32_t jj = b0 ? 0u : b1 ? 1u : b2 ? 2u : 3u;
            const uint64_t bj = b0 ? b0 : b1 ? b1 : b2 ? b2 : b3;
            const uint32_t l = (uint32_t)__builtin_ctzll(bj);
            top_s[r] = order_key_value(m);
            t.idx[r] = 64u * jj + l;
            const uint32_t mine = jj == 0 ? pes[0] : jj == 1 ? pes[1] : jj == 2 ? pes[2] : pes[3];
            gain[r] = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane(mine, l));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((uint32_t)j == jj && lane == l) key[j] = 0u;
        }
    }
    // softmax: lane r < 8 owns slot r's exponential; the sum runs in slot order
    const uint32_t r_l = lane & (kTopK - 1u);
    float my_s = top_s[0], my_gain = gain[0];
#pragma unroll
    for (uint32_t r = 1; r < kTopK; ++r)
        if (r_l == r) { my_s = top_s[r]; my_gain = gain[r]; }
    const float my_exp = expf(my_s - top_s[0]);
    float sum_exp = lane_value(my_exp, 0);
#pragma unroll
    for (uint32_t r = 1; r < kTopK; ++r) sum_exp += lane_value(my_exp, r);
    const uint32_t my_w = f32_to_f16(my_exp / sum_exp * my_gain);
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r) t.w[r] = (uint16_t)__builtin_amdgcn_readlane(my_w, r);
    return t;
}

// The same over logits in memory written earlier in this launch by other
// blocks (read with agent-coherent loads); lane 0 stores the result.
__device__ void wave_topk_softmax(const float* logits, uint32_t ne, const uint32_t (&pes)[4],
                                  uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w) {
    const uint32_t lane = threadIdx.x & 63u;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        v[j] = e < ne ? __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(logits) + e))
                      : -INFINITY;
    }
    const TopK t = wave_topk_softmax_regs(v, ne, pes);
    if (lane == 0) {
#pragma unroll
        for (uint32_t r = 0; r < kTopK; ++r) {
            out_idx[r] = t.idx[r];
            out_w[r] = t.w[r];
        }
    }
}

constexpr uint32_t kRouterRows = 16;      // rows sharing one weight read per wave
constexpr uint32_t kRouterWaves = 4;      // experts per block
constexpr int kRouterChunks = 8;          // 8-element chunks per lane: d <= 4096

// The canonical router sum over one row held in registers: lane l owns chunks
// l, l+64, ... (8 elements each, summed in order with fma(w, x*es, acc)), then
// a xor butterfly 32, 16, 8, 4, 2, 1; every lane returns the full sum.
__device__ __forceinline__ float router_chunks_dot(const uint4* wv, const uint4* xv,
                                                   const uint4* ev, uint32_t nchunks,
                                                   uint32_t lane) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouterChunks; ++i) {
        if (lane + 64u * i >= nchunks) break;  // lanes past the row end add nothing
        const uint32_t wa[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
        const uint32_t xa[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const uint32_t ea[4] = {ev[i].x, ev[i].y, ev[i].z, ev[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float x0 = f16_to_f32((uint16_t)(xa[k] & 0xFFFFu));
            const float x1 = f16_to_f32((uint16_t)(xa[k] >> 16));
            const float e0 = __uint_as_float(ea[k] << 16);
            const float e1 = __uint_as_float(ea[k] & 0xFFFF0000u);
            const float w0 = __uint_as_float(wa[k] << 16);
            const float w1 = __uint_as_float(wa[k] & 0xFFFF0000u);
            acc = __builtin_fmaf(w0, x0 * e0, acc);
            acc = __builtin_fmaf(w1, x1 * e1, acc);
        }
    }
    // 16-lane row sums on DPP, then the four rows in the order (0 + 1) + (2 + 3)
    acc = group16_sum(acc);
    return (lane_value(acc, 0) + lane_value(acc, 16)) + (lane_value(acc, 32) + lane_value(acc, 48));
}

// One router row (loads + canonical sum) on one wave.
__device__ __forceinline__ float router_dot(const uint16_t* __restrict__ w_row,
                                            const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ es, uint32_t d,
                                            uint32_t lane) {
    const uint32_t nchunks = d / 8u;
    uint4 wv[kRouterChunks], ev[kRouterChunks], xv[kRouterChunks];
#pragma unroll
    for (int i = 0; i < kRouterChunks; ++i) {
        const uint32_t cc = min(lane + 64u * i, nchunks - 1u);
        wv[i] = *reinterpret_cast<const uint4*>(w_row + cc * 8u);
        ev[i] = *reinterpret_cast<const uint4*>(es + cc * 8u);
        xv[i] = *reinterpret_cast<const uint4*>(x + cc * 8u);
    }
    return router_chunks_dot(wv, xv, ev, nchunks, lane);
}

// One expert row against up to kRouterRows activation rows in the canonical
// order: lane l sums chunks l, l+64, ... (elements in order, acc = fma(w,
// x*es, acc)); each 16-lane row then sums as group16_sum does (pairs, pairs of
// pairs, mirrored quads, mirrored 8s) and the four row sums add as
// (r0 + r1) + (r2 + r3). Every lane ends with the full sum. Loads for all chunks are issued before
// any arithmetic; out-of-range chunks load a clamped address and contribute
// nothing.
template <bool SELECT>
__global__ __launch_bounds__(256) void router_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ hidden, uint32_t hidden_stride,
    const uint16_t* __restrict__ es, const uint16_t* __restrict__ pes,
    float* __restrict__ logits, uint32_t logits_stride, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w, uint32_t ne, uint32_t d,
    uint32_t rows, uint32_t top_k) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t e = blockIdx.x * kRouterWaves + wave;
    const uint32_t r0 = blockIdx.y * kRouterRows;
    const uint32_t nr = min(kRouterRows, rows - r0);
    const uint32_t nchunks = d / 8u;
    uint32_t gains[4] = {0u, 0u, 0u, 0u};
    if constexpr (SELECT) load_expert_gains(pes, ne, gains);
    if (e < ne) {
        const uint16_t* wr = w + (uint64_t)e * d;
        uint4 wv[kRouterChunks], ev[kRouterChunks], xv[kRouterChunks];
#pragma unroll
        for (int i = 0; i < kRouterChunks; ++i) {
            const uint32_t cc = min(lane + 64u * i, nchunks - 1u);
            wv[i] = *reinterpret_cast<const uint4*>(wr + cc * 8u);
            ev[i] = *reinterpret_cast<const uint4*>(es + cc * 8u);
            xv[i] = *reinterpret_cast<const uint4*>(hidden + (uint64_t)r0 * hidden_stride + cc * 8u);
        }
        for (uint32_t r = 0; r < nr; ++r) {
            // next row's activations go out before this row's arithmetic
            uint4 xn[kRouterChunks];
            const uint32_t rn = (r + 1 < nr) ? r + 1 : r;
            const uint16_t* xnext = hidden + (uint64_t)(r0 + rn) * hidden_stride;
#pragma unroll
            for (int i = 0; i < kRouterChunks; ++i) {
                const uint32_t cc = min(lane + 64u * i, nchunks - 1u);
                xn[i] = *reinterpret_cast<const uint4*>(xnext + cc * 8u);
            }
            const float acc = router_chunks_dot(wv, xv, ev, nchunks, lane);
#pragma unroll
            for (int i = 0; i < kRouterChunks; ++i) xv[i] = xn[i];
            if (lane == 0)
                st_coherent(reinterpret_cast<uint32_t*>(logits) + (uint64_t)(r0 + r) * logits_stride + e,
                            __float_as_uint(acc));
        }
    }
    if constexpr (SELECT) {
        // logits travel by agent-coherent stores/loads: completing this
        // block's stores before it counts itself is all the last block needs
        __shared__ uint32_t is_last;
        wait_vector_memory();
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t done = atomicAdd(&counters[blockIdx.y], 1u);
            is_last = (done == gridDim.x - 1u) ? 1u : 0u;
        }
        __syncthreads();
        if (is_last) {
            for (uint32_t r = wave; r < nr; r += kRouterWaves)
                wave_topk_softmax(logits + (uint64_t)(r0 + r) * logits_stride, ne, gains,
                                  out_idx + (uint64_t)(r0 + r) * kTopK,
                                  out_w + (uint64_t)(r0 + r) * kTopK);
            if (threadIdx.x == 0) atomicExch(&counters[blockIdx.y], 0u);
        }
    }
}

// ------------------------------------------------------- phase geometry

// Phase 1: a block owns `pairs` (slot, f) row pairs, 32 lanes each (16 on the
// gate row, 16 on the up row). Phase 2: a block owns `rows` output rows, one
// wave each: 8 slots x 8 lanes. Blocks are sized so the grid is about one
// block per CU (Gemma: 5632 pairs = 256 x 22, 2816 rows = 256 x 11).
struct DecodeGeometry {
    uint32_t pairs_per_block;  // even
    uint32_t p1_blocks;
    uint32_t rows_per_block;
    uint32_t p2_blocks;
    uint32_t threads;          // max(32 * pairs, 64 * rows)
};

inline DecodeGeometry decode_geometry(uint32_t d, uint32_t f, uint32_t n_pairs_total,
                                      uint32_t target_blocks) {
    DecodeGeometry g{};
    uint32_t p = (n_pairs_total + target_blocks - 1) / target_blocks;
    p = p < 2u ? 2u : (p > 32u ? 32u : p);
    p += p & 1u;
    g.pairs_per_block = p;
    g.p1_blocks = (n_pairs_total + p - 1) / p;
    uint32_t q = (d + target_blocks - 1) / target_blocks;
    q = q < 1u ? 1u : (q > 16u ? 16u : q);
    g.rows_per_block = q;
    g.p2_blocks = (d + q - 1) / q;
    const uint32_t t1 = 32u * p, t2 = 64u * q;
    g.threads = t1 > t2 ? t1 : t2;
    (void)f;
    return g;
}

// ------------------------------------------------------ phase 1 / phase 2 bodies

// Addresses of one lane's gate or up row: 32 lanes per (slot, f) pair, lanes
// 0..15 on the gate row, 16..31 on the up row. A lane whose pair is not live
// (past the end, or a rejected subset slot) reads row 0 of slot 0 and stores
// nothing.
struct GULane {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint32_t slot, fr;
    bool live;
};

template <typename Src>
__device__ __forceinline__ GULane gu_lane(const Src& src, const tsg_expert_offsets& o,
                                          uint32_t d, uint32_t g, uint32_t slot, uint32_t fr,
                                          bool live) {
    const bool is_up = (threadIdx.x >> 4) & 1u;
    if (!live) { slot = 0u; fr = 0u; }
    const uint8_t* blob = src.blob(slot);
    const uint32_t ngroups = d / g;
    GULane l;
    l.w = blob + (is_up ? o.up_w : o.gate_w) + (uint64_t)fr * (d / 2u);
    l.s = reinterpret_cast<const uint16_t*>(blob + (is_up ? o.up_s : o.gate_s)) + (uint64_t)fr * ngroups;
    l.b = reinterpret_cast<const uint16_t*>(blob + (is_up ? o.up_b : o.gate_b)) + (uint64_t)fr * ngroups;
    l.slot = slot;
    l.fr = fr;
    l.live = live;
    return l;
}

// Gate/up dot products of one pair (x staged in LDS) and the activation
// half(act(gate) * up), the pair's entry acts[slot * f + fr]. Returns true on
// the one lane that holds it (in `out`). `bt` holds the first batch.
template <int G, bool SYM, int ACT>
__device__ __forceinline__ bool phase1_compute(const GULane& l, ChunkBatch<kGUBatch>& bt,
                                               const uint16_t* xs, const float* xsum,
                                               uint32_t d, uint16_t& out) {
    const uint32_t j = threadIdx.x & 15u;
    const bool is_up = (threadIdx.x >> 4) & 1u;
    const uint32_t nchunks = d / 32u;
    float acc[1] = {0.0f};
    for (uint32_t base = 0; base < nchunks; base += kGULanes * kGUBatch) {
        if (base) load_batch<G, SYM, kGUBatch, kGULanes>(l.w, l.s, l.b, base, j, nchunks, bt);
        compute_batch<G, SYM, kGUBatch, kGULanes, 1>(bt, base, j, nchunks, xs, 0u, xsum, 1u, acc);
    }
    acc[0] = group16_sum(acc[0]);
    const float up = shfl_xor(acc[0], 16);  // gate lanes receive the up sum
    out = f32_to_f16(gate_activation<ACT>(acc[0]) * up);
    return l.live && !is_up && j == 0;
}

// Down + combine for output row `row` (< d) on one wave: lane = slot * 8 + j.
// acts staged in LDS (slot stride slot_h). y[row] = half(res + sum_s w_s v_s)
// in slot order (moe.metal:678-686).
template <int G, bool SYM, typename Src>
__device__ __forceinline__ void phase2_body(const Src& src, const tsg_expert_offsets& o,
                                            const uint16_t* as, uint32_t slot_h,
                                            const float* asum, const uint16_t* __restrict__ rw,
                                            uint16_t res_bits, uint16_t* __restrict__ y,
                                            uint32_t d, uint32_t f, uint32_t row,
                                            ChunkBatch<kDBatch>& bt, bool preloaded) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t slot = lane >> 3, j = lane & 7u;
    const bool live = row < d;
    const uint32_t rr = live ? row : 0u;
    const uint8_t* blob = src.blob(slot);
    const uint32_t ngroups = f / G, nchunks = f / 32u;
    const uint8_t* w = blob + o.down_w + (uint64_t)rr * (f / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + o.down_s) + (uint64_t)rr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + o.down_b) + (uint64_t)rr * ngroups;
    float acc[1] = {0.0f};
    for (uint32_t base = 0; base < nchunks; base += kDLanes * kDBatch) {
        if (base || !preloaded) load_batch<G, SYM, kDBatch, kDLanes>(w, sc, bi, base, j, nchunks, bt);
        compute_batch<G, SYM, kDBatch, kDLanes, 1>(bt, base, j, nchunks, as + slot * slot_h, 0u,
                                                   asum + slot * nchunks, 1u, acc);
    }
    acc[0] = group8_sum(acc[0]);
    float vals[kTopK];
#pragma unroll
    for (int s = 0; s < (int)kTopK; ++s) vals[s] = lane_value(acc[0], s * 8);
    if (lane == 0 && live) {
        float out = f16_to_f32(res_bits);
#pragma unroll
        for (int s = 0; s < (int)kTopK; ++s) {
            const float p = f16_to_f32(rw[s]) * vals[s];
            out = out + p;
        }
        y[row] = f32_to_f16(out);
    }
}

// Prefetch of a lane's phase-2 weights and its row's residual (issued early,
// consumed after a rendezvous).
template <int G, bool SYM, typename Src>
__device__ __forceinline__ void phase2_prefetch(const Src& src, const tsg_expert_offsets& o,
                                                const uint16_t* __restrict__ residual,
                                                uint32_t d, uint32_t f, uint32_t row,
                                                ChunkBatch<kDBatch>& bt, uint16_t& res_bits) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t slot = lane >> 3, j = lane & 7u;
    const uint32_t rr = row < d ? row : 0u;
    res_bits = residual[rr];
    const uint8_t* blob = src.blob(slot);
    const uint32_t ngroups = f / G, nchunks = f / 32u;
    load_batch<G, SYM, kDBatch, kDLanes>(blob + o.down_w + (uint64_t)rr * (f / 2u),
                                         reinterpret_cast<const uint16_t*>(blob + o.down_s) + (uint64_t)rr * ngroups,
                                         reinterpret_cast<const uint16_t*>(blob + o.down_b) + (uint64_t)rr * ngroups,
                                         0u, j, nchunks, bt);
}

__host__ __device__ __forceinline__ uint32_t p2_slot_halves(uint32_t f) {
    return lds_chunks_halves(f) + 8u;
}

// ---------------------------------------------------------------- phase 1

// grid p1_blocks, block 32 * pairs_per_block: pair = blockIdx.x * ppb + t / 32,
// pair = slot * f + fr. Subset form: pair = a * f + fr with slot
// active_slots[a]. Weight loads go out before x is staged.
template <int G, bool SYM, int ACT, bool SUBSET>
__global__ __launch_bounds__(1024) void phase1_kernel(BlobSource src, tsg_expert_offsets o,
                                                      const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ acts, uint32_t d,
                                                      uint32_t f, uint32_t top_k,
                                                      uint32_t pairs_per_block) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + lds_chunks_halves(d) * 2u);
    const uint32_t n_pairs = (SUBSET ? src.active_count : top_k) * f;
    const uint32_t pair = blockIdx.x * pairs_per_block + (threadIdx.x >> 5);
    bool live = pair < n_pairs;
    const uint32_t pp = live ? pair : 0u;
    uint32_t slot = pp / f;
    const uint32_t fr = pp - slot * f;
    if constexpr (SUBSET) {
        slot = src.active_slots[slot];
        if (slot >= top_k) live = false;
    }
    const GULane l = gu_lane(src, o, d, G, slot, fr, live);
    ChunkBatch<kGUBatch> bt;
    load_batch<G, SYM, kGUBatch, kGULanes>(l.w, l.s, l.b, 0u, threadIdx.x & 15u, d / 32u, bt);
    stage_act_rows<SYM>(x, 0u, 1u, d, xs, 0u, xsum);
    __syncthreads();
    uint16_t v;
    if (phase1_compute<G, SYM, ACT>(l, bt, xs, xsum, d, v)) acts[l.slot * f + l.fr] = v;
}

// ---------------------------------------------------------------- phase 2

// grid p2_blocks, block 64 * rows_per_block: row = blockIdx.x * rpb + wave.
template <int G, bool SYM>
__global__ __launch_bounds__(1024) void phase2_kernel(BlobSource src, tsg_expert_offsets o,
                                                      const uint16_t* __restrict__ acts,
                                                      const uint16_t* __restrict__ routing_w,
                                                      const uint16_t* __restrict__ residual,
                                                      uint16_t* __restrict__ y, uint32_t d,
                                                      uint32_t f, uint32_t rows_per_block) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t slot_h = p2_slot_halves(f);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);
    float* asum = reinterpret_cast<float*>(smem + kTopK * slot_h * 2u);
    const uint32_t row = blockIdx.x * rows_per_block + (threadIdx.x >> 6);
    ChunkBatch<kDBatch> bt;
    uint16_t res_bits;
    phase2_prefetch<G, SYM>(src, o, residual, d, f, row, bt, res_bits);
    stage_act_rows<SYM>(acts, f, kTopK, f, as, slot_h, asum);
    __syncthreads();
    phase2_body<G, SYM>(src, o, as, slot_h, asum, routing_w, res_bits, y, d, f, row, bt, true);
}

// ------------------------------------------------- in-launch rendezvous

// The one-launch layer has two points where blocks need what others produced:
// the router logits (for the top-8) and the phase-1 activations (for phase 2).
// Neither uses a shared atomic counter (arrivals on one address serialize at
// the memory-side atomic unit) nor has every block poll every other (the
// polls then queue on the same few lines). Words travel by agent-coherent
// stores and loads, tagged with the launch's epoch, along a shallow tree:
//   - router: each expert's logit is posted as a (tag << 32 | bits) word;
//     block 0 gathers them, runs the top-8 and posts (tag, weight, id) words
//     to kSyncReplicas lines; block b reads line b % kSyncReplicas;
//   - phase 1 done: block b posts flag b; the leader of each 16 blocks
//     gathers its group and posts a group flag; block 0 gathers the groups
//     and posts the go word to kSyncReplicas lines.
// A word carries its own tag, so no reader can mistake an earlier launch's
// words for this one's. The epoch (read at launch start, advanced by block 0
// once every block has passed both rendezvous) makes each launch's tag new,
// also across HIP graph replays. Polls are bounded by kSpinLimit; a block
// that gives up sets the error word (reported by tsg_ctx_synchronize) and
// carries on, so every wave reaches the end of the kernel.
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kSyncFanIn = 16;

struct DecodeSync {
    uint32_t* epoch;
    uint32_t* error;
    uint32_t* flags;
    uint32_t* groups;
    uint32_t* go;       // kSyncReplicas lines
    uint64_t* topk;     // kSyncReplicas lines of kTopK words
    uint64_t* logits;   // kMaxExperts words
};

__device__ __forceinline__ DecodeSync decode_sync(uint32_t* words) {
    DecodeSync s;
    s.epoch = words + kSyncEpochWord;
    s.error = words + kSyncErrorWord;
    s.flags = words + kSyncFlagWord;
    s.groups = words + kSyncGroupWord;
    s.go = words + kSyncGoWord;
    s.topk = reinterpret_cast<uint64_t*>(words + kSyncTopkWord);
    s.logits = reinterpret_cast<uint64_t*>(words + kSyncLogitWord);
    return s;
}

// One wave polls until `ready()` holds on every lane (bounded).
template <typename F>
__device__ __forceinline__ void wave_poll(const DecodeSync& sy, F&& ready) {
    for (uint32_t spins = 0;; ++spins) {
        if (__all(ready())) return;
        if (spins > kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) atomicOr(sy.error, 1u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// One wave: `count` packed words at `w` all equal `tag`.
__device__ __forceinline__ void wave_wait_words(const DecodeSync& sy, const uint32_t* w,
                                                uint32_t count, uint32_t tag) {
    const uint32_t lane = threadIdx.x & 63u;
    wave_poll(sy, [&] {
        bool ok = true;
        for (uint32_t i = lane; i < count; i += 64u) ok = ok && ld_coherent(w + i) == tag;
        return ok;
    });
}

// One wave: every block of the launch has posted flag == tag.
__device__ __forceinline__ void rendezvous_all(const DecodeSync& sy, uint32_t nb, uint32_t tag) {
    const uint32_t b = blockIdx.x, lane = threadIdx.x & 63u;
    if (b % kSyncFanIn == 0) {
        const uint32_t n = min(kSyncFanIn, nb - b);
        wave_wait_words(sy, sy.flags + b, n, tag);
        if (lane == 0) st_coherent(sy.groups + b / kSyncFanIn, tag);
    }
    if (b == 0) {
        wave_wait_words(sy, sy.groups, (nb + kSyncFanIn - 1) / kSyncFanIn, tag);
        if (lane < kSyncReplicas) st_coherent(sy.go + lane * kSyncLineWords, tag);
    }
    wave_wait_words(sy, sy.go + (b % kSyncReplicas) * kSyncLineWords, 1u, tag);
}

// -------------------------------------------------- fused decode layer

struct DecodeLayerArgs {
    const uint8_t* layer_base;
    uint64_t expert_stride;
    tsg_expert_offsets o;
    const uint16_t* router_w;
    const uint16_t* router_hidden;
    const uint16_t* es;
    const uint16_t* pes;
    const uint16_t* x;
    const uint16_t* residual;
    uint16_t* y;
    uint32_t* out_idx;
    uint16_t* out_w;
    uint16_t* acts;
    uint16_t* act_rep;  // kActReplicas copies of the activations
    uint32_t* sync_words;
    uint32_t ne, d, f, pairs_per_block, rows_per_block;
};

// One decode MoE layer in one launch (grid = one block per CU, all
// co-resident): router logits (one expert row per block, the router kernel's
// canonical order) -> rendezvous, every block runs the top-k -> prefetch of
// its down-projection weights, gate/up + activation for its row pairs ->
// rendezvous -> down + slot-ordered combine for its output rows. The
// arithmetic of every phase is the separate kernels' (shared bodies), so the
// fused and unfused paths agree bit for bit.
template <int G, bool SYM, int ACT>
__global__ __launch_bounds__(1024) void decode_layer_kernel(DecodeLayerArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_tag;
    __shared__ uint16_t s_w[kTopK];
    __shared__ uint32_t s_idx[kTopK];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nb = gridDim.x;
    const DecodeSync sy = decode_sync(a.sync_words);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + lds_chunks_halves(a.d) * 2u);

    uint32_t gains[4] = {0u, 0u, 0u, 0u};
    if (blockIdx.x == 0 && wave == 0) load_expert_gains(a.pes, a.ne, gains);
    uint32_t tag = 0;
    if (threadIdx.x == 0) {
        tag = ld_coherent(sy.epoch) + 1u;
        tag = tag ? tag : 1u;
        s_tag = tag;
    }
    // router rows: wave 0 of block b takes experts b, b + nb, ...
    if (wave == 0)
        for (uint32_t e = blockIdx.x; e < a.ne; e += nb) {
            const float s = router_dot(a.router_w + (uint64_t)e * a.d, a.router_hidden, a.es,
                                       a.d, lane);
            if (lane == 0)
                st_coherent(sy.logits + e, ((uint64_t)tag << 32) | __float_as_uint(s));
        }
    stage_act_rows<SYM>(a.x, 0u, 1u, a.d, xs, 0u, xsum);
    __syncthreads();
    tag = s_tag;
    if (wave == 0) {
        if (blockIdx.x == 0) {
            // gather the logits, run the top-8, post it to every replica line
            float v[4];
            wave_poll(sy, [&] {
                bool ok = true;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t e = lane + 64u * j;
                    v[j] = -INFINITY;
                    if (e < a.ne) {
                        const uint64_t w = ld_coherent(sy.logits + e);
                        v[j] = __uint_as_float((uint32_t)w);
                        ok = ok && (uint32_t)(w >> 32) == tag;
                    }
                }
                return ok;
            });
            const TopK t = wave_topk_softmax_regs(v, a.ne, gains);
            const uint32_t r = lane & (kTopK - 1u);
            uint32_t id = 0, wb = 0;
#pragma unroll
            for (uint32_t q = 0; q < kTopK; ++q)
                if (r == q) { id = t.idx[q]; wb = t.w[q]; }
            for (uint32_t q = lane / kTopK; q < kSyncReplicas; q += 64u / kTopK)
                st_coherent(sy.topk + q * (kSyncLineWords / 2) + r,
                            ((uint64_t)tag << 32) | (wb << 16) | id);
            if (lane < kTopK) {
                a.out_idx[lane] = id;
                a.out_w[lane] = (uint16_t)wb;
            }
        }
        const uint64_t* line = sy.topk + (blockIdx.x % kSyncReplicas) * (kSyncLineWords / 2);
        uint64_t w = 0;
        wave_poll(sy, [&] {
            if (lane >= kTopK) return true;
            w = ld_coherent(line + lane);
            return (uint32_t)(w >> 32) == tag;
        });
        if (lane < kTopK) {
            s_idx[lane] = (uint32_t)w & 0xFFFFu;
            s_w[lane] = (uint16_t)(w >> 16);
        }
    }
    __syncthreads();

    const LdsBlobs src{a.layer_base, a.expert_stride, s_idx};
    const uint32_t row = blockIdx.x * a.rows_per_block + wave;
    ChunkBatch<kDBatch> dbt;
    uint16_t res_bits = 0;
    const bool p2_wave = wave < a.rows_per_block;
    if (p2_wave) phase2_prefetch<G, SYM>(src, a.o, a.residual, a.d, a.f, row, dbt, res_bits);
    {
        const uint32_t pair = blockIdx.x * a.pairs_per_block + (threadIdx.x >> 5);
        const bool live = (threadIdx.x >> 5) < a.pairs_per_block && pair < kTopK * a.f;
        const uint32_t pp = live ? pair : 0u;
        const uint32_t slot = pp / a.f;
        const GULane l = gu_lane(src, a.o, a.d, G, slot, pp - slot * a.f, live);
        ChunkBatch<kGUBatch> gbt;
        load_batch<G, SYM, kGUBatch, kGULanes>(l.w, l.s, l.b, 0u, threadIdx.x & 15u, a.d / 32u, gbt);
        uint16_t v;
        if (phase1_compute<G, SYM, ACT>(l, gbt, xs, xsum, a.d, v)) {
            const uint32_t at = l.slot * a.f + l.fr;
            a.acts[at] = v;
#pragma unroll
            for (uint32_t r = 0; r < kActReplicas; ++r)
                st_coherent(a.act_rep + (size_t)r * kActReplicaHalves + at, v);
        }
    }
    wait_vector_memory();  // this wave's activation stores have completed
    __syncthreads();
    if (threadIdx.x == 0) st_coherent(sy.flags + blockIdx.x, tag);
    if (wave == 0) rendezvous_all(sy, nb, tag);
    __syncthreads();

    const uint32_t slot_h = p2_slot_halves(a.f);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);
    float* asum = reinterpret_cast<float*>(smem + kTopK * slot_h * 2u);
    stage_act_rows<SYM, 4, true>(a.act_rep + (size_t)(blockIdx.x % kActReplicas) * kActReplicaHalves,
                                 a.f, kTopK, a.f, as, slot_h, asum);
    __syncthreads();
    if (p2_wave)
        phase2_body<G, SYM>(src, a.o, as, slot_h, asum, s_w, res_bits, a.y, a.d, a.f, row,
                            dbt, true);
    // every block has passed both rendezvous: the next launch may use tag + 1
    if (blockIdx.x == 0 && threadIdx.x == 0) st_coherent(sy.epoch, tag);
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
    TSG_REQUIRE(d > 0 && d % 8 == 0 && d <= 8u * 64u * kRouterChunks, TSG_ERR_INVALID_ARGUMENT,
                "d=%u must be a multiple of 8 and at most %u", d, 8u * 64u * kRouterChunks);
    TSG_REQUIRE(stride % 8 == 0, TSG_ERR_ALIGNMENT, "hidden stride %u must be a multiple of 8",
                stride);
    TSG_REQUIRE(w && hidden && es, TSG_ERR_INVALID_ARGUMENT, "NULL router operand");
    TSG_REQUIRE(aligned16(w) && aligned16(hidden) && aligned16(es), TSG_ERR_ALIGNMENT,
                "router weights, hidden and effective_scale must be 16-byte aligned");
    TSG_REQUIRE(rows > 0 && rows <= kMaxPromptRows, TSG_ERR_INVALID_ARGUMENT,
                "rows=%u not in 1..%u", rows, kMaxPromptRows);
    tsg_ctx* ctx = moe->ctx;
    const dim3 grid((ne + kRouterWaves - 1) / kRouterWaves, (rows + kRouterRows - 1) / kRouterRows);
    if (select) {
        TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK,
                    top_k);
        TSG_REQUIRE(pes && out_idx && out_w, TSG_ERR_INVALID_ARGUMENT, "NULL router output");
        hipLaunchKernelGGL(router_kernel<true>, grid, dim3(256), 0, stream, w, hidden, stride, es,
                           pes, ctx->logits, kMaxExperts, ctx->counters, out_idx, out_w, ne, d,
                           rows, top_k);
    } else {
        TSG_REQUIRE(logits_out, TSG_ERR_INVALID_ARGUMENT, "out_logits is NULL");
        hipLaunchKernelGGL(router_kernel<false>, grid, dim3(256), 0, stream, w, hidden, stride,
                           es, pes, logits_out, ne, ctx->counters, out_idx, out_w, ne, d, rows,
                           top_k);
    }
    return check_launch("router");
}

constexpr uint32_t kTargetBlocks = 256;  // about one block per CU

template <int G, bool SYM>
tsg_status launch_phase1(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                         const tsg_expert_offsets& o, const uint16_t* x, uint16_t* acts,
                         uint32_t d, uint32_t f, uint32_t top_k, bool subset) {
    const uint32_t n_pairs = (subset ? src.active_count : top_k) * f;
    if (n_pairs == 0) return TSG_OK;
    const DecodeGeometry g = decode_geometry(d, f, n_pairs, kTargetBlocks);
    const dim3 grid(g.p1_blocks), block(32u * g.pairs_per_block);
    const size_t lds = lds_chunks_halves(d) * 2u + (SYM ? 0u : (d / 32u) * 4u);
#define TSG_P1(ACT, SUB)                                                                      \
    hipLaunchKernelGGL((phase1_kernel<G, SYM, ACT, SUB>), grid, block, lds, stream, src, o, x, \
                       acts, d, f, top_k, g.pairs_per_block)
    if (moe->activation == TSG_ACT_SILU) {
        if (subset) TSG_P1(TSG_ACT_SILU, true);
        else TSG_P1(TSG_ACT_SILU, false);
    } else {
        if (subset) TSG_P1(TSG_ACT_GELU_TANH, true);
        else TSG_P1(TSG_ACT_GELU_TANH, false);
    }
#undef TSG_P1
    return check_launch("phase1");
}

tsg_status phase1_dispatch(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                           const tsg_expert_offsets& o, const uint16_t* x, uint16_t* acts,
                           uint32_t d, uint32_t f, uint32_t top_k, bool subset) {
    TSG_REQUIRE(x && acts, TSG_ERR_INVALID_ARGUMENT, "NULL x/acts");
    TSG_REQUIRE(aligned16(x), TSG_ERR_ALIGNMENT, "x must be 16-byte aligned");
    TSG_REQUIRE(lds_chunks_halves(d) * 2u + (d / 32u) * 4u <= 160u * 1024u, TSG_ERR_UNSUPPORTED,
                "d=%u does not fit the LDS staging", d);
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32)
        return sym ? launch_phase1<32, true>(moe, stream, src, o, x, acts, d, f, top_k, subset)
                   : launch_phase1<32, false>(moe, stream, src, o, x, acts, d, f, top_k, subset);
    return sym ? launch_phase1<64, true>(moe, stream, src, o, x, acts, d, f, top_k, subset)
               : launch_phase1<64, false>(moe, stream, src, o, x, acts, d, f, top_k, subset);
}

size_t phase2_lds(uint32_t f, bool sym) {
    return kTopK * p2_slot_halves(f) * 2u + (sym ? 0u : kTopK * (f / 32u) * 4u);
}

tsg_status phase2_dispatch(tsg_moe* moe, hipStream_t stream, const BlobSource& src,
                           const tsg_expert_offsets& o, const uint16_t* acts,
                           const uint16_t* rw, const uint16_t* residual, uint16_t* y,
                           uint32_t d, uint32_t f) {
    TSG_REQUIRE(acts && rw && residual && y, TSG_ERR_INVALID_ARGUMENT, "NULL phase-2 operand");
    TSG_REQUIRE(aligned16(acts), TSG_ERR_ALIGNMENT, "acts must be 16-byte aligned");
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const size_t lds = phase2_lds(f, sym);
    TSG_REQUIRE(lds <= 160u * 1024u, TSG_ERR_UNSUPPORTED, "f=%u does not fit the LDS staging", f);
    const DecodeGeometry g = decode_geometry(d, f, kTopK * f, kTargetBlocks);
    const dim3 grid(g.p2_blocks), block(64u * g.rows_per_block);
#define TSG_P2(GG, SS)                                                                       \
    hipLaunchKernelGGL((phase2_kernel<GG, SS>), grid, block, lds, stream, src, o, acts, rw, \
                       residual, y, d, f, g.rows_per_block)
    if (ctx->group_size == 32) {
        if (sym) TSG_P2(32, true);
        else TSG_P2(32, false);
    } else {
        if (sym) TSG_P2(64, true);
        else TSG_P2(64, false);
    }
#undef TSG_P2
    return check_launch("phase2");
}

// The fused one-launch decode layer, when every block fits on the device at
// once (the rendezvous need all blocks resident). Returns TSG_ERR_DECLINED
// otherwise and the caller runs the three-kernel sequence.
template <int G, bool SYM, int ACT>
tsg_status launch_fused(tsg_moe* moe, hipStream_t stream, const DecodeLayerArgs& a,
                        const DecodeGeometry& g) {
    const uint32_t nb = g.p1_blocks > g.p2_blocks ? g.p1_blocks : g.p2_blocks;
    const size_t lds_a = lds_chunks_halves(a.d) * 2u + (SYM ? 0u : (a.d / 32u) * 4u);
    const size_t lds_b = phase2_lds(a.f, SYM);
    const size_t lds = lds_a > lds_b ? lds_a : lds_b;
    auto kern = decode_layer_kernel<G, SYM, ACT>;
    int per_cu = 0;
    if (nb > kMaxFusedBlocks || a.ne > kMaxExperts || kTopK * a.f > kActReplicaHalves ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, (int)g.threads, lds) !=
            hipSuccess ||
        (uint64_t)per_cu * (uint64_t)moe->ctx->num_cus < nb)
        return TSG_ERR_DECLINED;
    hipLaunchKernelGGL(kern, dim3(nb), dim3(g.threads), lds, stream, a);
    return check_launch("decode_layer");
}

tsg_status fused_dispatch(tsg_moe* moe, hipStream_t stream, const DecodeLayerArgs& a,
                          const DecodeGeometry& g) {
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const bool silu = moe->activation == TSG_ACT_SILU;
#define TSG_FU(GG, SS)                                                             \
    return silu ? launch_fused<GG, SS, TSG_ACT_SILU>(moe, stream, a, g)            \
                : launch_fused<GG, SS, TSG_ACT_GELU_TANH>(moe, stream, a, g)
    if (ctx->group_size == 32) {
        if (sym) TSG_FU(32, true);
        TSG_FU(32, false);
    }
    if (sym) TSG_FU(64, true);
    TSG_FU(64, false);
#undef TSG_FU
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
    TSG_REQUIRE(ne > 0 && ne <= layer->num_experts && ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "router has %u experts but the layer holds %u", ne, layer->num_experts);
    TSG_REQUIRE(router_w && router_hidden && es && pes && x && residual && y && out_idx &&
                    out_w && acts,
                TSG_ERR_INVALID_ARGUMENT, "NULL decode-layer operand");
    TSG_REQUIRE(aligned16(router_w) && aligned16(router_hidden) && aligned16(es) &&
                    aligned16(x) && aligned16(acts),
                TSG_ERR_ALIGNMENT, "router weights, activations and acts must be 16-byte aligned");
    TSG_REQUIRE(d % 8 == 0 && d <= 8u * 64u * kRouterChunks, TSG_ERR_INVALID_ARGUMENT,
                "d=%u out of the router's range", d);
    hipStream_t s = as_stream(stream);
    const DecodeGeometry g = decode_geometry(d, f, kTopK * f, kTargetBlocks);
    DecodeLayerArgs a{};
    a.layer_base = layer->base;
    a.expert_stride = layer->expert_stride;
    a.o = layer->offsets;
    a.router_w = router_w;
    a.router_hidden = router_hidden;
    a.es = es;
    a.pes = pes;
    a.x = x;
    a.residual = residual;
    a.y = y;
    a.out_idx = out_idx;
    a.out_w = out_w;
    a.acts = acts;
    a.sync_words = moe->ctx->counters;
    a.act_rep = moe->ctx->act_replicas;
    a.ne = ne;
    a.d = d;
    a.f = f;
    a.pairs_per_block = g.pairs_per_block;
    a.rows_per_block = g.rows_per_block;
    if (!moe->unfused_decode) {
        st = fused_dispatch(moe, s, a, g);
        if (st != TSG_ERR_DECLINED) return st;
    }
    if ((st = router_launch(moe, s, router_w, router_hidden, d, es, pes, out_idx, out_w, nullptr,
                            1, ne, d, top_k, true)))
        return st;
    BlobSource src;
    if ((st = blobs_from_layer(layer, out_idx, &src))) return st;
    if ((st = phase1_dispatch(moe, s, src, layer->offsets, x, acts, d, f, top_k, false)))
        return st;
    return phase2_dispatch(moe, s, src, layer->offsets, acts, out_w, residual, y, d, f);
}

extern "C" tsg_status tsg_moe_set_fused_decode(tsg_moe* moe, int enabled) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    moe->unfused_decode = enabled ? false : true;
    return TSG_OK;
}

// Prompt router: the decode router body per row (bit-identical per row), all
// rows in one launch.
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
    TSG_REQUIRE(query_count <= kMaxPromptRows, TSG_ERR_UNSUPPORTED,
                "queryCount %u exceeds the %u-row prompt chunk", query_count, kMaxPromptRows);
    return router_launch(moe, as_stream(stream), w, hidden, stride, es, pes, out_idx, out_w,
                         nullptr, query_count, ne, d, top_k, true);
}
