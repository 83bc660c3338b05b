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
#include "qwen_shared.hpp"

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

// Softmax over the 8 selected slots (scores descending, unfilled = -inf) with
// the per-expert gains, rounded to fp16 (moe.metal:330-342): lane r < 8 holds
// slot r's score and gain and returns slot r's weight; the sum of the
// exponentials runs in slot order. Shared by the wave and block selections so
// both agree bit for bit.
__device__ __forceinline__ uint16_t slot_softmax_lane(float my_s, float my_gain) {
    const float my_exp = expf(my_s - lane_value(my_s, 0));
    float sum_exp = lane_value(my_exp, 0);
#pragma unroll
    for (uint32_t r = 1; r < kTopK; ++r) sum_exp += lane_value(my_exp, r);
    return (uint16_t)f32_to_f16(my_exp / sum_exp * my_gain);
}

// The same with the 8 slots' scores and gains held by every lane.
__device__ __forceinline__ void topk_softmax8(const float (&top_s)[kTopK],
                                              const float (&gain)[kTopK], uint16_t (&w)[kTopK]) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r_l = lane & (kTopK - 1u);
    float my_s = top_s[0], my_gain = gain[0];
#pragma unroll
    for (uint32_t r = 1; r < kTopK; ++r)
        if (r_l == r) { my_s = top_s[r]; my_gain = gain[r]; }
    const uint32_t my_w = slot_softmax_lane(my_s, my_gain);
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r) w[r] = (uint16_t)__builtin_amdgcn_readlane(my_w, r);
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
    topk_softmax8(top_s, gain, t.w);
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
template <int G, bool SYM, int ACT, int KB = kGUBatch>
__device__ __forceinline__ bool phase1_compute(const GULane& l, ChunkBatch<KB>& bt,
                                               const uint16_t* xs, const float* xsum,
                                               uint32_t d, uint16_t& out) {
    const uint32_t j = threadIdx.x & 15u;
    const bool is_up = (threadIdx.x >> 4) & 1u;
    const uint32_t nchunks = d / 32u;
    float acc[1] = {0.0f};
    gemv_batches<G, SYM, KB, kGULanes, 1>(l.w, l.s, l.b, j, nchunks, bt, xs, 0u, xsum, 1u, acc);
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
    if (!preloaded) load_batch<G, SYM, kDBatch, kDLanes>(w, sc, bi, 0u, j, nchunks, bt);
    gemv_batches<G, SYM, kDBatch, kDLanes, 1>(w, sc, bi, j, nchunks, bt, as + slot * slot_h, 0u,
                                              asum + slot * nchunks, 1u, acc);
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
    stage_act_rows_around<SYM>(x, 0u, 1u, d, xs, 0u, xsum, nullptr, [&] {
        load_batch<G, SYM, kGUBatch, kGULanes>(l.w, l.s, l.b, 0u, threadIdx.x & 15u, d / 32u, bt);
    });
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
    stage_act_rows_around<SYM>(acts, f, kTopK, f, as, slot_h, asum, nullptr, [&] {
        phase2_prefetch<G, SYM>(src, o, residual, d, f, row, bt, res_bits);
    });
    __syncthreads();
    phase2_body<G, SYM>(src, o, as, slot_h, asum, routing_w, res_bits, y, d, f, row, bt, true);
}

// ------------------------------------------------- in-launch hand-offs

// The one-launch layer runs as kDecodeGroups groups of kGroupMembers blocks,
// group g = block % 8 owning expert slot g. Workgroups go to the 8 XCDs
// round-robin by linear id, so a group's blocks share one XCD and its L2; the
// protocol below does not depend on that. No step waits for the whole grid,
// and every hand-off is a 64-bit word carrying the launch's tag above its
// payload, polled by its readers directly (no separate flag or counter):
//   - every group computes all router logits (each block a few expert rows);
//     every block gathers its group's logits and ranks them itself, so all
//     blocks obtain the same selection, bit for bit;
//   - each block posts the activations of its gate/up pairs; every block of
//     the group reads the slot's full activation row once all have arrived;
//   - each block posts fp32 partial down outputs of its slot; block (g, m)
//     then reads the 8 slots' partials of its share of row range m and
//     writes y = half(res + sum_s w_s v_s) in slot order.
// Tags come from the epoch word read at launch start, so no reader can take
// an earlier launch's word for this one's. Block 0 advances the epoch once
// its combine has read partials from all 8 groups: each of those blocks had
// read its whole group's activations, so by then all 256 blocks have read
// the epoch. Polls are bounded by kSpinLimit; a block that gives up sets the
// error word (reported by tsg_ctx_synchronize) and carries on, so every wave
// reaches the end.
constexpr uint32_t kSpinLimit = 1u << 20;

struct DecodeSync {
    uint32_t* epoch;
    uint32_t* error;
    uint64_t* logits;   // kMaxExperts words per group
};

__device__ __forceinline__ DecodeSync decode_sync(uint32_t* words) {
    DecodeSync s;
    s.epoch = words + kSyncEpochWord;
    s.error = words + kSyncErrorWord;
    s.logits = reinterpret_cast<uint64_t*>(words + kSyncLogitWord);
    return s;
}

__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t payload) {
    return ((uint64_t)tag << 32) | payload;
}

// One wave reads up to N tagged words per lane (word k at addr(k), for k in
// `live`, a lane's bit mask) until each carries `tag`, handing each payload to
// use(k, payload) once; every pass re-reads only the words still missing, so
// words already in cost no further traffic. Between passes the wave sleeps
// SLEEP x 64 cycles: the polls' agent-coherent loads are served from the
// memory side, and polling faster slowed the hand-offs and the expert stream
// they share it with (measured per hand-off, below). Bounded: after
// kSpinLimit passes the wave sets the error word and returns.
// Decode layer, sleep 1 / 2 / 3 on every hand-off, µs per layer: 14.55 / 13.80 /
// 13.97 on one box, 13.76 / 13.83 / (3 on two of three) 13.97 on another; 2 is
// within 0.5 % of the best on both.
constexpr int kPollSleepLogits = 2;
constexpr int kPollSleepActs = 2;
constexpr int kPollSleepParts = 2;
constexpr int kPollSleepRouter = 1;  // the staged router: one polling block
template <int N, int SLEEP, typename Addr, typename Use>
__device__ __forceinline__ void poll_tagged(const DecodeSync& sy, uint32_t tag, uint32_t live,
                                            Addr&& addr, Use&& use,
                                            uint32_t err_bit = kErrDecodeTimeout) {
    uint32_t pending = live;
    for (uint32_t spins = 0;; ++spins) {
        uint64_t w[N];
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (pending & (1u << k)) w[k] = ld_coherent(addr(k));
#pragma unroll
        for (int k = 0; k < N; ++k) {
            if ((pending & (1u << k)) && (uint32_t)(w[k] >> 32) == tag) {
                use(k, (uint32_t)w[k]);
                pending &= ~(1u << k);
            }
        }
        if (__all(pending == 0u)) return;
        if (spins > kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) atomicOr(sy.error, err_bit);
            return;
        }
        __builtin_amdgcn_s_sleep(SLEEP);
    }
}

// -------------------------------------------------- fused decode layer

struct DecodeLayerArgs {
    const uint8_t* layer_base;
    uint64_t expert_stride;
    tsg_expert_offsets o;
    const uint16_t* router_w;   // bf16 rows, or uint8 codes for the INT8 router
    const uint16_t* router_s;   // INT8 router: bf16 group scales and biases
    const uint16_t* router_b;
    const uint16_t* router_hidden;
    const uint16_t* es;
    const uint16_t* pes;
    const uint16_t* x;
    const uint16_t* residual;
    uint16_t* y;
    uint32_t* out_idx;
    uint16_t* out_w;
    uint16_t* acts;
    uint64_t* handoff;    // kDecodeGroups regions of kHandoffWords tagged words
    uint32_t* sync_words;
    uint32_t ne, d, f;
    uint32_t router_rows;  // expert rows per block: ceil(ne / kDecodeBlocks), one per wave
    uint32_t pairs;        // gate/up pairs per block: ceil(f / kGroupMembers)
    uint32_t rows;         // down rows per block: ceil(d / kGroupMembers)
    uint32_t as_off;       // dynamic LDS: staged activation row (after x)
    uint32_t xe_off;       // dynamic LDS: router products x * es, fp32
    // the Qwen-family shared expert (kernel flag SH): gate/up/down of one
    // expert blob, its bf16 gate row, intermediate size <= kMaxSharedF
    const uint8_t* sh_blob;
    tsg_expert_offsets sh_o;
    const uint16_t* sh_gate_w;
    uint16_t* sh_acts;     // the shared activations, also returned to the caller
    uint32_t sh_f;
    uint32_t ss_off;       // dynamic LDS: staged shared activations
    // the block size: blockDim.x is a kernarg load of its own, whose wait the
    // compiler put ahead of the first phase's loads
    uint32_t threads;
};

// Down row `row` of one slot on 8 lanes (lane = 8 r + j of the wave): the
// per-slot value of phase2_body, the same chunk split and the same sum, so
// the combine below reproduces the unfused path bit for bit.
template <int G, bool SYM, int KB = kDBatch>
__device__ __forceinline__ float slot_down_row(const uint8_t* w, const uint16_t* sc,
                                               const uint16_t* bi, const uint16_t* as,
                                               const float* asum, uint32_t f,
                                               ChunkBatch<KB>& bt) {
    const uint32_t j = threadIdx.x & 7u, nchunks = f / 32u;
    float acc[1] = {0.0f};
    gemv_batches<G, SYM, KB, kDLanes, 1>(w, sc, bi, j, nchunks, bt, as, 0u, asum, 1u, acc);
    return group8_sum(acc[0]);
}

// router_chunks_dot with the products x * es taken from LDS (fp32, element
// order): the same products and the same fma order, so the same sum.
__device__ __forceinline__ float router_dot_staged(const uint4 (&wv)[kRouterChunks],
                                                   const float* xe, uint32_t nchunks,
                                                   uint32_t lane) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouterChunks; ++i) {
        const uint32_t c = lane + 64u * i;
        if (c >= nchunks) break;
        const float4 p0 = *reinterpret_cast<const float4*>(xe + c * 8u);
        const float4 p1 = *reinterpret_cast<const float4*>(xe + c * 8u + 4u);
        const float p[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        const uint32_t wa[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc = __builtin_fmaf(__uint_as_float(wa[k] << 16), p[2 * k], acc);
            acc = __builtin_fmaf(__uint_as_float(wa[k] & 0xFFFF0000u), p[2 * k + 1], acc);
        }
    }
    acc = group16_sum(acc);
    return (lane_value(acc, 0) + lane_value(acc, 16)) + (lane_value(acc, 32) + lane_value(acc, 48));
}

__device__ __forceinline__ uint32_t row16_max(uint32_t k) {
    k = max(k, dpp_u32<0xB1>(k));   // quad_perm [1,0,3,2]
    k = max(k, dpp_u32<0x4E>(k));   // quad_perm [2,3,0,1]
    k = max(k, dpp_u32<0x141>(k));  // row_half_mirror
    k = max(k, dpp_u32<0x140>(k));  // row_mirror
    return k;
}

// Top-8 on one wave over the order keys of experts lane + 64 j (0 = not
// eligible; keys of experts >= ne are 0), with the reference's rule
// (moe.metal:281-329): descending score, ties to the lower index, -inf and
// NaN never enter. T, the least of the maxima of the eight 16-expert groups
// of experts 0..127 (the larger of that and the same over experts 128..255
// when there are more), has at least 8 keys at or above it, so an expert below
// T ranks 8th or later; the experts at or above T (the candidates, typically a
// few dozen) are ranked among themselves by composite key (key << 32 | ~e:
// by score, then lower expert, no two are equal) and rank r < 8 takes slot r.
// Candidates are compacted into `cand` by ballot and lane counts (no atomic
// round trip) and the list is padded with zeros (0 exceeds no candidate) to a
// multiple of kCandBatch. Up to kCandBatch candidates (the usual case), lanes
// 2i and 2i+1 count the list entries above candidate i, half each, and add
// the halves; beyond that, each lane ranks its own candidates against the
// whole list, kCandBatch keys per batch of reads. A slot whose expert is not eligible, or
// that no candidate reaches, keeps its preset (expert 0, unfilled, -inf).
// `cand` holds ne4 + kCandBatch words.
constexpr uint32_t kCandBatch = 32;

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// The least of the maxima of the eight 16-expert groups of keys k0 (lanes)
// and k1 (lanes): at least 8 keys are at or above it. Every lane returns it.
__device__ __forceinline__ uint32_t group_min_of_maxima(uint32_t k0, uint32_t k1) {
    uint32_t m = min(row16_max(k0), row16_max(k1));
    const auto a = __builtin_amdgcn_permlane16_swap(m, m, false, false);
    m = min(m, min((uint32_t)a[0], (uint32_t)a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(m, m, false, false);
    return min(m, min((uint32_t)b[0], (uint32_t)b[1]));
}

__device__ __forceinline__ void wave_select_top8(const uint32_t (&key)[4], uint32_t ne4,
                                                 uint64_t* cand, uint32_t* slot_id,
                                                 uint32_t* slot_fill, uint32_t* slot_key) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t m = group_min_of_maxima(key[0], key[1]);
    if (ne4 > 128u) m = max(m, group_min_of_maxima(key[2], key[3]));
    uint32_t pos[4], n = 0;  // n: candidates so far (uniform, counted on the VALU)
    bool is_cand[4];
    uint64_t ck[4];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        is_cand[j] = e < ne4 && key[j] >= m;
        ck[j] = ((uint64_t)key[j] << 32) | (uint32_t)~e;
        const uint64_t mask = __ballot(is_cand[j]);
        pos[j] = n + lanes_below(mask);
        n += __builtin_popcount((uint32_t)mask) + __builtin_popcount((uint32_t)(mask >> 32));
        if (is_cand[j]) cand[pos[j]] = ck[j];
    }
    const uint32_t padded = (n + kCandBatch - 1u) / kCandBatch * kCandBatch;
    if (n + lane < padded) cand[n + lane] = 0u;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // LDS ops of one wave run in order
    if (n <= kCandBatch) {
        // lanes 2i and 2i+1 rank candidate i, each against half of the list
        const uint32_t i = lane >> 1, h = (lane & 1u) * (kCandBatch / 2u);
        const uint64_t ki = cand[i];
        uint64_t kq[kCandBatch / 2];
#pragma unroll
        for (uint32_t q = 0; q < kCandBatch / 2; q += 2u) {
            const ulonglong2 kk = *reinterpret_cast<const ulonglong2*>(cand + h + q);
            kq[q] = kk.x;
            kq[q + 1] = kk.y;
        }
        uint32_t c = 0;
#pragma unroll
        for (uint32_t q = 0; q < kCandBatch / 2; ++q) c += kq[q] > ki ? 1u : 0u;
        c += __builtin_amdgcn_update_dpp(0u, c, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
        if ((lane & 1u) == 0 && i < n && c < kTopK) {
            const uint32_t k = (uint32_t)(ki >> 32);
            slot_id[c] = k ? ~(uint32_t)ki : 0u;
            slot_fill[c] = k ? 1u : 0u;
            slot_key[c] = k;
        }
        return;
    }
    uint32_t cnt[4] = {0u, 0u, 0u, 0u};
    for (uint32_t q0 = 0; q0 < padded; q0 += kCandBatch) {
        uint64_t kq[kCandBatch];
#pragma unroll
        for (uint32_t q = 0; q < kCandBatch; q += 2u) {
            const ulonglong2 kk = *reinterpret_cast<const ulonglong2*>(cand + q0 + q);
            kq[q] = kk.x;
            kq[q + 1] = kk.y;
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (64u * j >= ne4) break;
            if (is_cand[j]) {
#pragma unroll
                for (uint32_t q = 0; q < kCandBatch; ++q) cnt[j] += kq[q] > ck[j] ? 1u : 0u;
            }
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        if (64u * j >= ne4) break;
        if (is_cand[j] && cnt[j] < kTopK) {
            const uint32_t k = key[j];
            slot_id[cnt[j]] = k ? lane + 64u * j : 0u;
            slot_fill[cnt[j]] = k ? 1u : 0u;
            slot_key[cnt[j]] = k;
        }
    }
}

// Outputs of the grouping the rows router can append (GROUP): those of
// tsg_prefill_group_pairs_device for the routed rows.
struct RouterGroupOut {
    tsg_token_expert_pair* sorted;
    uint32_t* offsets;
    uint32_t* counts;
    tsg_routed_block* blocks;
    uint32_t* n_blocks;
};

// The grouping of the rows' n = rows * 8 pairs (token-major pair p = 8 t + r
// with expert pe[p], weight bits pw[p], in LDS; n <= 64) on one block, the
// device grouping's results: pairs stably sorted by expert, per-expert
// counts and exclusive offsets (0xFFFFFFFF for an expert with no pairs), and
// one routed block per expert present (an expert's <= 8 rows fit any tile),
// in expert order, which is the device grouping's largest-first order when
// every block is in the first size bucket. A counting sort: an LDS
// histogram, one scan over the experts (counts and presence packed in one
// word), and each pair's place = its expert's offset + the earlier tokens
// that chose the expert (a token's 8 experts are distinct; per-token expert
// bit masks in LDS). Every thread of the block calls it; it synchronises
// through LDS only and stores its results last.
constexpr uint32_t kGroupPairs = kMaxRouterRows * kTopK;  // 64
constexpr uint32_t kMaskWords = kMaxExperts / 32u;        // 8

struct RouterGroupLds {
    uint32_t cnt[kMaxExperts], off[kMaxExperts];
    uint32_t mask[kMaxRouterRows * kMaskWords];
    uint32_t wave_tot[kMaxExperts / 64u];
};

// Inclusive prefix sum over the wave on DPP moves (no LDS round trips): row
// shifts by 1, 2, 4, 8 within each 16-lane row (lanes shifted in from outside
// the row add 0), then lane 15's sum added to row 1 and row 3 (row_bcast:15)
// and lane 31's to rows 2 and 3 (row_bcast:31).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_add(uint32_t v) {
    return v + (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    v = dpp_add<0x111, 0xF>(v);  // row_shr:1
    v = dpp_add<0x112, 0xF>(v);  // row_shr:2
    v = dpp_add<0x114, 0xF>(v);  // row_shr:4
    v = dpp_add<0x118, 0xF>(v);  // row_shr:8
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ void group_router_rows(const uint32_t* pe, const uint32_t* pw, uint32_t n,
                                  uint32_t ne, RouterGroupLds& L, const RouterGroupOut& g) {
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    if (t < kMaxExperts) L.cnt[t] = 0u;
    if (t < kMaxRouterRows * kMaskWords) L.mask[t] = 0u;
    lds_barrier();
    const bool my_pair = t < n;
    const uint32_t my_e = my_pair ? pe[t] : 0u, my_w = my_pair ? pw[t] : 0u;
    const uint32_t tok = t / kTopK;
    if (my_pair) {
        atomicAdd(&L.cnt[my_e], 1u);
        atomicOr(&L.mask[tok * kMaskWords + (my_e >> 5)], 1u << (my_e & 31u));
    }
    lds_barrier();
    // offsets (low half) and block indices (high half) of the experts
    const uint32_t c = t < ne ? L.cnt[t] : 0u;
    const uint32_t packed = c | ((c ? 1u : 0u) << 16);
    const uint32_t incl = t < kMaxExperts ? wave_inclusive_scan(packed) : 0u;
    if (t < kMaxExperts && lane == 63u) L.wave_tot[wave] = incl;
    lds_barrier();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kMaxExperts / 64u; ++w) {
        base += w < wave ? L.wave_tot[w] : 0u;
        total += L.wave_tot[w];
    }
    const uint32_t excl = base + incl - packed;
    const uint32_t off = excl & 0xFFFFu, bidx = excl >> 16;
    if (t < ne) L.off[t] = off;
    lds_barrier();
    uint32_t pos = 0;
    if (my_pair) {
        // the earlier tokens' mask words, read together (tok < kMaxRouterRows)
        uint32_t rank = 0;
#pragma unroll
        for (uint32_t u = 0; u < kMaxRouterRows; ++u)
            rank += u < tok ? (L.mask[u * kMaskWords + (my_e >> 5)] >> (my_e & 31u)) & 1u : 0u;
        pos = L.off[my_e] + rank;
    }
    // every LDS read is done: the results leave
    if (my_pair) {
        tsg_token_expert_pair pr;
        pr.token = tok;
        pr.expert = my_e;
        pr.rank = t % kTopK;
        pr.weight_bits = my_w;
        g.sorted[pos] = pr;
    }
    if (t < ne) {
        g.counts[t] = c;
        g.offsets[t] = c ? off : 0xFFFFFFFFu;  // the device grouping's mark of an absent expert
        if (c) {
            tsg_routed_block b;
            b.local_slot = t;
            b.pair_start = off;
            b.row_count = c;
            b.local_row = off;
            g.blocks[bidx] = b;
        }
    }
    if (t == 0) g.n_blocks[0] = total >> 16;
}

// One expert row against up to kRouterRows activation rows in the canonical
// order: lane l sums chunks l, l+64, ... (elements in order, acc = fma(w,
// x*es, acc)); each 16-lane row then sums as group16_sum does (pairs, pairs of
// pairs, mirrored quads, mirrored 8s) and the four row sums add as
// (r0 + r1) + (r2 + r3). Every lane ends with the full sum. Loads for all
// chunks are issued before any arithmetic; out-of-range chunks load a clamped
// address and contribute nothing.
//  - one row or a prompt's rows: block b holds experts 4b .. 4b + 3, one per
//    wave, each wave taking the rows in turn (the next row's activations
//    requested before this row's sums); the last block ranks each row on one
//    wave (wave_topk_softmax).
//  - STAGE (2..8 rows, or GROUP): block e holds expert e and copies the rows
//    to LDS once, after its weight row is requested; wave w takes rows w,
//    w + 4. The last block ranks each row on one wave with the candidate
//    top-8 and the slot softmax of the one-launch layer (wave_select_top8,
//    slot_softmax_lane; the same indices and weights). Same sums as the
//    unstaged form.
//  - GROUP (with STAGE): the last block then groups the rows' pairs
//    (group_router_rows).
constexpr uint32_t kStageWaves = 8;  // the staged form: one wave per row
static_assert(kMaxRouterRows <= kStageWaves, "one row per wave");

template <bool SELECT, bool STAGE, bool GROUP>
// The parameters its first loads need come first (14 dwords, preloaded into
// SGPRs by the dispatch where the firmware does so).
__global__ __launch_bounds__(STAGE ? 64u * kStageWaves : 256u) void router_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ hidden,
    const uint16_t* __restrict__ es, const uint16_t* __restrict__ pes,
    uint32_t* __restrict__ counters, uint32_t hidden_stride, uint32_t ne, uint32_t d,
    uint32_t rows, float* __restrict__ logits, uint32_t logits_stride,
    uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w, uint32_t top_k,
    RouterGroupOut grp) {
    static_assert(!GROUP || (SELECT && STAGE), "the grouping follows a staged selection");
    static_assert(!STAGE || SELECT, "the staged form selects");
    extern __shared__ __align__(16) uint4 xrows[];  // STAGE: the block's rows, d / 8 units each
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t e = STAGE ? blockIdx.x : blockIdx.x * kRouterWaves + wave;
    const uint32_t r0 = blockIdx.y * kRouterRows;
    const uint32_t nr = min(kRouterRows, rows - r0);
    const uint32_t nchunks = d / 8u;
    uint32_t gains[4] = {0u, 0u, 0u, 0u};
    if constexpr (SELECT && !STAGE) load_expert_gains(pes, ne, gains);
    // STAGE: thread t's expert gain, for the selecting block (requested early),
    // and the launch epoch (the tag of this launch's logits is epoch + 1)
    const uint32_t my_gain = (STAGE && threadIdx.x < ne) ? pes[threadIdx.x] : 0u;
    uint32_t* const r_epoch = counters + kRouterEpochWord;
    uint64_t* const r_logits = reinterpret_cast<uint64_t*>(counters + kRouterLogitWord);
    // every thread reads the epoch (one request per wave), without a branch,
    // so its wait lands at the tag's first use and not before the weight loads
    const uint32_t epoch0 = STAGE ? ld_coherent(r_epoch) : 0u;
    uint4 wv[kRouterChunks], ev[kRouterChunks], xv[kRouterChunks];
    // (staged: the grid is one block per expert, so e < ne; unconditional
    // loads keep the compiler's waits on later loads precise)
    if (STAGE || e < ne) {
        const uint16_t* wr = w + (uint64_t)e * d;
#pragma unroll
        for (int i = 0; i < kRouterChunks; ++i) {
            const uint32_t cc = min(lane + 64u * i, nchunks - 1u);
            wv[i] = *reinterpret_cast<const uint4*>(wr + cc * 8u);
            ev[i] = *reinterpret_cast<const uint4*>(es + cc * 8u);
            if constexpr (!STAGE)
                xv[i] = *reinterpret_cast<const uint4*>(hidden + (uint64_t)r0 * hidden_stride + cc * 8u);
        }
    }
    __shared__ uint32_t s_tag;
    if constexpr (STAGE) {
        // the rows go to LDS in passes of kStageUnits 16-byte units per
        // thread, every load of a pass issued before any of its stores: one
        // memory round trip per pass, not one per unit (units past the end
        // repeat the last one and store nothing)
        constexpr uint32_t kStageUnits = 4;
        const uint32_t total = nr * nchunks;
        for (uint32_t q0 = 0; q0 < total; q0 += blockDim.x * kStageUnits) {
            u32x4_t v[kStageUnits];
#pragma unroll
            for (uint32_t i = 0; i < kStageUnits; ++i) {
                const uint32_t q = min(q0 + threadIdx.x + i * blockDim.x, total - 1u);
                const uint32_t r = q / nchunks, c = q - r * nchunks;
                v[i] = *reinterpret_cast<const u32x4_t*>(hidden + (uint64_t)(r0 + r) * hidden_stride + c * 8u);
            }
            // keeps the compiler from sinking each load into its conditional
            // store below (which would make the round trips serial again)
#pragma unroll
            for (uint32_t i = 0; i < kStageUnits; ++i) asm volatile("" : "+v"(v[i]));
#pragma unroll
            for (uint32_t i = 0; i < kStageUnits; ++i) {
                const uint32_t q = q0 + threadIdx.x + i * blockDim.x;
                if (q < total) xrows[q] = make_uint4(v[i].x, v[i].y, v[i].z, v[i].w);
            }
        }
        if (threadIdx.x == 0) s_tag = epoch0 + 1u == 0u ? 1u : epoch0 + 1u;  // words start at tag 0
        __syncthreads();
        const uint32_t tag = s_tag;
        for (uint32_t r = wave; r < nr; r += kStageWaves) {
#pragma unroll
            for (int i = 0; i < kRouterChunks; ++i)
                xv[i] = xrows[r * nchunks + min(lane + 64u * i, nchunks - 1u)];
            const float acc = router_chunks_dot(wv, xv, ev, nchunks, lane);
            if (lane == 0)
                st_coherent(r_logits + (uint64_t)r * kMaxExperts + e, tagged(tag, __float_as_uint(acc)));
        }
    } else if (e < ne) {
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
        // STAGE: block 0 selects, polling the other blocks' tagged logits (the
        // launch's blocks are co-resident: one per expert; the wait is
        // bounded); the other blocks leave once posted. Otherwise the last
        // block to finish selects: logits travel by agent-coherent
        // stores/loads, and completing this block's stores before it counts
        // itself is all the last block needs.
        __shared__ uint32_t is_last;
        if constexpr (STAGE) {
            if (blockIdx.x != 0) return;
        } else {
            wait_vector_memory();
            __syncthreads();
            if (threadIdx.x == 0) {
                const uint32_t done = atomicAdd(&counters[blockIdx.y], 1u);
                is_last = (done == gridDim.x - 1u) ? 1u : 0u;
            }
            __syncthreads();
        }
        if (STAGE || is_last) {
            if constexpr (STAGE) {
                __shared__ uint32_t s_gain[kMaxExperts];
                __shared__ __align__(16) uint64_t s_cand[kStageWaves][kMaxExperts + kCandBatch];
                __shared__ uint32_t s_sid[kStageWaves][kTopK], s_sfill[kStageWaves][kTopK];
                __shared__ uint32_t s_skey[kStageWaves][kTopK];
                __shared__ uint32_t s_pe[kGroupPairs], s_pw[kGroupPairs];
                static_assert(kMaxExperts <= 64u * kStageWaves, "one gain per thread");
                const uint32_t t = threadIdx.x;
                if (t < kMaxExperts) s_gain[t] = my_gain;
                lds_barrier();
                const uint32_t ne4 = (ne + 3u) & ~3u;
                const uint32_t r = wave;  // one row per wave
                if (r < nr) {
                    uint32_t key[4], bits[4] = {0u, 0u, 0u, 0u}, live = 0u;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (lane + 64u * j < ne) live |= 1u << j;
                    DecodeSync sy;
                    sy.error = counters + kSyncErrorWord;
                    poll_tagged<4, kPollSleepRouter>(sy, s_tag, live,
                                   [&](int j) { return r_logits + (uint64_t)r * kMaxExperts + lane + 64u * j; },
                                   [&](int j, uint32_t b) { bits[j] = b; }, kErrRouterWait);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t ej = lane + 64u * j;
                        const float v = ej < ne ? __uint_as_float(bits[j]) : -INFINITY;
                        key[j] = (v == v && v != -INFINITY) ? order_key(v) : 0u;
                    }
                    if (lane < kTopK) {
                        s_sid[wave][lane] = 0u;
                        s_sfill[wave][lane] = 0u;
                        s_skey[wave][lane] = 0u;
                    }
                    wave_select_top8(key, ne4, s_cand[wave], s_sid[wave], s_sfill[wave],
                                     s_skey[wave]);
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS in order
                    const uint32_t sl = lane & (kTopK - 1u);
                    const uint32_t id = s_sid[wave][sl];
                    const float my_s = s_sfill[wave][sl] ? order_key_value(s_skey[wave][sl]) : -INFINITY;
                    const uint16_t wb = slot_softmax_lane(my_s, bf16_to_f32((uint16_t)s_gain[id]));
                    if (lane < kTopK) {
                        s_pe[r * kTopK + lane] = id;
                        s_pw[r * kTopK + lane] = wb;
                    }
                }
                // the results leave after all the LDS work (a wave's next LDS
                // read would wait for its global stores in flight)
                lds_barrier();
                const bool my_pair = t < nr * kTopK;
                const uint32_t my_id = my_pair ? s_pe[t] : 0u, my_wb = my_pair ? s_pw[t] : 0u;
                if constexpr (GROUP) {
                    __shared__ RouterGroupLds gl;
                    group_router_rows(s_pe, s_pw, nr * kTopK, ne, gl, grp);
                }
                if (my_pair) {
                    out_idx[(uint64_t)r0 * kTopK + t] = my_id;
                    out_w[(uint64_t)r0 * kTopK + t] = (uint16_t)my_wb;
                }
                // every block has posted (the polls saw all tags): the next
                // launch may use tag + 1
                if (t == 0) st_coherent(r_epoch, s_tag);
            } else {
                for (uint32_t r = wave; r < nr; r += kRouterWaves)
                    wave_topk_softmax(logits + (uint64_t)(r0 + r) * logits_stride, ne, gains,
                                      out_idx + (uint64_t)(r0 + r) * kTopK,
                                      out_w + (uint64_t)(r0 + r) * kTopK);
                if (threadIdx.x == 0) atomicExch(&counters[blockIdx.y], 0u);
            }
        }
    }
}

// INT8-affine router (encodeRouterGemma4, MoE.swift:201-257; arithmetic of
// moe.metal:136-183): logit_e = sum_i (q_i * scale_g + bias_g) * x_i with
// x_i = hidden_i * es_i in fp32, as sum_g scale_g * (q . x)_g + bias_g *
// (sum x)_g. Block b holds experts 4b .. 4b + 3, one per wave. Lane l takes the
// 16-byte units u = l, l + 64, ... of its row (16 weights, each unit inside one
// group of G >= 16) with every load in flight before the arithmetic (units
// past the row end read the last unit again and add +0); per unit,
// in element order, qx = fma(q, x, qx) and sx = sx + x, then acc = fma(scale,
// qx, acc), acc = fma(bias, sx, acc). The lane sums reduce as the BF16
// router's (group16_sum, then (r0 + r1) + (r2 + r3)). The last block to
// finish selects on one wave (wave_topk_softmax), as the one-row BF16 router.
constexpr int kInt8Units = 4;  // 16-byte units per lane: d <= 4096

// One 16-weight unit against its 16 products x = hidden * es (fp32): qx =
// fma(q, x, qx) and sx = sx + x in element order, then acc = fma(scale, qx,
// acc), acc = fma(bias, sx, acc). Nothing is contracted.
__device__ __forceinline__ float int8_unit_dot_x(const u32x4_t& wq, const float (&x)[16],
                                                 float scale, float bias, float acc) {
#pragma clang fp contract(off)
    const uint32_t qa[4] = {wq.x, wq.y, wq.z, wq.w};
    float qx = 0.0f, sx = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float q = (float)((qa[k >> 2] >> (8 * (k & 3))) & 0xFFu);
        qx = __builtin_fmaf(q, x[k], qx);
        sx = sx + x[k];
    }
    acc = __builtin_fmaf(scale, qx, acc);
    return __builtin_fmaf(bias, sx, acc);
}

// The same with the products formed here from the fp16 hidden and bf16 es
// words (each rounded to fp32 before its two uses).
__device__ __forceinline__ float int8_unit_dot(const u32x4_t& wq, const u32x4_t (&xv)[2],
                                               const u32x4_t (&ev)[2], float scale, float bias,
                                               float acc) {
#pragma clang fp contract(off)
    const uint32_t xa[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w};
    const uint32_t ea[8] = {ev[0].x, ev[0].y, ev[0].z, ev[0].w, ev[1].x, ev[1].y, ev[1].z, ev[1].w};
    float x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t hw = xa[k >> 1], ew = ea[k >> 1];
        const float h = f16_to_f32((uint16_t)((k & 1) ? hw >> 16 : hw & 0xFFFFu));
        const float s = __uint_as_float((k & 1) ? ew & 0xFFFF0000u : ew << 16);
        x[k] = h * s;
    }
    return int8_unit_dot_x(wq, x, scale, bias, acc);
}

// One INT8 router row on one wave with the products x * es taken from LDS
// (fp32, element order): router_int8_kernel's units, sums and reduction, so
// the same logit bit for bit. wq[i] is unit lane + 64 i of the row (clamped),
// sb / bb its group's scale and bias bits.
__device__ __forceinline__ float router_dot_int8_staged(const uint4 (&wq)[kRouterChunks],
                                                        const uint32_t (&sb)[4],
                                                        const uint32_t (&bb)[4], const float* xe,
                                                        uint32_t nunits, uint32_t lane) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t uu = lane + 64u * i;
        const bool live = uu < nunits;
        const uint32_t u = live ? uu : nunits - 1u;
        float x[16];
#pragma unroll
        for (int k = 0; k < 16; k += 4) {
            const float4 v = *reinterpret_cast<const float4*>(xe + u * 16u + k);
            x[k] = v.x, x[k + 1] = v.y, x[k + 2] = v.z, x[k + 3] = v.w;
        }
        const u32x4_t w = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
        acc = int8_unit_dot_x(w, x, live ? bf16_to_f32((uint16_t)sb[i]) : 0.0f,
                              live ? bf16_to_f32((uint16_t)bb[i]) : 0.0f, acc);
    }
    acc = group16_sum(acc);
    return (lane_value(acc, 0) + lane_value(acc, 16)) + (lane_value(acc, 32) + lane_value(acc, 48));
}

template <int G>
__global__ __launch_bounds__(256) void router_int8_kernel(
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ hidden,
    const uint16_t* __restrict__ es, const uint16_t* __restrict__ pes,
    uint32_t* __restrict__ counters, uint32_t ne, uint32_t d, float* __restrict__ logits,
    uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w) {
    static_assert(G % 16 == 0, "a unit lies inside one group");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t e = blockIdx.x * kRouterWaves + wave;
    const uint32_t nunits = d / 16u, ngroups = d / G;
    uint32_t gains[4];
    load_expert_gains(pes, ne, gains);
    if (e < ne) {
        const uint8_t* wr = w + (uint64_t)e * d;
        u32x4_t wq[kInt8Units], xv[kInt8Units][2], ev[kInt8Units][2];
        uint32_t sb[kInt8Units], bb[kInt8Units];
#pragma unroll
        for (int i = 0; i < kInt8Units; ++i) {
            const uint32_t u = min(lane + 64u * i, nunits - 1u);
            wq[i] = *reinterpret_cast<const u32x4_t*>(wr + u * 16u);
            xv[i][0] = *reinterpret_cast<const u32x4_t*>(hidden + u * 16u);
            xv[i][1] = *reinterpret_cast<const u32x4_t*>(hidden + u * 16u + 8u);
            ev[i][0] = *reinterpret_cast<const u32x4_t*>(es + u * 16u);
            ev[i][1] = *reinterpret_cast<const u32x4_t*>(es + u * 16u + 8u);
            const uint32_t g = e * ngroups + u * 16u / G;
            sb[i] = scales[g];
            bb[i] = biases[g];
        }
        // every load is issued before the first use (the compiler would
        // otherwise interleave the units' loads with the arithmetic)
#pragma unroll
        for (int i = 0; i < kInt8Units; ++i)
            asm volatile("" : "+v"(wq[i]), "+v"(xv[i][0]), "+v"(xv[i][1]), "+v"(ev[i][0]),
                         "+v"(ev[i][1]), "+v"(sb[i]), "+v"(bb[i]));
        // units past the row end (a clamped copy of the last one) enter with
        // scale and bias 0 and add +0: no branch, so no load waits behind one
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kInt8Units; ++i) {
            const bool live = lane + 64u * i < nunits;
            acc = int8_unit_dot(wq[i], xv[i], ev[i], live ? bf16_to_f32((uint16_t)sb[i]) : 0.0f,
                                live ? bf16_to_f32((uint16_t)bb[i]) : 0.0f, acc);
        }
        acc = group16_sum(acc);
        const float logit =
            (lane_value(acc, 0) + lane_value(acc, 16)) + (lane_value(acc, 32) + lane_value(acc, 48));
        if (lane == 0) st_coherent(reinterpret_cast<uint32_t*>(logits) + e, __float_as_uint(logit));
    }
    // logits travel by agent-coherent stores/loads; completing this block's
    // stores before it counts itself is all the last block needs
    __shared__ uint32_t is_last;
    wait_vector_memory();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(&counters[0], 1u) == gridDim.x - 1u ? 1u : 0u;
    __syncthreads();
    if (!is_last) return;
    if (wave == 0) wave_topk_softmax(logits, ne, gains, out_idx, out_w);
    if (threadIdx.x == 0) atomicExch(&counters[0], 0u);
}

// One decode MoE layer in one launch (kDecodeBlocks blocks, all co-resident).
// Per group g: router logits -> top-8 (every block) -> gate/up + activation of
// slot g (pairs per block) -> down rows of slot g -> partials -> slot-ordered
// combine. The arithmetic of every phase is the separate kernels' (shared
// bodies), so the fused and unfused paths agree bit for bit. Wave roles:
// waves < router_rows compute a router row each; wave 0 gathers the logits,
// selects, and combines; wave w < pairs / 2 computes gate/up pairs 2w, 2w+1;
// wave w < rows / 8 computes 8 down rows; the last wave (no down rows, so no
// weight loads ahead of its polls) reads the slot's activations into LDS.
//
// With SH the layer also runs the Qwen-family shared branch
// (QwenForwardRunner.swift:1548-1578) and takes its output as the residual
// (:1583-1608), on the last wave of every block: at launch start, while the
// router runs, it loads its block's two shared gate/up pairs (the shared
// weights do not depend on the routing) and sums the gate logit; after the
// top-8 it posts the two shared activations (tagged words, a 9th hand-off
// region); it prefetches the shared down rows of the rows this block combines,
// reads all shared activations with the slot's, and leaves
// half(half(down . act) * sigmoid(logit)) for each of those rows in LDS for
// the combine. Each step is the dense GEMV's lane geometry and the separate
// kernels' arithmetic (qwen_shared.hpp), so the bits are tsg_moe_shared_expert's.
// The shared-branch form keeps more state per lane; its blocks are bounded at
// 768 threads (12 waves, 3 per SIMD) so it has 168 VGPRs instead of the 128 a
// 1024-thread bound allows, and does not spill.
__host__ __device__ constexpr uint32_t decode_layer_max_threads(bool sh) { return sh ? 768u : 1024u; }

template <int G, bool SYM, int ACT, bool SH, bool R8, bool Q>
// Q: chunk batches sized for d <= 2048 and f <= 512 (4 chunks a lane for a
// gate/up row, 2 for a down row), where the default sizes carry slots no lane
// uses; a row's bits do not depend on them.
// The values the first phase's loads need come as separate leading scalar
// arguments (14 dwords) so that, built with kernarg preloading, the dispatch
// hands them over in SGPRs: the loads go out with no memory round trip before
// them. k_ne_rr = ne | router_rows << 16, k_d_thr = d | threads << 16.
// R8: the router is INT8-affine (router_int8_kernel's arithmetic): k_router_w
// holds uint8 codes, a_arg.router_s / router_b the group scales and biases.
__global__ __launch_bounds__(decode_layer_max_threads(SH)) void decode_layer_kernel(
    const uint16_t* k_router_w, const uint16_t* k_hidden, const uint16_t* k_es,
    const uint16_t* k_pes, const uint16_t* k_x, uint32_t* k_sync, uint32_t k_ne_rr,
    uint32_t k_d_thr, DecodeLayerArgs a_arg) {
    constexpr int GUB = Q ? 4 : kGUBatch, DB = Q ? 2 : kDBatch;
    // The arguments are copied to LDS once: under SGPR pressure the compiler
    // re-reads kernel arguments instead of spilling, and a kernarg reload in
    // a loop costs a memory round trip each time; an LDS copy costs cycles.
    // One word per thread (blocks have at least 128 threads: a poll wave
    // beside the down rows), loaded by every thread (clamped) so the
    // compiler's waits on the loads after it stay exact, stored once the
    // first phase's loads are out.
    __shared__ DecodeLayerArgs a;
    constexpr uint32_t kArgWords = sizeof(DecodeLayerArgs) / 4;
    static_assert(sizeof(DecodeLayerArgs) % 4 == 0 && kArgWords <= 128,
                  "args copy: one word per thread");
    const uint32_t arg_word =
        reinterpret_cast<const uint32_t*>(&a_arg)[min((uint32_t)threadIdx.x, kArgWords - 1u)];
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_tag;
    __shared__ uint16_t s_w[kTopK];
    __shared__ uint32_t s_idx[kTopK], s_fill[kTopK], s_skey[kTopK];
    __shared__ uint32_t s_gains[kMaxExperts];
    __shared__ __align__(16) uint64_t s_cand[kMaxExperts + kCandBatch];
    __shared__ uint16_t s_sout[kMaxCombineRows];  // SH: shared output of the combine rows
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
    const uint32_t grp = blockIdx.x % kDecodeGroups, mem = blockIdx.x / kDecodeGroups;

    // Every load of the first phase goes out before any is waited for: this
    // wave's router row first (the routing waits on it), the epoch, the
    // per-expert gains, x for the gate/up dot products, and x and es for the
    // router products.
    const uint32_t d0 = k_d_thr & 0xFFFFu, nthreads = k_d_thr >> 16;
    const uint32_t ne0 = k_ne_rr & 0xFFFFu, router_rows = k_ne_rr >> 16;
    const uint32_t units = d0 / 8u;  // units <= 2 * blockDim (host-checked)
    const uint32_t er = blockIdx.x + kDecodeBlocks * wave;
    const bool router_wave = wave < router_rows && er < ne0;
    const bool router_block = blockIdx.x < ne0;  // holds at least one router row
    uint4 rw[kRouterChunks];
    uint32_t rsb[4], rbb[4];  // R8: the units' group scale and bias bits
    if (router_wave) {
        if constexpr (R8) {
            const uint32_t nunits = d0 / 16u;
            const uint8_t* w_row = reinterpret_cast<const uint8_t*>(global_ptr(k_router_w)) + (uint64_t)er * d0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                rw[i] = *reinterpret_cast<const uint4*>(w_row + min(lane + 64u * i, nunits - 1u) * 16u);
        } else {
            const uint16_t* w_row = global_ptr(k_router_w) + (uint64_t)er * d0;
#pragma unroll
            for (int i = 0; i < kRouterChunks; ++i)
                rw[i] = *reinterpret_cast<const uint4*>(w_row + min(lane + 64u * i, units - 1u) * 8u);
        }
    }
    // every thread reads the epoch (one request per wave), without a branch:
    // a load inside `if (t == 0)` left wave 0 waiting for it, and for its
    // router row issued before it, ahead of its x / es loads
    const uint32_t epoch = ld_coherent(global_ptr(k_sync) + kSyncEpochWord);
    const uint32_t gain = t < ne0 ? global_ptr(k_pes)[t] : 0u;
    const bool two = units > nthreads;
    const uint16_t* xg = global_ptr(k_x);
    const uint16_t* hg = global_ptr(k_hidden);
    const uint16_t* eg = global_ptr(k_es);
    uint4 xv[2], hv[2], ev[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (i == 1 && !two) break;
        const uint32_t q = min(t + i * nthreads, units - 1u) * 8u;
        xv[i] = *reinterpret_cast<const uint4*>(xg + q);
        if (router_block) {
            hv[i] = *reinterpret_cast<const uint4*>(hg + q);
            ev[i] = *reinterpret_cast<const uint4*>(eg + q);
        }
    }
    if constexpr (R8) {
        // the group scales and biases, whose pointers are kernel arguments
        // not preloaded: their loads wait for that read, so they go out after
        // every load that needs nothing but the preloaded arguments
        if (router_wave) {
            const uint16_t* rs = a_arg.router_s;
            const uint16_t* rb = a_arg.router_b;
            const uint32_t ngroups = d0 / G, nunits = d0 / 16u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t g = er * ngroups + min(lane + 64u * i, nunits - 1u) * 16u / G;
                rsb[i] = rs[g];
                rbb[i] = rb[g];
            }
        }
    }
    if (t < kArgWords) reinterpret_cast<uint32_t*>(&a)[t] = arg_word;
    if (t < kTopK) {
        s_idx[t] = 0u;
        s_fill[t] = 0u;
        s_skey[t] = 0u;
    }
    __syncthreads();
    const uint32_t d = a.d, f = a.f, ne = a.ne;
    const uint8_t* layer_base = global_ptr(a.layer_base);
    const DecodeSync sy = decode_sync(global_ptr(a.sync_words));
    uint64_t* handoff = global_ptr(a.handoff);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + lds_chunks_halves(d) * 2u);
    // the host places every region on 16 bytes; the masks let the compiler see
    // it and read the staged chunks 16 bytes at a time
    uint16_t* as = reinterpret_cast<uint16_t*>(smem + (a.as_off & ~15u));
    float* asum = reinterpret_cast<float*>(smem + (a.as_off & ~15u) + p2_slot_halves(f) * 2u);
    float* xe = reinterpret_cast<float*>(smem + (a.xe_off & ~15u));
    // expert row e's logit is computed once, by block e % kDecodeBlocks
    // (wave e / kDecodeBlocks), and posted to all kDecodeGroups regions; each
    // group polls its own copy, so 32 blocks, not 256, read each word
    uint64_t* logits = sy.logits + grp * kMaxExperts;
    uint64_t* gacts = handoff + (size_t)grp * kHandoffWords;
    const uint32_t nwaves = nthreads >> 6;
    const bool sh_wave = SH && wave == nwaves - 1u;
    const uint32_t share = (a.rows + kDecodeGroups - 1u) / kDecodeGroups;  // combine rows

    if (t < kMaxExperts) s_gains[t] = gain;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t q = t + i * nthreads;
        if (q >= units) break;
        *reinterpret_cast<uint4*>(xs + (q >> 2) * kChunkLds + (q & 3u) * 8u) = pair_permute(xv[i]);
        if (!router_block) continue;
        const uint32_t hw[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
        const uint32_t ew[4] = {ev[i].x, ev[i].y, ev[i].z, ev[i].w};
        float p[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            p[2 * k] = f16_to_f32((uint16_t)(hw[k] & 0xFFFFu)) * __uint_as_float(ew[k] << 16);
            p[2 * k + 1] = f16_to_f32((uint16_t)(hw[k] >> 16)) * __uint_as_float(ew[k] & 0xFFFF0000u);
        }
        *reinterpret_cast<float4*>(xe + q * 8u) = make_float4(p[0], p[1], p[2], p[3]);
        *reinterpret_cast<float4*>(xe + q * 8u + 4u) = make_float4(p[4], p[5], p[6], p[7]);
    }
    if (t == 0) {
        const uint32_t tag = epoch + 1u;
        s_tag = tag ? tag : 1u;
    }
    __syncthreads();
    const uint32_t tag = s_tag;
    if (router_wave) {
        const float s = R8 ? router_dot_int8_staged(rw, rsb, rbb, xe, d0 / 16u, lane)
                           : router_dot_staged(rw, xe, units, lane);
        if (lane < kDecodeGroups)
            st_coherent(sy.logits + lane * kMaxExperts + er, tagged(tag, __float_as_uint(s)));
    }
    if constexpr (!SYM) staged_chunk_sums(xs, 0u, 1u, d, xsum);
    // SH: this block's two shared gate/up pairs (lanes 0..31 pair 2b, 32..63
    // pair 2b + 1; 16 lanes per row) and the gate logit, while the logits are
    // gathered and ranked
    ChunkBatch<GUB> sbt;
    GULane sl{};
    float sh_scale = 0.0f;
    if constexpr (SH) {
        if (sh_wave) {
            const uint32_t p = 2u * blockIdx.x + (lane >> 5);
            const bool is_up = (lane >> 4) & 1u, live = p < a.sh_f;
            const uint32_t pr = live ? p : 0u, ng = d / G;
            const uint8_t* sb = global_ptr(a.sh_blob);
            sl.w = sb + (is_up ? a.sh_o.up_w : a.sh_o.gate_w) + (uint64_t)pr * (d / 2u);
            sl.s = reinterpret_cast<const uint16_t*>(sb + (is_up ? a.sh_o.up_s : a.sh_o.gate_s)) + (uint64_t)pr * ng;
            sl.b = reinterpret_cast<const uint16_t*>(sb + (is_up ? a.sh_o.up_b : a.sh_o.gate_b)) + (uint64_t)pr * ng;
            sl.fr = p;
            sl.live = live;
            load_batch<G, SYM, GUB, kGULanes>(sl.w, sl.s, sl.b, 0u, lane & 15u, d / 32u, sbt);
            sh_scale = qwen_sigmoid(gate_logit_wave(xg, global_ptr(a.sh_gate_w), d));
        }
    }

    // wave 0 gathers the group's logits and selects; the block waits once
    const uint32_t ne4 = (ne + 3u) & ~3u;
    if (wave == 0) {
        uint32_t key[4] = {0u, 0u, 0u, 0u};
        uint32_t live = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) live |= lane + 64u * j < ne ? 1u << j : 0u;
        poll_tagged<4, kPollSleepLogits>(sy, tag, live, [&](int j) { return logits + lane + 64u * j; },
                       [&](int j, uint32_t bits) {
                           const float v = __uint_as_float(bits);
                           key[j] = (v == v && v != -INFINITY) ? order_key(v) : 0u;
                       });
        wave_select_top8(key, ne4, s_cand, s_idx, s_fill, s_skey);
    }
    __syncthreads();

    // gate/up pairs of slot grp: mem * pairs + t / 32
    const uint32_t pl = t >> 5;
    const uint32_t fr = mem * a.pairs + pl;
    const bool pair_live = pl < a.pairs && fr < f;
    const LdsBlobs src{layer_base, a.expert_stride, s_idx};
    const bool gu_wave = 2u * wave < a.pairs;
    uint16_t s_wout = 0;  // wave 0: lane r's slot weight
    // this block's down rows (8 per wave), requested once the wave's gate/up
    // work is done: issued with the gate/up rows they share the memory
    // system with the gate/up stream and with the activation hand-off's
    // polls, and measured slower (the hand-off, not the down stream, is on
    // the critical path)
    const uint8_t* blob = layer_base + (uint64_t)s_idx[grp] * a.expert_stride;
    const uint32_t rl = 8u * wave + (lane >> 3);
    const uint32_t row = mem * a.rows + rl;
    const bool row_live = rl < a.rows && row < d;
    const bool down_wave = 8u * wave < a.rows;
    const uint32_t rr = row_live ? row : 0u;
    const uint32_t fgroups = f / G;
    const uint8_t* dw = blob + a.o.down_w + (uint64_t)rr * (f / 2u);
    const uint16_t* dsc = reinterpret_cast<const uint16_t*>(blob + a.o.down_s) + (uint64_t)rr * fgroups;
    const uint16_t* dbi = reinterpret_cast<const uint16_t*>(blob + a.o.down_b) + (uint64_t)rr * fgroups;
    ChunkBatch<DB> dbt;
    // Loads, the slot weights and the dot products in one straight-line
    // region per wave (wave 0 is always a gate/up wave: pairs >= 1), so the
    // waits before each chunk's dot product count only the loads after it.
    if (gu_wave) {
        ChunkBatch<GUB> gbt;
        const GULane l = gu_lane(src, a.o, d, G, pair_live ? grp : 0u, pair_live ? fr : 0u, pair_live);
        load_batch<G, SYM, GUB, kGULanes>(l.w, l.s, l.b, 0u, t & 15u, d / 32u, gbt);
        // the slot weights (needed only by the combine) while the loads fly
        if (wave == 0) {
            const uint32_t r = lane & (kTopK - 1u);
            const uint32_t id = s_idx[r];
            const float my_s = s_fill[r] ? order_key_value(s_skey[r]) : -INFINITY;
            const uint16_t w = slot_softmax_lane(my_s, bf16_to_f32((uint16_t)s_gains[id]));
            if (lane < kTopK) s_w[lane] = w;
            s_wout = w;
        }
        uint16_t act;
        if (phase1_compute<G, SYM, ACT, GUB>(l, gbt, xs, xsum, d, act)) {
            global_ptr(a.acts)[grp * f + fr] = act;
            st_coherent(gacts + fr, tagged(tag, act));
        }
        if (wave == 0 && blockIdx.x == 0 && lane < kTopK) {
            global_ptr(a.out_idx)[lane] = s_idx[lane];
            global_ptr(a.out_w)[lane] = s_wout;
        }
    }
    uint64_t* shacts = handoff + (size_t)kDecodeGroups * kHandoffWords;
    ChunkBatch<1> sdb[kMaxCombineRows / 4];
    if constexpr (SH) {
        if (sh_wave) {
            // act = half(silu(half(gate . x)) * half(up . x)) (shared_gate_up_kernel)
            const uint32_t j = lane & 15u, nck = d / 32u;
            float acc[1] = {0.0f};
            gemv_batches<G, SYM, GUB, kGULanes, 1>(sl.w, sl.s, sl.b, j, nck, sbt, xs, 0u, xsum, 1u,
                                                        acc);
            const float g = group16_sum(acc[0]);
            const float u = shfl_xor(g, 16);
            if (sl.live && ((lane >> 4) & 1u) == 0 && j == 0) {
                const uint16_t act = silu_mul_h(f32_to_f16(g), f32_to_f16(u));
                global_ptr(a.sh_acts)[sl.fr] = act;
                st_coherent(shacts + sl.fr, tagged(tag, act));
            }
            // the shared down rows of this block's combine rows, 4 per pass
            // (16 lanes per row, one chunk each: sh_f <= 512)
            const uint8_t* sb = global_ptr(a.sh_blob);
            const uint32_t fg = a.sh_f / G, fck = a.sh_f / 32u;
#pragma unroll
            for (uint32_t pp = 0; pp < kMaxCombineRows / 4; ++pp) {
                if (4u * pp >= share) break;
                const uint32_t i = 4u * pp + (lane >> 4);
                const uint32_t cl = grp * share + i, crow = mem * a.rows + cl;
                const uint32_t cr = (i < share && cl < a.rows && crow < d) ? crow : 0u;
                load_batch<G, SYM, 1, kGULanes>(
                    sb + a.sh_o.down_w + (uint64_t)cr * (a.sh_f / 2u),
                    reinterpret_cast<const uint16_t*>(sb + a.sh_o.down_s) + (uint64_t)cr * fg,
                    reinterpret_cast<const uint16_t*>(sb + a.sh_o.down_b) + (uint64_t)cr * fg, 0u, j,
                    fck, sdb[pp]);
            }
        }
    }

    if (down_wave) load_batch<G, SYM, DB, kDLanes>(dw, dsc, dbi, 0u, lane & 7u, f / 32u, dbt);

    // once this block's gate/up work is out, the last wave reads the slot's
    // activation row into LDS as its words arrive
    __syncthreads();
    if (wave == nwaves - 1u) {
        for (uint32_t i0 = 0; i0 < f; i0 += 64u * 16u) {
            uint32_t live = 0;
#pragma unroll
            for (uint32_t k = 0; k < 16; ++k) live |= i0 + lane + 64u * k < f ? 1u << k : 0u;
            poll_tagged<16, kPollSleepActs>(sy, tag, live, [&](int k) { return gacts + i0 + lane + 64u * k; },
                            [&](int k, uint32_t bits) {
                                const uint32_t i = i0 + lane + 64u * k, c = i & 31u;
                                as[(i >> 5) * kChunkLds + (c >> 3) * 8u + paired_pos(c & 7u)] =
                                    (uint16_t)bits;
                            });
        }
        if constexpr (SH) {
            uint16_t* ss = reinterpret_cast<uint16_t*>(smem + (a.ss_off & ~15u));
            float* ssum = reinterpret_cast<float*>(smem + (a.ss_off & ~15u) +
                                                   p2_slot_halves(a.sh_f) * 2u);
            uint32_t live = 0;
#pragma unroll
            for (uint32_t k = 0; k < kMaxSharedF / 64u; ++k) live |= lane + 64u * k < a.sh_f ? 1u << k : 0u;
            poll_tagged<kMaxSharedF / 64u, kPollSleepActs>(sy, tag, live, [&](int k) { return shacts + lane + 64u * k; },
                                           [&](int k, uint32_t bits) {
                                               const uint32_t i = lane + 64u * k, c = i & 31u;
                                               ss[(i >> 5) * kChunkLds + (c >> 3) * 8u + paired_pos(c & 7u)] =
                                                   (uint16_t)bits;
                                           });
            const uint32_t j = lane & 15u, fck = a.sh_f / 32u;
            if constexpr (!SYM) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS in order
                for (uint32_t q = lane; q < fck; q += 64u) {
                    const uint16_t* chunk = ss + q * kChunkLds;
                    float sum = 0.0f;
                    for (uint32_t k = 0; k < 32u; ++k)
                        sum += f16_to_f32(chunk[(k >> 3) * 8u + paired_pos(k & 7u)]);
                    ssum[q] = sum;
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // sharedOut of the combine rows (shared_down_kernel's arithmetic)
#pragma unroll
            for (uint32_t pp = 0; pp < kMaxCombineRows / 4; ++pp) {
                if (4u * pp >= share) break;
                float acc[1] = {0.0f};
                compute_batch<G, SYM, 1, kGULanes, 1>(sdb[pp], 0u, j, fck, ss, 0u, ssum, 1u, acc);
                const float v = group16_sum(acc[0]);
                const uint32_t i = 4u * pp + (lane >> 4);
                if (j == 0 && i < share)
                    s_sout[i] = f32_to_f16(f16_to_f32(f32_to_f16(v)) * sh_scale);
            }
        }
    }
    __syncthreads();
    if constexpr (!SYM) {
        staged_chunk_sums(as, 0u, 1u, f, asum);
        __syncthreads();
    }
    uint64_t* parts = handoff + kMaxFusedDim;  // slot g's partials at g * kHandoffWords
    if (down_wave) {
        const float v = slot_down_row<G, SYM, DB>(dw, dsc, dbi, as, asum, f, dbt);
        if ((lane & 7u) == 0 && row_live)
            st_coherent(parts + (size_t)grp * kHandoffWords + row, tagged(tag, __float_as_uint(v)));
    }

    // this block's share of row range mem: y = half(res + sum_s w_s v_s) in
    // slot order (moe.metal:678-686)
    if (wave == 0) {
        const uint32_t cl = grp * share + lane;
        const uint32_t crow = mem * a.rows + cl;
        const bool live = lane < share && cl < a.rows && crow < d;
        uint16_t res;
        if constexpr (SH) res = s_sout[lane < share ? lane : 0u];
        else res = global_ptr(a.residual)[live ? crow : 0u];
        float vq[kTopK];
        poll_tagged<kTopK, kPollSleepParts>(sy, tag, live ? 0xFFu : 0u,
                           [&](int q) { return parts + (size_t)q * kHandoffWords + crow; },
                           [&](int q, uint32_t bits) { vq[q] = __uint_as_float(bits); });
        if (live) {
            float out = f16_to_f32(res);
#pragma unroll
            for (uint32_t q = 0; q < kTopK; ++q) {
                const float p = f16_to_f32(s_w[q]) * vq[q];
                out = out + p;
            }
            global_ptr(a.y)[crow] = f32_to_f16(out);
        }
        // block 0 has now seen every group's partials: the next launch may
        // use tag + 1
        if (blockIdx.x == 0 && lane == 0) st_coherent(sy.epoch, tag);
    }
}

// ----------------------------------------------- one-launch verify layer

// One verify MoE layer of `rows` <= 8 tokens in one launch (kDecodeBlocks
// blocks of kVerifyThreads, all co-resident), the composition the verify step
// encodes per layer (RealForwardRunner.swift:1826-1872 router rows,
// :2116-2151 grouping, PrefillGroupedRoutedMoE.swift:793-917 encodeStreamedRows,
// PrefillMoE.swift:11-38 encodeReduceTokenMajor) with the same arithmetic as
// those separate launches, so every output is bit for bit theirs:
//  1. router: block e < ne holds router row e in registers; wave r < rows dots
//     it with token r's row (router_chunks_dot, the staged rows router's sum)
//     and posts the logit to the kDecodeGroups replicas (tagged words);
//  2. every block polls its group's replica and selects each token's top-8 on
//     wave r (wave_select_top8 + slot_softmax_lane, the rows router's steps),
//     then groups the rows * 8 pairs by a counting sort in LDS: slot u is the
//     u-th routed expert, its rows its pairs in token order (the device
//     grouping's sorted order);
//  3. gate/up: the U * f (slot, f) pairs are split over the blocks in
//     contiguous ranges of equal cost (a pair of a slot with m rows costs
//     kVerifyUnitBase + kVerifyRowCost * m); a 16-lane group holds a pair's
//     gate and up rows (the rows path's lane geometry and per-row steps over
//     the slot's rows, picked from the staged token rows); each activation is
//     posted as a tagged word;
//  4. down: the U * d (slot, row) outputs likewise, an 8-lane group holding
//     two adjacent rows; a block's range covers at most two slots, whose
//     activation rows it gathers into LDS (each wave's first rows requested
//     before the gather); each route partial half(down . act) is posted as a
//     tagged word;
//  5. the token-major sum h2[t, n] = half(sum_r fma(w[t, r], P[t, r, n]))
//     over the blocks' equal ranges of the rows * d outputs.
// The tag is the verify epoch + 1; every block posts an arrival word once it
// holds the tag, and block 0 advances the epoch after seeing all of them.
// Polls are bounded (timeouts set the error word). A token with fewer than 8
// eligible logits (NaN or -inf scores) makes every block write NaN outputs and
// the launch report the error.
// SH: the Qwen family's shared expert over the same rows (encodeSharedExpert
// per row, QwenForwardRunner.swift:1548-1578) is one more slot with every row,
// after the routed ones, in both splits; its pairs post
// half(silu(half(g)) * half(u)), its down rows take the shared down kernel's
// lane geometry (16 lanes a row) and are written as
// half(half(down . act) * sigmoid(gate_w . x_r)) with the logits summed by
// gate_logit_wave, so the shared output is bit for bit
// tsg_moe_shared_expert_rows'.
constexpr uint32_t kVerifyThreads = 512;  // 8 waves of up to 256 VGPRs
constexpr uint32_t kVerifyWaves = kVerifyThreads / 64u;
constexpr int kVerifyXUnits = (int)((kMaxRouterRows * 512u + kVerifyThreads - 1u) / kVerifyThreads);
// A unit (a gate/up pair or a down row) of a slot with m rows costs
// kVerifyUnitBase + kVerifyRowCost * m in the split of the units over the
// blocks: its weight bytes and its rows' dot products. Measured at configs[2]
// (bench.py, alternating runs): 3 + m 34.7-35.0 us per layer, 5 + m 35.7,
// 8 + m 36.4, 1 + m 35.8-36.0, 1 + 2 m 38.5, an equal split 37.8.
constexpr uint32_t kVerifyUnitBase = 3;
constexpr uint32_t kVerifyRowCost = 1;
constexpr uint32_t kRowsInOrder = 0xFAC688u;  // rows 0..7 as 3-bit picks
// Chunks per lane per batch of a shared-expert down row (16 lanes a row, as
// the shared down kernel; the batch size does not change a row's bits): one
// batch up to an intermediate size of 1024.
constexpr int kShDBatch = 2;

struct VerifyLayerArgs {
    const uint8_t* layer_base;
    uint64_t expert_stride;
    tsg_expert_offsets o;
    uint16_t* h2;
    uint32_t* out_idx;
    uint16_t* out_w;
    uint64_t* words;
    uint32_t* sync_words;
    uint32_t ne, d, f, rows;
    // SH: the Qwen-family shared expert over the same rows (its intermediate
    // size is f), its bf16 gate row and its [rows, d] output
    const uint8_t* sh_blob;
    tsg_expert_offsets sh_o;
    const uint16_t* sh_gate_w;
    uint16_t* sh_out;
};

// Dynamic LDS of the verify layer, in bytes from 0: the token rows in element
// order (router), the same rows in the GEMV's staged layout, their chunk sums
// (affine), and two slots' activation rows with their sums.
struct VerifyLds {
    uint32_t xs, xsum, as, asum, bytes;
};
__host__ __device__ __forceinline__ VerifyLds verify_lds(uint32_t rows, uint32_t d, uint32_t f,
                                                         bool sym) {
    VerifyLds l;
    // every region starts on 16 bytes (the rounding changes no offset, d being
    // a multiple of 64; it lets the compiler read the staged chunks 16 bytes
    // at a time)
    l.xs = (rows * d * 2u + 15u) & ~15u;
    l.xsum = l.xs + rows * lds_chunks_halves(d) * 2u;
    l.as = (l.xsum + (sym ? 0u : rows * (d / 32u) * 4u) + 15u) & ~15u;
    l.asum = l.as + 2u * rows * lds_chunks_halves(f) * 2u;
    l.bytes = l.asum + (sym ? 0u : 2u * rows * (f / 32u) * 4u);
    return l;
}

template <int G, bool SYM, int ACT, bool SH, bool Q>
// Q: chunk batches sized for d <= 2048 and f <= 512 (4 chunks a lane for a
// gate/up row, 2 for a down row, 1 for a shared down row), where the default
// sizes would carry slots no lane uses; a row's bits do not depend on them.
// The values the first loads need are leading scalar arguments (14 dwords,
// preloaded into SGPRs): k_ne_rows = ne | rows << 16, k_d_stride = d |
// hidden stride << 16.
__global__ __launch_bounds__(kVerifyThreads) void verify_layer_kernel(
    const uint16_t* k_router_w, const uint16_t* k_hidden, const uint16_t* k_es,
    const uint16_t* k_pes, const uint16_t* k_x, uint32_t* k_sync, uint32_t k_ne_rows,
    uint32_t k_d_stride, VerifyLayerArgs a_arg) {
    __shared__ VerifyLayerArgs a;
    constexpr uint32_t kArgWords = sizeof(VerifyLayerArgs) / 4;
    static_assert(sizeof(VerifyLayerArgs) % 4 == 0 && kArgWords <= kVerifyThreads, "args copy");
    constexpr int GUB = Q ? 4 : kGUBatch, DB = Q ? 2 : kDBatch, SDB = Q ? 1 : kShDBatch;
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
    const uint32_t arg_word = reinterpret_cast<const uint32_t*>(&a_arg)[min(t, kArgWords - 1u)];
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_tag, s_nslots;
    __shared__ uint32_t s_gains[kMaxExperts];
    __shared__ __align__(16) uint64_t s_cand[kMaxRouterRows][kMaxExperts + kCandBatch];
    __shared__ uint32_t s_sid[kMaxRouterRows][kTopK], s_sfill[kMaxRouterRows][kTopK];
    __shared__ uint32_t s_skey[kMaxRouterRows][kTopK];
    __shared__ uint32_t s_pe[kVerifyPairs], s_pw[kVerifyPairs];  // pair p = 8 t + r
    __shared__ uint32_t s_sp[kVerifyPairs];                      // sorted row -> pair
    __shared__ uint32_t s_uexp[kVerifyPairs], s_ustart[kVerifyPairs + 1];
    __shared__ uint32_t s_cnt[kMaxExperts], s_off[kMaxExperts];  // the grouping
    __shared__ uint32_t s_mask[kMaxRouterRows * kMaskWords], s_wtot[kMaxExperts / 64u];
    __shared__ uint32_t s_bad;
    __shared__ uint32_t s_split[4];  // gate/up pairs [0, 1), down outputs [2, 3)
    __shared__ float s_glog[SH ? kMaxRouterRows : 1];  // the rows' shared-expert gate logits

    const uint32_t ne = k_ne_rows & 0xFFFFu, rows = k_ne_rows >> 16;
    const uint32_t d = k_d_stride & 0xFFFFu, stride = k_d_stride >> 16;
    const uint32_t units = d / 8u;  // 16-byte units of a row
    const bool router_wave = blockIdx.x < ne && wave < rows;
    // every load of the first phase goes out before any is waited for: the
    // router row and es (router waves), the epoch, the gains, the token rows
    uint4 rw[kRouterChunks], rev[kRouterChunks];
    if (router_wave) {
        const uint16_t* w_row = global_ptr(k_router_w) + (uint64_t)blockIdx.x * d;
        const uint16_t* eg = global_ptr(k_es);
#pragma unroll
        for (int i = 0; i < kRouterChunks; ++i) {
            const uint32_t cc = min(lane + 64u * i, units - 1u);
            rw[i] = *reinterpret_cast<const uint4*>(w_row + cc * 8u);
            rev[i] = *reinterpret_cast<const uint4*>(eg + cc * 8u);
        }
    }
    const uint32_t epoch = ld_coherent(global_ptr(k_sync) + kVerifyEpochWord);
    const uint32_t gain = t < ne ? global_ptr(k_pes)[t] : 0u;
    const uint32_t total = rows * units;
    const bool same = k_x == k_hidden;
    const uint16_t* hg = global_ptr(k_hidden);
    const uint16_t* xg = global_ptr(k_x);
    uint4 hv[kVerifyXUnits], xv[kVerifyXUnits];
#pragma unroll
    for (int i = 0; i < kVerifyXUnits; ++i) {
        if ((uint32_t)i * kVerifyThreads >= total) break;
        const uint32_t q = min(t + (uint32_t)i * kVerifyThreads, total - 1u);
        const uint32_t r = q / units, c = q - r * units;
        hv[i] = *reinterpret_cast<const uint4*>(hg + (uint64_t)r * stride + c * 8u);
        if (!same) xv[i] = *reinterpret_cast<const uint4*>(xg + (uint64_t)r * stride + c * 8u);
    }
    if (t < kArgWords) reinterpret_cast<uint32_t*>(&a)[t] = arg_word;
    if (t < kMaxExperts) {
        s_gains[t] = gain;
        s_cnt[t] = 0u;
    }
    if (t < kMaxRouterRows * kMaskWords) s_mask[t] = 0u;
    if (t == 0) s_bad = 0u;
    const uint32_t row_h = lds_chunks_halves(d);
    const VerifyLds ld0 = verify_lds(rows, d, 0u, SYM);
    uint4* xn = reinterpret_cast<uint4*>(smem);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + ld0.xs);
    float* xsum = reinterpret_cast<float*>(smem + ld0.xsum);
#pragma unroll
    for (int i = 0; i < kVerifyXUnits; ++i) {
        if ((uint32_t)i * kVerifyThreads >= total) break;
        const uint32_t q = t + (uint32_t)i * kVerifyThreads;
        if (q < total) {
            const uint32_t r = q / units, c = q - r * units;
            xn[q] = hv[i];
            *reinterpret_cast<uint4*>(xs + r * row_h + (c >> 2) * kChunkLds + (c & 3u) * 8u) =
                pair_permute(same ? hv[i] : xv[i]);
        }
    }
    if (t == 0) {
        const uint32_t tg = epoch + 1u;
        s_tag = tg ? tg : 1u;  // the words start at tag 0
    }
    __syncthreads();
    const uint32_t tag = s_tag;
    const uint32_t f = a.f;
    uint64_t* words = global_ptr(a.words);
    DecodeSync sy{};
    sy.error = global_ptr(a.sync_words) + kSyncErrorWord;
    const uint32_t grp = blockIdx.x % kDecodeGroups;

    // 1. router row blockIdx.x against token row `wave`
    if (router_wave) {
        uint4 xr[kRouterChunks];
#pragma unroll
        for (int i = 0; i < kRouterChunks; ++i) xr[i] = xn[wave * units + min(lane + 64u * i, units - 1u)];
        const float s = router_chunks_dot(rw, xr, rev, units, lane);
        if (lane < kDecodeGroups)
            st_coherent(words + lane * kVerifyLogitRegion + wave * kMaxExperts + blockIdx.x,
                        tagged(tag, __float_as_uint(s)));
    }
    if (t == 0) st_coherent(words + kVerifyArriveWord + blockIdx.x, tagged(tag, 1u));
    if constexpr (!SYM) staged_chunk_sums(xs, row_h, rows, d, xsum);

    // 2. token `wave`'s top-8 from this group's replica
    if (wave < rows) {
        uint32_t key[4] = {0u, 0u, 0u, 0u};
        uint32_t live = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) live |= lane + 64u * j < ne ? 1u << j : 0u;
        const uint64_t* lg = words + grp * kVerifyLogitRegion + wave * kMaxExperts;
        poll_tagged<4, kPollSleepLogits>(sy, tag, live, [&](int j) { return lg + lane + 64u * j; },
                                         [&](int j, uint32_t bits) {
                                             const float v = __uint_as_float(bits);
                                             key[j] = (v == v && v != -INFINITY) ? order_key(v) : 0u;
                                         });
        if (lane < kTopK) {
            s_sid[wave][lane] = 0u;
            s_sfill[wave][lane] = 0u;
            s_skey[wave][lane] = 0u;
        }
        wave_select_top8(key, (ne + 3u) & ~3u, s_cand[wave], s_sid[wave], s_sfill[wave],
                         s_skey[wave]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS in order
        const uint32_t sl = lane & (kTopK - 1u);
        const uint32_t id = s_sid[wave][sl];
        const float my_s = s_sfill[wave][sl] ? order_key_value(s_skey[wave][sl]) : -INFINITY;
        const uint16_t wb = slot_softmax_lane(my_s, bf16_to_f32((uint16_t)s_gains[id]));
        if (lane < kTopK) {
            s_pe[wave * kTopK + lane] = id;
            s_pw[wave * kTopK + lane] = wb;
            if (!s_sfill[wave][lane]) s_bad = 1u;
        }
    }
    __syncthreads();
    // Fewer than 8 eligible logits for a token (NaN or -inf scores) leave
    // slots unfilled, naming expert 0 twice or more in one token: every block
    // sees it (the same selection everywhere), writes NaN for its outputs and
    // the launch reports it; the routing outputs are still written.
    const uint32_t np = rows * kTopK;
    const uint32_t nc_all = rows * d;
    const uint32_t cb0 = blockIdx.x * nc_all / kDecodeBlocks;
    const uint32_t cb1 = (blockIdx.x + 1u) * nc_all / kDecodeBlocks;
    const auto epoch_advance = [&] {
        // every block has read the epoch once its arrival word is in: the
        // next launch may use tag + 1
        if (blockIdx.x == 0 && wave == kVerifyWaves - 1u) {
            poll_tagged<kDecodeBlocks / 64u, kPollSleepActs>(
                sy, tag, (1u << (kDecodeBlocks / 64u)) - 1u,
                [&](int j) { return words + kVerifyArriveWord + lane + 64u * j; },
                [&](int, uint32_t) {});
            if (lane == 0) st_coherent(global_ptr(a.sync_words) + kVerifyEpochWord, tag);
        }
    };
    if (s_bad) {
        if (blockIdx.x == 0 && t < np) {
            global_ptr(a.out_idx)[t] = s_pe[t];
            global_ptr(a.out_w)[t] = (uint16_t)s_pw[t];
        }
        if (blockIdx.x == 0 && t == 0) atomicOr(sy.error, kErrVerifyRouting);
        for (uint32_t c = cb0 + t; c < cb1; c += kVerifyThreads) {
            global_ptr(a.h2)[c] = 0x7E00u;
            if constexpr (SH) global_ptr(a.sh_out)[c] = 0x7E00u;
        }
        epoch_advance();
        return;
    }
    // The grouping (group_router_rows' counting sort, in LDS): per-expert
    // counts and per-token expert masks, one scan over the experts (counts
    // and presence packed), then pair p's sorted row = its expert's offset +
    // the earlier tokens that chose the expert; slot u is the u-th expert
    // present, its rows those pairs in token order.
    const bool my_pair = t < np;
    const uint32_t my_e = my_pair ? s_pe[t] : 0u, my_tok = t / kTopK;
    if (my_pair) {
        atomicAdd(&s_cnt[my_e], 1u);
        atomicOr(&s_mask[my_tok * kMaskWords + (my_e >> 5)], 1u << (my_e & 31u));
    }
    lds_barrier();
    const uint32_t ecnt = t < ne ? s_cnt[t] : 0u;
    const uint32_t packed = ecnt | ((ecnt ? 1u : 0u) << 16);
    const uint32_t incl = t < kMaxExperts ? wave_inclusive_scan(packed) : 0u;
    if (t < kMaxExperts && lane == 63u) s_wtot[wave] = incl;
    lds_barrier();
    if (t < kMaxExperts) {
        uint32_t base = 0, total = 0;
#pragma unroll
        for (uint32_t w = 0; w < kMaxExperts / 64u; ++w) {
            base += w < wave ? s_wtot[w] : 0u;
            total += s_wtot[w];
        }
        const uint32_t excl = base + incl - packed;
        s_off[t] = excl & 0xFFFFu;
        if (ecnt) {
            s_uexp[excl >> 16] = t;
            s_ustart[excl >> 16] = excl & 0xFFFFu;
        }
        if (t == 0) {
            s_nslots = total >> 16;
            s_ustart[total >> 16] = np;
        }
    }
    lds_barrier();
    if (my_pair) {
        uint32_t rank = 0;
#pragma unroll
        for (uint32_t q = 0; q < kMaxRouterRows; ++q)
            rank += q < my_tok ? (s_mask[q * kMaskWords + (my_e >> 5)] >> (my_e & 31u)) & 1u : 0u;
        s_sp[s_off[my_e] + rank] = t;
        if (blockIdx.x == 0) {
            global_ptr(a.out_idx)[t] = my_e;
            global_ptr(a.out_w)[t] = (uint16_t)s_pw[t];
        }
    }
    // This block's ranges of the gate/up pairs (per slot f, 0) and the down
    // outputs (per slot d, 2): block b takes the units whose cost falls in
    // [b C / NB, (b + 1) C / NB) of the total C; down ranges start on even
    // outputs (row pairs never straddle a slot: d is even). One wave: lane u
    // holds slot u's unit cost and its inclusive prefix; the slot of a cost
    // position is the first lane whose prefix passes it. SH: the shared
    // expert is one more slot after the routed ones, with every row.
    if (wave == 1) {
        const uint32_t nsl = s_nslots;
        const uint32_t w = lane < nsl ? kVerifyUnitBase + kVerifyRowCost * (s_ustart[lane + 1u] - s_ustart[lane]) : 0u;
        const uint32_t wsum = wave_inclusive_scan(w);
        const uint32_t wtot = (uint32_t)__builtin_amdgcn_readlane((int)wsum, 63);
        const uint32_t wsh = SH ? kVerifyUnitBase + kVerifyRowCost * rows : 0u;
        // 32-bit arithmetic: per <= kMaxFusedDim and the costs sum to at most
        // 64 pairs' (3 + 1) plus the shared slot's 3 + 8, so (b + 1) * total
        // < 256 * 4096 * 267 < 2^32
        static_assert((uint64_t)kDecodeBlocks * kMaxFusedDim *
                              (kVerifyPairs * (kVerifyUnitBase + kVerifyRowCost) +
                               kVerifyUnitBase + kVerifyRowCost * kMaxRouterRows) <
                          (1ull << 32), "verify split in 32 bits");
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t per = q < 2u ? a.f : d;
            const uint32_t routed = per * wtot, total = routed + per * wsh;
            const uint32_t cpos = (blockIdx.x + (q & 1u)) * total / kDecodeBlocks;
            const uint64_t past = __ballot(lane < nsl && per * wsum > cpos);
            uint32_t unit = (nsl + (SH ? 1u : 0u)) * per;
            if (past) {
                const uint32_t us = (uint32_t)__builtin_ctzll(past);
                const uint32_t wu = (uint32_t)__builtin_amdgcn_readlane((int)w, (int)us);
                const uint32_t pu = (uint32_t)__builtin_amdgcn_readlane((int)wsum, (int)us) - wu;
                unit = us * per + (cpos - per * pu + wu - 1u) / wu;
            } else if (SH && cpos < total) {
                unit = nsl * per + (cpos - routed + wsh - 1u) / wsh;
            }
            if (lane == 0) s_split[q] = q < 2u ? unit : unit & ~1u;
        }
    }
    __syncthreads();
    const uint32_t nslots = s_nslots;
    const uint8_t* layer_base = global_ptr(a.layer_base);
    uint64_t* acts_w = words + kVerifyActWord;

    // 3. gate/up: this block's pairs [pb0, pb0 + npb) of the nslots * f. A
    // 16-lane group takes one pair, its gate row and its up row (lane j holds
    // chunks j, j + 16, ... of both, the rows path's lane geometry and per-row
    // steps over the slot's rows, picked from the staged token rows), so each
    // staged activation chunk is read from LDS once for the two rows; a wave
    // takes 4 pairs per pass.
    // SH: units past the routed pairs are the shared expert's pairs (every
    // row, the shared kernels' epilogue half(silu(half(g)) * half(u)))
    const uint32_t np_all = nslots * f, np_units = np_all + (SH ? f : 0u);
    const uint32_t pb0 = s_split[0], npb = s_split[1] - pb0;
    const uint32_t j16 = lane & 15u;
    const uint32_t nck_d = d / 32u;
    uint64_t* sh_acts_w = words + kVerifySharedActWord;
    for (uint32_t k0 = 4u * wave; k0 < npb; k0 += 4u * kVerifyWaves) {  // wave-uniform
        const uint32_t k = k0 + (lane >> 4);
        const bool live = k < npb;
        const uint32_t p = min(pb0 + k, np_units - 1u);
        const bool shp = SH && p >= np_all;
        const uint32_t u = shp ? 0u : p / f, fi = shp ? p - np_all : p - u * f;
        const uint32_t start = shp ? 0u : s_ustart[u];
        const uint32_t m = shp ? rows : s_ustart[u + 1u] - start;
        const uint8_t* blob = shp ? global_ptr(a.sh_blob) : layer_base + (uint64_t)s_uexp[u] * a.expert_stride;
        const tsg_expert_offsets& eo = shp ? a.sh_o : a.o;
        const uint32_t ng = d / G;
        const uint8_t* gw = blob + eo.gate_w + (uint64_t)fi * (d / 2u);
        const uint8_t* uw = blob + eo.up_w + (uint64_t)fi * (d / 2u);
        const uint16_t* gs = reinterpret_cast<const uint16_t*>(blob + eo.gate_s) + (uint64_t)fi * ng;
        const uint16_t* us = reinterpret_cast<const uint16_t*>(blob + eo.up_s) + (uint64_t)fi * ng;
        const uint16_t* gb = reinterpret_cast<const uint16_t*>(blob + eo.gate_b) + (uint64_t)fi * ng;
        const uint16_t* ub = reinterpret_cast<const uint16_t*>(blob + eo.up_b) + (uint64_t)fi * ng;
        ChunkBatch<GUB> bg, bu;
        load_batch<G, SYM, GUB, kGULanes>(gw, gs, gb, 0u, j16, nck_d, bg);
        load_batch<G, SYM, GUB, kGULanes>(uw, us, ub, 0u, j16, nck_d, bu);
        uint32_t rt = kRowsInOrder;  // the rows' tokens, 3 bits each
        if (!shp) {
            rt = 0u;
#pragma unroll
            for (uint32_t r = 0; r < kMaxRouterRows; ++r)
                rt |= (s_sp[start + min(r, m - 1u)] >> 3) << (3u * r);
        }
        float ag[kMaxRouterRows], au[kMaxRouterRows];
#pragma unroll
        for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
            ag[r] = 0.0f;
            au[r] = 0.0f;
        }
        gemv_batches_picked2<G, SYM, GUB, kGULanes, (int)kMaxRouterRows>(
            gw, gs, gb, uw, us, ub, j16, nck_d, bg, bu, xs, row_h, xsum, rt, m, ag, au);
#pragma unroll
        for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
            const float gsum = group16_sum(ag[r]), usum = group16_sum(au[r]);
            if (live && j16 == 0 && r < m) {
                if (shp)
                    st_coherent(sh_acts_w + (uint64_t)r * f + fi,
                                tagged(tag, silu_mul_h(f32_to_f16(gsum), f32_to_f16(usum))));
                else
                    st_coherent(acts_w + (uint64_t)(start + r) * f + fi,
                                tagged(tag, f32_to_f16(gate_activation<ACT>(gsum) * usum)));
            }
        }
    }

    // 4. down: this block's outputs [qb0, qb0 + nqb) of the nslots * d (at
    // most d of them: two slots at most). An 8-lane group takes two adjacent
    // output rows (the ranges start on even outputs and d is even, so both
    // are of one slot; lane j holds chunks j, j + 8, ... of both, decode's
    // per-row steps), so each staged activation chunk is read once for the
    // two rows; a wave takes 16 rows per pass and requests its first pass's
    // rows before the activations are in. SH: outputs past the routed ones
    // are the shared expert's rows, two per 16-lane group (the shared down
    // kernel's lane geometry and steps), scaled by the token's gate.
    const uint32_t nq_all = nslots * d;
    const uint32_t qb0 = s_split[2], nqb = s_split[3] - qb0;
    const uint32_t nqr = qb0 < nq_all ? min(nqb, nq_all - qb0) : 0u;  // routed outputs
    const uint32_t nqs = nqb - nqr;                                    // shared rows (SH)
    const uint32_t qs0 = nqs != 0u ? qb0 + nqr - nq_all : 0u;          // the first of them
    const uint32_t j8 = lane & 7u;
    const uint32_t nck_f = f / 32u;
    struct DownPair {
        const uint8_t* w;
        const uint16_t* s;
        const uint16_t* b;
        uint32_t u, n;
        bool live;
    };
    // rows q0 + 2 k and q0 + 2 k + 1 share u; the second row's weights are
    // f / 2 bytes and f / G groups further on
    const auto dn_pair = [&](uint32_t k, ChunkBatch<DB>& b0, ChunkBatch<DB>& b1) {
        DownPair p;
        p.live = 2u * k < nqr;
        const uint32_t q = min(qb0 + 2u * k, nq_all - 2u);
        p.u = q / d;
        p.n = q - p.u * d;
        const uint8_t* blob = layer_base + (uint64_t)s_uexp[p.u] * a.expert_stride;
        const uint32_t ng = f / G;
        p.w = blob + a.o.down_w + (uint64_t)p.n * (f / 2u);
        p.s = reinterpret_cast<const uint16_t*>(blob + a.o.down_s) + (uint64_t)p.n * ng;
        p.b = reinterpret_cast<const uint16_t*>(blob + a.o.down_b) + (uint64_t)p.n * ng;
        load_batch<G, SYM, DB, kDLanes>(p.w, p.s, p.b, 0u, j8, nck_f, b0);
        load_batch<G, SYM, DB, kDLanes>(p.w + f / 2u, p.s + ng, p.b + ng, 0u, j8, nck_f, b1);
        return p;
    };
    constexpr uint32_t kDnPass = 8u * kVerifyWaves;  // row pairs per pass of the block
    const bool dn_a = 16u * wave < nqr;
    DownPair da{};
    ChunkBatch<DB> da0, da1;
    if (dn_a) da = dn_pair(8u * wave + (lane >> 3), da0, da1);
    // SH: the gate logits of the rows this block's shared outputs scale by
    if (SH && nqs != 0 && wave < rows) {
        const float g = gate_logit_wave(xg + (uint64_t)wave * stride, global_ptr(a.sh_gate_w), d);
        if (lane == 0) s_glog[wave] = g;
    }
    epoch_advance();
    uint64_t* parts = words + kVerifyPartWord;
    // the activation rows of the (at most two) slots the range covers
    // (nqb == 0, block-uniform, only when nslots * d < kDecodeBlocks)
    if (nqb != 0) {
        const uint32_t u_lo = qb0 / d, u_hi = (qb0 + nqb - 1u) / d;
        // slot u's activation rows: the sorted rows from s_ustart[u], or
        // (SH, u == nslots) the shared expert's rows in token order
        const auto slot_rows = [&](uint32_t u, uint32_t& st, uint32_t& m) {
            const bool sh = SH && u == nslots;
            st = sh ? 0u : s_ustart[u];
            m = sh ? rows : s_ustart[u + 1u] - st;
            return sh ? sh_acts_w : acts_w + (uint64_t)st * f;
        };
        uint32_t st_lo, m_lo, st_hi = 0u, m_hi = 0u;
        const uint64_t* src_lo = slot_rows(u_lo, st_lo, m_lo);
        const uint64_t* src_hi = src_lo;
        if (u_hi != u_lo) src_hi = slot_rows(u_hi, st_hi, m_hi);
        const uint32_t arows = m_lo + m_hi;  // <= 2 * rows
        const VerifyLds ldf = verify_lds(rows, d, f, SYM);
        uint16_t* as = reinterpret_cast<uint16_t*>(smem + ldf.as);
        float* asum = reinterpret_cast<float*>(smem + ldf.asum);
        const uint32_t row_hf = lds_chunks_halves(f);
        // thread t gathers column fi = t (+ kVerifyThreads ...) of every
        // staged row, 8 rows per poll
        for (uint32_t fi0 = 0; fi0 < f; fi0 += kVerifyThreads) {
            const uint32_t fi = fi0 + t;
            const uint32_t c = fi & 31u;
            uint16_t* dst = as + (fi >> 5) * kChunkLds + (c >> 3) * 8u + paired_pos(c & 7u);
            for (uint32_t r0 = 0; r0 < arows; r0 += kMaxRouterRows) {
                const uint32_t nr = min(arows - r0, kMaxRouterRows);
                poll_tagged<kMaxRouterRows, kPollSleepActs>(
                    sy, tag, fi < f ? (1u << nr) - 1u : 0u,
                    [&](int k) {
                        const uint32_t r = r0 + k;
                        return r < m_lo ? src_lo + (uint64_t)r * f + fi
                                        : src_hi + (uint64_t)(r - m_lo) * f + fi;
                    },
                    [&](int k, uint32_t bits) { dst[(r0 + k) * row_hf] = (uint16_t)bits; });
            }
        }
        __syncthreads();
        if constexpr (!SYM) {
            staged_chunk_sums(as, row_hf, arows, f, asum);
            __syncthreads();
        }
        const auto dn_run = [&](const DownPair& p, ChunkBatch<DB>& b0, ChunkBatch<DB>& b1) {
            const bool hi = p.u != u_lo;
            const uint32_t st = hi ? st_hi : st_lo, m = hi ? m_hi : m_lo;
            const uint32_t ng = f / G;
            float a0[kMaxRouterRows], a1[kMaxRouterRows];
#pragma unroll
            for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
                a0[r] = 0.0f;
                a1[r] = 0.0f;
            }
            gemv_batches_picked2<G, SYM, DB, kDLanes, (int)kMaxRouterRows>(
                p.w, p.s, p.b, p.w + f / 2u, p.s + ng, p.b + ng, j8, nck_f, b0, b1,
                as + (hi ? m_lo : 0u) * row_hf, row_hf, asum + (hi ? m_lo : 0u) * nck_f,
                kRowsInOrder, m, a0, a1);
#pragma unroll
            for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
                const float v0 = group8_sum(a0[r]), v1 = group8_sum(a1[r]);
                if (p.live && j8 == 0 && r < m) {
                    uint64_t* dst = parts + (uint64_t)s_sp[st + r] * d + p.n;
                    st_coherent(dst, tagged(tag, (uint32_t)f32_to_f16(v0)));
                    st_coherent(dst + 1, tagged(tag, (uint32_t)f32_to_f16(v1)));
                }
            }
        };
        if (dn_a) dn_run(da, da0, da1);
        for (uint32_t k0 = kDnPass; 2u * k0 < nqr; k0 += kDnPass) {
            if (2u * (k0 + 8u * wave) >= nqr) break;  // wave-uniform
            ChunkBatch<DB> dc0, dc1;
            const DownPair dc = dn_pair(k0 + 8u * wave + (lane >> 3), dc0, dc1);
            dn_run(dc, dc0, dc1);
        }
        if constexpr (SH) {
            // the shared rows [qs0, qs0 + nqs): 4 row pairs per wave per pass
            const uint32_t sh_row0 = u_lo == nslots ? 0u : m_lo;  // their staged rows
            const uint8_t* sb = global_ptr(a.sh_blob);
            const uint32_t ng = f / G;
            for (uint32_t k0 = 4u * wave; 2u * k0 < nqs; k0 += 4u * kVerifyWaves) {  // wave-uniform
                const uint32_t k = k0 + (lane >> 4);
                const bool live = 2u * k < nqs;
                const uint32_t n = min(qs0 + 2u * k, d - 2u);
                const uint8_t* w = sb + a.sh_o.down_w + (uint64_t)n * (f / 2u);
                const uint16_t* sc = reinterpret_cast<const uint16_t*>(sb + a.sh_o.down_s) + (uint64_t)n * ng;
                const uint16_t* bi = reinterpret_cast<const uint16_t*>(sb + a.sh_o.down_b) + (uint64_t)n * ng;
                ChunkBatch<SDB> b0, b1;
                load_batch<G, SYM, SDB, kGULanes>(w, sc, bi, 0u, j16, nck_f, b0);
                load_batch<G, SYM, SDB, kGULanes>(w + f / 2u, sc + ng, bi + ng, 0u, j16, nck_f, b1);
                float a0[kMaxRouterRows], a1[kMaxRouterRows];
#pragma unroll
                for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
                    a0[r] = 0.0f;
                    a1[r] = 0.0f;
                }
                gemv_batches_picked2<G, SYM, SDB, kGULanes, (int)kMaxRouterRows>(
                    w, sc, bi, w + f / 2u, sc + ng, bi + ng, j16, nck_f, b0, b1,
                    as + sh_row0 * row_hf, row_hf, asum + sh_row0 * nck_f, kRowsInOrder, rows, a0,
                    a1);
#pragma unroll
                for (uint32_t r = 0; r < kMaxRouterRows; ++r) {
                    const float v0 = group16_sum(a0[r]), v1 = group16_sum(a1[r]);
                    if (live && j16 == 0 && r < rows) {
                        const float gs = qwen_sigmoid(s_glog[r]);
                        uint16_t* dst = global_ptr(a.sh_out) + (uint64_t)r * d + n;
                        dst[0] = f32_to_f16(f16_to_f32(f32_to_f16(v0)) * gs);
                        dst[1] = f32_to_f16(f16_to_f32(f32_to_f16(v1)) * gs);
                    }
                }
            }
        }
    }

    // 5. the token-major sum over this block's outputs [cb0, cb1)
    for (uint32_t c0 = cb0; c0 < cb1; c0 += kVerifyThreads) {
        const uint32_t c = c0 + t;
        const bool live = c < cb1;
        const uint32_t tok = live ? c / d : 0u, n = live ? c - tok * d : 0u;
        uint32_t pv[kTopK];
        poll_tagged<kTopK, kPollSleepParts>(
            sy, tag, live ? (1u << kTopK) - 1u : 0u,
            [&](int r) { return parts + (uint64_t)(tok * kTopK + r) * d + n; },
            [&](int r, uint32_t bits) { pv[r] = bits; });
        if (live) {
            float acc = 0.0f;
#pragma unroll
            for (uint32_t r = 0; r < kTopK; ++r)
                acc = __builtin_fmaf(f16_to_f32((uint16_t)s_pw[tok * kTopK + r]),
                                     f16_to_f32((uint16_t)pv[r]), acc);
            global_ptr(a.h2)[(uint64_t)tok * d + n] = f32_to_f16(acc);
        }
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
                         uint32_t top_k, bool select, const RouterGroupOut* group = nullptr) {
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
    TSG_REQUIRE(moe->router_weight_bits == 16, TSG_ERR_INVALID_ARGUMENT,
                "BF16 router encode on a %u-bit router", moe->router_weight_bits);
    tsg_ctx* ctx = moe->ctx;
    const dim3 grid((ne + kRouterWaves - 1) / kRouterWaves, (rows + kRouterRows - 1) / kRouterRows);
    // a few rows of one y-block are staged in LDS (same sums, no per-row
    // round trip to memory); the one-row and prompt-sized forms are not
    const size_t stage = (size_t)rows * d * 2u;
    const bool staged = select && (rows > 1 || group) && rows <= kMaxRouterRows &&
                        stage <= 64u * 1024u;
    TSG_REQUIRE(!group || staged, TSG_ERR_UNSUPPORTED,
                "the grouped router takes 1..%u rows of at most %zu bytes", kMaxRouterRows,
                (size_t)64u * 1024u);
    const dim3 sgrid(ne, 1);  // staged: one expert per block
    if (select) {
        TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK,
                    top_k);
        TSG_REQUIRE(pes && out_idx && out_w, TSG_ERR_INVALID_ARGUMENT, "NULL router output");
        if (staged) {
            auto kern = group ? router_kernel<true, true, true> : router_kernel<true, true, false>;
            // the staged rows take up to 64 KiB of dynamic LDS (idempotent)
            TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            64 * 1024));
            hipLaunchKernelGGL(kern, sgrid, dim3(64u * kStageWaves), stage, stream, w, hidden,
                               es, pes, ctx->counters, stride, ne, d, rows, ctx->logits,
                               kMaxExperts, out_idx, out_w, top_k,
                               group ? *group : RouterGroupOut{});
        }
        else
            hipLaunchKernelGGL((router_kernel<true, false, false>), grid, dim3(256), 0, stream, w,
                               hidden, es, pes, ctx->counters, stride, ne, d, rows, ctx->logits,
                               kMaxExperts, out_idx, out_w, top_k, RouterGroupOut{});
    } else {
        TSG_REQUIRE(logits_out, TSG_ERR_INVALID_ARGUMENT, "out_logits is NULL");
        hipLaunchKernelGGL((router_kernel<false, false, false>), grid, dim3(256), 0, stream, w,
                           hidden, es, pes, ctx->counters, stride, ne, d, rows, logits_out, ne,
                           out_idx, out_w, top_k, RouterGroupOut{});
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
template <int G, bool SYM, int ACT, bool SH, bool R8, bool Q = false>
tsg_status launch_fused(tsg_moe* moe, hipStream_t stream, DecodeLayerArgs a) {
    const auto up64 = [](uint32_t v) { return (v + 63u) / 64u * 64u; };
    uint32_t threads = 32u * a.pairs;                               // gate/up pairs
    if (SH) threads = 64u * ((a.pairs + 1u) / 2u + 1u);             // + the shared wave
    threads = std::max(threads, 64u * ((a.rows + 7u) / 8u + 1u));    // down rows, 8 per wave, + poll wave
    threads = std::max(threads, 64u * a.router_rows);                // router rows
    threads = std::max(threads, up64((a.d / 8u + 1u) / 2u));         // x in two 16-byte units
    const uint32_t xs_bytes = lds_chunks_halves(a.d) * 2u + (SYM ? 0u : (a.d / 32u) * 4u);
    const uint32_t as_bytes = p2_slot_halves(a.f) * 2u + (SYM ? 0u : (a.f / 32u) * 4u);
    a.as_off = (xs_bytes + 15u) & ~15u;
    a.xe_off = (a.as_off + as_bytes + 15u) & ~15u;
    size_t lds = a.xe_off + a.d * 4u;
    if (SH) {
        a.ss_off = (uint32_t)((lds + 15u) & ~(size_t)15u);
        lds = a.ss_off + p2_slot_halves(a.sh_f) * 2u + (SYM ? 0u : (a.sh_f / 32u) * 4u);
    }
    auto kern = decode_layer_kernel<G, SYM, ACT, SH, R8, Q>;
    int per_cu = 0;
    if (threads > decode_layer_max_threads(SH) || a.ne > kMaxExperts || a.f > kMaxFusedDim || a.d > kMaxFusedDim ||
        (a.rows + kDecodeGroups - 1u) / kDecodeGroups > kMaxCombineRows ||
        (SH && (a.sh_f > kMaxSharedF || a.sh_f > 2u * kDecodeBlocks)) ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, (int)threads, lds) !=
            hipSuccess ||
        (uint64_t)per_cu * (uint64_t)moe->ctx->num_cus < kDecodeBlocks)
        return TSG_ERR_DECLINED;
    a.threads = threads;
    hipLaunchKernelGGL(kern, dim3(kDecodeBlocks), dim3(threads), lds, stream, a.router_w,
                       a.router_hidden, a.es, a.pes, a.x, a.sync_words, a.ne | (a.router_rows << 16),
                       a.d | (threads << 16), a);
    return check_launch("decode_layer");
}

template <bool SH, bool R8>
tsg_status fused_dispatch(tsg_moe* moe, hipStream_t stream, const DecodeLayerArgs& a) {
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const bool silu = moe->activation == TSG_ACT_SILU;
    if constexpr (SH && !R8) {
        // the Qwen family's shapes (d = 2048, f = 512) take the compact batches
        if (silu && a.d <= 2048u && a.f <= 512u) {
            if (ctx->group_size == 32)
                return sym ? launch_fused<32, true, TSG_ACT_SILU, true, false, true>(moe, stream, a)
                           : launch_fused<32, false, TSG_ACT_SILU, true, false, true>(moe, stream, a);
            return sym ? launch_fused<64, true, TSG_ACT_SILU, true, false, true>(moe, stream, a)
                       : launch_fused<64, false, TSG_ACT_SILU, true, false, true>(moe, stream, a);
        }
    }
#define TSG_FU(GG, SS)                                                             \
    return silu ? launch_fused<GG, SS, TSG_ACT_SILU, SH, R8>(moe, stream, a)       \
                : launch_fused<GG, SS, TSG_ACT_GELU_TANH, SH, R8>(moe, stream, a)
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

extern "C" tsg_status tsg_moe_router_bf16_rows_grouped(
    tsg_moe* moe, tsg_stream stream, const uint16_t* w, const uint16_t* hidden, uint32_t stride,
    const uint16_t* es, const uint16_t* pes, uint32_t* out_idx, uint16_t* out_w, uint32_t rows,
    uint32_t ne, uint32_t d, uint32_t top_k, tsg_token_expert_pair* sorted, uint32_t* offsets,
    uint32_t* counts, tsg_routed_block* blocks, uint32_t max_blocks, uint32_t* n_blocks) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK, top_k);
    TSG_REQUIRE(ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT, "numExperts %u > %u", ne, kMaxExperts);
    if (rows == 0 || rows > kMaxRouterRows)
        return fail(TSG_ERR_DECLINED, "rows router takes 1..%u rows, got %u", kMaxRouterRows,
                    rows);
    TSG_REQUIRE(sorted && offsets && counts && blocks && n_blocks, TSG_ERR_INVALID_ARGUMENT,
                "NULL grouping output");
    TSG_REQUIRE(max_blocks >= std::min(rows * kTopK, ne), TSG_ERR_INVALID_ARGUMENT,
                "max_blocks %u cannot hold the work list: need min(rows*8, numExperts) = %u",
                max_blocks, std::min(rows * kTopK, ne));
    const RouterGroupOut g{sorted, offsets, counts, blocks, n_blocks};
    return router_launch(moe, as_stream(stream), w, hidden, stride, es, pes, out_idx, out_w,
                         nullptr, rows, ne, d, top_k, true, &g);
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

// encodeRouterGemma4 (MoE.swift:201-257): the INT8-affine router on a MoE
// created with 8-bit router weights, at the context's group size.
tsg_status router_int8_launch(tsg_moe* moe, hipStream_t stream, const uint8_t* w,
                              const uint16_t* scales, const uint16_t* biases,
                              const uint16_t* hidden, const uint16_t* es, const uint16_t* pes,
                              uint32_t* out_idx, uint16_t* out_w, uint32_t ne, uint32_t d,
                              uint32_t top_k) {
    TSG_REQUIRE(moe->router_weight_bits == 8, TSG_ERR_INVALID_ARGUMENT,
                "INT8 router encode on a %u-bit router", moe->router_weight_bits);
    const uint32_t g = moe->ctx->group_size;
    TSG_REQUIRE(top_k == kTopK, TSG_ERR_INVALID_ARGUMENT, "topK must be %u, got %u", kTopK, top_k);
    TSG_REQUIRE(ne > 0 && ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "numExperts %u not in 1..%u", ne, kMaxExperts);
    // the reference walks a row in 64-element steps (MoE.swift:215-217)
    TSG_REQUIRE(d > 0 && d % 64u == 0 && d % g == 0 && d <= 16u * 64u * kInt8Units,
                TSG_ERR_INVALID_ARGUMENT,
                "d=%u must be a positive multiple of 64 and of the group size %u, at most %u", d,
                g, 16u * 64u * kInt8Units);
    TSG_REQUIRE(w && scales && biases && hidden && es && pes && out_idx && out_w,
                TSG_ERR_INVALID_ARGUMENT, "NULL router operand");
    TSG_REQUIRE(aligned16(w) && aligned16(hidden) && aligned16(es), TSG_ERR_ALIGNMENT,
                "router weights, hidden and effective_scale must be 16-byte aligned");
    TSG_REQUIRE(((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases) |
                  reinterpret_cast<uintptr_t>(pes)) & 1u) == 0,
                TSG_ERR_ALIGNMENT, "scales, biases and per_expert_scale must be 2-byte aligned");
    tsg_ctx* ctx = moe->ctx;
    const dim3 grid((ne + kRouterWaves - 1) / kRouterWaves);
    auto kern = g == 32 ? router_int8_kernel<32> : router_int8_kernel<64>;
    hipLaunchKernelGGL(kern, grid, dim3(64u * kRouterWaves), 0, stream, w, scales, biases,
                       hidden, es, pes, ctx->counters, ne, d, ctx->logits, out_idx, out_w);
    return check_launch("router_int8");
}

extern "C" tsg_status tsg_moe_router_int8(tsg_moe* moe, tsg_stream stream, const uint8_t* w,
                                          const uint16_t* scales, const uint16_t* biases,
                                          const uint16_t* hidden, const uint16_t* es,
                                          const uint16_t* pes, uint32_t* out_idx,
                                          uint16_t* out_w, uint32_t ne, uint32_t d,
                                          uint32_t top_k) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    return router_int8_launch(moe, as_stream(stream), w, scales, biases, hidden, es, pes,
                              out_idx, out_w, ne, d, top_k);
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

struct SharedBranch {
    const uint8_t* blob;
    tsg_expert_offsets o;
    const uint16_t* gate_w;
    uint16_t* acts;
    uint32_t f;
};

// The INT8 router's tensors (encodeRouterGemma4's weights, scales, biases).
struct RouterInt8 {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
};

tsg_status decode_layer_impl(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                             const uint16_t* router_w, const uint16_t* router_hidden,
                             const uint16_t* es, const uint16_t* pes, const uint16_t* x,
                             const uint16_t* residual, uint16_t* y, uint32_t* out_idx,
                             uint16_t* out_w, uint16_t* acts, uint32_t ne, uint32_t d,
                             uint32_t f, uint32_t top_k, const SharedBranch* sh,
                             const RouterInt8* r8 = nullptr) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    TSG_REQUIRE(moe->router_weight_bits == (r8 ? 8u : 16u), TSG_ERR_INVALID_ARGUMENT,
                "%s router weights on a MoE created with %u-bit router weights",
                r8 ? "INT8" : "BF16", moe->router_weight_bits);
    if (r8) {
        router_w = reinterpret_cast<const uint16_t*>(r8->w);
        const uint32_t g = moe->ctx->group_size;
        TSG_REQUIRE(r8->s && r8->b, TSG_ERR_INVALID_ARGUMENT, "NULL router scales/biases");
        TSG_REQUIRE(((reinterpret_cast<uintptr_t>(r8->s) | reinterpret_cast<uintptr_t>(r8->b)) & 1u) == 0,
                    TSG_ERR_ALIGNMENT, "router scales and biases must be 2-byte aligned");
        TSG_REQUIRE(d % 64u == 0 && d % g == 0, TSG_ERR_INVALID_ARGUMENT,
                    "d=%u must be a multiple of 64 and of the group size %u (INT8 router)", d, g);
    }
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
    DecodeLayerArgs a{};
    a.layer_base = layer->base;
    a.expert_stride = layer->expert_stride;
    a.o = layer->offsets;
    a.router_w = router_w;
    a.router_s = r8 ? r8->s : nullptr;
    a.router_b = r8 ? r8->b : nullptr;
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
    a.handoff = reinterpret_cast<uint64_t*>(moe->ctx->act_replicas);
    a.ne = ne;
    a.d = d;
    a.f = f;
    a.router_rows = (ne + kDecodeBlocks - 1u) / kDecodeBlocks;
    a.pairs = (f + kGroupMembers - 1u) / kGroupMembers;
    a.rows = (d + kGroupMembers - 1u) / kGroupMembers;
    if (sh) {
        a.sh_blob = sh->blob;
        a.sh_o = sh->o;
        a.sh_gate_w = sh->gate_w;
        a.sh_acts = sh->acts;
        a.sh_f = sh->f;
    }
    if (!moe->unfused_decode) {
        // (no one-launch form of the shared branch with the INT8 router)
        st = r8 ? (sh ? TSG_ERR_DECLINED : fused_dispatch<false, true>(moe, s, a))
                : (sh ? fused_dispatch<true, false>(moe, s, a) : fused_dispatch<false, false>(moe, s, a));
        if (st != TSG_ERR_DECLINED) return st;
    }
    if (sh) {
        // the shared branch into y, then the routed experts on top of it
        // (QwenForwardRunner.swift:1583-1608: residual = y = sharedOut)
        if ((st = tsg_moe_shared_expert(moe, stream, sh->blob, &sh->o, x, sh->gate_w, sh->acts,
                                        y, d, sh->f)))
            return st;
        residual = y;
    }
    if ((st = r8 ? router_int8_launch(moe, s, r8->w, r8->s, r8->b, router_hidden, es, pes,
                                      out_idx, out_w, ne, d, top_k)
                 : router_launch(moe, s, router_w, router_hidden, d, es, pes, out_idx, out_w,
                                 nullptr, 1, ne, d, top_k, true)))
        return st;
    BlobSource src;
    if ((st = blobs_from_layer(layer, out_idx, &src))) return st;
    if ((st = phase1_dispatch(moe, s, src, layer->offsets, x, acts, d, f, top_k, false)))
        return st;
    return phase2_dispatch(moe, s, src, layer->offsets, acts, out_w, residual, y, d, f);
}

extern "C" tsg_status tsg_moe_decode_layer(tsg_moe* moe, tsg_stream stream,
                                           const tsg_layer* layer, const uint16_t* router_w,
                                           const uint16_t* router_hidden, const uint16_t* es,
                                           const uint16_t* pes, const uint16_t* x,
                                           const uint16_t* residual, uint16_t* y,
                                           uint32_t* out_idx, uint16_t* out_w,
                                           uint16_t* acts, uint32_t ne, uint32_t d, uint32_t f,
                                           uint32_t top_k) {
    return decode_layer_impl(moe, stream, layer, router_w, router_hidden, es, pes, x, residual, y,
                             out_idx, out_w, acts, ne, d, f, top_k, nullptr);
}

extern "C" tsg_status tsg_moe_decode_layer_int8(
    tsg_moe* moe, tsg_stream stream, const tsg_layer* layer, const uint8_t* router_w,
    const uint16_t* router_scales, const uint16_t* router_biases, const uint16_t* router_hidden,
    const uint16_t* es, const uint16_t* pes, const uint16_t* x, const uint16_t* residual,
    uint16_t* y, uint32_t* out_idx, uint16_t* out_w, uint16_t* acts, uint32_t ne, uint32_t d,
    uint32_t f, uint32_t top_k) {
    const RouterInt8 r8{router_w, router_scales, router_biases};
    return decode_layer_impl(moe, stream, layer, nullptr, router_hidden, es, pes, x, residual, y,
                             out_idx, out_w, acts, ne, d, f, top_k, nullptr, &r8);
}

extern "C" tsg_status tsg_moe_decode_layer_shared(
    tsg_moe* moe, tsg_stream stream, const tsg_layer* layer, const uint16_t* router_w,
    const uint16_t* router_hidden, const uint16_t* es, const uint16_t* pes, const uint16_t* x,
    uint16_t* y, uint32_t* out_idx, uint16_t* out_w, uint16_t* acts, const void* shared_blob,
    const tsg_expert_offsets* shared_offsets, const uint16_t* shared_gate_weight,
    uint16_t* shared_acts, uint32_t ne, uint32_t d, uint32_t f, uint32_t shared_f,
    uint32_t top_k) {
    TSG_REQUIRE(shared_blob && shared_offsets && shared_gate_weight && shared_acts,
                TSG_ERR_INVALID_ARGUMENT, "NULL shared-expert operand");
    TSG_REQUIRE(moe && moe->ctx, TSG_ERR_INVALID_ARGUMENT, "moe is NULL");
    const uint32_t g = moe->ctx->group_size;
    TSG_REQUIRE(shared_f > 0 && shared_f % g == 0, TSG_ERR_INVALID_ARGUMENT,
                "shared_f=%u must be a positive multiple of the group size %u", shared_f, g);
    const tsg_expert_offsets& o = *shared_offsets;
    const uint8_t* b = static_cast<const uint8_t*>(shared_blob);
    TSG_REQUIRE(aligned16(b + o.gate_w) && aligned16(b + o.up_w) && aligned16(b + o.down_w),
                TSG_ERR_ALIGNMENT, "shared weight sub-tensors must start on 16 bytes");
    TSG_REQUIRE(((o.gate_s | o.up_s | o.down_s | o.gate_b | o.up_b | o.down_b) & 1u) == 0,
                TSG_ERR_ALIGNMENT, "shared scale/bias offsets must be even");
    TSG_REQUIRE(aligned16(shared_gate_weight) && aligned16(shared_acts), TSG_ERR_ALIGNMENT,
                "the shared gate row and shared_acts must be 16-byte aligned");
    const SharedBranch sh{b, o, shared_gate_weight, shared_acts, shared_f};
    // y is the residual too (the reference's sharedOut is both)
    return decode_layer_impl(moe, stream, layer, router_w, router_hidden, es, pes, x, y, y,
                             out_idx, out_w, acts, ne, d, f, top_k, &sh);
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

// ------------------------------------------------------ verify layer (host)

namespace tsg {
namespace {

template <int G, bool SYM, int ACT, bool SH, bool Q = false>
tsg_status launch_verify(tsg_moe* moe, hipStream_t stream, const uint16_t* router_w,
                         const uint16_t* hidden, const uint16_t* es, const uint16_t* pes,
                         const uint16_t* x, uint32_t stride, const VerifyLayerArgs& a) {
    const size_t lds = verify_lds(a.rows, a.d, a.f, SYM).bytes;
    auto kern = verify_layer_kernel<G, SYM, ACT, SH, Q>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return fail(TSG_ERR_DECLINED, "verify layer: %zu bytes of LDS do not fit", lds);
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, (int)kVerifyThreads, lds) !=
            hipSuccess ||
        (uint64_t)per_cu * (uint64_t)moe->ctx->num_cus < kDecodeBlocks) {
        (void)hipGetLastError();
        return fail(TSG_ERR_DECLINED, "verify layer: %u blocks are not co-resident",
                    kDecodeBlocks);
    }
    hipLaunchKernelGGL(kern, dim3(kDecodeBlocks), dim3(kVerifyThreads), lds, stream, router_w,
                       hidden, es, pes, x, a.sync_words, a.ne | (a.rows << 16),
                       a.d | (stride << 16), a);
    return check_launch("verify_layer");
}

// The checks and arguments both verify entry points share.
tsg_status verify_args(tsg_moe* moe, const tsg_layer* layer, const uint16_t* router_w,
                       const uint16_t* router_hidden, const uint16_t* es, const uint16_t* pes,
                       const uint16_t* x, uint32_t hidden_stride, uint16_t* h2,
                       uint32_t* out_idx, uint16_t* out_w, uint32_t row_count, uint32_t ne,
                       uint32_t d, uint32_t f, uint32_t top_k, VerifyLayerArgs& a) {
    tsg_status st = check_moe(moe);
    if (st) return st;
    TSG_REQUIRE(moe->router_weight_bits == 16u, TSG_ERR_INVALID_ARGUMENT,
                "the verify layer takes BF16 router weights (a MoE created with 16-bit router "
                "weights), this MoE has %u-bit ones", moe->router_weight_bits);
    if ((st = check_decode_shape(moe->ctx, d, f, top_k))) return st;
    TSG_REQUIRE(layer, TSG_ERR_INVALID_ARGUMENT, "layer is NULL");
    TSG_REQUIRE(ne > 0 && ne <= layer->num_experts && ne <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "router has %u experts but the layer holds %u", ne, layer->num_experts);
    TSG_REQUIRE(router_w && router_hidden && es && pes && x && h2 && out_idx && out_w,
                TSG_ERR_INVALID_ARGUMENT, "NULL verify-layer operand");
    TSG_REQUIRE(aligned16(router_w) && aligned16(router_hidden) && aligned16(es) &&
                    aligned16(x) && hidden_stride % 8u == 0,
                TSG_ERR_ALIGNMENT, "router weights and token rows must be 16-byte aligned");
    TSG_REQUIRE(hidden_stride >= d, TSG_ERR_INVALID_ARGUMENT, "hidden stride %u < d=%u",
                hidden_stride, d);
    if (row_count == 0 || row_count > kMaxRouterRows)
        return fail(TSG_ERR_DECLINED, "the verify layer takes 1..%u rows, got %u", kMaxRouterRows,
                    row_count);
    if (ne < kTopK || d % 64u || f % 64u || d > kMaxFusedDim || f > kMaxFusedDim ||
        hidden_stride > 0xFFFFu)
        return fail(TSG_ERR_DECLINED, "verify layer shape (ne=%u, d=%u, f=%u, stride %u) not "
                                      "taken by the one launch", ne, d, f, hidden_stride);
    a = VerifyLayerArgs{};
    a.layer_base = layer->base;
    a.expert_stride = layer->expert_stride;
    a.o = layer->offsets;
    a.h2 = h2;
    a.out_idx = out_idx;
    a.out_w = out_w;
    a.words = moe->ctx->verify_words;
    a.sync_words = moe->ctx->counters;
    a.ne = ne;
    a.d = d;
    a.f = f;
    a.rows = row_count;
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

extern "C" tsg_status tsg_moe_verify_layer(tsg_moe* moe, tsg_stream stream,
                                           const tsg_layer* layer, const uint16_t* router_w,
                                           const uint16_t* router_hidden, const uint16_t* es,
                                           const uint16_t* pes, const uint16_t* x,
                                           uint32_t hidden_stride, uint16_t* h2,
                                           uint32_t* out_idx, uint16_t* out_w,
                                           uint32_t row_count, uint32_t ne, uint32_t d,
                                           uint32_t f, uint32_t top_k) {
    VerifyLayerArgs a;
    tsg_status st = verify_args(moe, layer, router_w, router_hidden, es, pes, x, hidden_stride,
                                h2, out_idx, out_w, row_count, ne, d, f, top_k, a);
    if (st) return st;
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const bool silu = moe->activation == TSG_ACT_SILU;
    hipStream_t s = as_stream(stream);
#define TSG_VL(GG, SS)                                                                        \
    return silu ? launch_verify<GG, SS, TSG_ACT_SILU, false>(moe, s, router_w, router_hidden, \
                                                             es, pes, x, hidden_stride, a)    \
                : launch_verify<GG, SS, TSG_ACT_GELU_TANH, false>(moe, s, router_w,           \
                                                                  router_hidden, es, pes, x,  \
                                                                  hidden_stride, a)
    if (ctx->group_size == 32) {
        if (sym) TSG_VL(32, true);
        TSG_VL(32, false);
    }
    if (sym) TSG_VL(64, true);
    TSG_VL(64, false);
#undef TSG_VL
}

extern "C" tsg_status tsg_moe_verify_layer_shared(
    tsg_moe* moe, tsg_stream stream, const tsg_layer* layer, const uint16_t* router_w,
    const uint16_t* router_hidden, const uint16_t* es, const uint16_t* pes, const uint16_t* x,
    uint32_t hidden_stride, uint16_t* h2, uint32_t* out_idx, uint16_t* out_w,
    const void* shared_blob, const tsg_expert_offsets* shared_offsets,
    const uint16_t* shared_gate_weight, uint16_t* shared_out, uint32_t row_count, uint32_t ne,
    uint32_t d, uint32_t f, uint32_t top_k) {
    VerifyLayerArgs a;
    tsg_status st = verify_args(moe, layer, router_w, router_hidden, es, pes, x, hidden_stride,
                                h2, out_idx, out_w, row_count, ne, d, f, top_k, a);
    if (st) return st;
    TSG_REQUIRE(shared_blob && shared_offsets && shared_gate_weight && shared_out,
                TSG_ERR_INVALID_ARGUMENT, "NULL shared-expert operand");
    const tsg_expert_offsets& o = *shared_offsets;
    const uint8_t* b = static_cast<const uint8_t*>(shared_blob);
    TSG_REQUIRE(aligned16(b + o.gate_w) && aligned16(b + o.up_w) && aligned16(b + o.down_w),
                TSG_ERR_ALIGNMENT, "shared weight sub-tensors must start on 16 bytes");
    TSG_REQUIRE(((o.gate_s | o.up_s | o.down_s | o.gate_b | o.up_b | o.down_b) & 1u) == 0,
                TSG_ERR_ALIGNMENT, "shared scale/bias offsets must be even");
    TSG_REQUIRE(aligned16(shared_gate_weight), TSG_ERR_ALIGNMENT,
                "the shared gate row must be 16-byte aligned");
    if (moe->activation != TSG_ACT_SILU)
        return fail(TSG_ERR_DECLINED, "the shared expert's one-launch form takes SiLU layers "
                                      "(the Qwen family)");
    a.sh_blob = b;
    a.sh_o = o;
    a.sh_gate_w = shared_gate_weight;
    a.sh_out = shared_out;
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    hipStream_t s = as_stream(stream);
    // the Qwen family's shapes (d = 2048, f = 512) take the compact batches
    const bool q = d <= 2048u && f <= 512u;
#define TSG_VLS(GG, SS)                                                                        \
    return q ? launch_verify<GG, SS, TSG_ACT_SILU, true, true>(moe, s, router_w, router_hidden, \
                                                               es, pes, x, hidden_stride, a)    \
             : launch_verify<GG, SS, TSG_ACT_SILU, true, false>(moe, s, router_w,               \
                                                                router_hidden, es, pes, x,      \
                                                                hidden_stride, a)
    if (ctx->group_size == 32) {
        if (sym) TSG_VLS(32, true);
        TSG_VLS(32, false);
    }
    if (sym) TSG_VLS(64, true);
    TSG_VLS(64, false);
#undef TSG_VLS
}
