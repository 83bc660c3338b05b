// shared.hip — the Qwen-family shared expert with its sigmoid gate
// (QwenForwardRunner.swift:1548-1578):
//
//   act       = half(silu(half(gate · x)) · half(up · x))
//   sharedOut = half(half(down · act) · sigmoid(w_g · x))
//
// as the reference's separate steps — the three projections are the dense int4
// GEMV (tsg_qmv_int4, DequantInt4GEMV), qwen_silu_mul (qwen.metal:466),
// qwen_moe_shared_gate (qwen.metal:432-455) and qwen_moe_shared_gate_logit
// (qwen.metal:1038-1046) — and fused into two launches that give the same
// bits: gate/up and down rows use the GEMV's lane geometry and sum order, and
// the gate logit is gate_logit_wave (qwen_shared.hpp) everywhere.
#include "qwen_shared.hpp"

namespace tsg {
namespace {

constexpr uint32_t kGateThreads = 256;

// gate_logit_wave on wave 0 of the block, handed to every thread through LDS.
__device__ float gate_logit_block(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                  uint32_t d, float* red) {
    if (threadIdx.x < 64u) {
        const float s = gate_logit_wave(x, w, d);
        if (threadIdx.x == 0) red[0] = s;
    }
    __syncthreads();
    const float s = red[0];
    __syncthreads();
    return s;
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up,
                                                       uint16_t* __restrict__ out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_mul_h(gate[i], up[i]);
}

// out = half(gelu_tanh(float(gate)) * float(up)) (utility.metal:7-18), the
// Gemma shared expert's activation.
__global__ __launch_bounds__(256) void gelu_mul_kernel(const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up,
                                                       uint16_t* __restrict__ out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        out[i] = f32_to_f16(gate_activation<TSG_ACT_GELU_TANH>(f16_to_f32(gate[i])) *
                            f16_to_f32(up[i]));
}

// y *= sigmoid(w_g · x) in place, one block (qwen.metal:432-455).
__global__ __launch_bounds__(kGateThreads) void shared_gate_kernel(uint16_t* __restrict__ y,
                                                                   const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ w,
                                                                   uint32_t d) {
    __shared__ float red[1];
    const float scale = qwen_sigmoid(gate_logit_block(x, w, d, red));
    for (uint32_t i = threadIdx.x; i < d; i += kGateThreads)
        y[i] = f32_to_f16(f16_to_f32(y[i]) * scale);
}

// y *= sigmoid(logit[0]) in place (qwen.metal:1038-1046).
__global__ __launch_bounds__(256) void shared_gate_logit_kernel(uint16_t* __restrict__ y,
                                                                const uint16_t* __restrict__ logit,
                                                                uint32_t d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < d) y[i] = f32_to_f16(f16_to_f32(y[i]) * qwen_sigmoid(f16_to_f32(logit[0])));
}

// act[r, p] = half(silu(half(gate_p · x_r)) * half(up_p · x_r)) for the
// rows r < rows (R = 1: one token; R = kSharedRowsMax: up to that many). 8
// weight rows p per block: lanes 0..15 of each 32 sum the gate row, lanes
// 16..31 the up row, in the dense GEMV's geometry (16 lanes per row,
// kGUBatch chunks per batch), each weight read once for every token row; each
// row's sum and its fp16 rounding equal tsg_qmv_int4's on that row.
constexpr uint32_t kSharedRowsMax = 8;

template <int G, bool SYM, int R>
__global__ __launch_bounds__(256) void shared_gate_up_kernel(const uint8_t* __restrict__ blob,
                                                             tsg_expert_offsets o,
                                                             const uint16_t* __restrict__ x,
                                                             uint32_t x_stride, uint32_t rows,
                                                             uint16_t* __restrict__ act,
                                                             uint32_t d, uint32_t f) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t row_h = R == 1 ? 0u : lds_chunks_halves(d);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + (R == 1 ? lds_chunks_halves(d) : R * row_h) * 2u);
    const uint32_t t = threadIdx.x, j = t & 15u;
    const bool is_up = (t >> 4) & 1u;
    const uint32_t p = blockIdx.x * 8u + (t >> 5);
    const bool live = p < f;
    const uint32_t pr = live ? p : 0u;
    const uint32_t ngroups = d / G, nchunks = d / 32u;
    const uint8_t* w = blob + (is_up ? o.up_w : o.gate_w) + (uint64_t)pr * (d / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + (is_up ? o.up_s : o.gate_s)) +
                         (uint64_t)pr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + (is_up ? o.up_b : o.gate_b)) +
                         (uint64_t)pr * ngroups;
    ChunkBatch<kGUBatch> bt;
    stage_act_rows_around<SYM>(x, x_stride, R == 1 ? 1u : rows, d, xs, row_h, xsum, nullptr, [&] {
        load_batch<G, SYM, kGUBatch, kGULanes>(w, sc, bi, 0u, j, nchunks, bt);
    });
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    gemv_batches<G, SYM, kGUBatch, kGULanes, R>(w, sc, bi, j, nchunks, bt, xs, row_h, xsum,
                                                R == 1 ? 1u : rows, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float s = group16_sum(acc[r]);
        const float u = shfl_xor(s, 16);  // gate lanes receive the up sum
        if (live && !is_up && j == 0 && (uint32_t)r < rows)
            act[(uint64_t)r * f + p] = silu_mul_h(f32_to_f16(s), f32_to_f16(u));
    }
}

// out[r, i] = half(half(down_i · act_r) * sigmoid(w_g · x_r)) for the rows
// r < rows: 16 output rows i per block in the dense GEMV's geometry, each
// weight read once for every token row, the gate logits summed by every block
// as shared_gate_kernel sums them (one wave per token row).
template <int G, bool SYM, int R>
__global__ __launch_bounds__(kGateThreads) void shared_down_kernel(
    const uint8_t* __restrict__ blob, tsg_expert_offsets o, const uint16_t* __restrict__ act,
    const uint16_t* __restrict__ x, uint32_t x_stride, uint32_t rows,
    const uint16_t* __restrict__ gate_w, uint16_t* __restrict__ out, uint32_t d, uint32_t f) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[R];
    const uint32_t row_h = R == 1 ? 0u : lds_chunks_halves(f);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);
    float* asum = reinterpret_cast<float*>(smem + (R == 1 ? lds_chunks_halves(f) : R * row_h) * 2u);
    const uint32_t t = threadIdx.x, j = t & 15u;
    const uint32_t row = blockIdx.x * 16u + (t >> 4);
    const bool live = row < d;
    const uint32_t rr = live ? row : 0u;
    const uint32_t ngroups = f / G, nchunks = f / 32u;
    const uint8_t* w = blob + o.down_w + (uint64_t)rr * (f / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + o.down_s) + (uint64_t)rr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + o.down_b) + (uint64_t)rr * ngroups;
    ChunkBatch<kGUBatch> bt;
    const uint32_t nr = R == 1 ? 1u : rows;
    stage_act_rows_around<SYM>(act, f, nr, f, as, row_h, asum, nullptr, [&] {
        load_batch<G, SYM, kGUBatch, kGULanes>(w, sc, bi, 0u, j, nchunks, bt);
    });
    float logit0 = 0.0f;
    if constexpr (R == 1) {
        logit0 = gate_logit_block(x, gate_w, d, red);  // synchronises
    } else {
        for (uint32_t r = t >> 6; r < nr; r += kGateThreads / 64u) {
            const float s = gate_logit_wave(x + (uint64_t)r * x_stride, gate_w, d);
            if ((t & 63u) == 0) red[r] = s;
        }
        __syncthreads();
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    gemv_batches<G, SYM, kGUBatch, kGULanes, R>(w, sc, bi, j, nchunks, bt, as, row_h, asum, nr, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = group16_sum(acc[r]);
        if (live && j == 0 && (uint32_t)r < nr)
            out[(uint64_t)r * d + row] =
                f32_to_f16(f16_to_f32(f32_to_f16(v)) * qwen_sigmoid(R == 1 ? logit0 : red[r]));
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

tsg_status check_gate_args(const tsg_ctx* ctx, const void* y, const void* a, const void* b,
                           uint32_t n) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(y && a && b, TSG_ERR_INVALID_ARGUMENT, "NULL operand");
    // The reference's encoders return false (nothing encoded) for an empty size.
    TSG_REQUIRE(n > 0, TSG_ERR_DECLINED, "empty size: nothing to encode");
    return TSG_OK;
}

// LDS of the staged rows (and affine row sums) of one shared-expert kernel.
size_t shared_lds(uint32_t n, uint32_t rows, bool sym) {
    return (size_t)rows * (lds_chunks_halves(n) * 2u + (sym ? 0u : (n / 32u) * 4u));
}

template <int G, bool SYM>
tsg_status launch_shared(hipStream_t s, const uint8_t* blob, const tsg_expert_offsets& o,
                         const uint16_t* x, uint32_t x_stride, uint32_t rows,
                         const uint16_t* gate_w, uint16_t* act, uint16_t* out, uint32_t d,
                         uint32_t f) {
    const dim3 g1((f + 7u) / 8u), g2((d + 15u) / 16u);
    if (rows == 1) {
        hipLaunchKernelGGL((shared_gate_up_kernel<G, SYM, 1>), g1, dim3(256),
                           shared_lds(d, 1u, SYM), s, blob, o, x, 0u, 1u, act, d, f);
        hipLaunchKernelGGL((shared_down_kernel<G, SYM, 1>), g2, dim3(kGateThreads),
                           shared_lds(f, 1u, SYM), s, blob, o, act, x, 0u, 1u, gate_w, out, d, f);
    } else {
        constexpr int R = (int)kSharedRowsMax;
        hipLaunchKernelGGL((shared_gate_up_kernel<G, SYM, R>), g1, dim3(256),
                           shared_lds(d, R, SYM), s, blob, o, x, x_stride, rows, act, d, f);
        hipLaunchKernelGGL((shared_down_kernel<G, SYM, R>), g2, dim3(kGateThreads),
                           shared_lds(f, R, SYM), s, blob, o, act, x, x_stride, rows, gate_w, out,
                           d, f);
    }
    return check_launch("shared_expert");
}

}  // namespace
}  // namespace tsg

using namespace tsg;

extern "C" tsg_status tsg_qwen_silu_mul(tsg_ctx* ctx, tsg_stream stream, const uint16_t* gate,
                                        const uint16_t* up, uint16_t* out, uint32_t count) {
    tsg_status st = check_gate_args(ctx, out, gate, up, count);
    if (st) return st;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((count + 255u) / 256u), dim3(256), 0,
                       as_stream(stream), gate, up, out, count);
    return check_launch("qwen_silu_mul");
}

extern "C" tsg_status tsg_gelu_mul_f16(tsg_ctx* ctx, tsg_stream stream, const uint16_t* gate,
                                       const uint16_t* up, uint16_t* out, uint32_t count) {
    tsg_status st = check_gate_args(ctx, out, gate, up, count);
    if (st) return st;
    hipLaunchKernelGGL(gelu_mul_kernel, dim3((count + 255u) / 256u), dim3(256), 0,
                       as_stream(stream), gate, up, out, count);
    return check_launch("gelu_mul");
}

static tsg_status check_gate_row(const uint16_t* x, const uint16_t* w, uint32_t d) {
    TSG_REQUIRE(d % 8u == 0 && d <= 64u * 8u * kGateUnits, TSG_ERR_UNSUPPORTED,
                "hidden=%u: the gate sum takes a multiple of 8 up to %u", d, 64u * 8u * kGateUnits);
    TSG_REQUIRE(aligned16(x) && aligned16(w), TSG_ERR_ALIGNMENT,
                "x and the gate weight row must be 16-byte aligned");
    return TSG_OK;
}

extern "C" tsg_status tsg_qwen_moe_shared_gate(tsg_ctx* ctx, tsg_stream stream, uint16_t* y,
                                               const uint16_t* x, const uint16_t* weight,
                                               uint32_t hidden) {
    tsg_status st = check_gate_args(ctx, y, x, weight, hidden);
    if (st) return st;
    if ((st = check_gate_row(x, weight, hidden))) return st;
    hipLaunchKernelGGL(shared_gate_kernel, dim3(1), dim3(kGateThreads), 0, as_stream(stream), y,
                       x, weight, hidden);
    return check_launch("qwen_moe_shared_gate");
}

extern "C" tsg_status tsg_qwen_moe_shared_gate_logit(tsg_ctx* ctx, tsg_stream stream,
                                                     uint16_t* y, const uint16_t* logit,
                                                     uint32_t hidden) {
    tsg_status st = check_gate_args(ctx, y, logit, logit, hidden);
    if (st) return st;
    hipLaunchKernelGGL(shared_gate_logit_kernel, dim3((hidden + 255u) / 256u), dim3(256), 0,
                       as_stream(stream), y, logit, hidden);
    return check_launch("qwen_moe_shared_gate_logit");
}

static tsg_status shared_expert(tsg_moe* moe, tsg_stream stream, const void* blob,
                                const tsg_expert_offsets* offsets, const uint16_t* x,
                                uint32_t x_stride, uint32_t rows, const uint16_t* gate_weight,
                                uint16_t* act_scratch, uint16_t* out, uint32_t d, uint32_t f) {
    TSG_REQUIRE(moe && moe->ctx, TSG_ERR_INVALID_ARGUMENT, "moe is NULL");
    TSG_REQUIRE(blob && offsets && x && gate_weight && act_scratch && out,
                TSG_ERR_INVALID_ARGUMENT, "NULL shared-expert operand");
    const tsg_ctx* ctx = moe->ctx;
    const uint32_t g = ctx->group_size;
    TSG_REQUIRE(d > 0 && f > 0 && d % g == 0 && f % g == 0, TSG_ERR_INVALID_ARGUMENT,
                "d=%u and f=%u must be positive multiples of the group size %u", d, f, g);
    const tsg_expert_offsets& o = *offsets;
    const uint8_t* b = static_cast<const uint8_t*>(blob);
    TSG_REQUIRE(aligned16(b + o.gate_w) && aligned16(b + o.up_w) && aligned16(b + o.down_w),
                TSG_ERR_ALIGNMENT, "weight sub-tensors must start on 16 bytes");
    TSG_REQUIRE(((o.gate_s | o.up_s | o.down_s | o.gate_b | o.up_b | o.down_b) & 1u) == 0,
                TSG_ERR_ALIGNMENT, "scale/bias offsets must be even");
    TSG_REQUIRE(aligned16(x) && aligned16(act_scratch) && x_stride % 8u == 0, TSG_ERR_ALIGNMENT,
                "x rows and act_scratch must be 16-byte aligned");
    tsg_status st = check_gate_row(x, gate_weight, d);
    if (st) return st;
    const uint32_t lr = rows == 1 ? 1u : kSharedRowsMax;
    const bool sym = ctx->scheme == TSG_SYM;
    TSG_REQUIRE(shared_lds(d, lr, sym) <= 64u * 1024u && shared_lds(f, lr, sym) <= 64u * 1024u,
                TSG_ERR_UNSUPPORTED, "d=%u / f=%u do not fit the LDS staging of %u rows", d, f,
                lr);
    hipStream_t s = as_stream(stream);
    if (g == 32)
        return sym ? launch_shared<32, true>(s, b, o, x, x_stride, rows, gate_weight, act_scratch, out, d, f)
                   : launch_shared<32, false>(s, b, o, x, x_stride, rows, gate_weight, act_scratch, out, d, f);
    return sym ? launch_shared<64, true>(s, b, o, x, x_stride, rows, gate_weight, act_scratch, out, d, f)
               : launch_shared<64, false>(s, b, o, x, x_stride, rows, gate_weight, act_scratch, out, d, f);
}

extern "C" tsg_status tsg_moe_shared_expert(tsg_moe* moe, tsg_stream stream, const void* blob,
                                            const tsg_expert_offsets* offsets, const uint16_t* x,
                                            const uint16_t* gate_weight, uint16_t* act_scratch,
                                            uint16_t* out, uint32_t d, uint32_t f) {
    return shared_expert(moe, stream, blob, offsets, x, 0u, 1u, gate_weight, act_scratch, out, d,
                         f);
}

extern "C" tsg_status tsg_moe_shared_expert_rows(tsg_moe* moe, tsg_stream stream,
                                                 const void* blob,
                                                 const tsg_expert_offsets* offsets,
                                                 const uint16_t* x, uint32_t x_stride,
                                                 const uint16_t* gate_weight,
                                                 uint16_t* act_scratch, uint16_t* out,
                                                 uint32_t rows, uint32_t d, uint32_t f) {
    TSG_REQUIRE(rows > 0 && rows <= kSharedRowsMax, TSG_ERR_DECLINED,
                "the shared expert's rows form takes 1..%u rows, got %u", kSharedRowsMax, rows);
    return shared_expert(moe, stream, blob, offsets, x, x_stride, rows, gate_weight, act_scratch,
                         out, d, f);
}
