// qmv.hip — dense int4 GEMV (DequantInt4GEMV.swift:6-364,
// dequant_int4.metal:135-358) and the bit-exact dequantisation check.
//
// One output row per 16 lanes, 16-byte weight chunks (one g32 group, half a
// g64 group) streamed with all loads in flight, nibbles -> fp16 by the 0x6400
// exponent trick, v_dot2_f32_f16 against x staged in LDS, fp32 scale fma.
// The rows form keeps T <= 8 accumulators per lane so a weight chunk is read
// once for all rows; each row's sum runs in exactly the one-row order.
#include "gemv_lane.hpp"

namespace tsg {
namespace {

constexpr uint32_t kMaxRows = 8;

// WA: the weights' alignment, 16 or 2 (a weights pointer bound at a 2-byte
// offset, DequantInt4GEMV.swift:93-96: every row starts at the same offset
// modulo 16, since a row is a multiple of 16 bytes).
// RPB rows per block (16 lanes each), so the block size is a constant. The
// parameters the first loads need fill the first 14 dwords, which the
// dispatch preloads into SGPRs: no kernel-argument load comes before them.
template <int G, bool SYM, int T, int WA, uint32_t RPB>
__global__ __launch_bounds__(16 * RPB) void qmv_kernel(const uint8_t* __restrict__ w,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint16_t* __restrict__ biases,
                                                       const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, uint32_t n,
                                                       uint32_t m, uint32_t t, uint32_t x_stride,
                                                       uint32_t y_stride) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t row_h = lds_chunks_halves(n);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                        // T rows
    float* xsum = reinterpret_cast<float*>(smem + (size_t)T * row_h * 2u);  // T * n / 32

    const uint32_t row = blockIdx.x * RPB + (threadIdx.x >> 4);
    const uint32_t j = threadIdx.x & 15u;
    const bool live = row < m;
    const uint32_t rr = live ? row : 0u;
    const uint32_t ngroups = n / G, nchunks = n / 32u;
    const uint8_t* wr = w + (uint64_t)rr * (n / 2u);
    const uint16_t* sr = scales + (uint64_t)rr * ngroups;
    const uint16_t* br = biases + (uint64_t)rr * ngroups;
    ChunkBatch<kGUBatch> bt;
    auto issue_weights = [&] {
        load_batch<G, SYM, kGUBatch, kGULanes, WA>(wr, sr, br, 0u, j, nchunks, bt);
    };
    stage_act_rows_around<SYM, decltype(issue_weights)&, 4, 16u * RPB>(x, x_stride, t, n, xs, row_h,
                                                                       xsum, nullptr, issue_weights);
    __syncthreads();
    float acc[T];
#pragma unroll
    for (int r = 0; r < T; ++r) acc[r] = 0.0f;
    gemv_batches<G, SYM, kGUBatch, kGULanes, T, WA>(wr, sr, br, j, nchunks, bt, xs, row_h, xsum, t, acc);
#pragma unroll
    for (int r = 0; r < T; ++r) {
        acc[r] = group16_sum(acc[r]);
    }
    if (live && j == 0) {
#pragma unroll
        for (int r = 0; r < T; ++r)
            if ((uint32_t)r < t) y[(uint64_t)r * y_stride + row] = f32_to_f16(acc[r]);
    }
}

// out[r, k] = half(fma(q, s, b)), b = -8 s under sym (prefill.metal:1021-1026).
template <int G, bool SYM>
__global__ void dequant_f16_kernel(const uint8_t* __restrict__ w,
                                   const uint16_t* __restrict__ scales,
                                   const uint16_t* __restrict__ biases,
                                   uint16_t* __restrict__ out, uint32_t rows, uint32_t n) {
    const uint64_t total = (uint64_t)rows * n;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / n;
        const uint32_t k = (uint32_t)(i - r * n);
        const uint8_t byte = w[r * (n / 2u) + k / 2u];
        const uint32_t q = (k & 1u) ? (byte >> 4) : (byte & 0xFu);
        const uint32_t g = k / G;
        const float s = bf16_to_f32(scales[r * (n / G) + g]);
        const float b = SYM ? -8.0f * s : bf16_to_f32(biases[r * (n / G) + g]);
        out[i] = f32_to_f16(__builtin_fmaf((float)q, s, b));
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int G, bool SYM, int WA>
tsg_status launch_qmv(hipStream_t s, const uint8_t* w, const uint16_t* sc, const uint16_t* bi,
                      const uint16_t* x, uint32_t xs, uint16_t* y, uint32_t ys, uint32_t t,
                      uint32_t m, uint32_t n) {
    // 16 lanes per row; 4 rows per block (one wave) below 4096 rows so a
    // small matrix still spreads over the CUs, 16 above
    const uint32_t rpb = m < 4096u ? 4u : 16u;
    const dim3 grid((m + rpb - 1u) / rpb), block(16u * rpb);
    const size_t lds_per_row = (size_t)lds_chunks_halves(n) * 2u + (SYM ? 0u : (n / 32u) * 4u);
#define TSG_QMV_CASE(TT)                                                                        \
    case TT:                                                                                    \
        if (rpb == 4u)                                                                          \
            hipLaunchKernelGGL((qmv_kernel<G, SYM, TT, WA, 4u>), grid, block, lds_per_row * TT, \
                               s, w, sc, bi, x, y, n, m, t, xs, ys);                            \
        else                                                                                    \
            hipLaunchKernelGGL((qmv_kernel<G, SYM, TT, WA, 16u>), grid, block, lds_per_row * TT, \
                               s, w, sc, bi, x, y, n, m, t, xs, ys);                            \
        break;
    switch (t) {
        TSG_QMV_CASE(1)
        TSG_QMV_CASE(2)
        TSG_QMV_CASE(3)
        TSG_QMV_CASE(4)
        TSG_QMV_CASE(5)
        TSG_QMV_CASE(6)
        TSG_QMV_CASE(7)
        TSG_QMV_CASE(8)
        default: return fail(TSG_ERR_INVALID_ARGUMENT, "t=%u not in 1..8", t);
    }
#undef TSG_QMV_CASE
    return check_launch("qmv_int4");
}

tsg_status qmv_dispatch(tsg_ctx* ctx, hipStream_t s, const uint8_t* w, const uint16_t* sc,
                        const uint16_t* bi, const uint16_t* x, uint32_t xs, uint16_t* y,
                        uint32_t ys, uint32_t t, uint32_t m, uint32_t n) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(w && sc && x && y, TSG_ERR_INVALID_ARGUMENT, "NULL operand");
    TSG_REQUIRE(ctx->scheme == TSG_SYM || bi, TSG_ERR_INVALID_ARGUMENT,
                "biases is NULL under the affine scheme");
    TSG_REQUIRE(n > 0 && n % ctx->group_size == 0, TSG_ERR_INVALID_ARGUMENT,
                "N must be a multiple of %u, got %u", ctx->group_size, n);
    TSG_REQUIRE(m > 0, TSG_ERR_INVALID_ARGUMENT, "m must be positive");
    // The reference reads weights through ushort* and needs a 2-aligned
    // weightsOffset (DequantInt4GEMV.swift:91-96). Rows are n / 2 bytes, a
    // multiple of 16 (n % 32 == 0), so every 16-byte chunk has the base's
    // alignment: 16-byte loads when the base is 16-byte aligned, else the
    // 2-byte-safe load (load16_a2).
    TSG_REQUIRE((reinterpret_cast<uintptr_t>(w) & 1u) == 0, TSG_ERR_ALIGNMENT,
                "weights need a 2-aligned offset (got %p)", (const void*)w);
    TSG_REQUIRE((reinterpret_cast<uintptr_t>(sc) & 1u) == 0 &&
                    (reinterpret_cast<uintptr_t>(bi ? bi : sc) & 1u) == 0,
                TSG_ERR_ALIGNMENT, "scales and biases must be 2-byte aligned");
    const bool w16 = aligned16(w);
    TSG_REQUIRE(aligned16(x) && xs % 8 == 0, TSG_ERR_ALIGNMENT,
                "x rows must be 16-byte aligned");
    // Rows are independent (each is summed exactly as on its own), so rows
    // that do not fit the LDS staging together run in several launches.
    const size_t per_row = (size_t)lds_chunks_halves(n) * 2u + (n / 32u) * 4u;
    const uint32_t fit = (uint32_t)std::min<size_t>(kMaxRows, (160u * 1024u) / per_row);
    TSG_REQUIRE(fit >= 1, TSG_ERR_UNSUPPORTED, "a row of n=%u does not fit the LDS staging", n);
    const bool sym = ctx->scheme == TSG_SYM;
    for (uint32_t r0 = 0; r0 < t; r0 += fit) {
        const uint32_t tt = std::min(fit, t - r0);
        const uint16_t* xr = x + (size_t)r0 * xs;
        uint16_t* yr = y + (size_t)r0 * ys;
        tsg_status st;
#define TSG_QMV_WA(WA)                                                                 \
    if (ctx->group_size == 32)                                                         \
        st = sym ? launch_qmv<32, true, WA>(s, w, sc, sc, xr, xs, yr, ys, tt, m, n)    \
                 : launch_qmv<32, false, WA>(s, w, sc, bi, xr, xs, yr, ys, tt, m, n);  \
    else                                                                               \
        st = sym ? launch_qmv<64, true, WA>(s, w, sc, sc, xr, xs, yr, ys, tt, m, n)    \
                 : launch_qmv<64, false, WA>(s, w, sc, bi, xr, xs, yr, ys, tt, m, n);
        if (w16) {
            TSG_QMV_WA(16)
        } else {
            TSG_QMV_WA(2)
        }
#undef TSG_QMV_WA
        if (st) return st;
    }
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

using namespace tsg;

extern "C" tsg_status tsg_qmv_int4(tsg_ctx* ctx, tsg_stream stream, const uint8_t* w,
                                   const uint16_t* scales, const uint16_t* biases,
                                   const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n) {
    return qmv_dispatch(ctx, as_stream(stream), w, scales, biases, x, n, y, m, 1, m, n);
}

extern "C" tsg_status tsg_qmv_int4_rows(tsg_ctx* ctx, tsg_stream stream, const uint8_t* w,
                                        const uint16_t* scales, const uint16_t* biases,
                                        const uint16_t* x, uint32_t x_stride, uint16_t* y,
                                        uint32_t y_stride, uint32_t t, uint32_t m,
                                        uint32_t n) {
    TSG_REQUIRE(t >= 1 && t <= kMaxRows, TSG_ERR_INVALID_ARGUMENT, "t=%u not in 1..%u", t,
                kMaxRows);
    return qmv_dispatch(ctx, as_stream(stream), w, scales, biases, x, x_stride, y, y_stride, t,
                        m, n);
}

// SharedExpertInt4.encode (Kernels/MoE/SharedExpertInt4.swift:30-93): the
// dense int4 MLP y = down(gelu(gate x) * up x) as the reference encodes it:
// QMV gate and up into fp16 scratch, gelu_mul_fp16, QMV down.
extern "C" tsg_status tsg_shared_expert_int4(
    tsg_ctx* ctx, tsg_stream stream, const uint16_t* x, uint64_t x_bytes,
    const tsg_int4_projection* gate, const tsg_int4_projection* up,
    const tsg_int4_projection* down, uint16_t* y, uint64_t y_bytes, uint16_t* scratch_gate,
    uint64_t scratch_gate_bytes, uint16_t* scratch_up, uint64_t scratch_up_bytes,
    uint16_t* scratch_act, uint64_t scratch_act_bytes) {
    TSG_REQUIRE(ctx && gate && up && down, TSG_ERR_INVALID_ARGUMENT, "NULL ctx or projection");
    if (!(gate->rows == up->rows && gate->cols == up->cols && down->rows == gate->cols &&
          down->cols == gate->rows))
        return fail(TSG_ERR_INVALID_ARGUMENT,
                    "dimensionMismatch: gate=(%u,%u) up=(%u,%u) down=(%u,%u)", gate->rows,
                    gate->cols, up->rows, up->cols, down->rows, down->cols);
    const uint64_t required = (uint64_t)gate->rows * 2u;
    if (scratch_gate_bytes < required || scratch_up_bytes < required || scratch_act_bytes < required)
        return fail(TSG_ERR_INVALID_ARGUMENT,
                    "scratchTooSmall: need %llu bytes per intermediate buffer",
                    (unsigned long long)required);
    if (x_bytes < (uint64_t)gate->cols * 2u)
        return fail(TSG_ERR_INVALID_ARGUMENT, "scratchTooSmall: input range exceeds x buffer");
    if (y_bytes < (uint64_t)down->rows * 2u)
        return fail(TSG_ERR_INVALID_ARGUMENT, "scratchTooSmall: output range exceeds y buffer");
    tsg_status st;
    if ((st = tsg_qmv_int4(ctx, stream, gate->weights, gate->scales, gate->biases, x,
                           scratch_gate, gate->rows, gate->cols)))
        return st;
    if ((st = tsg_qmv_int4(ctx, stream, up->weights, up->scales, up->biases, x, scratch_up,
                           up->rows, up->cols)))
        return st;
    if ((st = tsg_gelu_mul_f16(ctx, stream, scratch_gate, scratch_up, scratch_act, gate->rows)))
        return st;
    return tsg_qmv_int4(ctx, stream, down->weights, down->scales, down->biases, scratch_act, y,
                        down->rows, down->cols);
}

extern "C" tsg_status tsg_debug_dequant_f16(tsg_ctx* ctx, tsg_stream stream, const uint8_t* w,
                                            const uint16_t* scales, const uint16_t* biases,
                                            uint16_t* out, uint32_t rows, uint32_t n) {
    TSG_REQUIRE(ctx && w && scales && out, TSG_ERR_INVALID_ARGUMENT, "NULL operand");
    TSG_REQUIRE(ctx->scheme == TSG_SYM || biases, TSG_ERR_INVALID_ARGUMENT,
                "biases is NULL under the affine scheme");
    TSG_REQUIRE(n > 0 && n % ctx->group_size == 0 && rows > 0, TSG_ERR_INVALID_ARGUMENT,
                "bad shape rows=%u n=%u", rows, n);
    const uint64_t total = (uint64_t)rows * n;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t s = as_stream(stream);
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32) {
        if (sym) hipLaunchKernelGGL((dequant_f16_kernel<32, true>), dim3(blocks), dim3(256), 0, s, w, scales, scales, out, rows, n);
        else hipLaunchKernelGGL((dequant_f16_kernel<32, false>), dim3(blocks), dim3(256), 0, s, w, scales, biases, out, rows, n);
    } else {
        if (sym) hipLaunchKernelGGL((dequant_f16_kernel<64, true>), dim3(blocks), dim3(256), 0, s, w, scales, scales, out, rows, n);
        else hipLaunchKernelGGL((dequant_f16_kernel<64, false>), dim3(blocks), dim3(256), 0, s, w, scales, biases, out, rows, n);
    }
    return check_launch("debug_dequant_f16");
}
