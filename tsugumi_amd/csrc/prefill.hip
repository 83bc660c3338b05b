// prefill.hip — prompt-chunk routed MoE for gfx950.
//
//   device grouping   PrefillMoEGrouping.swift:90-202 (stable counting sort)
//   grouped GEMMs     prefill.metal:913-1092, 3664-3864 (encodeStreamedTiled)
//   token-major sum   prefill.metal:796-817
//   verify rows path  prefill.metal:1489-1721 (encodeStreamedRows)
//
// The grouped GEMMs' kernels are in prefill_gemm_impl.hpp.
#include "prefill_gemm.hpp"

namespace tsg {
namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------- device grouping

// Exclusive prefix sum of one value per thread over a block of NT threads
// (NT a multiple of 64, at most 1024); every thread also gets the total.
template <uint32_t NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tot,
                                                         uint32_t& total) {
    constexpr uint32_t kWaves = NT / 64u;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(x, off, 64);
        if ((int)lane >= off) x += o;
    }
    if (lane == 63) wave_tot[wave] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) {
        const uint32_t c = wave_tot[w];
        before += w < wave ? c : 0u;
        all += c;
    }
    total = all;
    return before + x - v;
}

// One block per expert e: rank_of[p] = position of pair p among the pairs of
// expert e in (token, rank) order; counts[e] = their number. Thread i owns
// the consecutive tokens [i * tpt, (i + 1) * tpt): it counts its matches,
// one block scan places them, and a second pass over the same indices (kept
// in registers for top-8 up to 4096 tokens, else re-read from the cache)
// writes the ranks.
__global__ __launch_bounds__(1024) void group_rank_kernel(const uint32_t* __restrict__ idx,
                                                          uint32_t t, uint32_t k,
                                                          uint32_t* __restrict__ rank_of,
                                                          uint32_t* __restrict__ counts) {
    __shared__ uint32_t wave_tot[16];
    const uint32_t e = blockIdx.x;
    const uint32_t tpt = (t + 1023u) / 1024u;
    const uint32_t p0 = min(threadIdx.x * tpt, t) * k, p1 = min(threadIdx.x * tpt + tpt, t) * k;
    uint32_t c = 0;
    constexpr uint32_t kKeep = 4;  // tokens per thread kept in registers (t <= 4096)
    if (k == 8u && tpt <= kKeep && (reinterpret_cast<uintptr_t>(idx) & 15u) == 0) {
        // top-8 routing up to 4096 tokens: the thread's indices stay in
        // registers between the count and the rank pass
        uint4 va[kKeep], vb[kKeep];
#pragma unroll
        for (uint32_t i = 0; i < kKeep; ++i) {
            const uint32_t p = p0 + 8u * i;
            if (p < p1) {
                va[i] = *reinterpret_cast<const uint4*>(idx + p);
                vb[i] = *reinterpret_cast<const uint4*>(idx + p + 4u);
            } else {
                va[i] = vb[i] = make_uint4(~0u, ~0u, ~0u, ~0u);  // matches no expert
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < kKeep; ++i)
            c += (va[i].x == e) + (va[i].y == e) + (va[i].z == e) + (va[i].w == e) +
                 (vb[i].x == e) + (vb[i].y == e) + (vb[i].z == e) + (vb[i].w == e);
        uint32_t total;
        uint32_t before = block_exclusive_scan<1024>(c, wave_tot, total);
        if (c) {
#pragma unroll
            for (uint32_t i = 0; i < kKeep; ++i) {
                const uint32_t v[8] = {va[i].x, va[i].y, va[i].z, va[i].w,
                                       vb[i].x, vb[i].y, vb[i].z, vb[i].w};
#pragma unroll
                for (uint32_t q = 0; q < 8u; ++q)
                    if (v[q] == e) rank_of[p0 + 8u * i + q] = before++;
            }
        }
        if (threadIdx.x == 0) counts[e] = total;
        return;
    }
    if (k == 8u && (reinterpret_cast<uintptr_t>(idx) & 15u) == 0) {
        for (uint32_t p = p0; p < p1; p += 8u) {
            const uint4 a = *reinterpret_cast<const uint4*>(idx + p);
            const uint4 b = *reinterpret_cast<const uint4*>(idx + p + 4u);
            c += (a.x == e) + (a.y == e) + (a.z == e) + (a.w == e) + (b.x == e) + (b.y == e) +
                 (b.z == e) + (b.w == e);
        }
    } else {
        for (uint32_t p = p0; p < p1; ++p) c += idx[p] == e ? 1u : 0u;
    }
    uint32_t total;
    uint32_t before = block_exclusive_scan<1024>(c, wave_tot, total);
    if (c) {
        for (uint32_t p = p0; p < p1; ++p)
            if (idx[p] == e) rank_of[p] = before++;
    }
    if (threadIdx.x == 0) counts[e] = total;
}

// Scatter pairs to their sorted positions; block 0 also writes offsets and
// the GEMM work list. An expert id >= num_experts is the reference's
// expertOutOfRange (PrefillMoEGrouping.swift:52-88): its pair is left out and
// the error word gets kErrGroupExpertRange, which tsg_ctx_synchronize reports;
// a work list longer than max_blocks is cut there and sets kErrGroupBlocks.
// Each block scans the expert counts (ne <= 256, one per thread) for the
// expert offsets. The work list comes largest first: routed blocks by
// size bucket ceil(rows / 32) (capped at 8) descending, then by (expert,
// position in the expert), so the GEMM takes it in order (long items start
// early, short ones fill the tail) without sorting it again.
__global__ __launch_bounds__(256) void group_scatter_kernel(
    const uint32_t* __restrict__ idx, const uint16_t* __restrict__ w, uint32_t t, uint32_t k,
    uint32_t ne, const uint32_t* __restrict__ rank_of, const uint32_t* __restrict__ counts,
    tsg_token_expert_pair* __restrict__ sorted, uint32_t* __restrict__ offsets,
    tsg_routed_block* __restrict__ blocks, uint32_t max_blocks, uint32_t* __restrict__ n_blocks,
    uint32_t tile_rows, uint32_t* __restrict__ error_word) {
    static_assert(kMaxExperts <= 256, "one expert per thread");
    __shared__ uint32_t off_s[kMaxExperts];
    __shared__ uint32_t wave_tot[4];
    const uint32_t e = threadIdx.x;
    const uint32_t c = e < ne ? counts[e] : 0u;
    uint32_t total_rows;
    const uint32_t off = block_exclusive_scan<256>(c, wave_tot, total_rows);
    if (e < ne) off_s[e] = off;
    if (blockIdx.x == 0) {
        const uint32_t full = c / tile_rows, rem = c - full * tile_rows;
        const uint32_t bfull = min(tile_rows / 32u, 8u);
        const uint32_t brem = rem ? min((rem + 31u) / 32u, 8u) : 0u;
        uint32_t first_full = 0, first_rem = 0, running = 0;
        for (uint32_t bk = 8; bk >= 1; --bk) {
            const uint32_t n_e = (bfull == bk ? full : 0u) + (brem == bk ? 1u : 0u);
            __syncthreads();  // the previous scan's totals are read
            uint32_t total;
            const uint32_t before = block_exclusive_scan<256>(n_e, wave_tot, total);
            if (bfull == bk) first_full = running + before;
            if (brem == bk) first_rem = running + before + (bfull == bk ? full : 0u);
            running += total;
        }
        if (e == 0) {
            *n_blocks = running < max_blocks ? running : max_blocks;
            if (running > max_blocks) atomicOr(error_word, kErrGroupBlocks);
        }
        if (e < ne) {
            offsets[e] = c ? off : 0xFFFFFFFFu;
            for (uint32_t b = 0; b < full; ++b) {
                const uint32_t bi = first_full + b;
                const uint32_t start = off + b * tile_rows;
                if (bi < max_blocks) blocks[bi] = tsg_routed_block{e, start, tile_rows, start};
            }
            if (rem) {
                const uint32_t start = off + full * tile_rows;
                if (first_rem < max_blocks) blocks[first_rem] = tsg_routed_block{e, start, rem, start};
            }
        }
    }
    __syncthreads();
    const uint64_t n = (uint64_t)t * k;
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < n;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t ex = idx[p];
        if (ex >= ne) {
            atomicOr(error_word, kErrGroupExpertRange);
            continue;
        }
        const uint32_t tok = (uint32_t)(p / k), r = (uint32_t)(p - (uint64_t)tok * k);
        sorted[off_s[ex] + rank_of[p]] = tsg_token_expert_pair{tok, ex, r, (uint32_t)w[p]};
    }
}

// ---------------------------------------------------- token-major reduce

__global__ __launch_bounds__(256) void reduce_token_major_kernel(
    const uint16_t* __restrict__ p, const uint16_t* __restrict__ w, uint16_t* __restrict__ h2,
    uint32_t t, uint32_t k, uint32_t d) {
    const uint64_t total = (uint64_t)t * d;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t tok = i / d;
        const uint64_t j = i - tok * d;
        float acc = 0.0f;
        for (uint32_t r = 0; r < k; ++r)
            acc = __builtin_fmaf(f16_to_f32(w[tok * k + r]), f16_to_f32(p[(tok * k + r) * d + j]), acc);
        h2[i] = f32_to_f16(acc);
    }
}

// The same sum, eight elements per thread: 16-byte loads of the K partial
// rows (all in flight at once) and one 16-byte store. Per element the fma
// order over the ranks is the scalar kernel's, so the results are identical.
// K is a template parameter so the K loaded rows stay in registers. Needs
// d % 8 == 0 and 16-byte aligned partials and output.
template <uint32_t K>
__global__ __launch_bounds__(256) void reduce_token_major_vec_kernel(
    const uint16_t* __restrict__ p, const uint16_t* __restrict__ w, uint16_t* __restrict__ h2,
    uint32_t t, uint32_t d) {
    const uint32_t d8 = d / 8u;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= t * d8) return;
    const uint32_t tok = i / d8, j8 = i - tok * d8;
    uint4 v[K];
    uint16_t wr[K];
#pragma unroll
    for (uint32_t r = 0; r < K; ++r) {
        const uint64_t row = (uint64_t)tok * K + r;
        v[r] = *reinterpret_cast<const uint4*>(p + row * d + 8u * j8);
        wr[r] = w[row];
    }
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t r = 0; r < K; ++r) {
        const float wf = f16_to_f32(wr[r]);
        const uint32_t u[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[2 * q] = __builtin_fmaf(wf, f16_to_f32((uint16_t)(u[q] & 0xFFFFu)), acc[2 * q]);
            acc[2 * q + 1] = __builtin_fmaf(wf, f16_to_f32((uint16_t)(u[q] >> 16)), acc[2 * q + 1]);
        }
    }
    uint4 o;
    o.x = (uint32_t)f32_to_f16(acc[0]) | ((uint32_t)f32_to_f16(acc[1]) << 16);
    o.y = (uint32_t)f32_to_f16(acc[2]) | ((uint32_t)f32_to_f16(acc[3]) << 16);
    o.z = (uint32_t)f32_to_f16(acc[4]) | ((uint32_t)f32_to_f16(acc[5]) << 16);
    o.w = (uint32_t)f32_to_f16(acc[6]) | ((uint32_t)f32_to_f16(acc[7]) << 16);
    *reinterpret_cast<uint4*>(h2 + (uint64_t)tok * d + 8u * j8) = o;
}

// --------------------------------------------------------- rows path

constexpr uint32_t kRowsMax = 8;
constexpr uint32_t kRowsBlocksPerLaunch = 64;

constexpr uint32_t kRowsThreads = 512;  // 16 gate/up pairs or 64 down rows per block

// The rows path's block list travels in the kernel arguments, as the
// reference passes it with setBytes (PrefillGroupedRoutedMoE.swift:835-870).
// lds_rows: the most rows of any block in the launch (<= kRowsMax), the rows
// the LDS is sized for.
struct RowsBlocks {
    tsg_routed_block b[kRowsBlocksPerLaunch];
    uint32_t lds_rows;
};

// grid (ceil(F / 16), n_blocks), block 512: 32 lanes per f row (16 on the
// gate row, 16 on the up row), every row of the routed block (<= 8) against
// one weight read; the block's 16 f rows share one staging of the activation
// rows. Per row the arithmetic is decode phase 1's (decode.hip
// phase1_compute): the same gemv_lane.hpp steps, batch and reduction, so one
// row here is bit-identical to decode.
template <int G, bool SYM, int ACT>
__device__ __forceinline__ void rows_gate_up_body(const GemmArgs& args, const tsg_routed_block& blk,
                                                  uint32_t lds_rows) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t tok[kRowsMax];
    const uint32_t rows = blk.row_count < kRowsMax ? blk.row_count : kRowsMax;
    const uint32_t d = args.d, f = args.f;
    const uint32_t row_h = lds_chunks_halves(d);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + (size_t)lds_rows * row_h * 2u);

    const uint32_t fr_raw = blockIdx.x * (kRowsThreads / 32u) + (threadIdx.x >> 5);
    const uint32_t j = threadIdx.x & 15u;
    const bool is_up = (threadIdx.x >> 4) & 1u;
    const bool live = fr_raw < f;
    const uint32_t fr = live ? fr_raw : 0u;
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    const uint32_t ngroups = d / G, nchunks = d / 32u;
    const uint8_t* w = blob + (is_up ? args.o.up_w : args.o.gate_w) + (uint64_t)fr * (d / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + (is_up ? args.o.up_s : args.o.gate_s)) + (uint64_t)fr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + (is_up ? args.o.up_b : args.o.gate_b)) + (uint64_t)fr * ngroups;
    // the staging's loads go out before the weights (stage_act_rows_around);
    // its row indices cost one round trip first
    if (threadIdx.x < rows) tok[threadIdx.x] = args.pairs[blk.pair_start + threadIdx.x].token;
    __syncthreads();
    ChunkBatch<kGUBatch> bt;
    stage_act_rows_around<SYM>(args.a, args.a_stride, rows, d, xs, row_h, xsum, tok, [&] {
        load_batch<G, SYM, kGUBatch, kGULanes>(w, sc, bi, 0u, j, nchunks, bt);
    });
    __syncthreads();
    float acc[kRowsMax];
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) acc[r] = 0.0f;
    gemv_batches<G, SYM, kGUBatch, kGULanes, kRowsMax>(w, sc, bi, j, nchunks, bt, xs, row_h, xsum,
                                                       rows, acc);
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) {
        acc[r] = group16_sum(acc[r]);
        const float up = shfl_xor(acc[r], 16);
        if (live && !is_up && j == 0 && r < rows)
            args.out[(uint64_t)(blk.local_row + r) * f + fr] =
                f32_to_f16(gate_activation<ACT>(acc[r]) * up);
    }
}

// grid (ceil(D / 64), n_blocks), block 512: 8 lanes per output row, each of
// the block's rows against one weight read; the block's 64 output rows share
// one staging of the activation rows. Per row the arithmetic is decode phase
// 2's per-slot GEMV (decode.hip phase2_body): the same gemv_lane.hpp steps.
template <int G, bool SYM>
__device__ __forceinline__ void rows_down_body(const GemmArgs& args, const tsg_routed_block& blk,
                                               uint32_t lds_rows, uint16_t* partials) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t dst[kRowsMax];
    const uint32_t rows = blk.row_count < kRowsMax ? blk.row_count : kRowsMax;
    const uint32_t d = args.d, f = args.f;
    const uint32_t row_h = lds_chunks_halves(f);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);
    float* asum = reinterpret_cast<float*>(smem + (size_t)lds_rows * row_h * 2u);

    const uint32_t j = threadIdx.x & 7u;
    const uint32_t row = blockIdx.x * (kRowsThreads / 8u) + (threadIdx.x >> 3);
    const bool live_row = row < d;
    const uint32_t rr = live_row ? row : 0u;
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    const uint32_t ngroups = f / G, nchunks = f / 32u;
    const uint8_t* w = blob + args.o.down_w + (uint64_t)rr * (f / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + args.o.down_s) + (uint64_t)rr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + args.o.down_b) + (uint64_t)rr * ngroups;
    // the staging's loads go out before the weights (stage_act_rows_around)
    ChunkBatch<kDBatch> bt;
    stage_act_rows_around<SYM>(args.a + (uint64_t)blk.local_row * f, f, rows, f, as, row_h, asum,
                               nullptr, [&] {
                                   load_batch<G, SYM, kDBatch, kDLanes>(w, sc, bi, 0u, j, nchunks, bt);
                                   if (threadIdx.x < rows) {
                                       const tsg_token_expert_pair pr = args.pairs[blk.pair_start + threadIdx.x];
                                       dst[threadIdx.x] = (pr.token * args.top_k + pr.rank) * d;
                                   }
                               });
    __syncthreads();
    float acc[kRowsMax];
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) acc[r] = 0.0f;
    gemv_batches<G, SYM, kDBatch, kDLanes, kRowsMax>(w, sc, bi, j, nchunks, bt, as, row_h, asum, rows,
                                                     acc);
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) {
        acc[r] = group8_sum(acc[r]);
    }
    if (live_row && j == 0)
        for (uint32_t r = 0; r < rows; ++r) partials[dst[r] + row] = f32_to_f16(acc[r]);
}

template <int G, bool SYM, int ACT>
__global__ __launch_bounds__(kRowsThreads) void rows_gate_up_kernel(GemmArgs args, RowsBlocks rb) {
    rows_gate_up_body<G, SYM, ACT>(args, rb.b[blockIdx.y], rb.lds_rows);
}

template <int G, bool SYM>
__global__ __launch_bounds__(kRowsThreads) void rows_down_kernel(GemmArgs args, RowsBlocks rb,
                                                                 uint16_t* partials) {
    rows_down_body<G, SYM>(args, rb.b[blockIdx.y], rb.lds_rows, partials);
}

// The device-list forms: the block list and its count were written on the
// device (tsg_prefill_group_pairs_device), the grid covers the list's
// capacity and blocks past the count exit. A block the rows path cannot take
// (no rows, more than kRowsMax, rows past the activation scratch, an expert
// past the layer) is skipped and sets kErrRowsBlock, which
// tsg_ctx_synchronize reports.
// The list, its device count and its capacity come as leading scalar kernel
// arguments (preloaded into SGPRs by the dispatch), so the first load needs
// no kernarg round trip; the struct's fields arrive meanwhile.
__device__ __forceinline__ bool rows_device_block(const GemmArgs& args,
                                                  const tsg_routed_block* blocks,
                                                  const uint32_t* n_dev, uint32_t n_blocks,
                                                  tsg_routed_block& blk) {
    const uint32_t n = min(*n_dev, n_blocks);
    if (blockIdx.y >= n) return false;
    blk = blocks[blockIdx.y];
    if (blk.row_count == 0 || blk.row_count > kRowsMax || blk.local_slot >= args.num_experts ||
        (uint64_t)blk.local_row + blk.row_count > args.max_rows) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicOr(args.error, kErrRowsBlock);
        return false;
    }
    return true;
}

template <int G, bool SYM, int ACT>
__global__ __launch_bounds__(kRowsThreads) void rows_gate_up_dev_kernel(
    const tsg_routed_block* k_blocks, const uint32_t* k_n_dev, uint32_t k_n_blocks,
    GemmArgs args) {
    tsg_routed_block blk;
    if (rows_device_block(args, k_blocks, k_n_dev, k_n_blocks, blk))
        rows_gate_up_body<G, SYM, ACT>(args, blk, kRowsMax);
}

template <int G, bool SYM>
__global__ __launch_bounds__(kRowsThreads) void rows_down_dev_kernel(
    const tsg_routed_block* k_blocks, const uint32_t* k_n_dev, uint32_t k_n_blocks,
    uint16_t* partials, GemmArgs args) {
    tsg_routed_block blk;
    if (rows_device_block(args, k_blocks, k_n_dev, k_n_blocks, blk))
        rows_down_body<G, SYM>(args, blk, kRowsMax, partials);
}

// ------------------------------------------------------------ host side

tsg_status check_layer_moe(const tsg_moe* moe, const tsg_layer* layer) {
    TSG_REQUIRE(moe && moe->ctx, TSG_ERR_INVALID_ARGUMENT, "moe is NULL");
    TSG_REQUIRE(layer, TSG_ERR_INVALID_ARGUMENT, "layer is NULL");
    return TSG_OK;
}

template <int MODE>
tsg_status gemm_dispatch(const tsg_moe* moe, hipStream_t s, const GemmArgs& a, uint32_t max_blocks) {
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32)
        return sym ? routed_gemm_launch<32, true>(moe, s, MODE, a, max_blocks)
                   : routed_gemm_launch<32, false>(moe, s, MODE, a, max_blocks);
    return sym ? routed_gemm_launch<64, true>(moe, s, MODE, a, max_blocks)
               : routed_gemm_launch<64, false>(moe, s, MODE, a, max_blocks);
}

tsg_status fill_gemm_args(const tsg_moe* moe, const tsg_layer* layer, GemmArgs* a,
                          const uint16_t* act_in, uint32_t a_stride,
                          const tsg_token_expert_pair* pairs, const tsg_routed_block* blocks,
                          uint32_t n_blocks, const uint32_t* n_dev, uint16_t* out, uint32_t d,
                          uint32_t f, uint32_t top_k) {
    const tsg_ctx* ctx = moe->ctx;
    TSG_REQUIRE(act_in && pairs && blocks && out, TSG_ERR_INVALID_ARGUMENT, "NULL GEMM operand");
    TSG_REQUIRE(d > 0 && f > 0 && d % ctx->group_size == 0 && f % ctx->group_size == 0,
                TSG_ERR_INVALID_ARGUMENT, "d=%u, f=%u must be multiples of the group size %u",
                d, f, ctx->group_size);
    TSG_REQUIRE(d % kGemmKC == 0 && f % kGemmKC == 0, TSG_ERR_UNSUPPORTED,
                "the grouped GEMM needs d=%u and f=%u to be multiples of %u", d, f, kGemmKC);
    TSG_REQUIRE(aligned16(act_in) && a_stride % 8 == 0, TSG_ERR_ALIGNMENT,
                "activation rows must be 16-byte aligned");
    TSG_REQUIRE(aligned16(out), TSG_ERR_ALIGNMENT, "GEMM output must be 16-byte aligned");
    // scale windows are fetched as dwords: 8-group windows (G = 32) need
    // 4-byte aligned rows; 7-group windows (G = 64) tolerate 2-byte ones
    const tsg_expert_offsets& o = layer->offsets;
    TSG_REQUIRE(ctx->group_size != 32 || ((o.gate_s | o.up_s | o.down_s | o.gate_b | o.up_b |
                                           o.down_b) % 4u) == 0,
                TSG_ERR_ALIGNMENT,
                "the grouped GEMM needs 4-byte aligned scale/bias sub-tensors at group size 32");
    *a = GemmArgs{};
    a->layer_base = layer->base;
    a->expert_stride = layer->expert_stride;
    a->o = layer->offsets;
    a->a = act_in;
    a->a_stride = a_stride;
    a->pairs = pairs;
    a->blocks = blocks;
    a->n_blocks = n_blocks;
    a->n_blocks_device = n_dev;
    a->out = out;
    a->d = d;
    a->f = f;
    a->top_k = top_k;
    a->num_experts = layer->num_experts;
    a->error = ctx->counters + kSyncErrorWord;
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

using namespace tsg;

extern "C" size_t tsg_prefill_group_scratch_bytes(uint32_t query_count, uint32_t top_k,
                                                  uint32_t) {
    return (size_t)query_count * top_k * sizeof(uint32_t);
}

// Scratch of tsg_prefill_group_pairs_device_noalloc: the rank of each pair
// among its expert's pairs, one word per pair, for up to kNoAllocPairs pairs
// (256 KiB). A file-scope device array, so that entry point allocates
// nothing: each GPU the library runs on holds its own copy until the process
// ends. Host code passes the per-device address that
// tsg::group_noalloc_setup looks up, never the array's name.
static __device__ __align__(256) uint32_t noalloc_rank_scratch[kNoAllocPairs];

namespace tsg {

tsg_status group_noalloc_setup(tsg_ctx* ctx) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_rank_scratch));
    TSG_REQUIRE(e == hipSuccess && p != nullptr, TSG_ERR_HIP,
                "device %d: address of the no-alloc grouping scratch: %s", ctx->device,
                hipGetErrorString(e));
    ctx->group_rank_scratch = static_cast<uint32_t*>(p);
    return TSG_OK;
}

namespace {

// The device grouping of both entry points; rank_of holds t * k words.
tsg_status group_pairs_device(tsg_ctx* ctx, hipStream_t s, const uint32_t* idx,
                              const uint16_t* w, uint32_t t, uint32_t k, uint32_t ne,
                              uint32_t tile_rows, tsg_token_expert_pair* sorted,
                              uint32_t* offsets, uint32_t* counts, tsg_routed_block* blocks,
                              uint32_t max_blocks, uint32_t* n_blocks, uint32_t* rank_of) {
    // an expert's c pairs make ceil(c / tile_rows) <= c / tile_rows + 1 blocks
    // of at least one row, so this many always hold the list
    const uint64_t pairs_total = (uint64_t)t * k;
    const uint64_t need = std::min<uint64_t>(pairs_total, (pairs_total + tile_rows - 1) / tile_rows + ne);
    TSG_REQUIRE(max_blocks >= need, TSG_ERR_INVALID_ARGUMENT,
                "max_blocks %u cannot hold the work list: need min(t*k, ceil(t*k/%u) + %u) = %llu",
                max_blocks, tile_rows, ne, (unsigned long long)need);
    hipLaunchKernelGGL(group_rank_kernel, dim3(ne), dim3(1024), 0, s, idx, t, k, rank_of, counts);
    tsg_status st = check_launch("group_rank");
    if (st) return st;
    const uint64_t n = (uint64_t)t * k;
    uint64_t grid = (n + 255) / 256;
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(group_scatter_kernel, dim3(grid), dim3(256), 0, s, idx, w, t, k, ne,
                       rank_of, counts, sorted, offsets, blocks, max_blocks, n_blocks, tile_rows,
                       ctx->counters + kSyncErrorWord);
    return check_launch("group_scatter");
}

tsg_status check_group_args(const tsg_ctx* ctx, uint32_t t, uint32_t k, uint32_t ne,
                            uint32_t tile_rows) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(t > 0, TSG_ERR_GROUPING_INVALID_QUERY_COUNT, "queryCount must be positive");
    TSG_REQUIRE(k > 0, TSG_ERR_GROUPING_INVALID_TOP_K, "topK must be positive");
    TSG_REQUIRE(ne > 0 && ne <= kMaxExperts, TSG_ERR_GROUPING_INVALID_NUM_EXPERTS,
                "numExperts %u not in 1..%u", ne, kMaxExperts);
    TSG_REQUIRE(tile_rows == 32 || tile_rows == 64 || tile_rows == 128 || tile_rows == 256,
                TSG_ERR_INVALID_ARGUMENT, "tile_rows must be 32, 64, 128 or 256, got %u", tile_rows);
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

extern "C" tsg_status tsg_prefill_group_pairs_device(
    tsg_ctx* ctx, tsg_stream stream, const uint32_t* idx, const uint16_t* w, uint32_t t,
    uint32_t k, uint32_t ne, uint32_t tile_rows, tsg_token_expert_pair* sorted,
    uint32_t* offsets, uint32_t* counts, tsg_routed_block* blocks, uint32_t max_blocks,
    uint32_t* n_blocks, void* scratch) {
    tsg_status st = check_group_args(ctx, t, k, ne, tile_rows);
    if (st) return st;
    TSG_REQUIRE(idx && w && sorted && offsets && counts && blocks && n_blocks && scratch,
                TSG_ERR_INVALID_ARGUMENT, "NULL grouping operand");
    return group_pairs_device(ctx, as_stream(stream), idx, w, t, k, ne, tile_rows, sorted, offsets,
                              counts, blocks, max_blocks, n_blocks, static_cast<uint32_t*>(scratch));
}

extern "C" tsg_status tsg_prefill_group_pairs_device_noalloc(
    tsg_ctx* ctx, tsg_stream stream, const uint32_t* idx, const uint16_t* w, uint32_t t,
    uint32_t k, uint32_t ne, uint32_t tile_rows, tsg_token_expert_pair* sorted,
    uint32_t* offsets, uint32_t* counts, tsg_routed_block* blocks, uint32_t max_blocks,
    uint32_t* n_blocks) {
    tsg_status st = check_group_args(ctx, t, k, ne, tile_rows);
    if (st) return st;
    TSG_REQUIRE(idx && w && sorted && offsets && counts && blocks && n_blocks,
                TSG_ERR_INVALID_ARGUMENT, "NULL grouping operand");
    TSG_REQUIRE((uint64_t)t * k <= kNoAllocPairs, TSG_ERR_UNSUPPORTED,
                "t*k = %llu pairs exceed the no-alloc grouping scratch (%u pairs); use "
                "tsg_prefill_group_pairs_device with a workspace",
                (unsigned long long)t * k, kNoAllocPairs);
    TSG_REQUIRE(ctx->group_rank_scratch, TSG_ERR_HIP, "context has no no-alloc grouping scratch");
    return group_pairs_device(ctx, as_stream(stream), idx, w, t, k, ne, tile_rows, sorted, offsets,
                              counts, blocks, max_blocks, n_blocks, ctx->group_rank_scratch);
}

extern "C" tsg_status tsg_prefill_moe_gate_up(tsg_moe* moe, tsg_stream stream,
                                              const tsg_layer* layer, const uint16_t* hidden,
                                              uint32_t hidden_stride,
                                              const tsg_token_expert_pair* pairs,
                                              const tsg_routed_block* blocks, uint32_t n_blocks,
                                              const uint32_t* n_dev, uint16_t* act, uint32_t d,
                                              uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    if (n_blocks == 0) return TSG_OK;
    GemmArgs a;
    if ((st = fill_gemm_args(moe, layer, &a, hidden, hidden_stride, pairs, blocks, n_blocks,
                             n_dev, act, d, f, kTopK)))
        return st;
    return gemm_dispatch<0>(moe, as_stream(stream), a, n_blocks);
}

extern "C" tsg_status tsg_prefill_moe_gate_up_down(
    tsg_moe* moe, tsg_stream stream, const tsg_layer* layer, const uint16_t* hidden,
    uint32_t hidden_stride, const tsg_token_expert_pair* pairs, const tsg_routed_block* blocks,
    uint32_t n_blocks, const uint32_t* n_dev, uint16_t* act, uint16_t* partials, uint32_t top_k,
    uint32_t d, uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    TSG_REQUIRE(top_k > 0, TSG_ERR_INVALID_ARGUMENT, "topK must be positive");
    if (n_blocks == 0) return TSG_OK;
    TSG_REQUIRE(n_blocks <= kGemmSchedBlocks, TSG_ERR_UNSUPPORTED,
                "the fused GEMM takes up to %u routed blocks, got %u", kGemmSchedBlocks, n_blocks);
    TSG_REQUIRE(((uintptr_t)act & 127u) == 0, TSG_ERR_ALIGNMENT,
                "the fused GEMM's activation buffer must be 128-byte aligned");
    GemmArgs gu, dn;
    if ((st = fill_gemm_args(moe, layer, &gu, hidden, hidden_stride, pairs, blocks, n_blocks, n_dev,
                             act, d, f, kTopK)))
        return st;
    if ((st = fill_gemm_args(moe, layer, &dn, act, f, pairs, blocks, n_blocks, n_dev, partials, d,
                             f, top_k)))
        return st;
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    hipStream_t s = as_stream(stream);
    if (ctx->gemm_queues == 0) {
        // XCD count unknown or not one queue per XCD: the two launches (the
        // same results; the hand-off between the GEMMs is the launch boundary)
        if ((st = gemm_dispatch<0>(moe, s, gu, n_blocks))) return st;
        return gemm_dispatch<1>(moe, s, dn, n_blocks);
    }
    if (ctx->group_size == 32)
        return sym ? routed_gemm_fused_launch<32, true>(moe, s, gu, dn, n_blocks)
                   : routed_gemm_fused_launch<32, false>(moe, s, gu, dn, n_blocks);
    return sym ? routed_gemm_fused_launch<64, true>(moe, s, gu, dn, n_blocks)
               : routed_gemm_fused_launch<64, false>(moe, s, gu, dn, n_blocks);
}

extern "C" tsg_status tsg_prefill_moe_down(tsg_moe* moe, tsg_stream stream,
                                           const tsg_layer* layer, const uint16_t* act,
                                           const tsg_token_expert_pair* pairs,
                                           const tsg_routed_block* blocks, uint32_t n_blocks,
                                           const uint32_t* n_dev, uint16_t* partials,
                                           uint32_t top_k, uint32_t d, uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    TSG_REQUIRE(top_k > 0, TSG_ERR_INVALID_ARGUMENT, "topK must be positive");
    if (n_blocks == 0) return TSG_OK;
    GemmArgs a;
    if ((st = fill_gemm_args(moe, layer, &a, act, f, pairs, blocks, n_blocks, n_dev, partials, d,
                             f, top_k)))
        return st;
    return gemm_dispatch<1>(moe, as_stream(stream), a, n_blocks);
}

extern "C" tsg_status tsg_prefill_moe_rows(tsg_moe* moe, tsg_stream stream,
                                           const tsg_layer* layer, const uint16_t* hidden,
                                           uint32_t hidden_stride,
                                           const tsg_token_expert_pair* pairs,
                                           const tsg_routed_block* blocks, uint32_t n_blocks,
                                           uint16_t* act_scratch, uint32_t max_rows,
                                           uint16_t* partials, uint32_t top_k, uint32_t d,
                                           uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    if (n_blocks == 0) return TSG_OK;
    TSG_REQUIRE(blocks, TSG_ERR_INVALID_ARGUMENT, "blocks is NULL");
    // The host chooses the rows path from the grouping, and it declines blocks
    // wider than its cap and a tile whose activation rows exceed the scratch
    // it was sized for (PrefillGroupedRoutedMoE.swift:808-830).
    for (uint32_t i = 0; i < n_blocks; ++i) {
        if (blocks[i].row_count == 0 || blocks[i].row_count > kRowsMax)
            return fail(TSG_ERR_DECLINED, "rows path takes 1..%u rows per block, block %u has %u",
                        kRowsMax, i, blocks[i].row_count);
        if ((uint64_t)blocks[i].local_row + blocks[i].row_count > max_rows)
            return fail(TSG_ERR_DECLINED,
                        "block %u's activation rows %u..%u reach past the scratch's %u rows", i,
                        blocks[i].local_row, blocks[i].local_row + blocks[i].row_count - 1u,
                        max_rows);
        // the block list is on the host: an expert id past the layer would
        // make the kernels read outside it
        TSG_REQUIRE(blocks[i].local_slot < layer->num_experts, TSG_ERR_INVALID_ARGUMENT,
                    "block %u names expert %u but the layer holds %u", i, blocks[i].local_slot,
                    layer->num_experts);
        TSG_REQUIRE((uint64_t)blocks[i].local_row + blocks[i].row_count <= 0xFFFFFFFFull &&
                        (uint64_t)blocks[i].pair_start + blocks[i].row_count <= 0xFFFFFFFFull,
                    TSG_ERR_INVALID_ARGUMENT, "block %u's rows overflow 32 bits", i);
    }
    TSG_REQUIRE(top_k > 0 && act_scratch && partials, TSG_ERR_INVALID_ARGUMENT,
                "NULL rows operand");
    GemmArgs a;
    if ((st = fill_gemm_args(moe, layer, &a, hidden, hidden_stride, pairs, blocks, n_blocks,
                             nullptr, act_scratch, d, f, top_k)))
        return st;
    TSG_REQUIRE(aligned16(act_scratch), TSG_ERR_ALIGNMENT, "act_scratch must be 16-byte aligned");
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    const size_t lds1 = (size_t)kRowsMax * lds_chunks_halves(d) * 2u + (sym ? 0u : kRowsMax * (d / 32u) * 4u);
    const size_t lds2 = (size_t)kRowsMax * lds_chunks_halves(f) * 2u + (sym ? 0u : kRowsMax * (f / 32u) * 4u);
    TSG_REQUIRE(lds1 <= 160u * 1024u && lds2 <= 160u * 1024u, TSG_ERR_UNSUPPORTED,
                "d=%u / f=%u do not fit the rows path's LDS staging", d, f);
    hipStream_t s = as_stream(stream);
    GemmArgs a2 = a;
    a2.a = act_scratch;
    a2.a_stride = f;
    for (uint32_t b0 = 0; b0 < n_blocks; b0 += kRowsBlocksPerLaunch) {
        const uint32_t nb = n_blocks - b0 < kRowsBlocksPerLaunch ? n_blocks - b0 : kRowsBlocksPerLaunch;
        RowsBlocks rb{};
        rb.lds_rows = 1;
        for (uint32_t i = 0; i < nb; ++i) {
            rb.b[i] = blocks[b0 + i];
            rb.lds_rows = std::max(rb.lds_rows, std::min(blocks[b0 + i].row_count, kRowsMax));
        }
        // LDS for the launch's widest block (the maximum checked above)
        const size_t l1 = (size_t)rb.lds_rows * lds_chunks_halves(d) * 2u + (sym ? 0u : rb.lds_rows * (d / 32u) * 4u);
        const size_t l2 = (size_t)rb.lds_rows * lds_chunks_halves(f) * 2u + (sym ? 0u : rb.lds_rows * (f / 32u) * 4u);
        const dim3 g1((f + kRowsThreads / 32u - 1u) / (kRowsThreads / 32u), nb);
        const dim3 g2((d + kRowsThreads / 8u - 1u) / (kRowsThreads / 8u), nb);
#define TSG_ROWS_LAUNCH(GG, SS)                                                                    \
    do {                                                                                           \
        if (moe->activation == TSG_ACT_SILU)                                                       \
            hipLaunchKernelGGL((rows_gate_up_kernel<GG, SS, TSG_ACT_SILU>), g1,                    \
                               dim3(kRowsThreads), l1, s, a, rb);                                  \
        else                                                                                       \
            hipLaunchKernelGGL((rows_gate_up_kernel<GG, SS, TSG_ACT_GELU_TANH>), g1,               \
                               dim3(kRowsThreads), l1, s, a, rb);                                  \
        if ((st = check_launch("rows gate/up"))) return st;                                       \
        hipLaunchKernelGGL((rows_down_kernel<GG, SS>), g2, dim3(kRowsThreads), l2, s, a2, rb,      \
                           partials);                                                              \
        if ((st = check_launch("rows down"))) return st;                                          \
    } while (0)
        if (ctx->group_size == 32) {
            if (sym) TSG_ROWS_LAUNCH(32, true);
            else TSG_ROWS_LAUNCH(32, false);
        } else {
            if (sym) TSG_ROWS_LAUNCH(64, true);
            else TSG_ROWS_LAUNCH(64, false);
        }
#undef TSG_ROWS_LAUNCH
    }
    return TSG_OK;
}

extern "C" tsg_status tsg_prefill_moe_rows_device(tsg_moe* moe, tsg_stream stream,
                                                  const tsg_layer* layer, const uint16_t* hidden,
                                                  uint32_t hidden_stride,
                                                  const tsg_token_expert_pair* pairs,
                                                  const tsg_routed_block* blocks,
                                                  uint32_t max_blocks,
                                                  const uint32_t* n_blocks_device,
                                                  uint16_t* act_scratch, uint32_t max_rows,
                                                  uint16_t* partials, uint32_t top_k, uint32_t d,
                                                  uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    TSG_REQUIRE(n_blocks_device && top_k > 0 && act_scratch && partials, TSG_ERR_INVALID_ARGUMENT,
                "NULL rows operand");
    TSG_REQUIRE(max_blocks > 0 && max_blocks <= 65535u, TSG_ERR_INVALID_ARGUMENT,
                "max_blocks must be in 1..65535, got %u", max_blocks);
    GemmArgs a;
    if ((st = fill_gemm_args(moe, layer, &a, hidden, hidden_stride, pairs, blocks, max_blocks,
                             n_blocks_device, act_scratch, d, f, top_k)))
        return st;
    TSG_REQUIRE(aligned16(act_scratch), TSG_ERR_ALIGNMENT, "act_scratch must be 16-byte aligned");
    a.max_rows = max_rows;
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    // LDS for the widest block the rows path takes
    const size_t l1 = (size_t)kRowsMax * lds_chunks_halves(d) * 2u + (sym ? 0u : kRowsMax * (d / 32u) * 4u);
    const size_t l2 = (size_t)kRowsMax * lds_chunks_halves(f) * 2u + (sym ? 0u : kRowsMax * (f / 32u) * 4u);
    TSG_REQUIRE(l1 <= 64u * 1024u && l2 <= 64u * 1024u, TSG_ERR_UNSUPPORTED,
                "d=%u / f=%u do not fit the rows path's LDS staging", d, f);
    hipStream_t s = as_stream(stream);
    GemmArgs a2 = a;
    a2.a = act_scratch;
    a2.a_stride = f;
    const dim3 g1((f + kRowsThreads / 32u - 1u) / (kRowsThreads / 32u), max_blocks);
    const dim3 g2((d + kRowsThreads / 8u - 1u) / (kRowsThreads / 8u), max_blocks);
#define TSG_ROWS_DEV(GG, SS)                                                                       \
    do {                                                                                           \
        if (moe->activation == TSG_ACT_SILU)                                                       \
            hipLaunchKernelGGL((rows_gate_up_dev_kernel<GG, SS, TSG_ACT_SILU>), g1,                \
                               dim3(kRowsThreads), l1, s, blocks, n_blocks_device, max_blocks, a); \
        else                                                                                       \
            hipLaunchKernelGGL((rows_gate_up_dev_kernel<GG, SS, TSG_ACT_GELU_TANH>), g1,           \
                               dim3(kRowsThreads), l1, s, blocks, n_blocks_device, max_blocks, a); \
        if ((st = check_launch("rows gate/up (device list)"))) return st;                         \
        hipLaunchKernelGGL((rows_down_dev_kernel<GG, SS>), g2, dim3(kRowsThreads), l2, s, blocks,  \
                           n_blocks_device, max_blocks, partials, a2);                             \
        return check_launch("rows down (device list)");                                           \
    } while (0)
    if (ctx->group_size == 32) {
        if (sym) TSG_ROWS_DEV(32, true);
        TSG_ROWS_DEV(32, false);
    }
    if (sym) TSG_ROWS_DEV(64, true);
    TSG_ROWS_DEV(64, false);
#undef TSG_ROWS_DEV
}

extern "C" tsg_status tsg_prefill_moe_reduce_token_major(tsg_ctx* ctx, tsg_stream stream,
                                                         const uint16_t* partials,
                                                         const uint16_t* w, uint16_t* h2,
                                                         uint32_t t, uint32_t k, uint32_t d) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(t > 0, TSG_ERR_INVALID_ARGUMENT, "queryCount must be positive");
    TSG_REQUIRE(k > 0, TSG_ERR_INVALID_ARGUMENT, "topK must be positive");
    TSG_REQUIRE(d > 0, TSG_ERR_INVALID_ARGUMENT, "D must be positive");
    TSG_REQUIRE(partials && w && h2, TSG_ERR_INVALID_ARGUMENT, "NULL reduce operand");
    const uint64_t total = (uint64_t)t * d;
    if (d % 8u == 0 && aligned16(partials) && aligned16(h2) && total / 8u < (1ull << 31)) {
        const dim3 grid((uint32_t)((total / 8u + 255) / 256)), block(256);
        hipStream_t hs = as_stream(stream);
        bool launched = true;
        switch (k) {
            case 1: hipLaunchKernelGGL(reduce_token_major_vec_kernel<1>, grid, block, 0, hs, partials, w, h2, t, d); break;
            case 2: hipLaunchKernelGGL(reduce_token_major_vec_kernel<2>, grid, block, 0, hs, partials, w, h2, t, d); break;
            case 4: hipLaunchKernelGGL(reduce_token_major_vec_kernel<4>, grid, block, 0, hs, partials, w, h2, t, d); break;
            case 8: hipLaunchKernelGGL(reduce_token_major_vec_kernel<8>, grid, block, 0, hs, partials, w, h2, t, d); break;
            default: launched = false;
        }
        if (launched) return check_launch("reduce_token_major_vec");
    }
    uint64_t grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(reduce_token_major_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                       partials, w, h2, t, k, d);
    return check_launch("reduce_token_major");
}

extern "C" tsg_status tsg_prefill_int4_qmm(tsg_ctx* ctx, tsg_stream stream,
                                           const uint8_t* weights, const uint16_t* scales,
                                           const uint16_t* biases, const uint16_t* x,
                                           uint16_t* y, uint32_t t, uint32_t n, uint32_t k) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    const uint32_t g = ctx->group_size;
    const bool sym = ctx->scheme == TSG_SYM;
    TSG_REQUIRE(t > 0 && n > 0 && k > 0, TSG_ERR_INVALID_ARGUMENT, "t, n and k must be positive");
    TSG_REQUIRE(k % g == 0, TSG_ERR_INVALID_ARGUMENT, "K must be a multiple of %u", g);
    TSG_REQUIRE(weights && scales && x && y && (sym || biases), TSG_ERR_INVALID_ARGUMENT,
                "NULL QMM operand");
    TSG_REQUIRE(g == 32 || g == 64, TSG_ERR_UNSUPPORTED,
                "the tiled QMM supports group sizes 32 and 64, not %u", g);
    TSG_REQUIRE(k % kGemmKC == 0 && n % 64u == 0, TSG_ERR_UNSUPPORTED,
                "the tiled QMM needs K=%u and N=%u to be multiples of 64", k, n);
    TSG_REQUIRE(aligned16(weights) && aligned16(x) && aligned16(y), TSG_ERR_ALIGNMENT,
                "weights, x and y must be 16-byte aligned");
    TSG_REQUIRE((uint64_t)t * n < (1ull << 32) && (uint64_t)t * k < (1ull << 32),
                TSG_ERR_UNSUPPORTED, "t*n and t*k must stay below 2^32 elements");
    const uint16_t* b = sym ? scales : biases;
    // scale and bias windows are fetched as dwords from the sub-tensor bases
    TSG_REQUIRE(((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(b)) % 4u) == 0,
                TSG_ERR_ALIGNMENT, "scales and biases must be 4-byte aligned");
    TSG_REQUIRE((uint64_t)n * k / 2u < (1ull << 32), TSG_ERR_UNSUPPORTED,
                "the weight matrix must stay below 4 GiB");
    GemmArgs a{};  // all nine offsets 0: each sub-tensor has its own base
    a.layer_base = weights;
    a.dense_s = reinterpret_cast<const uint8_t*>(scales);
    a.dense_b = reinterpret_cast<const uint8_t*>(b);
    a.a = x;
    a.a_stride = k;
    a.out = y;
    a.d = n;
    a.f = k;
    a.top_k = 1;
    a.dense_rows = t;
    hipStream_t hs = as_stream(stream);
    const uint32_t cus = (uint32_t)ctx->num_cus;
    if (g == 32)
        return sym ? dense_qmm_launch<32, true>(hs, a, cus) : dense_qmm_launch<32, false>(hs, a, cus);
    return sym ? dense_qmm_launch<64, true>(hs, a, cus) : dense_qmm_launch<64, false>(hs, a, cus);
}

// The GEMM's own fp16 staging, un-paired (test hook for bit-exact dequant).
extern "C" tsg_status tsg_debug_gemm_dequant_f16(tsg_ctx* ctx, tsg_stream stream,
                                                 const uint8_t* w, const uint16_t* scales,
                                                 const uint16_t* biases, uint16_t* out,
                                                 uint32_t rows, uint32_t n) {
    TSG_REQUIRE(ctx && w && scales && out, TSG_ERR_INVALID_ARGUMENT, "NULL operand");
    TSG_REQUIRE(ctx->scheme == TSG_SYM || biases, TSG_ERR_INVALID_ARGUMENT,
                "biases is NULL under the affine scheme");
    TSG_REQUIRE(n % ctx->group_size == 0 && n % 16 == 0 && rows > 0, TSG_ERR_INVALID_ARGUMENT,
                "bad shape rows=%u n=%u", rows, n);
    TSG_REQUIRE(reinterpret_cast<uintptr_t>(w) % 4 == 0 && aligned16(out), TSG_ERR_ALIGNMENT,
                "weights must be 4-byte and out 16-byte aligned");
    const uint64_t pieces = (uint64_t)rows * (n / 8u);
    uint64_t grid = (pieces + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipStream_t s = as_stream(stream);
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32) {
        if (sym) hipLaunchKernelGGL((gemm_dequant_probe_kernel<32, true>), dim3(grid), dim3(256), 0, s, w, scales, scales, out, rows, n);
        else hipLaunchKernelGGL((gemm_dequant_probe_kernel<32, false>), dim3(grid), dim3(256), 0, s, w, scales, biases, out, rows, n);
    } else {
        if (sym) hipLaunchKernelGGL((gemm_dequant_probe_kernel<64, true>), dim3(grid), dim3(256), 0, s, w, scales, scales, out, rows, n);
        else hipLaunchKernelGGL((gemm_dequant_probe_kernel<64, false>), dim3(grid), dim3(256), 0, s, w, scales, biases, out, rows, n);
    }
    return check_launch("gemm_dequant_probe");
}
