// gemv_lane.hpp — the per-lane steps of the int4 GEMVs (decode phase 1/2, the
// verify rows path and QMV), shared so that every caller performs the same
// operations in the same order on a given row: one row through the rows path
// is bit-identical to decode (PrefillRoutedMoERowsVsDecodeTests.swift:23-166).
//
// A weight row of K int4 values is K/32 16-byte chunks (one g32 group, half a
// g64 group). `LANES` lanes share a row; lane j owns chunks j, j+LANES, ...,
// loaded KB at a time with every load of a batch issued before any use.
// Chunks are 16-byte aligned (WA = 16) or, for weights bound at a 2-byte
// aligned offset, read by load16_a2 (WA = 2).
// Chunks past the row end load a clamped address and leave the sum untouched,
// so a row's bits do not depend on KB (how many chunk slots a lane carries).
#pragma once

#include "tsg_internal.hpp"

namespace tsg {

// Lane geometry shared by every caller so a row's arithmetic is the same
// everywhere: a gate or up row (K = hidden, 88 chunks for Gemma) is split over
// 16 lanes, a down row (K = intermediate, 22 chunks) over 8.
constexpr int kGULanes = 16;
constexpr int kGUBatch = 6;   // chunks per lane per batch: one batch up to K = 3072
constexpr int kDLanes = 8;
constexpr int kDBatch = 3;    // one batch up to K = 768

template <int KB>
struct ChunkBatch {
    uint4 w[KB];
    uint32_t s[KB];
    uint32_t b[KB];
};

template <int G, bool SYM, int KB, int LANES, int WA = 16>
__device__ __forceinline__ void load_batch(const uint8_t* __restrict__ w_row,
                                           const uint16_t* __restrict__ s_row,
                                           const uint16_t* __restrict__ b_row, uint32_t base,
                                           uint32_t j, uint32_t nchunks, ChunkBatch<KB>& bt) {
    // scales (and biases) first, then the chunks in the order compute_batch
    // uses them: loads return in issue order, so chunk i is usable once the
    // loads after it are the only ones outstanding, and the dot products of
    // early chunks run while later chunks are still in flight
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const uint32_t cc = min(base + j + LANES * i, nchunks - 1u);
        bt.s[i] = s_row[cc * 32u / G];
        if constexpr (!SYM) bt.b[i] = b_row[cc * 32u / G];
    }
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const uint32_t cc = min(base + j + LANES * i, nchunks - 1u);
        bt.w[i] = load_weights16<WA>(w_row + 16u * cc);
    }
}

// acc[r] += sum over the batch's chunks of scale * dot(chunk, x_r) (+ bias *
// chunk-sum of x_r for affine), for rows r < nrows of the staged activations
// (row r at xs + r * row_h, sums at xsum + r * nchunks).
template <int G, bool SYM, int KB, int LANES, int R>
__device__ __forceinline__ void compute_batch(const ChunkBatch<KB>& bt, uint32_t base, uint32_t j,
                                              uint32_t nchunks, const uint16_t* xs,
                                              uint32_t row_h, const float* xsum,
                                              uint32_t nrows, float* acc) {
    const h2_t bias = SYM ? h2_t{(_Float16)1032.0f, (_Float16)1032.0f}
                          : h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const uint32_t c = base + j + LANES * i;
        const uint32_t cc = min(c, nchunks - 1u);
        const bool live = c < nchunks;
        const float s = bf16_to_f32((uint16_t)bt.s[i]);
        float b = 0.0f;
        if constexpr (!SYM) b = bf16_to_f32((uint16_t)bt.b[i]);
        if constexpr (R == 1) {
            float v = __builtin_fmaf(s, chunk_dot(bt.w[i], staged_chunk(xs, cc), bias), acc[0]);
            if constexpr (!SYM) v = __builtin_fmaf(b, xsum[cc], v);
            acc[0] = live ? v : acc[0];  // a chunk past the row end leaves acc as it is
        } else {
            // several rows: the chunk's weights are unpacked once for all of them
            h2_t q[16];
            chunk_pairs(bt.w[i], bias, q);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if ((uint32_t)r >= nrows) break;
                float v = __builtin_fmaf(s, chunk_dot_pairs(q, staged_chunk(xs + (size_t)r * row_h, cc)),
                                         acc[r]);
                if constexpr (!SYM) v = __builtin_fmaf(b, xsum[r * nchunks + cc], v);
                acc[r] = live ? v : acc[r];
            }
        }
    }
}

// compute_batch's several-row form for two weight rows of one lane with the
// same chunk positions (a gate row in bt0, its up row in bt1), over rows
// picked from a larger staging: row r is staged row (rt >> 3r) & 7 (at xs +
// row * row_h, sums at xsum + row * nchunks). Each staged chunk of a picked
// row is read from LDS once for both weight rows, and each weight row takes
// compute_batch's steps (the same dot2 sequence per chunk, the same fma per
// chunk), so its bits are the same as when it is computed alone.
template <int G, bool SYM, int KB, int LANES, int R>
__device__ __forceinline__ void compute_batch_picked2(const ChunkBatch<KB>& bt0,
                                                      const ChunkBatch<KB>& bt1, uint32_t base,
                                                      uint32_t j, uint32_t nchunks,
                                                      const uint16_t* xs, uint32_t row_h,
                                                      const float* xsum, uint32_t rt,
                                                      uint32_t nrows, float* acc0, float* acc1) {
    static_assert(R <= 8, "three bits per picked row");
    const h2_t bias = SYM ? h2_t{(_Float16)1032.0f, (_Float16)1032.0f}
                          : h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const uint32_t c = base + j + LANES * i;
        const uint32_t cc = min(c, nchunks - 1u);
        const bool live = c < nchunks;
        const float s0 = bf16_to_f32((uint16_t)bt0.s[i]), s1 = bf16_to_f32((uint16_t)bt1.s[i]);
        float b0 = 0.0f, b1 = 0.0f;
        if constexpr (!SYM) {
            b0 = bf16_to_f32((uint16_t)bt0.b[i]);
            b1 = bf16_to_f32((uint16_t)bt1.b[i]);
        }
        h2_t q0[16], q1[16];
        chunk_pairs(bt0.w[i], bias, q0);
        chunk_pairs(bt1.w[i], bias, q1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if ((uint32_t)r >= nrows) break;
            const uint32_t row = (rt >> (3 * r)) & 7u;
            const h2_t* xp = staged_chunk(xs + (size_t)row * row_h, cc);
            float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const h2_t x = xp[k];
                d0 = dot2(q0[k], x, d0);
                d1 = dot2(q1[k], x, d1);
            }
            float v0 = __builtin_fmaf(s0, d0, acc0[r]);
            float v1 = __builtin_fmaf(s1, d1, acc1[r]);
            if constexpr (!SYM) {
                const float xsm = xsum[row * nchunks + cc];
                v0 = __builtin_fmaf(b0, xsm, v0);
                v1 = __builtin_fmaf(b1, xsm, v1);
            }
            acc0[r] = live ? v0 : acc0[r];
            acc1[r] = live ? v1 : acc1[r];
        }
        // one chunk at a time: the scheduler would otherwise unpack later
        // chunks' weights ahead (32 registers each) and spill
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Both rows' whole segments (compute_batch_picked2); bt0 / bt1 hold the first
// batches, requested by the caller.
template <int G, bool SYM, int KB, int LANES, int R, int WA = 16>
__device__ __forceinline__ void gemv_batches_picked2(
    const uint8_t* __restrict__ w0, const uint16_t* __restrict__ s0,
    const uint16_t* __restrict__ b0, const uint8_t* __restrict__ w1,
    const uint16_t* __restrict__ s1, const uint16_t* __restrict__ b1, uint32_t j,
    uint32_t nchunks, ChunkBatch<KB>& bt0, ChunkBatch<KB>& bt1, const uint16_t* xs,
    uint32_t row_h, const float* xsum, uint32_t rt, uint32_t nrows, float* acc0, float* acc1) {
    compute_batch_picked2<G, SYM, KB, LANES, R>(bt0, bt1, 0u, j, nchunks, xs, row_h, xsum, rt, nrows,
                                                acc0, acc1);
    for (uint32_t base = LANES * KB; base < nchunks; base += LANES * KB) {
        load_batch<G, SYM, KB, LANES, WA>(w0, s0, b0, base, j, nchunks, bt0);
        load_batch<G, SYM, KB, LANES, WA>(w1, s1, b1, base, j, nchunks, bt1);
        compute_batch_picked2<G, SYM, KB, LANES, R>(bt0, bt1, base, j, nchunks, xs, row_h, xsum, rt,
                                                    nrows, acc0, acc1);
    }
}

// A whole row segment: the first batch, already requested into `bt` by the
// caller with load_batch (so its loads can go out early), then the rest
// batch by batch. The first batch sits outside the loop so the compiler's
// waits before its chunks count only the loads issued after each (inside a
// loop they are merged with the back edge's and wait for every load).
template <int G, bool SYM, int KB, int LANES, int R, int WA = 16>
__device__ __forceinline__ void gemv_batches(const uint8_t* __restrict__ w_row,
                                             const uint16_t* __restrict__ s_row,
                                             const uint16_t* __restrict__ b_row, uint32_t j,
                                             uint32_t nchunks, ChunkBatch<KB>& bt,
                                             const uint16_t* xs, uint32_t row_h,
                                             const float* xsum, uint32_t nrows, float* acc) {
    compute_batch<G, SYM, KB, LANES, R>(bt, 0u, j, nchunks, xs, row_h, xsum, nrows, acc);
    for (uint32_t base = LANES * KB; base < nchunks; base += LANES * KB) {
        load_batch<G, SYM, KB, LANES, WA>(w_row, s_row, b_row, base, j, nchunks, bt);
        compute_batch<G, SYM, KB, LANES, R>(bt, base, j, nchunks, xs, row_h, xsum, nrows, acc);
    }
}

}  // namespace tsg
