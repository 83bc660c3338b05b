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
