// prefill.hip — prompt-chunk routed MoE for gfx950.
//
//   device grouping   PrefillMoEGrouping.swift:90-202 (stable counting sort)
//   grouped GEMMs     prefill.metal:913-1092, 3664-3864 (encodeStreamedTiled)
//   token-major sum   prefill.metal:796-817
//   verify rows path  prefill.metal:1489-1721 (encodeStreamedRows)
//
// GEMM design: a 256-thread block owns one routed block (<= 64 rows of one
// expert) x 128 weight rows. Per 32-wide K step the block gathers the 64
// activation rows into LDS (fp16, k permuted into the "paired" order the
// nibble conversion produces) and dequantises 128 x 32 int4 weights into LDS as
// fp16, each value RNE(fma(q, s, b)) exactly as the reference stages it. Four
// waves (2 x 2) each accumulate 32 x 64 of the output with
// v_mfma_f32_32x32x16_f16 (fp32 accumulation). Gate and up share the block:
// weight rows 0..63 are gate f0..f0+63, 64..127 up f0..f0+63, so the GeGLU
// epilogue finds both halves in the same lane.
#include "gemv_lane.hpp"

namespace tsg {
namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------- device grouping

// One block per expert e: rank_of[p] = position of pair p among the pairs of
// expert e in (token, rank) order; counts[e] = their number.
__global__ __launch_bounds__(1024) void group_rank_kernel(const uint32_t* __restrict__ idx,
                                                          uint32_t t, uint32_t k,
                                                          uint32_t* __restrict__ rank_of,
                                                          uint32_t* __restrict__ counts) {
    __shared__ uint32_t wave_tot[16];
    __shared__ uint32_t carry_s;
    const uint32_t e = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t carry = 0;
    for (uint32_t t0 = 0; t0 < t; t0 += 1024u) {
        const uint32_t tok = t0 + threadIdx.x;
        uint32_t c = 0;
        if (tok < t)
            for (uint32_t r = 0; r < k; ++r) c += idx[(uint64_t)tok * k + r] == e ? 1u : 0u;
        // inclusive scan of c across the block
        uint32_t v = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(v, off, 64);
            if ((int)lane >= off) v += o;
        }
        if (lane == 63) wave_tot[wave] = v;
        __syncthreads();
        if (threadIdx.x < 64) {
            uint32_t w = threadIdx.x < 16 ? wave_tot[threadIdx.x] : 0u;
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const uint32_t o = __shfl_up(w, off, 64);
                if ((int)threadIdx.x >= off) w += o;
            }
            if (threadIdx.x < 16) wave_tot[threadIdx.x] = w;  // inclusive
        }
        __syncthreads();
        const uint32_t before = carry + (wave ? wave_tot[wave - 1] : 0u) + (v - c);
        if (c) {
            uint32_t j = 0;
            for (uint32_t r = 0; r < k; ++r)
                if (idx[(uint64_t)tok * k + r] == e) rank_of[(uint64_t)tok * k + r] = before + j++;
        }
        if (threadIdx.x == 0) carry_s = carry + wave_tot[15];
        __syncthreads();
        carry = carry_s;
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[e] = carry;
}

// Scatter pairs to their sorted positions; block 0 also writes offsets and
// the GEMM work list. Expert ids >= num_experts are dropped (never routed).
__global__ __launch_bounds__(256) void group_scatter_kernel(
    const uint32_t* __restrict__ idx, const uint16_t* __restrict__ w, uint32_t t, uint32_t k,
    uint32_t ne, const uint32_t* __restrict__ rank_of, const uint32_t* __restrict__ counts,
    tsg_token_expert_pair* __restrict__ sorted, uint32_t* __restrict__ offsets,
    tsg_routed_block* __restrict__ blocks, uint32_t max_blocks, uint32_t* __restrict__ n_blocks,
    uint32_t tile_rows) {
    __shared__ uint32_t off_s[kMaxExperts];
    __shared__ uint32_t blk_s[kMaxExperts];
    if (threadIdx.x == 0) {
        uint32_t run = 0, brun = 0;
        for (uint32_t e = 0; e < ne; ++e) {
            off_s[e] = run;
            blk_s[e] = brun;
            run += counts[e];
            brun += (counts[e] + tile_rows - 1) / tile_rows;
        }
        if (blockIdx.x == 0) *n_blocks = brun < max_blocks ? brun : max_blocks;
    }
    __syncthreads();
    if (blockIdx.x == 0) {
        for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) {
            const uint32_t c = counts[e];
            offsets[e] = c ? off_s[e] : 0xFFFFFFFFu;
            const uint32_t nb = (c + tile_rows - 1) / tile_rows;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint32_t bi = blk_s[e] + b;
                if (bi >= max_blocks) break;
                const uint32_t start = off_s[e] + b * tile_rows;
                const uint32_t rows = (c - b * tile_rows) < tile_rows ? (c - b * tile_rows) : tile_rows;
                blocks[bi] = tsg_routed_block{e, start, rows, start};
            }
        }
    }
    const uint64_t n = (uint64_t)t * k;
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < n;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t e = idx[p];
        if (e >= ne) continue;
        const uint32_t tok = (uint32_t)(p / k), r = (uint32_t)(p - (uint64_t)tok * k);
        sorted[off_s[e] + rank_of[p]] = tsg_token_expert_pair{tok, e, r, (uint32_t)w[p]};
    }
}

// ------------------------------------------------------- fp16 dequant

// Sixteen weights (two packed u32, elements 0..15 of a K run) -> eight fp16
// pairs in paired order per 8-element half: out[0..3] from w0, out[4..7] from
// w1. Each value is RNE(fma(q, s, b)) with b = -8 s under sym
// (prefill.metal:1021-1026). The fp16 FMA is exact-then-round-once, so when s
// and -8 s are exact in fp16 it reproduces half(fp32 fma) bit for bit; any
// other group (tiny scales, and every affine group, whose bias would be
// rounded twice) takes the fp32 route.
template <bool SYM>
__device__ __forceinline__ void dequant16_f16(uint32_t w0, uint32_t w1, float s, float b,
                                              h2_t out[8]) {
    const h2_t k1024 = h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
    h2_t q[8];
    nib8_to_pairs(w0, k1024, q);
    nib8_to_pairs(w1, k1024, q + 4);
    bool fast = false;
    _Float16 sh = (_Float16)s, bh = (_Float16)b;
    if constexpr (SYM) fast = ((float)sh == s) && ((float)bh == b);
    if (fast) {
        const h2_t s2 = h2_t{sh, sh}, b2 = h2_t{bh, bh};
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = __builtin_elementwise_fma(q[i], s2, b2);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float lo = __builtin_fmaf((float)q[i].x, s, b);
            const float hi = __builtin_fmaf((float)q[i].y, s, b);
            out[i] = h2_t{(_Float16)lo, (_Float16)hi};
        }
    }
}

// Un-paired debug dump of the same staging (tsg_debug_dequant_f16's twin for
// the GEMM path): out[k] for the 16 weights of (w0, w1).
template <int G, bool SYM>
__global__ void gemm_dequant_probe_kernel(const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ scales,
                                          const uint16_t* __restrict__ biases,
                                          uint16_t* __restrict__ out, uint32_t rows,
                                          uint32_t n) {
    const uint64_t pieces = (uint64_t)rows * (n / 16u);
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < pieces;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = p / (n / 16u);
        const uint32_t k0 = (uint32_t)(p - r * (n / 16u)) * 16u;
        const uint2 v = *reinterpret_cast<const uint2*>(w + r * (n / 2u) + k0 / 2u);
        const uint32_t g = k0 / G;
        const float s = bf16_to_f32(scales[r * (n / G) + g]);
        const float b = SYM ? -8.0f * s : bf16_to_f32(biases[r * (n / G) + g]);
        h2_t o[8];
        dequant16_f16<SYM>(v.x, v.y, s, b, o);
        for (int half = 0; half < 2; ++half)
            for (int kk = 0; kk < 8; ++kk) {
                const h2_t pr = o[half * 4 + (kk & 3)];
                const _Float16 val = (kk >> 2) ? pr.y : pr.x;
                out[r * n + k0 + half * 8 + kk] = __builtin_bit_cast(uint16_t, val);
            }
    }
}

// --------------------------------------------------------------- GEMM

constexpr uint32_t kTM = 64;    // rows per routed block
constexpr uint32_t kTN = 128;   // weight rows per block
constexpr uint32_t kTK = 32;    // K per step
constexpr uint32_t kLdsStride = kTK + 8;  // halves; pads rows off the same banks

typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ h8v_t lds_h8(const uint16_t* p) {
    return __builtin_bit_cast(h8v_t, *reinterpret_cast<const uint4*>(p));
}

struct GemmArgs {
    const uint8_t* layer_base;
    uint64_t expert_stride;
    tsg_expert_offsets o;
    const uint16_t* a;          // hidden (gate/up) or act (down)
    uint32_t a_stride;          // elements
    const tsg_token_expert_pair* pairs;
    const tsg_routed_block* blocks;
    uint32_t n_blocks;
    const uint32_t* n_blocks_device;
    uint16_t* out;              // act (gate/up) or route partials (down)
    uint32_t d, f, top_k;
};

// MODE 0: gate/up + activation; MODE 1: down + scatter.
template <int G, bool SYM, int ACT, int MODE>
__global__ __launch_bounds__(256) void moe_gemm_kernel(GemmArgs args) {
    __shared__ __align__(16) uint16_t As[kTM * kLdsStride];
    __shared__ __align__(16) uint16_t Bs[kTN * kLdsStride];
    __shared__ uint32_t row_src[kTM];
    __shared__ uint32_t row_dst[kTM];

    const uint32_t nb = args.n_blocks_device ? *args.n_blocks_device : args.n_blocks;
    if (blockIdx.y >= nb) return;
    const tsg_routed_block blk = args.blocks[blockIdx.y];
    const uint32_t tid = threadIdx.x;
    const uint32_t K = MODE == 0 ? args.d : args.f;       // reduction length
    const uint32_t N = MODE == 0 ? args.f : args.d;       // output columns
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;

    if (tid < kTM) {
        uint32_t src = 0, dst = 0;
        if (tid < blk.row_count) {
            const tsg_token_expert_pair pr = args.pairs[blk.pair_start + tid];
            if (MODE == 0) {
                src = pr.token * args.a_stride;
                dst = (blk.local_row + tid) * args.f;
            } else {
                src = (blk.local_row + tid) * args.a_stride;
                dst = (pr.token * args.top_k + pr.rank) * args.d;
            }
        }
        row_src[tid] = src;
        row_dst[tid] = dst;
    }

    // Weight rows this thread dequantises: 128 rows x 2 halves of 16 weights.
    const uint32_t wrow = tid >> 1, whalf = tid & 1u;
    uint32_t n_w;
    const uint8_t* wbase;
    const uint16_t* sbase;
    const uint16_t* bbase;
    if (MODE == 0) {
        const bool up = wrow >= 64u;
        n_w = blockIdx.x * 64u + (wrow & 63u);
        wbase = blob + (up ? args.o.up_w : args.o.gate_w);
        sbase = reinterpret_cast<const uint16_t*>(blob + (up ? args.o.up_s : args.o.gate_s));
        bbase = reinterpret_cast<const uint16_t*>(blob + (up ? args.o.up_b : args.o.gate_b));
    } else {
        n_w = blockIdx.x * kTN + wrow;
        wbase = blob + args.o.down_w;
        sbase = reinterpret_cast<const uint16_t*>(blob + args.o.down_s);
        bbase = reinterpret_cast<const uint16_t*>(blob + args.o.down_b);
    }
    const bool w_live = n_w < N;
    const uint32_t ngroups = K / G;
    const uint8_t* wrow_p = wbase + (uint64_t)(w_live ? n_w : 0u) * (K / 2u);
    const uint16_t* srow_p = sbase + (uint64_t)(w_live ? n_w : 0u) * ngroups;
    const uint16_t* brow_p = bbase + (uint64_t)(w_live ? n_w : 0u) * ngroups;

    // Activation piece this thread gathers: row tid/4, 8 halves at (tid%4)*8.
    const uint32_t arow = tid >> 2, apiece = tid & 3u;
    __syncthreads();
    const bool a_live = arow < blk.row_count;
    const uint16_t* a_p = args.a + row_src[arow] + apiece * 8u;

    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    f16v_t acc0 = {}, acc1 = {};
    // B rows for this wave's two 32-column accumulators.
    const uint32_t b0 = MODE == 0 ? wn * 32u : wn * 64u;
    const uint32_t b1 = MODE == 0 ? 64u + wn * 32u : wn * 64u + 32u;

    for (uint32_t k0 = 0; k0 < K; k0 += kTK) {
        uint4 av = make_uint4(0, 0, 0, 0);
        if (a_live) av = *reinterpret_cast<const uint4*>(a_p + k0);
        uint2 wv = make_uint2(0, 0);
        uint16_t sv = 0, bv = 0;
        const uint32_t kk = k0 + whalf * 16u;
        if (w_live) {
            wv = *reinterpret_cast<const uint2*>(wrow_p + kk / 2u);
            sv = srow_p[kk / G];
            if constexpr (!SYM) bv = brow_p[kk / G];
        }
        *reinterpret_cast<uint4*>(&As[arow * kLdsStride + apiece * 8u]) = pair_permute(av);
        {
            const float s = bf16_to_f32(sv);
            const float b = SYM ? -8.0f * s : bf16_to_f32(bv);
            h2_t o[8];
            dequant16_f16<SYM>(wv.x, wv.y, s, b, o);
            uint16_t* dst = &Bs[wrow * kLdsStride + whalf * 16u];
            *reinterpret_cast<uint4*>(dst) = __builtin_bit_cast(uint4, (h8v_t){o[0].x, o[0].y, o[1].x, o[1].y, o[2].x, o[2].y, o[3].x, o[3].y});
            *reinterpret_cast<uint4*>(dst + 8) = __builtin_bit_cast(uint4, (h8v_t){o[4].x, o[4].y, o[5].x, o[5].y, o[6].x, o[6].y, o[7].x, o[7].y});
        }
        __syncthreads();
#pragma unroll
        for (uint32_t ks = 0; ks < kTK; ks += 16u) {
            const uint32_t kof = ks + 8u * (lane >> 5);
            const h8v_t a = lds_h8(&As[(wm * 32u + (lane & 31u)) * kLdsStride + kof]);
            const h8v_t bb0 = lds_h8(&Bs[(b0 + (lane & 31u)) * kLdsStride + kof]);
            const h8v_t bb1 = lds_h8(&Bs[(b1 + (lane & 31u)) * kLdsStride + kof]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bb0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bb1, acc1, 0, 0, 0);
        }
        __syncthreads();
    }

    // acc[v] of lane l holds row 8*(v/4) + 4*(l/32) + v%4, column l%32.
    const uint32_t col = lane & 31u;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const uint32_t m = wm * 32u + 8u * (v >> 2) + 4u * (lane >> 5) + (v & 3);
        if (m >= blk.row_count) continue;
        if (MODE == 0) {
            const uint32_t fcol = blockIdx.x * 64u + wn * 32u + col;
            if (fcol >= args.f) continue;
            const float g = f16_to_f32(f32_to_f16(acc0[v]));
            const float u = f16_to_f32(f32_to_f16(acc1[v]));
            args.out[row_dst[m] + fcol] = f32_to_f16(gate_activation<ACT>(g) * u);
        } else {
            const uint32_t dcol0 = blockIdx.x * kTN + wn * 64u + col;
            if (dcol0 < args.d) args.out[row_dst[m] + dcol0] = f32_to_f16(acc0[v]);
            if (dcol0 + 32u < args.d) args.out[row_dst[m] + dcol0 + 32u] = f32_to_f16(acc1[v]);
        }
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

// --------------------------------------------------------- rows path

constexpr uint32_t kRowsMax = 8;
constexpr uint32_t kRowsBlocksPerLaunch = 64;

// The rows path's block list travels in the kernel arguments, as the
// reference passes it with setBytes (PrefillGroupedRoutedMoE.swift:835-870).
struct RowsBlocks {
    tsg_routed_block b[kRowsBlocksPerLaunch];
};

// grid (ceil(F / 8), n_blocks), block 256: 32 lanes per f row (16 on the gate
// row, 16 on the up row), every row of the routed block (<= 8) against one
// weight read. Per row the arithmetic is decode phase 1's (decode.hip
// phase1_compute): the same gemv_lane.hpp steps, batch and reduction, so one
// row here is bit-identical to decode.
template <int G, bool SYM, int ACT>
__global__ __launch_bounds__(256) void rows_gate_up_kernel(GemmArgs args, RowsBlocks rb) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t tok[kRowsMax];
    const tsg_routed_block blk = rb.b[blockIdx.y];
    const uint32_t rows = blk.row_count < kRowsMax ? blk.row_count : kRowsMax;
    const uint32_t d = args.d, f = args.f;
    const uint32_t row_h = lds_chunks_halves(d);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + (size_t)kRowsMax * row_h * 2u);

    const uint32_t fr_raw = blockIdx.x * 8u + (threadIdx.x >> 5);
    const uint32_t j = threadIdx.x & 15u;
    const bool is_up = (threadIdx.x >> 4) & 1u;
    const bool live = fr_raw < f;
    const uint32_t fr = live ? fr_raw : 0u;
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    const uint32_t ngroups = d / G, nchunks = d / 32u;
    const uint8_t* w = blob + (is_up ? args.o.up_w : args.o.gate_w) + (uint64_t)fr * (d / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + (is_up ? args.o.up_s : args.o.gate_s)) + (uint64_t)fr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + (is_up ? args.o.up_b : args.o.gate_b)) + (uint64_t)fr * ngroups;
    ChunkBatch<kGUBatch> bt;
    load_batch<G, SYM, kGUBatch, kGULanes>(w, sc, bi, 0u, j, nchunks, bt);
    if (threadIdx.x < rows) tok[threadIdx.x] = args.pairs[blk.pair_start + threadIdx.x].token;
    __syncthreads();
    stage_act_rows<SYM>(args.a, args.a_stride, rows, d, xs, row_h, xsum, tok);
    __syncthreads();
    float acc[kRowsMax];
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) acc[r] = 0.0f;
    for (uint32_t base = 0; base < nchunks; base += kGULanes * kGUBatch) {
        if (base) load_batch<G, SYM, kGUBatch, kGULanes>(w, sc, bi, base, j, nchunks, bt);
        compute_batch<G, SYM, kGUBatch, kGULanes, kRowsMax>(bt, base, j, nchunks, xs, row_h, xsum,
                                                            rows, acc);
    }
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) {
        acc[r] = group16_sum(acc[r]);
        const float up = shfl_xor(acc[r], 16);
        if (live && !is_up && j == 0 && r < rows)
            args.out[(uint64_t)(blk.local_row + r) * f + fr] =
                f32_to_f16(gate_activation<ACT>(acc[r]) * up);
    }
}

// grid (ceil(D / 8), n_blocks), block 64: 8 lanes per output row, each of the
// block's rows against one weight read. Per row the arithmetic is decode phase
// 2's per-slot GEMV (decode.hip phase2_body): the same gemv_lane.hpp steps.
template <int G, bool SYM>
__global__ __launch_bounds__(64) void rows_down_kernel(GemmArgs args, RowsBlocks rb,
                                                       uint16_t* partials) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t dst[kRowsMax];
    const tsg_routed_block blk = rb.b[blockIdx.y];
    const uint32_t rows = blk.row_count < kRowsMax ? blk.row_count : kRowsMax;
    const uint32_t d = args.d, f = args.f;
    const uint32_t row_h = lds_chunks_halves(f);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);
    float* asum = reinterpret_cast<float*>(smem + (size_t)kRowsMax * row_h * 2u);

    const uint32_t j = threadIdx.x & 7u;
    const uint32_t row = blockIdx.x * 8u + (threadIdx.x >> 3);
    const bool live_row = row < d;
    const uint32_t rr = live_row ? row : 0u;
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    const uint32_t ngroups = f / G, nchunks = f / 32u;
    const uint8_t* w = blob + args.o.down_w + (uint64_t)rr * (f / 2u);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(blob + args.o.down_s) + (uint64_t)rr * ngroups;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(blob + args.o.down_b) + (uint64_t)rr * ngroups;
    ChunkBatch<kDBatch> bt;
    load_batch<G, SYM, kDBatch, kDLanes>(w, sc, bi, 0u, j, nchunks, bt);
    if (threadIdx.x < rows) {
        const tsg_token_expert_pair pr = args.pairs[blk.pair_start + threadIdx.x];
        dst[threadIdx.x] = (pr.token * args.top_k + pr.rank) * d;
    }
    stage_act_rows<SYM>(args.a + (uint64_t)blk.local_row * f, f, rows, f, as, row_h, asum);
    __syncthreads();
    float acc[kRowsMax];
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) acc[r] = 0.0f;
    for (uint32_t base = 0; base < nchunks; base += kDLanes * kDBatch) {
        if (base) load_batch<G, SYM, kDBatch, kDLanes>(w, sc, bi, base, j, nchunks, bt);
        compute_batch<G, SYM, kDBatch, kDLanes, kRowsMax>(bt, base, j, nchunks, as, row_h, asum,
                                                          rows, acc);
    }
#pragma unroll
    for (uint32_t r = 0; r < kRowsMax; ++r) {
        acc[r] = group8_sum(acc[r]);
    }
    if (live_row && j == 0)
        for (uint32_t r = 0; r < rows; ++r) partials[dst[r] + row] = f32_to_f16(acc[r]);
}

// ------------------------------------------------------------ host side

tsg_status check_layer_moe(const tsg_moe* moe, const tsg_layer* layer) {
    TSG_REQUIRE(moe && moe->ctx, TSG_ERR_INVALID_ARGUMENT, "moe is NULL");
    TSG_REQUIRE(layer, TSG_ERR_INVALID_ARGUMENT, "layer is NULL");
    return TSG_OK;
}

template <int G, bool SYM, int MODE>
tsg_status launch_gemm(const tsg_moe* moe, hipStream_t s, const GemmArgs& a, uint32_t max_blocks) {
    const uint32_t ntiles = MODE == 0 ? (a.f + 63u) / 64u : (a.d + kTN - 1u) / kTN;
    const dim3 grid(ntiles, max_blocks);
    if (moe->activation == TSG_ACT_SILU)
        hipLaunchKernelGGL((moe_gemm_kernel<G, SYM, TSG_ACT_SILU, MODE>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((moe_gemm_kernel<G, SYM, TSG_ACT_GELU_TANH, MODE>), grid, dim3(256), 0, s, a);
    return check_launch(MODE == 0 ? "moe_gemm gate/up" : "moe_gemm down");
}

template <int MODE>
tsg_status gemm_dispatch(const tsg_moe* moe, hipStream_t s, const GemmArgs& a, uint32_t max_blocks) {
    const tsg_ctx* ctx = moe->ctx;
    const bool sym = ctx->scheme == TSG_SYM;
    if (ctx->group_size == 32)
        return sym ? launch_gemm<32, true, MODE>(moe, s, a, max_blocks)
                   : launch_gemm<32, false, MODE>(moe, s, a, max_blocks);
    return sym ? launch_gemm<64, true, MODE>(moe, s, a, max_blocks)
               : launch_gemm<64, false, MODE>(moe, s, a, max_blocks);
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
    TSG_REQUIRE(aligned16(act_in) && a_stride % 8 == 0, TSG_ERR_ALIGNMENT,
                "activation rows must be 16-byte aligned");
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
    return TSG_OK;
}

}  // namespace
}  // namespace tsg

using namespace tsg;

extern "C" size_t tsg_prefill_group_scratch_bytes(uint32_t query_count, uint32_t top_k,
                                                  uint32_t) {
    return (size_t)query_count * top_k * sizeof(uint32_t);
}

extern "C" tsg_status tsg_prefill_group_pairs_device(
    tsg_ctx* ctx, tsg_stream stream, const uint32_t* idx, const uint16_t* w, uint32_t t,
    uint32_t k, uint32_t ne, uint32_t tile_rows, tsg_token_expert_pair* sorted,
    uint32_t* offsets, uint32_t* counts, tsg_routed_block* blocks, uint32_t max_blocks,
    uint32_t* n_blocks, void* scratch) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(t > 0, TSG_ERR_GROUPING_INVALID_QUERY_COUNT, "queryCount must be positive");
    TSG_REQUIRE(k > 0, TSG_ERR_GROUPING_INVALID_TOP_K, "topK must be positive");
    TSG_REQUIRE(ne > 0 && ne <= kMaxExperts, TSG_ERR_GROUPING_INVALID_NUM_EXPERTS,
                "numExperts %u not in 1..%u", ne, kMaxExperts);
    TSG_REQUIRE(tile_rows == 32 || tile_rows == 64, TSG_ERR_INVALID_ARGUMENT,
                "tile_rows must be 32 or 64, got %u", tile_rows);
    TSG_REQUIRE(idx && w && sorted && offsets && counts && blocks && n_blocks && scratch,
                TSG_ERR_INVALID_ARGUMENT, "NULL grouping operand");
    hipStream_t s = as_stream(stream);
    uint32_t* rank_of = static_cast<uint32_t*>(scratch);
    hipLaunchKernelGGL(group_rank_kernel, dim3(ne), dim3(1024), 0, s, idx, t, k, rank_of, counts);
    tsg_status st = check_launch("group_rank");
    if (st) return st;
    const uint64_t n = (uint64_t)t * k;
    uint64_t grid = (n + 255) / 256;
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(group_scatter_kernel, dim3(grid), dim3(256), 0, s, idx, w, t, k, ne,
                       rank_of, counts, sorted, offsets, blocks, max_blocks, n_blocks, tile_rows);
    return check_launch("group_scatter");
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
                                           uint16_t* act_scratch, uint16_t* partials,
                                           uint32_t top_k, uint32_t d, uint32_t f) {
    tsg_status st = check_layer_moe(moe, layer);
    if (st) return st;
    if (n_blocks == 0) return TSG_OK;
    TSG_REQUIRE(blocks, TSG_ERR_INVALID_ARGUMENT, "blocks is NULL");
    // The host chooses the rows path from the grouping and it declines blocks
    // wider than its cap (PrefillGroupedRoutedMoE.swift:808-830).
    for (uint32_t i = 0; i < n_blocks; ++i)
        if (blocks[i].row_count == 0 || blocks[i].row_count > kRowsMax)
            return fail(TSG_ERR_DECLINED, "rows path takes 1..%u rows per block, block %u has %u",
                        kRowsMax, i, blocks[i].row_count);
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
        for (uint32_t i = 0; i < nb; ++i) rb.b[i] = blocks[b0 + i];
        const dim3 g1((f + 7) / 8, nb), g2((d + 7) / 8, nb);
#define TSG_ROWS_LAUNCH(GG, SS)                                                                  \
    do {                                                                                         \
        if (moe->activation == TSG_ACT_SILU)                                                     \
            hipLaunchKernelGGL((rows_gate_up_kernel<GG, SS, TSG_ACT_SILU>), g1, dim3(256), lds1, \
                               s, a, rb);                                                        \
        else                                                                                     \
            hipLaunchKernelGGL((rows_gate_up_kernel<GG, SS, TSG_ACT_GELU_TANH>), g1, dim3(256),  \
                               lds1, s, a, rb);                                                  \
        if ((st = check_launch("rows gate/up"))) return st;                                     \
        hipLaunchKernelGGL((rows_down_kernel<GG, SS>), g2, dim3(64), lds2, s, a2, rb, partials); \
        if ((st = check_launch("rows down"))) return st;                                        \
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
    uint64_t grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(reduce_token_major_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                       partials, w, h2, t, k, d);
    return check_launch("reduce_token_major");
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
    TSG_REQUIRE(reinterpret_cast<uintptr_t>(w) % 8 == 0, TSG_ERR_ALIGNMENT,
                "weights must be 8-byte aligned");
    const uint64_t pieces = (uint64_t)rows * (n / 16u);
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
