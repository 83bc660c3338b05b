// prefill.hip — prompt-chunk routed MoE for gfx950.
//
//   device grouping   PrefillMoEGrouping.swift:90-202 (stable counting sort)
//   grouped GEMMs     prefill.metal:913-1092, 3664-3864 (encodeStreamedTiled)
//   token-major sum   prefill.metal:796-817
//   verify rows path  prefill.metal:1489-1721 (encodeStreamedRows)
//
// GEMM design (moe_gemm_kernel below): a work item is one routed block of up
// to 128 rows of one expert x one column tile of the weights (128 gate+up
// rows, or 256 down rows). Four waves each own two 32-row weight tiles and
// dequantise them in registers, RNE_f16(fma(q, s, b)) exactly as the
// reference stages them, against every live 32-row slice of the block's
// activation rows held in LDS; v_mfma_f32_32x32x16_f16 accumulates in fp32.
// Operands arrive by direct global->LDS loads in a 3-stage ring. Gate and up
// rows of the same f share a wave, so the GeGLU/SiLU epilogue runs in
// registers; the output tile leaves through LDS as 16-byte stores.
#include "gemv_lane.hpp"

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

// ------------------------------------------------------- fp16 dequant

typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));

// Per (weight row, group) dequantisation parameters. Every weight is staged
// as RNE_f16(fmaf(q, s, b)) with b = -8 s under sym (prefill.metal:1021-1026):
// fmaf rounds q * s + b to fp32, the conversion rounds that to fp16. The
// nibble q is isolated inside a 16-bit half, where as an fp16 bit pattern it
// is the subnormal q * 2^-24 (bits 0..3) or q * 2^-20 (bits 4..7); the scale
// is pre-multiplied by 2^24 or 2^20, so v_fma_mix forms the exact product
// q * s (for |s| < 2^103, where s * 2^24 stays finite), with no per-group test.
//  - sym: q * s - 8 s = (q - 8) * s has at most 12 significant bits, exact in
//    fp32, so v_fma_mix{lo,hi}_f16, which round the exact sum once to fp16,
//    give the reference's bits.
//  - affine: q * s + b can need more than 24 bits (b far smaller or larger
//    than s), and rounding it to fp32 first can land on an fp16 tie that a
//    single rounding would not; the sum is therefore taken to fp32 with
//    v_fma_mix_f32 and converted with its own instruction.
struct GroupScale {
    float s_lo, s_hi, b;  // s * 2^24, s * 2^20, b
};

template <bool SYM>
__device__ __forceinline__ GroupScale group_scale(uint16_t s_bits, uint16_t b_bits) {
    const float s = bf16_to_f32(s_bits);
    GroupScale g;
    g.s_lo = s * 16777216.0f;
    g.s_hi = s * 1048576.0f;
    g.b = SYM ? -8.0f * s : bf16_to_f32(b_bits);
    return g;
}

// Eight weights (one packed u32, elements 0..7 of a K run), in element order.
// Two ANDs of the word and two of the word shifted right by 8 leave every
// nibble alone in a 16-bit half, at bits 0..3 (elements 0, 2 | 4, 6: the low
// nibbles of bytes 0, 1 | 2, 3) or 4..7 (elements 1, 3 | 5, 7); one v_fma_mix
// per element reads its half. 13 VALU per 8 weights under sym (the pair
// packing folds into v_fma_mix{lo,hi}_f16), 17 under affine (fp32 sums, one
// v_cvt_pk_f16_f32 per pair). Split into the extraction and four pairs so the
// GEMM can spread the work between its MFMAs.
struct Nibbles {
    h2_t n0, n1, n2, n3;  // e0|e4, e1|e5, e2|e6, e3|e7
};

__device__ __forceinline__ Nibbles nibbles8(uint32_t w) {
    const uint32_t w8 = w >> 8;
    return Nibbles{__builtin_bit_cast(h2_t, w & 0x000F000Fu), __builtin_bit_cast(h2_t, w & 0x00F000F0u),
                   __builtin_bit_cast(h2_t, w8 & 0x000F000Fu), __builtin_bit_cast(h2_t, w8 & 0x00F000F0u)};
}

// Pair j (elements 2j, 2j+1) of the eight.
template <bool SYM, int J>
__device__ __forceinline__ h2_t dequant_pair(const Nibbles& n, const GroupScale& g) {
    const _Float16 lo_src = J == 0 ? n.n0.x : J == 1 ? n.n2.x : J == 2 ? n.n0.y : n.n2.y;
    const _Float16 hi_src = J == 0 ? n.n1.x : J == 1 ? n.n3.x : J == 2 ? n.n1.y : n.n3.y;
    if constexpr (SYM) {
        // the empty asm makes the low half a value of its own, so the pair
        // becomes v_fma_mixlo_f16 + v_fma_mixhi_f16 rather than two
        // v_fma_mix_f32 and a v_cvt_pk_f16_f32
        _Float16 lo = (_Float16)__builtin_fmaf((float)lo_src, g.s_lo, g.b);
        asm("" : "+v"(lo));
        return h2_t{lo, (_Float16)__builtin_fmaf((float)hi_src, g.s_hi, g.b)};
    } else {
        float lo = __builtin_fmaf((float)lo_src, g.s_lo, g.b);
        float hi = __builtin_fmaf((float)hi_src, g.s_hi, g.b);
        asm("" : "+v"(lo), "+v"(hi));
        return h2_t{(_Float16)lo, (_Float16)hi};
    }
}

__device__ __forceinline__ h8v_t pack_pairs(h2_t p0, h2_t p1, h2_t p2, h2_t p3) {
    return h8v_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

template <bool SYM>
__device__ __forceinline__ h8v_t dequant8(uint32_t w, const GroupScale& g) {
    const Nibbles n = nibbles8(w);
    return pack_pairs(dequant_pair<SYM, 0>(n, g), dequant_pair<SYM, 1>(n, g),
                      dequant_pair<SYM, 2>(n, g), dequant_pair<SYM, 3>(n, g));
}

// Dump of the GEMM's staging (tsg_debug_gemm_dequant_f16): one thread per 8
// weights. The eight values leave as one 16-byte vector: extracting them one
// by one into 16-bit stores made this hipcc fold all eight to the first.
template <int G, bool SYM>
__global__ void gemm_dequant_probe_kernel(const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ scales,
                                          const uint16_t* __restrict__ biases,
                                          uint16_t* __restrict__ out, uint32_t rows,
                                          uint32_t n) {
    const uint64_t pieces = (uint64_t)rows * (n / 8u);
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < pieces;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = p / (n / 8u);
        const uint32_t k0 = (uint32_t)(p - r * (n / 8u)) * 8u;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(w + r * (n / 2u) + k0 / 2u);
        const uint32_t g = k0 / G;
        const GroupScale gs = group_scale<SYM>(scales[r * (n / G) + g],
                                               SYM ? (uint16_t)0 : biases[r * (n / G) + g]);
        *reinterpret_cast<uint4*>(out + r * n + k0) = __builtin_bit_cast(uint4, dequant8<SYM>(v, gs));
    }
}

// --------------------------------------------------------------- GEMM

// Grouped int4 GEMM over routed blocks of up to kGemmRows rows of one expert.
// Block = 4 waves, two blocks per CU; each wave owns 64 weight rows as two
// 32-row MFMA tiles (gate/up: 32 gate + the same 32 up rows, so the GeGLU
// epilogue finds both in one lane; down: 64 output rows) against every live
// 32-row slice of the block's activation rows (NT = 1..4, a template
// parameter, so the inner loop has no per-slice tests). Each activation
// fragment read from LDS feeds two MFMAs, which keeps LDS read traffic near
// half its bandwidth at full MFMA rate. K runs in 64-element chunks. Operands
// arrive by direct global->LDS loads laid out so that each 64-lane load
// touches as few cache sectors as its data allows: the vector L1's access
// rate, not bandwidth, bounds scattered loads.
//  - activations, shared by the block: a 3-stage ring; row r's 16-byte piece
//    p sits in slot p ^ swz(r), swz(r) = (r & 7) ^ ((r >> 3) & 1); waves
//    w < NT load rows [32w, 32w + 32).
//  - weights, per (wave, tile): a 3-stage ring of 32 rows x 32 bytes (one
//    chunk), two lanes per row; row r's half h sits in slot h ^ swzb(r),
//    swzb(r) = ((r >> 2) ^ (r >> 3)) & 1.
//  - group scales (and affine biases), per wave: windows of 8 groups (16
//    bytes of each of its 64 rows; 7 groups when rows are only 2-byte
//    aligned, G = 64), double-buffered, loaded once per window, four lanes
//    per row.
// The swizzles keep the MFMA-side LDS reads conflict-free whether the LDS
// serves 8 lanes of a 16-byte read per cycle over 32 banks or 16 over 64.
// Word s of a lane's 16 weight bytes is dequantised into the B operand of
// MFMA step s, whose logical K 8h..8h+7 is physical 64c + 32h + 8s + (0..7);
// the activations are read with the same mapping. Step s + 1's activation
// reads and dequantisation are issued ahead of step s's MFMAs.
constexpr uint32_t kGemmRows = 128;
constexpr uint32_t kGemmWaves = 4;
constexpr uint32_t kGemmThreads = kGemmWaves * 64u;
constexpr uint32_t kGemmKC = 64;
constexpr uint32_t kGemmStages = 3;
constexpr uint32_t kGemmAStage = kGemmRows * kGemmKC * 2u;            // 16 KiB
constexpr uint32_t kGemmBTile = 32u * kGemmKC / 2u;                   // 1 KiB
constexpr uint32_t kGemmBWave = 2u * kGemmBTile;
constexpr uint32_t kGemmBStage = kGemmWaves * kGemmBWave;             // 8 KiB
constexpr uint32_t kGemmSWave = 64u * 16u;                            // 1 KiB
constexpr uint32_t kGemmSSlot = kGemmWaves * kGemmSWave;              // 4 KiB
constexpr uint32_t kGemmBBase = kGemmStages * kGemmAStage;            // 48 KiB
constexpr uint32_t kGemmSBase = kGemmBBase + kGemmStages * kGemmBStage;
constexpr uint32_t kGemmZBase = kGemmSBase + 2u * kGemmSSlot;
// sym: 80 KiB (two blocks per CU), affine: 88 KiB (one)
__host__ __device__ constexpr uint32_t gemm_lds_bytes(bool sym) {
    return kGemmZBase + (sym ? 0u : 2u * kGemmSSlot);
}
static_assert(gemm_lds_bytes(true) * 2u <= 160u * 1024u, "two sym blocks per CU");

// Chunks per scale window: 8 groups of 32 (two per chunk), or 7 of 64.
template <int G>
__host__ __device__ constexpr uint32_t gemm_window() { return G == 32 ? 4u : 7u; }

// LDS reads as inline ds_read: the compiler cannot tell them from the
// direct-to-LDS writes of other stages and would drain every outstanding load
// before each one. lds_wait() waits for them; its operands tie the results to
// the wait so no use (or copy) is scheduled before it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
template <uint32_t OFF>
__device__ __forceinline__ u32x4_t lds_read16(uint32_t addr) {
    static_assert(OFF < 65536u, "ds offset is 16 bits");
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
template <int NT>
__device__ __forceinline__ void lds_wait(u32x4_t (&a)[NT]) {
    if constexpr (NT == 1) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]));
    if constexpr (NT == 2) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]));
    if constexpr (NT == 3)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]));
    if constexpr (NT == 4)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]));
    if constexpr (NT == 5)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]));
    if constexpr (NT == 6)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]));
    if constexpr (NT == 7)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                       "+v"(a[6]));
    if constexpr (NT == 8)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                       "+v"(a[6]), "+v"(a[7]));
}
template <int NT>
__device__ __forceinline__ void lds_wait(u32x4_t (&a)[NT], u32x4_t& b0, u32x4_t& b1, uint32_t& s0,
                                         uint32_t& s1, uint32_t& z0, uint32_t& z1) {
    asm volatile("" : "+v"(b0), "+v"(b1), "+v"(s0), "+v"(s1), "+v"(z0), "+v"(z1));
    lds_wait<NT>(a);
    asm volatile("" : "+v"(b0), "+v"(b1), "+v"(s0), "+v"(s1), "+v"(z0), "+v"(z1));
}
template <int NT, uint32_t BASE>
__device__ __forceinline__ void lds_read_slices(u32x4_t (&a)[NT], uint32_t addr) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        switch (i) {
            case 0: a[i] = lds_read16<BASE + 0u * 4096u>(addr); break;
            case 1: a[i] = lds_read16<BASE + 1u * 4096u>(addr); break;
            case 2: a[i] = lds_read16<BASE + 2u * 4096u>(addr); break;
            default: a[i] = lds_read16<BASE + 3u * 4096u>(addr); break;
        }
    }
}

// Wait until at most N of this wave's vector memory loads are outstanding
// (loads complete in issue order); also a compiler barrier.
template <uint32_t N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the memory fence of __syncthreads(), whose release
// would wait for every outstanding load (the prefetches included). The
// explicit vmcnt waits order the direct-to-LDS data; the asm statements keep
// the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void lds_dma16(const void* src, uint8_t* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds_wave_base,
                                     16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* src, uint8_t* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds_wave_base,
                                     4, 0, 0);
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
    uint16_t* out;              // act (gate/up), route partials (down) or y (dense)
    uint32_t d, f, top_k;
    uint32_t dense_rows;        // MODE 2: rows of x and y
    const uint8_t* dense_s;     // MODE 2: scales (the weights are at layer_base)
    const uint8_t* dense_b;     // MODE 2: biases (the scales again under sym)
    uint32_t ntiles;            // weight-row tiles per routed block
    uint32_t dense_narrow;      // MODE 2: 128-column tiles, one 32-row weight tile per wave
    uint32_t num_experts;       // experts of the layer (device block lists are checked)
    uint32_t max_rows;          // rows path, device list: rows of the activation scratch
    uint32_t* error;            // the context's device error word
};

// Per-lane state of one block's GEMM.
struct GemmLane {
    const uint8_t* blob;
    const uint8_t* sblob;       // base of the scale offsets (the blob, or dense scales)
    const uint8_t* zblob;       // base of the bias offsets
    const uint16_t* a_src[4];   // the lane's activation piece for DMA j (chunk 0)
    const uint8_t* w_src[2];    // the lane's weight piece per tile (chunk 0)
    uint32_t s_ld[4], z_ld[4];  // scale / bias row starts of the rows this lane loads
    uint32_t s_own[2], z_own[2];  // scale / bias row starts of the lane's own rows (m, tile)
    uint32_t s_last, z_last;    // last dword of the scale / bias sub-tensors
    uint32_t a_rd[4];           // LDS activation read address per MFMA step (stage 0, slice 0)
    uint32_t b_rd;              // LDS weight read address (stage 0)
    uint32_t s_rd;              // LDS scale read address of row m (slot 0)
    uint32_t wave, nchunks, nwin;
    bool a_wave, live;
};

// Byte offset of the first group of scale window w within a row, and of the
// lane's group for chunk c (half h).
template <int G>
__device__ __forceinline__ uint32_t window_byte(uint32_t w) {
    return 2u * w * (G == 32 ? 8u : 7u);
}
template <int G>
__device__ __forceinline__ uint32_t group_byte(uint32_t c, uint32_t h) {
    return G == 32 ? 4u * c + 2u * h : 2u * c;
}

// Chunk c (clamped to the last one) into ring stage ST: activations (4 loads
// if the wave moves activation rows) and weights (2 loads).
template <int ST>
__device__ __forceinline__ void gemm_issue(const GemmLane& L, uint8_t* smem, uint32_t c) {
    const uint32_t cc = c < L.nchunks ? c : L.nchunks - 1u;
    if (L.a_wave) {
        uint8_t* dst = smem + ST * kGemmAStage + L.wave * 32u * kGemmKC * 2u;
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_dma16(L.a_src[j] + cc * kGemmKC, dst + j * 8u * kGemmKC * 2u);
    }
    uint8_t* bst = smem + kGemmBBase + ST * kGemmBStage + L.wave * kGemmBWave;
    lds_dma16(L.w_src[0] + cc * (kGemmKC / 2u), bst);
    lds_dma16(L.w_src[1] + cc * (kGemmKC / 2u), bst + kGemmBTile);
}

// Scale (and bias) window w (clamped) into slot w & 1: 4 loads (8 affine).
template <int G, bool SYM>
__device__ __forceinline__ void gemm_issue_scales(const GemmLane& L, uint8_t* smem, uint32_t w) {
    const uint32_t wc = w < L.nwin ? w : L.nwin - 1u;
    const uint32_t wb = window_byte<G>(wc);
    const uint32_t dw = 4u * (threadIdx.x & 3u);
    uint8_t* dst = smem + kGemmSBase + (w & 1u) * kGemmSSlot + L.wave * kGemmSWave;
    // a window may reach past its row; bytes past the sub-tensor are never
    // used, so those addresses are clamped to stay inside it
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t o = ((L.s_ld[j] + wb) & ~3u) + dw;
        lds_dma4(L.sblob + (o < L.s_last ? o : L.s_last), dst + j * 256u);
    }
    if constexpr (!SYM) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t o = ((L.z_ld[j] + wb) & ~3u) + dw;
            lds_dma4(L.zblob + (o < L.z_last ? o : L.z_last), dst + (kGemmZBase - kGemmSBase) + j * 256u);
        }
    }
}

// The MFMA work of one chunk (stage ST) for the wave's two weight tiles. The
// next step's dequantisation (10 pieces: two nibble extractions, eight
// pairs) is spread between this step's 2 NT MFMAs, and scheduling fences keep
// the order, so the wave issues its conversions while its own MFMAs run.
// HALF: the wave runs one tile (bw0, g0) into acc[.][0]: NT MFMAs and 5
// pieces per step.
template <bool SYM, int NT, int ST, bool HALF>
__device__ __forceinline__ void gemm_mma(const GemmLane& L, u32x4_t (&af)[2][NT], const u32x4_t& bw0,
                                         const u32x4_t& bw1, const GroupScale& g0,
                                         const GroupScale& g1, f16v_t (&acc)[NT][2]) {
    constexpr int kT = HALF ? 1 : 2;       // tiles per wave
    constexpr int kP = HALF ? 5 : 10;      // conversion pieces per step
    h8v_t bf[2][2];
    bf[0][0] = dequant8<SYM>(bw0[0], g0);
    if constexpr (!HALF) bf[0][1] = dequant8<SYM>(bw1[0], g1);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const int cur = st & 1, nxt = cur ^ 1;
        if (st < 3) lds_read_slices<NT, ST * kGemmAStage>(af[nxt], L.a_rd[st + 1]);
        Nibbles n0{}, n1{};
        h2_t p0[4], p1[4];
        // piece k of the next step's conversion (k < kP)
        auto piece = [&](int k) {
            if (st >= 3) return;
            if constexpr (HALF) {
                switch (k) {
                    case 0: n0 = nibbles8(bw0[st + 1]); break;
                    case 1: p0[0] = dequant_pair<SYM, 0>(n0, g0); break;
                    case 2: p0[1] = dequant_pair<SYM, 1>(n0, g0); break;
                    case 3: p0[2] = dequant_pair<SYM, 2>(n0, g0); break;
                    default: p0[3] = dequant_pair<SYM, 3>(n0, g0); break;
                }
                return;
            }
            switch (k) {
                case 0: n0 = nibbles8(bw0[st + 1]); break;
                case 1: n1 = nibbles8(bw1[st + 1]); break;
                case 2: p0[0] = dequant_pair<SYM, 0>(n0, g0); break;
                case 3: p1[0] = dequant_pair<SYM, 0>(n1, g1); break;
                case 4: p0[1] = dequant_pair<SYM, 1>(n0, g0); break;
                case 5: p1[1] = dequant_pair<SYM, 1>(n1, g1); break;
                case 6: p0[2] = dequant_pair<SYM, 2>(n0, g0); break;
                case 7: p1[2] = dequant_pair<SYM, 2>(n1, g1); break;
                case 8: p0[3] = dequant_pair<SYM, 3>(n0, g0); break;
                default: p1[3] = dequant_pair<SYM, 3>(n1, g1); break;
            }
        };
        constexpr int kM = kT * NT;  // MFMAs this step
#pragma unroll
        for (int q = 0; q < kM; ++q) {
            const int i = q / kT, t = q % kT;
            const h8v_t a8 = __builtin_bit_cast(h8v_t, af[cur][i]);
            acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, bf[cur][t], acc[i][t], 0, 0, 0);
#pragma unroll
            for (int k = q * kP / kM; k < (q + 1) * kP / kM; ++k) piece(k);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (st < 3) {
            bf[nxt][0] = pack_pairs(p0[0], p0[1], p0[2], p0[3]);
            if constexpr (!HALF) bf[nxt][1] = pack_pairs(p1[0], p1[1], p1[2], p1[3]);
            lds_wait<NT>(af[nxt]);
        }
    }
}

// One chunk: wait for it, start chunk c + 2 (into the stage chunk c - 1 used)
// and, at the first chunk of a scale window, the next window, then read its
// weights, scale and step-0 activations and run its MFMAs.
template <int G, bool SYM, int NT, int ST, bool HALF>
__device__ __forceinline__ void gemm_chunk(const GemmLane& L, uint8_t* smem, uint32_t c,
                                           f16v_t (&acc)[NT][2]) {
    constexpr uint32_t W = gemm_window<G>();
    constexpr uint32_t kNS = SYM ? 4u : 8u;
    // Loads allowed in flight: chunk c + 1's (4 activation + 2 weight), if
    // there is one, and the scale window started at chunk c - 1 or c - 2, if
    // any (nothing past the last chunk or window is requested).
    const bool next = c + 1u < L.nchunks;
    const bool s_recent = (c >= 1u && (c - 1u) % W == 0u && (c - 1u) / W + 1u < L.nwin) ||
                          (c >= 2u && (c - 2u) % W == 0u && (c - 2u) / W + 1u < L.nwin);
    if (next) {
        if (L.a_wave) {
            if (s_recent) wait_vmcnt<6u + kNS>();
            else wait_vmcnt<6u>();
        } else {
            if (s_recent) wait_vmcnt<2u + kNS>();
            else wait_vmcnt<2u>();
        }
    } else {
        if (s_recent) wait_vmcnt<kNS>();
        else wait_vmcnt<0u>();
    }
    block_barrier();
    // Chunk c - 1's stage and the scale window before this one are free now
    // (every wave has passed the barrier): start chunk c + 2 and, at a
    // window's first chunk, the next window before this chunk's MFMAs, so two
    // chunks are in flight while one is computed.
    if (c + 2u < L.nchunks) gemm_issue<(ST + 2) % 3>(L, smem, c + 2u);
    if (c % W == 0u && c / W + 1u < L.nwin) gemm_issue_scales<G, SYM>(L, smem, c / W + 1u);
    if (L.live) {
        const uint32_t win = c / W, lane = threadIdx.x & 63u, h = lane >> 5;
        const uint32_t wb = window_byte<G>(win), gb = group_byte<G>(c, h);
        const uint32_t slot = (win & 1u) * kGemmSSlot;
        u32x4_t af[2][NT];
        u32x4_t bw0 = lds_read16<ST * kGemmBStage>(L.b_rd);
        u32x4_t bw1 = HALF ? bw0 : lds_read16<ST * kGemmBStage + kGemmBTile>(L.b_rd);
        uint32_t sw0 = lds_read_u16(L.s_rd + slot + (L.s_own[0] + gb) - ((L.s_own[0] + wb) & ~3u));
        uint32_t sw1 = HALF ? sw0 : lds_read_u16(L.s_rd + 512u + slot + (L.s_own[1] + gb) - ((L.s_own[1] + wb) & ~3u));
        uint32_t zw0 = 0u, zw1 = 0u;
        if constexpr (!SYM) {
            constexpr uint32_t zo = kGemmZBase - kGemmSBase;
            zw0 = lds_read_u16(L.s_rd + zo + slot + (L.z_own[0] + gb) - ((L.z_own[0] + wb) & ~3u));
            zw1 = HALF ? zw0 : lds_read_u16(L.s_rd + zo + 512u + slot + (L.z_own[1] + gb) - ((L.z_own[1] + wb) & ~3u));
        }
        lds_read_slices<NT, ST * kGemmAStage>(af[0], L.a_rd[0]);
        lds_wait<NT>(af[0], bw0, bw1, sw0, sw1, zw0, zw1);
        const GroupScale g0 = group_scale<SYM>((uint16_t)sw0, (uint16_t)zw0);
        const GroupScale g1 = group_scale<SYM>((uint16_t)sw1, (uint16_t)zw1);
        gemm_mma<SYM, NT, ST, HALF>(L, af, bw0, bw1, g0, g1, acc);
    }
}

// MODE 0: gate/up + activation; MODE 1: down + scatter; MODE 2: dense
// projection y[t, n] (the down sub-tensor's geometry, rows taken in order).
// HALF, dense GEMM: a 128-column tile, wave w the 32 weight rows 32 w .. of
// it as one tile (acc[.][0]).
// HALF, gate/up (a column tile with 64 live columns): waves 0-1 run the
// gate rows of columns 0-31 and 32-63 and waves 2-3 the up rows of the same
// columns, one weight tile each instead of two tiles on two waves with two
// idle; the up accumulators reach waves 0-1 through the LDS before the
// activation. Every accumulator sees the same MFMA sequence as in a full
// tile, so the results are identical.
// The fused launch's next work item index: the last dword of the weight
// ring's stage 2, which every epilogue leaves free and an item first writes
// (by direct-to-LDS load) only after its first barrier.
constexpr uint32_t kNextWord = kGemmBBase + 3u * kGemmBStage - 4u;

template <int G, bool SYM, int ACT, int MODE, int NT, bool HALF>
__device__ __forceinline__ void gemm_block(const GemmArgs& args, const tsg_routed_block& blk,
                                           uint32_t rows, uint32_t tile, uint8_t* smem,
                                           bool post, uint32_t next) {
    static_assert(!HALF || MODE != 1, "the down GEMM has no half tiles");
    const uint32_t lane = threadIdx.x & 63u, h = lane >> 5, m = lane & 31u;
    GemmLane L;
    L.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t K = MODE == 0 ? args.d : args.f;
    L.nchunks = K / kGemmKC;
    L.nwin = (L.nchunks + gemm_window<G>() - 1u) / gemm_window<G>();
    L.blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    L.sblob = MODE == 2 ? args.dense_s : L.blob;
    L.zblob = MODE == 2 ? args.dense_b : L.blob;
    L.a_wave = L.wave < (uint32_t)NT;

    // the wave's weight rows: tile t row r is row0[t] + r of sub-tensor t
    const uint32_t ngroups = K / G;
    uint32_t row0[2], w_off[2], s_off[2], z_off[2];
    if (MODE == 0) {
        row0[0] = row0[1] = tile * 128u + 32u * (HALF ? (L.wave & 1u) : L.wave);
        L.live = row0[0] < args.f;
        w_off[0] = args.o.gate_w, w_off[1] = args.o.up_w;
        s_off[0] = args.o.gate_s, s_off[1] = args.o.up_s;
        z_off[0] = args.o.gate_b, z_off[1] = args.o.up_b;
    } else {
        // HALF (dense only): 128 columns, wave w one tile of 32 (both tile
        // slots load it; the second copy is not read)
        row0[0] = HALF ? tile * 128u + 32u * L.wave : tile * 256u + 64u * L.wave;
        row0[1] = HALF ? row0[0] : row0[0] + 32u;
        L.live = row0[0] < args.d;
        w_off[0] = w_off[1] = args.o.down_w;
        s_off[0] = s_off[1] = args.o.down_s;
        z_off[0] = z_off[1] = args.o.down_b;
    }
    if (!L.live) row0[0] = row0[1] = 0u;  // dead waves load row 0's data and drop it
    auto srow = [&](int t, uint32_t r) { return s_off[t] + (row0[t] + r) * ngroups * 2u; };
    auto zrow = [&](int t, uint32_t r) { return z_off[t] + (row0[t] + r) * ngroups * 2u; };
    {
        const uint32_t r = lane >> 1;
        const uint32_t swzb = ((r >> 2) ^ (r >> 3)) & 1u;
#pragma unroll
        for (int t = 0; t < 2; ++t)
            L.w_src[t] = L.blob + w_off[t] + (row0[t] + r) * (K / 2u) + 16u * ((lane & 1u) ^ swzb);
    }
    // scale DMA j brings rows 16j .. 16j + 15 of the wave's 64 (tile j / 2)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        L.s_ld[j] = srow(j >> 1, 16u * (j & 1) + (lane >> 2));
        L.z_ld[j] = zrow(j >> 1, 16u * (j & 1) + (lane >> 2));
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        L.s_own[t] = srow(t, m);
        L.z_own[t] = zrow(t, m);
    }
    {
        const uint32_t nrows = MODE == 0 ? args.f : args.d;  // rows x groups is even
        const uint32_t s_hi = s_off[0] > s_off[1] ? s_off[0] : s_off[1];
        const uint32_t z_hi = z_off[0] > z_off[1] ? z_off[0] : z_off[1];
        L.s_last = s_hi + nrows * ngroups * 2u - 4u;
        L.z_last = z_hi + nrows * ngroups * 2u - 4u;
    }

    // activation DMA j of wave w moves rows 32w + 8j + l/8, lane l bringing
    // the piece stored in slot l % 8; rows past the block repeat row 0
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t row = 32u * L.wave + 8u * j + (lane >> 3);
        row = row < rows ? row : 0u;
        const uint32_t piece = (lane & 7u) ^ (lane >> 3) ^ ((uint32_t)j & 1u);
        const uint32_t src = MODE == 0 ? args.pairs[blk.pair_start + row].token * args.a_stride
                                       : (blk.local_row + row) * args.a_stride;
        L.a_src[j] = args.a + src + piece * 8u;
    }
    const uint32_t base = lds_addr(smem);
    const uint32_t swz = (m & 7u) ^ ((m >> 3) & 1u);
#pragma unroll
    for (int st = 0; st < 4; ++st) L.a_rd[st] = base + m * kGemmKC * 2u + (((h * 4u + st) ^ swz) << 4);
    const uint32_t swzb_m = ((m >> 2) ^ (m >> 3)) & 1u;
    L.b_rd = base + kGemmBBase + L.wave * kGemmBWave + 32u * m + 16u * (h ^ swzb_m);
    L.s_rd = base + kGemmSBase + L.wave * kGemmSWave + 16u * m;
    if (MODE == 0 && HALF && L.wave >= 2u) {  // waves 2-3 read their up tile in the tile-0 slots
        L.b_rd += kGemmBTile;
        L.s_rd += 512u;
        L.s_own[0] = L.s_own[1];
        L.z_own[0] = L.z_own[1];
    }

    f16v_t acc[NT][2];
#pragma unroll
    for (int i = 0; i < NT; ++i) acc[i][0] = acc[i][1] = f16v_t{};

    // down: this thread's row destination (token * top_k + rank) * d, loaded
    // now so that its latency hides behind the K loop (it is the oldest load,
    // so the loop's counted waits retire it first)
    uint32_t row_dst = 0u;
    if (MODE == 1 && threadIdx.x < rows) {
        const tsg_token_expert_pair pr = args.pairs[blk.pair_start + threadIdx.x];
        row_dst = (pr.token * args.top_k + pr.rank) * args.d;
    }
    gemm_issue_scales<G, SYM>(L, smem, 0u);
    gemm_issue<0>(L, smem, 0u);
    if (L.nchunks > 1u) gemm_issue<1>(L, smem, 1u);
    for (uint32_t c = 0;;) {
        gemm_chunk<G, SYM, NT, 0, HALF>(L, smem, c, acc);
        if (++c == L.nchunks) break;
        gemm_chunk<G, SYM, NT, 1, HALF>(L, smem, c, acc);
        if (++c == L.nchunks) break;
        gemm_chunk<G, SYM, NT, 2, HALF>(L, smem, c, acc);
        if (++c == L.nchunks) break;
    }
    wait_vmcnt<0>();  // no LDS write may land after this point

    // Output: the block's tile goes through LDS (idle now) so
    // that global stores are 16 bytes per lane along output rows.
    // acc[i][t][v] of lane l: row 32 i + 8 (v / 4) + 4 h + v % 4 of the block,
    // weight row n_t (column m of tile t). Rows are padded by 16 bytes so the
    // two half-waves' 2-byte writes (4 rows apart) fall in different banks.
    constexpr uint32_t kCols = MODE == 0 || HALF ? 128u : 256u;  // columns per block
    constexpr uint32_t kStride = kCols + 8u;             // halves per LDS row
    static_assert(kGemmRows * kStride * 2u <= gemm_lds_bytes(true), "output tile fits the LDS");
    uint16_t* otile = reinterpret_cast<uint16_t*>(smem);
    // down: each row's destination, staged once per block
    uint32_t* odst = reinterpret_cast<uint32_t*>(smem + kGemmRows * kStride * 2u);
    static_assert(kGemmRows * kStride * 2u + kGemmRows * 4u <= gemm_lds_bytes(true),
                  "output tile and row destinations fit the LDS");
    block_barrier();  // every wave is done reading the rings
    // the fused launch's next item index, posted where the epilogue does not
    // write (its atomic is long complete: the loads are drained above)
    static_assert(kGemmRows * kStride * 2u + kGemmRows * 4u <= kNextWord, "next word is free");
    if (post && threadIdx.x == 0)
        asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(smem + kNextWord)), "v"(next) : "memory");
    if (MODE == 1 && threadIdx.x < rows) odst[threadIdx.x] = row_dst;
    if (MODE == 2 && threadIdx.x < rows) odst[threadIdx.x] = (blk.local_row + threadIdx.x) * args.d;
    if constexpr (HALF && MODE == 0) {
        // waves 2-3 hand their up accumulators to waves 0-1, past the tile
        constexpr uint32_t kXch = kGemmRows * kStride * 2u;
        static_assert(kXch + 2u * NT * 16u * 64u * 4u <= kNextWord, "exchange fits below the next word");
        float* xch = reinterpret_cast<float*>(smem + kXch);
        const uint32_t pair = L.wave & 1u;
        if (L.wave >= 2u) {
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) xch[((pair * NT + i) * 16u + v) * 64u + lane] = acc[i][0][v];
        }
        lds_barrier();
        if (L.wave < 2u) {
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][1][v] = xch[((pair * NT + i) * 16u + v) * 64u + lane];
        }
    }
    if (L.live && (!HALF || MODE != 0 || L.wave < 2u)) {
        const uint32_t c0 = MODE == 0 || HALF ? 32u * L.wave + m : 64u * L.wave + m;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t mm = 32u * i + 8u * (v >> 2) + 4u * h + (v & 3);
                if (MODE == 0) {
                    const float gt = f16_to_f32(f32_to_f16(acc[i][0][v]));
                    const float up = f16_to_f32(f32_to_f16(acc[i][1][v]));
                    otile[mm * kStride + c0] = f32_to_f16(gate_activation<ACT>(gt) * up);
                } else {
                    otile[mm * kStride + c0] = f32_to_f16(acc[i][0][v]);
                    if constexpr (!HALF) otile[mm * kStride + c0 + 32u] = f32_to_f16(acc[i][1][v]);
                }
            }
        }
    }
    block_barrier();
    const uint32_t col0 = MODE == 0 || HALF ? tile * 128u : tile * 256u;
    const uint32_t ncols = MODE == 0 ? args.f : args.d;
    const uint32_t live = ncols - col0 < kCols ? ncols - col0 : kCols;  // multiple of 64
    constexpr uint32_t kPieces = kCols / 8u;  // 16-byte pieces per row
    // The tile's LDS reads are inline ds_reads: a plain LDS read after the
    // direct-to-LDS loads makes the compiler wait for every outstanding vector
    // memory operation first, and on gfx9 that count includes this loop's own
    // global stores, so each store waited for the one before it to complete.
    for (uint32_t p = threadIdx.x; p < rows * kPieces; p += kGemmThreads) {
        const uint32_t r = p / kPieces, cg = p - r * kPieces;
        if (cg * 8u >= live) continue;
        u32x4_t v = lds_read16<0>(lds_addr(otile + r * kStride + cg * 8u));
        uint32_t dst = MODE == 0 ? (blk.local_row + r) * args.f : lds_read_b32(lds_addr(odst + r));
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v), "+v"(dst));
        *reinterpret_cast<u32x4_t*>(args.out + dst + col0 + cg * 8u) = v;
    }
}

// Work item of workgroup pid. Routed blocks are taken largest first (stable
// in block order), so the long items start early and short ones fill the
// tail; groups of 8 consecutive routed blocks are dealt one per XCD
// (workgroups go to the 8 XCDs round-robin by linear id, each XCD with its
// own L2) with their ntiles items on that XCD, tile-major, so the items of a
// routed block share its activation rows in one L2. Blocks past
// kSortBlocks keep block order, and so does a list whose count the device
// wrote (tsg_prefill_group_pairs_device writes it largest first). `scratch`
// is 64 words of LDS the caller does not use yet. Bijective on
// [0, nb * ntiles).
constexpr uint32_t kSortBlocks = 1024;

__device__ __forceinline__ uint32_t size_bucket(uint32_t rows) {
    const uint32_t b = (rows + 31u) / 32u;
    return b < 8u ? b : 8u;
}

__device__ void gemm_work_item(const GemmArgs& args, uint32_t nb, uint32_t pid, uint32_t* scratch,
                               bool presorted, uint32_t& yb, uint32_t& tile) {
    const uint32_t T = args.ntiles, G = nb / 8u;
    uint32_t j;
    if (pid < 8u * T * G) {
        const uint32_t rem = pid % (8u * T);
        j = 8u * (pid / (8u * T)) + rem % 8u;
        tile = rem / 8u;
    } else {
        const uint32_t q = pid - 8u * T * G;
        j = 8u * G + q / T;
        tile = q % T;
    }
    if (presorted || nb > kSortBlocks || args.n_blocks_device) {
        // too many to sort here, or a list from tsg_prefill_group_pairs_device
        // (largest first already)
        yb = j;
        return;
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    uint32_t bq[kSortBlocks / kGemmThreads];
#pragma unroll
    for (uint32_t q = 0; q < kSortBlocks / kGemmThreads; ++q) {
        const uint32_t jj = tid + kGemmThreads * q;
        bq[q] = jj < nb ? size_bucket(args.blocks[jj].row_count) : 0u;
    }
    // per-wave bucket counts (buckets 0..8) -> scratch[9 * wave + bucket]
#pragma unroll
    for (uint32_t k = 0; k <= 8u; ++k) {
        uint32_t c = 0;
#pragma unroll
        for (uint32_t q = 0; q < kSortBlocks / kGemmThreads; ++q)
            c += (uint32_t)__builtin_popcountll(__ballot(bq[q] == k));
        if (lane == 0) scratch[9u * wv + k] = c;
    }
    __syncthreads();
    // rank j in (bucket descending, block index) order: bucket kk, rank r in it
    uint32_t kk = 0, r = 0, base = 0;
    for (int k = 8; k >= 0; --k) {
        uint32_t c = 0;
        for (uint32_t w = 0; w < kGemmWaves; ++w) c += scratch[9u * w + (uint32_t)k];
        if (j < base + c) {
            kk = (uint32_t)k;
            r = j - base;
            break;
        }
        base += c;
    }
    __syncthreads();
    // matches of bucket kk per (q, wave) segment, in block index order
    uint64_t mask[kSortBlocks / kGemmThreads];
#pragma unroll
    for (uint32_t q = 0; q < kSortBlocks / kGemmThreads; ++q) {
        mask[q] = __ballot(bq[q] == kk);
        if (lane == 0) scratch[kGemmWaves * q + wv] = (uint32_t)__builtin_popcountll(mask[q]);
    }
    __syncthreads();
    uint32_t acc = 0;
    for (uint32_t q = 0; q < kSortBlocks / kGemmThreads; ++q) {
        for (uint32_t w = 0; w < kGemmWaves; ++w) {
            const uint32_t c = scratch[kGemmWaves * q + w];
            if (r < acc + c) {
                if (w == wv && ((mask[q] >> lane) & 1u) &&
                    (uint32_t)__builtin_popcountll(mask[q] & ((1ull << lane) - 1ull)) == r - acc)
                    scratch[63] = kGemmThreads * q + 64u * w + lane;
                q = kSortBlocks;  // done
                break;
            }
            acc += c;
        }
    }
    __syncthreads();
    yb = scratch[63];
}

// One work item: column tile `tile` of routed block blk; a block wider than
// kGemmRows runs as consecutive passes.
template <int G, bool SYM, int ACT, int MODE>
__device__ __forceinline__ void gemm_item(const GemmArgs& args, const tsg_routed_block& blk,
                                          uint32_t tile, uint8_t* smem, bool post = false,
                                          uint32_t next = 0u) {
    // a block list written on the device is not checked on the host: an
    // expert past the layer is skipped (its weights would lie outside it)
    const bool bad_expert = MODE != 2 && blk.local_slot >= args.num_experts;
    if (bad_expert || blk.row_count == 0) {
        // No pass runs (a block with no rows is a no-op, as in the two-launch
        // form), so the fused launch's next index is posted here instead of in
        // the epilogue; the barrier first lets every wave read the index the
        // previous item posted in the same word (the block takes this branch
        // as a whole: blk is uniform).
        if (bad_expert && threadIdx.x == 0) atomicOr(args.error, kErrGemmBlock);
        if (post) {
            lds_barrier();
            if (threadIdx.x == 0)
                asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(smem + kNextWord)), "v"(next) : "memory");
        }
        return;
    }
    for (uint32_t r0 = 0; r0 < blk.row_count; r0 += kGemmRows) {
        if (r0) block_barrier();  // every wave is done with the previous pass's LDS
        tsg_routed_block sub = blk;
        sub.pair_start += r0;
        sub.local_row += r0;
        const uint32_t rows = blk.row_count - r0 < kGemmRows ? blk.row_count - r0 : kGemmRows;
        // gate/up column tiles hold 128 columns, the last one 64 when F is an
        // odd multiple of 64; dense tiles hold 128 columns when dense_narrow
        const bool half = MODE == 0 ? args.f - tile * 128u <= 64u : MODE == 2 && args.dense_narrow;
        if (half) {
            switch ((rows + 31u) / 32u) {
                case 1: gemm_block<G, SYM, ACT, MODE, 1, MODE != 1>(args, sub, rows, tile, smem, post, next); break;
                case 2: gemm_block<G, SYM, ACT, MODE, 2, MODE != 1>(args, sub, rows, tile, smem, post, next); break;
                case 3: gemm_block<G, SYM, ACT, MODE, 3, MODE != 1>(args, sub, rows, tile, smem, post, next); break;
                default: gemm_block<G, SYM, ACT, MODE, 4, MODE != 1>(args, sub, rows, tile, smem, post, next); break;
            }
        } else {
            switch ((rows + 31u) / 32u) {
                case 1: gemm_block<G, SYM, ACT, MODE, 1, false>(args, sub, rows, tile, smem, post, next); break;
                case 2: gemm_block<G, SYM, ACT, MODE, 2, false>(args, sub, rows, tile, smem, post, next); break;
                case 3: gemm_block<G, SYM, ACT, MODE, 3, false>(args, sub, rows, tile, smem, post, next); break;
                default: gemm_block<G, SYM, ACT, MODE, 4, false>(args, sub, rows, tile, smem, post, next); break;
            }
        }
    }
}

// 1-D grid of ntiles x (routed block capacity) workgroups; those past the
// live count exit at once.
template <int G, bool SYM, int ACT, int MODE>
__global__ __launch_bounds__(kGemmThreads, 2) void moe_gemm_kernel(GemmArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];  // gemm_lds_bytes(SYM)
    const uint32_t nb = args.n_blocks_device ? *args.n_blocks_device : args.n_blocks;
    const uint32_t total = nb * args.ntiles;
    if (blockIdx.x >= total) return;
    uint32_t yb, tile;
    // the weight ring's last stage is first written after chunk 0's barrier
    gemm_work_item(args, nb, blockIdx.x, reinterpret_cast<uint32_t*>(smem + kGemmBBase + 2u * kGemmBStage),
                   MODE == 2, yb, tile);
    tsg_routed_block blk;
    if (MODE == 2) {  // dense: block yb is rows 128 yb .. of x, all full but the last
        blk.local_slot = 0;
        blk.pair_start = blk.local_row = yb * kGemmRows;
        blk.row_count = args.dense_rows - blk.local_row < kGemmRows ? args.dense_rows - blk.local_row
                                                                    : kGemmRows;
    } else {
        blk = args.blocks[yb];
    }
    gemm_item<G, SYM, ACT, MODE>(args, blk, tile, smem);
}

// The gate/up and down GEMMs of one layer in one persistent launch. With Q
// queues (the device's XCDs), routed block b of the list (largest first as
// the device grouping writes it) belongs to queue b % Q; each queue holds its blocks' work items, all
// gate/up items (block by block, largest first) before any down item. A
// workgroup takes items from queue XCC_ID % Q (the XCD it runs on, a hardware
// register), so every item of a block runs on one XCD and the activations
// pass between its gate/up and down items through that XCD's L2: a gate/up
// item's stores complete (vmcnt), then it counts itself in done[b]; a down
// item of b waits until done[b] holds all gate/up tiles of b. The L1 of a CU
// is invalidated at launch, and an activation row is whole 128-byte lines
// (f % 64 == 0, a 128-byte aligned buffer), so a CU's L1 holds no line of b's
// activations from before b's gate/up items wrote them: a line it holds was
// loaded by a down item of its own block, after the block's gate/up items.
// No wait can block the gate/up items (they wait on nothing, and a down item
// is taken only after every gate/up item of its queue was), and each wait is
// bounded (kErrGemmWait on a timeout). The last workgroup to leave resets the
// queues and counters for the next launch, and reports a queue no workgroup
// drained (kErrGemmWait). Down items fill the gate/up tail, and there is no
// launch between the two GEMMs. Launches that share a context's schedule
// words must not overlap (one stream, or ordered streams).
struct FusedSched {
    uint32_t* next;    // kMaxGemmQueues queue heads
    uint32_t* exited;  // workgroups that have left
    uint32_t* done;    // gate/up tiles finished, per routed block (cap entries)
    uint32_t cap;
    uint32_t queues;   // 1, 2, 4 or 8
};
constexpr uint32_t kFusedSpinLimit = 1u << 18;

template <int G, bool SYM, int ACT>
__global__ __launch_bounds__(kGemmThreads, 2) void moe_gemm_fused_kernel(GemmArgs gu, GemmArgs dn,
                                                                         FusedSched sc) {
    extern __shared__ __align__(16) uint8_t smem[];  // gemm_lds_bytes(SYM)
    // The item index travels through the weight ring's last stage, which an
    // item first writes after its first barrier (every wave has read the
    // index by then). No static LDS: two sym workgroups fill a CU's 160 KiB.
    uint32_t* word = reinterpret_cast<uint32_t*>(smem + kGemmBBase + 2u * kGemmBStage);
    const uint32_t nb_dev = gu.n_blocks_device ? *gu.n_blocks_device : gu.n_blocks;
    const uint32_t nb = nb_dev < sc.cap ? nb_dev : sc.cap;
    const uint32_t Q = sc.queues;
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= Q - 1u;
    const uint32_t T0 = gu.ntiles, T1 = dn.ntiles;
    const uint32_t nbx = nb > xcc ? (nb - xcc + Q - 1u) / Q : 0u;
    const uint32_t n_gu = nbx * T0, n_all = nbx * (T0 + T1);
    if (threadIdx.x == 0) word[0] = atomicAdd(&sc.next[xcc], 1u);
    __syncthreads();
    uint32_t item = word[0];
    while (item < n_all) {
        // the next item is taken now; its index arrives while this one runs
        uint32_t next = 0;
        if (threadIdx.x == 0) next = atomicAdd(&sc.next[xcc], 1u);
        if (item < n_gu) {
            const uint32_t yb = xcc + Q * (item / T0), tile = item % T0;
            gemm_item<G, SYM, ACT, 0>(gu, gu.blocks[yb], tile, smem, true, next);
            wait_vmcnt<0>();  // this wave's activation stores are in the L2
            __syncthreads();
            if (threadIdx.x == 0) atomicAdd(&sc.done[yb], 1u);
        } else {
            const uint32_t j = item - n_gu, yb = xcc + Q * (j / T1), tile = j % T1;
            if (threadIdx.x == 0) {
                for (uint32_t spins = 0; ld_coherent(&sc.done[yb]) < T0; ++spins) {
                    if (spins > kFusedSpinLimit) {
                        atomicOr(gu.error, kErrGemmWait);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            __syncthreads();
            gemm_item<G, SYM, ACT, 1>(dn, dn.blocks[yb], tile, smem, true, next);
        }
        // An LDS-only barrier and an LDS read the compiler does not see: a
        // __syncthreads() (its release fence) or a plain LDS access after the
        // direct-to-LDS loads would wait for this item's epilogue stores to
        // complete, and nothing in this launch reads a down item's partials.
        // The item posted the next index at its epilogue (gemm_block).
        lds_barrier();  // the item's LDS is free, the next index visible
        item = lds_read_b32(lds_addr(smem + kNextWord));
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(item));
        item = __builtin_amdgcn_readfirstlane(item);
    }
    if (threadIdx.x == 0) word[1] = atomicAdd(sc.exited, 1u) == gridDim.x - 1u ? 1u : 0u;
    __syncthreads();
    if (word[1]) {
        // every other workgroup has left: nobody reads the schedule any more
        // (agent-coherent stores: the counters live at the memory side, where
        // the other XCDs' atomics of the next launch find them)
        for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) st_coherent(sc.done + i, 0u);
        if (threadIdx.x < Q) {
            const uint32_t x = threadIdx.x;
            const uint32_t nx = nb > x ? (nb - x + Q - 1u) / Q : 0u;
            if (ld_coherent(sc.next + x) < nx * (T0 + T1)) atomicOr(gu.error, kErrGemmWait);
            st_coherent(sc.next + x, 0u);
        }
        if (threadIdx.x == 0) st_coherent(sc.exited, 0u);
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

template <int G, bool SYM, int MODE>
tsg_status launch_gemm(const tsg_moe* moe, hipStream_t s, const GemmArgs& a, uint32_t max_blocks) {
    GemmArgs args = a;
    args.ntiles = MODE == 0 ? (a.f + 127u) / 128u : (a.d + 255u) / 256u;  // 4 waves x 32 / 64 rows
    TSG_REQUIRE((uint64_t)args.ntiles * max_blocks <= 0x7FFFFFFFu, TSG_ERR_INVALID_ARGUMENT,
                "moe_gemm: %u routed blocks x %u tiles exceed the grid", max_blocks, args.ntiles);
    const dim3 grid(args.ntiles * max_blocks);
    auto kern = moe->activation == TSG_ACT_SILU ? moe_gemm_kernel<G, SYM, TSG_ACT_SILU, MODE>
                                                : moe_gemm_kernel<G, SYM, TSG_ACT_GELU_TANH, MODE>;
    // more than 64 KiB of dynamic LDS must be allowed per kernel (idempotent)
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)gemm_lds_bytes(SYM)));
    hipLaunchKernelGGL(kern, grid, dim3(kGemmThreads), gemm_lds_bytes(SYM), s, args);
    return check_launch(MODE == 0 ? "moe_gemm gate/up" : "moe_gemm down");
}

template <int G, bool SYM>
tsg_status launch_fused(const tsg_moe* moe, hipStream_t s, GemmArgs gu, GemmArgs dn,
                        uint32_t max_blocks) {
    gu.ntiles = (gu.f + 127u) / 128u;
    dn.ntiles = (dn.d + 255u) / 256u;
    const tsg_ctx* ctx = moe->ctx;
    FusedSched sc;
    sc.next = ctx->gemm_sched;
    sc.exited = ctx->gemm_sched + kMaxGemmQueues;
    sc.done = ctx->gemm_sched + 16u;
    sc.cap = max_blocks;
    sc.queues = ctx->gemm_queues;
    auto kern = moe->activation == TSG_ACT_SILU ? moe_gemm_fused_kernel<G, SYM, TSG_ACT_SILU>
                                                : moe_gemm_fused_kernel<G, SYM, TSG_ACT_GELU_TANH>;
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)gemm_lds_bytes(SYM)));
    // two workgroups per CU (the GEMM's occupancy), every one of them resident
    const dim3 grid(2u * (uint32_t)ctx->num_cus);
    hipLaunchKernelGGL(kern, grid, dim3(kGemmThreads), gemm_lds_bytes(SYM), s, gu, dn, sc);
    return check_launch("moe_gemm fused gate/up + down");
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

// Dense projection: blocks of 128 rows of x in order, 256 output columns per
// workgroup (the down GEMM's tiling).
template <int G, bool SYM>
tsg_status launch_dense_qmm(hipStream_t s, const GemmArgs& a, uint32_t num_cus) {
    GemmArgs args = a;
    args.n_blocks = (a.dense_rows + kGemmRows - 1u) / kGemmRows;
    // 256-column tiles while they cover the device's CUs; below that, 128-column
    // tiles (one 32-row weight tile per wave, the same MFMA sequence per
    // column, so the same results), twice the workgroups. T = 2048: N = 2816
    // runs 352 narrow workgroups instead of 176 wide ones, 0.84-0.92 of the
    // N = 4096 call's time in the same run against 0.92-0.95 wide; N = 4096 (256
    // wide workgroups) was no faster as 512 narrow ones and keeps wide tiles
    args.dense_narrow = (uint64_t)((a.d + 255u) / 256u) * args.n_blocks < num_cus ? 1u : 0u;
    args.ntiles = args.dense_narrow ? (a.d + 127u) / 128u : (a.d + 255u) / 256u;
    TSG_REQUIRE((uint64_t)args.ntiles * args.n_blocks <= 0x7FFFFFFFu, TSG_ERR_UNSUPPORTED,
                "qmm: %u row blocks x %u tiles exceed the grid", args.n_blocks, args.ntiles);
    auto kern = moe_gemm_kernel<G, SYM, TSG_ACT_GELU_TANH, 2>;  // ACT unused in mode 2
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)gemm_lds_bytes(SYM)));
    hipLaunchKernelGGL(kern, dim3(args.ntiles * args.n_blocks), dim3(kGemmThreads),
                       gemm_lds_bytes(SYM), s, args);
    return check_launch("moe_gemm dense qmm");
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
        return sym ? launch_fused<32, true>(moe, s, gu, dn, n_blocks)
                   : launch_fused<32, false>(moe, s, gu, dn, n_blocks);
    return sym ? launch_fused<64, true>(moe, s, gu, dn, n_blocks)
               : launch_fused<64, false>(moe, s, gu, dn, n_blocks);
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
        return sym ? launch_dense_qmm<32, true>(hs, a, cus) : launch_dense_qmm<32, false>(hs, a, cus);
    return sym ? launch_dense_qmm<64, true>(hs, a, cus) : launch_dense_qmm<64, false>(hs, a, cus);
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
