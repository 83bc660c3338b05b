// prefill_gemm_impl.hpp — the grouped int4 GEMM kernels of the prompt-chunk
// routed MoE (prefill.metal:913-1092, 3664-3864, encodeStreamedTiled) and the
// dense projection QMM that shares them, with their launchers. Included by the
// four gemm_g*_*.hip translation units only, each instantiating one
// (group size, scheme).
#pragma once

#include "prefill_gemm.hpp"

namespace tsg {
namespace {

// --------------------------------------------------------------- GEMM

// Grouped int4 GEMM over routed blocks of one expert, in passes of R = 128
// rows. Workgroup = 4 waves, two workgroups per CU (two waves per SIMD, so
// one wave's barrier and memory waits overlap the other's MFMAs); each wave
// owns 64 weight rows as two 32-row MFMA tiles (gate/up: 32 gate + the same
// 32 up rows, so the GeGLU epilogue finds both in one lane; down: 64 output
// rows) against every live 32-row slice of the pass's activation rows (NT =
// 1 .. 4, a template parameter, so the inner loop has no per-slice tests). A
// dequantised weight fragment feeds NT MFMAs per tile and an activation
// fragment read from LDS feeds two. A routed block of more than 128 rows
// runs as consecutive passes of the same work item. (One 256-row workgroup
// per CU, its 8 x 2 accumulator tiles in AGPRs, halves the dequantisation
// per MFMA but runs at well under half the MFMA rate: a single wave per SIMD
// leaves every barrier and memory wait exposed.)
//
// K runs in 64-element chunks through a 3-stage ring. Every wave issues the
// same loads per chunk, all direct global->LDS: NT activation loads (load j
// = wave + 4 i moves rows 8 j .. 8 j + 7, 16 bytes a lane), its two weight
// tiles (32 rows x 32 bytes each, two lanes per row) and one dword of group
// scales per weight row (one more of biases under affine). The chunk's single
// workgroup barrier sits before its last MFMA step: by then every wave has
// its last activation fragments in registers, so the barrier both frees the
// chunk's stage (chunk c + 3 is issued into it) and publishes chunk c + 1,
// whose weights, scales and first activation fragments are read and
// dequantised while the last step's MFMAs run. The next chunk starts on its
// MFMAs at once.
//  - activations: row r's 16-byte piece p sits in slot p ^ swz(r),
//    swz(r) = (r & 7) ^ ((r >> 3) & 1);
//  - weights: row r's half h sits in slot h ^ swzb(r),
//    swzb(r) = ((r >> 2) ^ (r >> 3)) & 1;
//  - scales: lane l of a wave brings the dword holding the chunk's group(s)
//    of its row l (tile l / 32, row l % 32).
// The swizzles keep the MFMA-side LDS reads conflict-free whether the LDS
// serves 8 lanes of a 16-byte read per cycle over 32 banks or 16 over 64.
// Word s of a lane's 16 weight bytes is dequantised into the B operand of
// MFMA step s, whose logical K 8h..8h+7 is physical 64c + 32h + 8s + (0..7);
// the activations are read with the same mapping. Step s + 1's activation
// reads and dequantisation are issued ahead of step s's MFMAs.
constexpr uint32_t kGemmRows = 128;       // routed blocks: rows per pass
constexpr uint32_t kDenseRows = 128;      // dense projection: rows per pass
constexpr uint32_t kGemmWaves = 4;
constexpr uint32_t kGemmThreads = kGemmWaves * 64u;
constexpr uint32_t kGemmAStages = 3;     // activation ring (shared by the workgroup)
constexpr uint32_t kGemmBStages = 2;     // weight ring (each wave its own tiles)
constexpr uint32_t kGemmBTile = 32u * kGemmKC / 2u;                   // 1 KiB
constexpr uint32_t kGemmBWave = 2u * kGemmBTile;
constexpr uint32_t kGemmBStage = kGemmWaves * kGemmBWave;             // 8 KiB
constexpr uint32_t kGemmSWin = 4u;                                    // chunks per scale window
constexpr uint32_t kGemmSWave = 64u * 16u;                            // 1 KiB: 64 rows x 16 B
constexpr uint32_t kGemmSBuf = kGemmWaves * kGemmSWave;               // 4 KiB

// LDS of a workgroup running passes of R rows: the activation ring
// (3 x R x 128 bytes), the weight ring (2 stages), two buffers of scale
// windows (and two of bias windows under affine); the epilogue reuses it from
// offset 0 and leaves the fused launch's item word and exit flag just past
// its data. R = 128: 73,728 bytes sym, 81,920 affine, two workgroups per CU.
template <uint32_t R>
struct GemmLds {
    static constexpr uint32_t kSlices = R / 32u;                 // 32-row MFMA slices
    static constexpr uint32_t kAStage = R * kGemmKC * 2u;        // 16 KiB
    static constexpr uint32_t kBBase = kGemmAStages * kAStage;
    static constexpr uint32_t kSBase = kBBase + kGemmBStages * kGemmBStage;
    static constexpr uint32_t kZBase = kSBase + 2u * kGemmSBuf;
    static constexpr uint32_t pipe(bool sym) { return kZBase + (sym ? 0u : 2u * kGemmSBuf); }
    // the largest epilogue: R x (256 + 8) halves and R row destinations, or
    // R x (128 + 8) halves and the half-tile exchange of 2 x kSlices x 4 KiB
    static constexpr uint32_t kEpiDown = R * 264u * 2u + R * 4u;
    static constexpr uint32_t kEpiHalf = R * 136u * 2u + 2u * kSlices * 4096u;
    static constexpr uint32_t kEpi = kEpiDown > kEpiHalf ? kEpiDown : kEpiHalf;
    static constexpr uint32_t kWord = (kEpi + 15u) / 16u * 16u;  // item index, exit flag
    static constexpr uint32_t bytes(bool sym) {
        return pipe(sym) > kWord + 16u ? pipe(sym) : kWord + 16u;
    }
};
static_assert(GemmLds<kGemmRows>::bytes(false) * 2u <= 160u * 1024u, "two workgroups per CU");
static_assert(GemmLds<kDenseRows>::bytes(false) * 2u <= 160u * 1024u, "two workgroups per CU");

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
// Slice i of the activation stage at byte OFF: addr + OFF + 4096 i. The ds
// offset field holds 16 bits, so a stage whose slices reach past it is read
// from addr + 65536.
template <int NT, uint32_t BASE, int I = 0>
__device__ __forceinline__ void lds_read_slices(u32x4_t (&a)[NT], uint32_t addr) {
    if constexpr (I < NT) {
        a[I] = lds_read16<BASE + (uint32_t)I * 4096u>(addr);
        lds_read_slices<NT, BASE, I + 1>(a, addr);
    }
}
template <int NT, uint32_t OFF>
__device__ __forceinline__ void lds_read_act(u32x4_t (&a)[NT], uint32_t addr) {
    if constexpr (OFF + (uint32_t)(NT - 1) * 4096u > 65535u) {
        static_assert(OFF >= 65536u, "a stage straddles the 64 KiB offset limit");
        // added at the use (volatile asm): a hoisted copy would be spilled
        uint32_t hi;
        asm volatile("v_add_u32 %0, %1, %2" : "=v"(hi) : "s"(65536u), "v"(addr));
        lds_read_slices<NT, OFF - 65536u>(a, hi);
    } else
        lds_read_slices<NT, OFF>(a, addr);
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

// Buffer form: rsrc (a raw byte buffer), a 32-bit per-lane offset and a
// uniform one (SGPR), so a load needs no per-lane address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
    // stride 0, offsets below `bytes` in range (a load past it reads zero),
    // 32-bit data format
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ void lds_buf16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          uint8_t* lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave_base,
                                             16, voff, soff, 0, 0);
}
__device__ __forceinline__ void lds_buf4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                         uint8_t* lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave_base,
                                             4, voff, soff, 0, 0);
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

// LDS address of MFMA step st's activation piece: a ^ (st << 4). Issued as
// volatile asm at its use, so the compiler does not hoist the three step
// addresses out of the K loop (where they would be spilled, and each reload's
// vmcnt(0) wait would drain the chunk prefetch).
__device__ __forceinline__ uint32_t step_addr(uint32_t a, uint32_t st) {
    uint32_t r;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "s"(st << 4), "v"(a));
    return r;
}

// Per-lane state of one pass's GEMM: NT activation loads per chunk.
template <int NT>
struct GemmLane {
    __amdgpu_buffer_rsrc_t abuf;  // activation bytes (hidden, act or x)
    __amdgpu_buffer_rsrc_t wbuf;  // weights (the expert's blob)
    __amdgpu_buffer_rsrc_t sbuf;  // base of the scale offsets (the blob, or dense scales)
    __amdgpu_buffer_rsrc_t zbuf;  // base of the bias offsets
    uint32_t a_off[NT];         // byte offset of the lane's piece of activation load i (chunk 0)
    uint32_t w_off[2];          // byte offset of the lane's weight piece per tile (chunk 0)
    uint32_t s_ld[2], z_ld[2];  // scale / bias row start of the row the lane loads in window
                                // pieces 0-1 (tile 0) and 2-3 (tile 1); G = 32: + 4 (lane % 4)
    uint32_t s_q1;              // window piece q adds (q & 1) x 16 rows of scale bytes
    uint32_t s_own[2], z_own[2];  // scale / bias row starts of the lane's own rows (G = 64)
    uint32_t a_rd;              // LDS activation read address of MFMA step 0 (stage 0, slice 0)
    uint32_t b_rd;              // LDS weight read address (stage 0)
    uint32_t s_rd[2];           // LDS scale read address of the lane's row per tile (buffer 0)
    uint32_t wave, nchunks;
};

// Scale (and bias) windows: window V is chunks 4V .. 4V + 3, 16 bytes of
// each weight row: G = 32, groups 8V .. 8V + 7 (a 4-byte aligned row, as the
// launch checks); G = 64, the 16 bytes from the dword holding group 4V,
// which hold groups 4V .. 4V + 3 however the row is aligned. A window is
// four loads of 16 rows x 4 dwords (piece q: rows 16 q .. 16 q + 15 of the
// wave's 64), one per chunk: piece q of window V goes out with chunk
// X = 4V - 3 + q. Buffer V % 2.
template <int G, bool SYM, int NT>
__device__ __forceinline__ void window_piece(const GemmLane<NT>& L, uint8_t* smem_sbase,
                                             uint32_t q, uint32_t V) {
    const uint32_t lane = threadIdx.x & 63u;
    uint8_t* dst = smem_sbase + (V & 1u) * kGemmSBuf + L.wave * kGemmSWave + q * 256u;
    const uint32_t srow = q >= 2u ? L.s_ld[1] : L.s_ld[0];
    const uint32_t zrow = q >= 2u ? L.z_ld[1] : L.z_ld[0];
    if constexpr (G == 32) {
        lds_buf4(L.sbuf, srow, (q & 1u) * L.s_q1 + 16u * V, dst);
        if constexpr (!SYM) lds_buf4(L.zbuf, zrow, (q & 1u) * L.s_q1 + 16u * V, dst + 2u * kGemmSBuf);
    } else {
        const uint32_t d4 = 4u * (lane & 3u);
        lds_buf4(L.sbuf, ((srow + (q & 1u) * L.s_q1 + 8u * V) & ~3u) + d4, 0u, dst);
        if constexpr (!SYM)
            lds_buf4(L.zbuf, ((zrow + (q & 1u) * L.s_q1 + 8u * V) & ~3u) + d4, 0u, dst + 2u * kGemmSBuf);
    }
}
// Byte of the lane's group for chunk c within its row's 16 window bytes
// (G = 32: the lane's half h is folded into its read address).
template <int G>
__device__ __forceinline__ uint32_t scale_sel(uint32_t row, uint32_t c) {
    if constexpr (G == 32) {
        return 4u * (c & 3u);
    } else {
        return row + 2u * c - ((row + 8u * (c >> 2)) & ~3u);
    }
}

// Chunk X's loads, issued while chunk X - 3 runs: NT activation loads into
// ring stage ST (= X % 3), the two weight tiles into stage X % 2, and the
// scale (and bias) window piece that goes out with it.
template <uint32_t R, int G, bool SYM, int NT, int ST>
__device__ __forceinline__ void gemm_issue(const GemmLane<NT>& L, uint8_t* smem, uint32_t X) {
    using Y = GemmLds<R>;
    uint8_t* adst = smem + ST * Y::kAStage + L.wave * 1024u;
#pragma unroll
    for (int i = 0; i < NT; ++i) lds_buf16(L.abuf, L.a_off[i], X * (kGemmKC * 2u), adst + (uint32_t)i * 4096u);
    uint8_t* bst = smem + Y::kBBase + (X & 1u) * kGemmBStage + L.wave * kGemmBWave;
    lds_buf16(L.wbuf, L.w_off[0], X * (kGemmKC / 2u), bst);
    lds_buf16(L.wbuf, L.w_off[1], X * (kGemmKC / 2u), bst + kGemmBTile);
    window_piece<G, SYM, NT>(L, smem + Y::kSBase, (X + 3u) & 3u, (X + 3u) >> 2);
}

// One chunk's weights and group parameters in registers.
struct ChunkRegs {
    u32x4_t bw0, bw1;           // raw weight words per tile (word s: MFMA step s)
    GroupScale g0, g1;
};

// Chunk c's weights and scales: the LDS reads (head_issue), then the wait for
// them and the group parameters (head_finish).
struct HeadRaw {
    u32x4_t bw0, bw1;
    uint32_t sw0, sw1, zw0, zw1;
};
template <uint32_t R, int G, bool SYM, int NT, bool HALF>
__device__ __forceinline__ void head_issue(const GemmLane<NT>& L, uint32_t c, HeadRaw& h) {
    using Y = GemmLds<R>;
    const uint32_t brd = L.b_rd + (c & 1u) * kGemmBStage;
    h.bw0 = lds_read16<0>(brd);
    h.bw1 = HALF ? h.bw0 : lds_read16<kGemmBTile>(brd);
    const uint32_t buf = ((c >> 2) & 1u) * kGemmSBuf;
    h.sw0 = lds_read_u16(L.s_rd[0] + buf + scale_sel<G>(L.s_own[0], c));
    h.sw1 = HALF ? h.sw0 : lds_read_u16(L.s_rd[1] + buf + scale_sel<G>(L.s_own[1], c));
    h.zw0 = h.zw1 = 0u;
    if constexpr (!SYM) {
        constexpr uint32_t zo = Y::kZBase - Y::kSBase;
        h.zw0 = lds_read_u16(L.s_rd[0] + zo + buf + scale_sel<G>(L.z_own[0], c));
        h.zw1 = HALF ? h.zw0 : lds_read_u16(L.s_rd[1] + zo + buf + scale_sel<G>(L.z_own[1], c));
    }
}
template <bool SYM>
__device__ __forceinline__ void head_finish(HeadRaw& h, ChunkRegs& cr) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(h.bw0), "+v"(h.bw1), "+v"(h.sw0), "+v"(h.sw1), "+v"(h.zw0), "+v"(h.zw1));
    cr.bw0 = h.bw0;
    cr.bw1 = h.bw1;
    cr.g0 = group_scale<SYM>((uint16_t)h.sw0, (uint16_t)h.zw0);
    cr.g1 = group_scale<SYM>((uint16_t)h.sw1, (uint16_t)h.zw1);
}

// Piece k of the dequantisation of step `st` of a chunk into p0 / p1 (k <
// 10; 5 for HALF, one tile): two nibble extractions, then eight pairs.
template <bool SYM, bool HALF>
__device__ __forceinline__ void dequant_piece(int k, int st, const ChunkRegs& cr, Nibbles& n0,
                                              Nibbles& n1, h2_t (&p0)[4], h2_t (&p1)[4]) {
    if constexpr (HALF) {
        switch (k) {
            case 0: n0 = nibbles8(cr.bw0[st]); break;
            case 1: p0[0] = dequant_pair<SYM, 0>(n0, cr.g0); break;
            case 2: p0[1] = dequant_pair<SYM, 1>(n0, cr.g0); break;
            case 3: p0[2] = dequant_pair<SYM, 2>(n0, cr.g0); break;
            default: p0[3] = dequant_pair<SYM, 3>(n0, cr.g0); break;
        }
        return;
    }
    switch (k) {
        case 0: n0 = nibbles8(cr.bw0[st]); break;
        case 1: n1 = nibbles8(cr.bw1[st]); break;
        case 2: p0[0] = dequant_pair<SYM, 0>(n0, cr.g0); break;
        case 3: p1[0] = dequant_pair<SYM, 0>(n1, cr.g1); break;
        case 4: p0[1] = dequant_pair<SYM, 1>(n0, cr.g0); break;
        case 5: p1[1] = dequant_pair<SYM, 1>(n1, cr.g1); break;
        case 6: p0[2] = dequant_pair<SYM, 2>(n0, cr.g0); break;
        case 7: p1[2] = dequant_pair<SYM, 2>(n1, cr.g1); break;
        case 8: p0[3] = dequant_pair<SYM, 3>(n0, cr.g0); break;
        default: p1[3] = dequant_pair<SYM, 3>(n1, cr.g1); break;
    }
}

// One chunk (activation stage ST) of the K loop. On entry af[0] holds step
// 0's activation fragments, bf[0] its dequantised weights and cr the chunk's
// raw weights and scales; on exit the same for chunk c + 1. Steps 0-2: the
// next step's activation reads go out first and its dequantisation (10
// pieces) is spread between this step's 2 NT MFMAs. Step 3 (af[1], bf[1]):
// after its first MFMA, the chunk's barrier (chunk c + 1 has landed for
// every wave; nobody reads this chunk's activation stage any more) and chunk
// c + 1's weight and scale reads; a few MFMAs later the wait for them, chunk
// c + 3's loads (into this activation stage and the weight stage chunk c + 1
// has just been read from), chunk c + 1's step-0 activation reads and group
// parameters, then its step-0 dequantisation between the remaining MFMAs.
// Branch-free: past the last chunk the loads and reads repeat the last chunk
// (clamped) and their results go unused, so every chunk issues the same
// loads and waits for the same counts.
template <uint32_t R, int G, bool SYM, int NT, int ST, bool HALF>
__device__ __forceinline__ void gemm_chunk(const GemmLane<NT>& L, uint8_t* smem, uint32_t c,
                                           u32x4_t (&af)[2][NT], h8v_t (&bf)[2][2], ChunkRegs& cr,
                                           f16v_t (&acc)[NT][2]) {
    using Y = GemmLds<R>;
    constexpr int kT = HALF ? 1 : 2;       // tiles per wave
    constexpr int kP = HALF ? 5 : 10;      // conversion pieces per step
    constexpr int kM = kT * NT;            // MFMAs per step
    constexpr uint32_t kLoads = (uint32_t)NT + (SYM ? 3u : 4u);  // per chunk and wave
    constexpr int kNext = (ST + 1) % 3;
#pragma unroll
    for (int st = 0; st < 3; ++st) {
        const int cur = st & 1, nxt = cur ^ 1;
        lds_read_act<NT, ST * Y::kAStage>(af[nxt], step_addr(L.a_rd, (uint32_t)(st + 1)));
        Nibbles n0{}, n1{};
        h2_t p0[4], p1[4];
#pragma unroll
        for (int q = 0; q < kM; ++q) {
            const int i = q / kT, t = q % kT;
            acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v_t, af[cur][i]),
                                                               bf[cur][t], acc[i][t], 0, 0, 0);
#pragma unroll
            for (int k = q * kP / kM; k < (q + 1) * kP / kM; ++k)
                dequant_piece<SYM, HALF>(k, st + 1, cr, n0, n1, p0, p1);
            __builtin_amdgcn_sched_barrier(0);
        }
        bf[nxt][0] = pack_pairs(p0[0], p0[1], p0[2], p0[3]);
        if constexpr (!HALF) bf[nxt][1] = pack_pairs(p1[0], p1[1], p1[2], p1[3]);
        lds_wait<NT>(af[nxt]);
    }
    const uint32_t last = L.nchunks - 1u;
    const uint32_t c1 = c + 1u < last ? c + 1u : last;
    const uint32_t c3 = c + 3u < last ? c + 3u : last;
    // MFMA index after which chunk c + 1's head is waited for, chunk c + 3's
    // loads go out and the dequantisation pieces start
    constexpr int kQ1 = kM > 3 ? 3 : kM - 1;
    HeadRaw hr;
    ChunkRegs nr;
    Nibbles n0{}, n1{};
    h2_t p0[4], p1[4];
#pragma unroll
    for (int q = 0; q < kM; ++q) {
        const int i = q / kT, t = q % kT;
        acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v_t, af[1][i]),
                                                           bf[1][t], acc[i][t], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (q == 0) {
            // chunk c + 1 has landed for this wave (chunk c + 2's loads may
            // still be in flight), then for every wave
            wait_vmcnt<kLoads>();
            block_barrier();
            head_issue<R, G, SYM, NT, HALF>(L, c1, hr);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (q == kQ1) {
            // chunk c + 1's weight stage and the scale buffer of the window
            // two ahead are free (read, and waited for, by this wave)
            head_finish<SYM>(hr, nr);
            gemm_issue<R, G, SYM, NT, ST>(L, smem, c3);
            lds_read_act<NT, kNext * Y::kAStage>(af[0], L.a_rd);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (q >= kQ1) {
            // pieces spread over MFMAs kQ1 .. kM - 1
            constexpr int kSpan = kM - kQ1;
            const int r = q - kQ1;
#pragma unroll
            for (int k = r * kP / kSpan; k < (r + 1) * kP / kSpan; ++k)
                dequant_piece<SYM, HALF>(k, 0, nr, n0, n1, p0, p1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    bf[0][0] = pack_pairs(p0[0], p0[1], p0[2], p0[3]);
    if constexpr (!HALF) bf[0][1] = pack_pairs(p1[0], p1[1], p1[2], p1[3]);
    lds_wait<NT>(af[0]);
    cr = nr;
}

// The K loop of one pass: window 0's first three pieces and chunks 0-1 go
// out; once chunk 0 has landed its head is read, chunk 2 goes out (into the
// weight stage chunk 0 was read from) and chunk 0's first fragments are
// read and dequantised; then each chunk runs as above. The loads past the
// last chunk are still in flight at the end; the epilogue waits for them
// before it writes the LDS.
template <uint32_t R, int G, bool SYM, int NT, bool HALF>
__device__ __forceinline__ void gemm_kloop(const GemmLane<NT>& L, uint8_t* smem,
                                           f16v_t (&acc)[NT][2]) {
    using Y = GemmLds<R>;
    constexpr uint32_t kLoads = (uint32_t)NT + (SYM ? 3u : 4u);
    const uint32_t last = L.nchunks - 1u;
#pragma unroll
    for (uint32_t q = 0; q < 3u; ++q) window_piece<G, SYM, NT>(L, smem + Y::kSBase, q, 0u);
    gemm_issue<R, G, SYM, NT, 0>(L, smem, 0u);
    gemm_issue<R, G, SYM, NT, 1>(L, smem, 1u < last ? 1u : last);
    wait_vmcnt<kLoads>();
    block_barrier();
    u32x4_t af[2][NT];
    h8v_t bf[2][2];
    ChunkRegs cr;
    HeadRaw hr;
    head_issue<R, G, SYM, NT, HALF>(L, 0u, hr);
    head_finish<SYM>(hr, cr);
    gemm_issue<R, G, SYM, NT, 2>(L, smem, 2u < last ? 2u : last);
    lds_read_act<NT, 0u>(af[0], L.a_rd);
    bf[0][0] = dequant8<SYM>(cr.bw0[0], cr.g0);
    if constexpr (!HALF) bf[0][1] = dequant8<SYM>(cr.bw1[0], cr.g1);
    lds_wait<NT>(af[0]);
    for (uint32_t c = 0;;) {
        gemm_chunk<R, G, SYM, NT, 0, HALF>(L, smem, c, af, bf, cr, acc);
        if (++c == L.nchunks) break;
        gemm_chunk<R, G, SYM, NT, 1, HALF>(L, smem, c, af, bf, cr, acc);
        if (++c == L.nchunks) break;
        gemm_chunk<R, G, SYM, NT, 2, HALF>(L, smem, c, af, bf, cr, acc);
        if (++c == L.nchunks) break;
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
// The routed GEMMs (MODE 0, 1) run passes of kGemmRows rows, the dense
// projection (MODE 2) passes of kDenseRows.
template <int MODE>
__host__ __device__ constexpr uint32_t gemm_rows() { return MODE == 2 ? kDenseRows : kGemmRows; }
// The fused launch's next work item index: posted just past the epilogue's
// data, after the item's loads have all landed, and read by every wave
// (followed by a barrier) before the next item's first loads.
template <bool SYM>
__host__ __device__ constexpr uint32_t next_word() { return GemmLds<kGemmRows>::kWord; }

template <int G, bool SYM, int ACT, int MODE, int NT, bool HALF>
__device__ __forceinline__ void gemm_block(const GemmArgs& args, const tsg_routed_block& blk,
                                           uint32_t rows, uint32_t tile, uint8_t* smem,
                                           bool post, uint32_t next) {
    static_assert(!HALF || MODE != 1, "the down GEMM has no half tiles");
    constexpr uint32_t R = gemm_rows<MODE>();
    using Y = GemmLds<R>;
    static_assert(NT >= 1 && (uint32_t)NT <= Y::kSlices, "slices per pass");
    const uint32_t lane = threadIdx.x & 63u, h = lane >> 5, m = lane & 31u;
    GemmLane<NT> L;
    L.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t K = MODE == 0 ? args.d : args.f;
    L.nchunks = K / kGemmKC;
    const uint8_t* blob = args.layer_base + (uint64_t)blk.local_slot * args.expert_stride;
    // routed GEMMs: loads past the expert's stride read zero (a window past
    // the last row of the last expert), never another allocation
    const uint32_t wlim = MODE == 2 ? 0xFFFFFFFFu
                                    : (uint32_t)(args.expert_stride < 0xFFFFFFFFull ? args.expert_stride
                                                                                    : 0xFFFFFFFFull);
    L.wbuf = raw_rsrc(blob, wlim);
    L.sbuf = raw_rsrc(MODE == 2 ? args.dense_s : blob, wlim);
    L.zbuf = raw_rsrc(MODE == 2 ? args.dense_b : blob, wlim);
    L.abuf = raw_rsrc(args.a, 0xFFFFFFFFu);

    // the wave's weight rows: tile t row r is row0[t] + r of sub-tensor t
    const uint32_t srow = K / G * 2u;  // scale bytes per weight row
    uint32_t row0[2], w_off[2], s_off[2], z_off[2];
    bool wave_live;
    if (MODE == 0) {
        row0[0] = row0[1] = tile * 128u + 32u * (HALF ? (L.wave & 1u) : L.wave);
        wave_live = row0[0] < args.f;
        w_off[0] = args.o.gate_w, w_off[1] = args.o.up_w;
        s_off[0] = args.o.gate_s, s_off[1] = args.o.up_s;
        z_off[0] = args.o.gate_b, z_off[1] = args.o.up_b;
    } else {
        // HALF (dense only): 128 columns, wave w one tile of 32 (both tile
        // slots load it; the second copy is not read)
        row0[0] = HALF ? tile * 128u + 32u * L.wave : tile * 256u + 64u * L.wave;
        row0[1] = HALF ? row0[0] : row0[0] + 32u;
        wave_live = row0[0] < args.d;
        w_off[0] = w_off[1] = args.o.down_w;
        s_off[0] = s_off[1] = args.o.down_s;
        z_off[0] = z_off[1] = args.o.down_b;
    }
    // dead waves (a tile past the last weight row) load row 0's data, run
    // the same loop and store nothing
    if (!wave_live) row0[0] = row0[1] = 0u;
    {
        const uint32_t r = lane >> 1;
        const uint32_t swzb = ((r >> 2) ^ (r >> 3)) & 1u;
#pragma unroll
        for (int t = 0; t < 2; ++t)
            L.w_off[t] = w_off[t] + (row0[t] + r) * (K / 2u) + 16u * ((lane & 1u) ^ swzb);
    }
    {
        // window piece q: lane l loads dword l % 4 of row 16 (q & 1) + l / 4
        // of tile q / 2 (G = 32: that dword's offset is folded in here)
        const uint32_t r = lane >> 2, d4 = G == 32 ? 4u * (lane & 3u) : 0u;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            L.s_ld[t] = s_off[t] + (row0[t] + r) * srow + d4;
            L.z_ld[t] = z_off[t] + (row0[t] + r) * srow + d4;
        }
        L.s_q1 = 16u * srow;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        L.s_own[t] = s_off[t] + (row0[t] + m) * srow;
        L.z_own[t] = z_off[t] + (row0[t] + m) * srow;
    }

    // activation load i of wave w is load j = w + 4 i: rows 8 j + l / 8,
    // lane l bringing the piece stored in slot l % 8; rows past the pass
    // repeat row 0
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const uint32_t j = L.wave + 4u * (uint32_t)i;
        uint32_t row = 8u * j + (lane >> 3);
        row = row < rows ? row : 0u;
        const uint32_t piece = (lane & 7u) ^ (lane >> 3) ^ (j & 1u);
        const uint32_t src = MODE == 0 ? args.pairs[blk.pair_start + row].token * args.a_stride
                                       : (blk.local_row + row) * args.a_stride;
        L.a_off[i] = (src + piece * 8u) * 2u;
    }
    const uint32_t base = lds_addr(smem);
    const uint32_t swz = (m & 7u) ^ ((m >> 3) & 1u);
    // step st reads slot (4h + st) ^ swz: a_rd ^ (st << 4), the LDS base
    // being 128-byte aligned
    L.a_rd = base + m * kGemmKC * 2u + (((h * 4u) ^ swz) << 4);
    const uint32_t swzb_m = ((m >> 2) ^ (m >> 3)) & 1u;
    L.b_rd = base + Y::kBBase + L.wave * kGemmBWave + 32u * m + 16u * (h ^ swzb_m);
    // the lane's row's 16 window bytes; G = 32: half h reads group 2c + h,
    // the second half of the chunk's dword
#pragma unroll
    for (int t = 0; t < 2; ++t)
        L.s_rd[t] = base + Y::kSBase + L.wave * kGemmSWave + (32u * t + m) * 16u + (G == 32 ? 2u * h : 0u);
    if (MODE == 0 && HALF && L.wave >= 2u) {  // waves 2-3 run their up tile in the tile-0 slots
        L.b_rd += kGemmBTile;
        L.s_rd[0] = L.s_rd[1];
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
    gemm_kloop<R, G, SYM, NT, HALF>(L, smem, acc);
    wait_vmcnt<0>();  // no LDS write may land after this point

    // Output: the block's tile goes through LDS (idle now) so
    // that global stores are 16 bytes per lane along output rows.
    // acc[i][t][v] of lane l: row 32 i + 8 (v / 4) + 4 h + v % 4 of the block,
    // weight row n_t (column m of tile t). Rows are padded by 16 bytes so the
    // two half-waves' 2-byte writes (4 rows apart) fall in different banks.
    constexpr uint32_t kCols = MODE == 0 || HALF ? 128u : 256u;  // columns per block
    constexpr uint32_t kStride = kCols + 8u;             // halves per LDS row
    uint16_t* otile = reinterpret_cast<uint16_t*>(smem);
    // down: each row's destination, staged once per block
    uint32_t* odst = reinterpret_cast<uint32_t*>(smem + R * kStride * 2u);
    static_assert(R * kStride * 2u + R * 4u <= Y::kEpi, "output tile and row destinations fit");
    block_barrier();  // every wave is done reading the rings
    // the fused launch's next item index, posted where the epilogue does not
    // write (its atomic is long complete: the loads are drained above)
    static_assert(Y::kEpi <= Y::kWord && Y::kWord + 8u <= Y::bytes(SYM), "the item words are free");
    if (post && threadIdx.x == 0)
        asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(smem + Y::kWord)), "v"(next) : "memory");
    if (MODE == 1 && threadIdx.x < rows) odst[threadIdx.x] = row_dst;
    if (MODE == 2 && threadIdx.x < rows) odst[threadIdx.x] = (blk.local_row + threadIdx.x) * args.d;
    if constexpr (HALF && MODE == 0) {
        // waves 2-3 hand their up accumulators to waves 0-1, past the tile
        constexpr uint32_t kXch = R * kStride * 2u;
        static_assert(kXch + 2u * NT * 16u * 64u * 4u <= Y::kEpi, "exchange fits below the next word");
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
    if (wave_live && (!HALF || MODE != 0 || L.wave < 2u)) {
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
    __syncthreads();  // the scratch may be overwritten from here on
}

// gemm_block with NT = nt slices (1 <= nt <= the pass's slices).
template <int G, bool SYM, int ACT, int MODE, bool HALF, int NT = 1>
__device__ __forceinline__ void gemm_block_nt(uint32_t nt, const GemmArgs& args,
                                              const tsg_routed_block& blk, uint32_t rows,
                                              uint32_t tile, uint8_t* smem, bool post,
                                              uint32_t next) {
    if constexpr ((uint32_t)NT < GemmLds<gemm_rows<MODE>()>::kSlices) {
        if (nt > (uint32_t)NT) {
            gemm_block_nt<G, SYM, ACT, MODE, HALF, NT + 1>(nt, args, blk, rows, tile, smem, post, next);
            return;
        }
    }
    gemm_block<G, SYM, ACT, MODE, NT, HALF>(args, blk, rows, tile, smem, post, next);
}

// One work item: column tile `tile` of routed block blk; a block wider than
// the pass (kGemmRows, or kDenseRows for the dense projection) runs as
// consecutive passes.
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
                asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(smem + next_word<SYM>())), "v"(next) : "memory");
        }
        return;
    }
    constexpr uint32_t R = gemm_rows<MODE>();
    for (uint32_t r0 = 0; r0 < blk.row_count; r0 += R) {
        if (r0) block_barrier();  // every wave is done with the previous pass's LDS
        tsg_routed_block sub = blk;
        sub.pair_start += r0;
        sub.local_row += r0;
        const uint32_t rows = blk.row_count - r0 < R ? blk.row_count - r0 : R;
        const uint32_t nt = (rows + 31u) / 32u;
        // gate/up column tiles hold 128 columns, the last one 64 when F is an
        // odd multiple of 64; dense tiles hold 128 columns when dense_narrow
        const bool half = MODE == 0 ? args.f - tile * 128u <= 64u : MODE == 2 && args.dense_narrow;
        if (half)
            gemm_block_nt<G, SYM, ACT, MODE, MODE != 1>(nt, args, sub, rows, tile, smem, post, next);
        else
            gemm_block_nt<G, SYM, ACT, MODE, false>(nt, args, sub, rows, tile, smem, post, next);
    }
}

// 1-D grid of ntiles x (routed block capacity) workgroups; those past the
// live count exit at once. Two workgroups per CU.
template <int G, bool SYM, int ACT, int MODE>
__global__ __launch_bounds__(kGemmThreads, 2) void moe_gemm_kernel(GemmArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];  // GemmLds<gemm_rows<MODE>()>::bytes(SYM)
    constexpr uint32_t R = gemm_rows<MODE>();
    const uint32_t nb = args.n_blocks_device ? *args.n_blocks_device : args.n_blocks;
    const uint32_t total = nb * args.ntiles;
    if (blockIdx.x >= total) return;
    uint32_t yb, tile;
    // the ranking's scratch is the activation ring, free until the item's
    // first loads (gemm_work_item ends on a barrier after every wave has
    // read the result)
    gemm_work_item(args, nb, blockIdx.x, reinterpret_cast<uint32_t*>(smem), MODE == 2, yb, tile);
    tsg_routed_block blk;
    if (MODE == 2) {  // dense: block yb is rows R yb .. of x, all full but the last
        blk.local_slot = 0;
        blk.pair_start = blk.local_row = yb * R;
        blk.row_count = args.dense_rows - blk.local_row < R ? args.dense_rows - blk.local_row : R;
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
    extern __shared__ __align__(16) uint8_t smem[];  // GemmLds<kGemmRows>::bytes(SYM)
    // item indices travel through schedule word 0, the exit flag word 1
    uint32_t* word = reinterpret_cast<uint32_t*>(smem + next_word<SYM>());
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
    __syncthreads();  // every wave has the index before the first item's loads
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
        item = lds_read_b32(lds_addr(smem + next_word<SYM>()));
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(item));
        item = __builtin_amdgcn_readfirstlane(item);
        lds_barrier();  // every wave has the index before the next item's loads land on it
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

// ------------------------------------------------------------- launchers

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
    constexpr uint32_t lds = GemmLds<gemm_rows<MODE>()>::bytes(SYM);
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, grid, dim3(kGemmThreads), lds, s, args);
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
    constexpr uint32_t lds = GemmLds<kGemmRows>::bytes(SYM);
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    // two workgroups per CU (the GEMM's occupancy), every one of them resident
    const dim3 grid(2u * (uint32_t)ctx->num_cus);
    hipLaunchKernelGGL(kern, grid, dim3(kGemmThreads), lds, s, gu, dn, sc);
    return check_launch("moe_gemm fused gate/up + down");
}

// Dense projection: blocks of kDenseRows (128) rows of x in order, 256
// output columns per workgroup (the down GEMM's tiling).
template <int G, bool SYM>
tsg_status launch_dense_qmm(hipStream_t s, const GemmArgs& a, uint32_t num_cus) {
    GemmArgs args = a;
    args.n_blocks = (a.dense_rows + kDenseRows - 1u) / kDenseRows;
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
    constexpr uint32_t lds = GemmLds<kDenseRows>::bytes(SYM);
    TSG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(args.ntiles * args.n_blocks), dim3(kGemmThreads), lds, s, args);
    return check_launch("moe_gemm dense qmm");
}

}  // namespace

template <int G, bool SYM>
tsg_status routed_gemm_launch(const tsg_moe* moe, hipStream_t s, int mode, const GemmArgs& a,
                              uint32_t max_blocks) {
    return mode == 0 ? launch_gemm<G, SYM, 0>(moe, s, a, max_blocks)
                     : launch_gemm<G, SYM, 1>(moe, s, a, max_blocks);
}

template <int G, bool SYM>
tsg_status routed_gemm_fused_launch(const tsg_moe* moe, hipStream_t s, GemmArgs gu, GemmArgs dn,
                                    uint32_t max_blocks) {
    return launch_fused<G, SYM>(moe, s, gu, dn, max_blocks);
}

template <int G, bool SYM>
tsg_status dense_qmm_launch(hipStream_t s, const GemmArgs& a, uint32_t num_cus) {
    return launch_dense_qmm<G, SYM>(s, a, num_cus);
}

}  // namespace tsg
