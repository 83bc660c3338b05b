// tsg_internal.hpp — shared state, error plumbing and device helpers of the
// gfx950 int4 MoE library. Not part of the public ABI (include/tsugumi_hip.h).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/tsugumi_hip.h"

namespace tsg {

// ------------------------------------------------------------------ errors

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
tsg_status fail(tsg_status status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define TSG_HIP_TRY(expr)                                                        \
    do {                                                                         \
        hipError_t _e = (expr);                                                  \
        if (_e != hipSuccess)                                                    \
            return ::tsg::fail(TSG_ERR_HIP, "%s: %s (%s:%d)", #expr,             \
                               hipGetErrorString(_e), __FILE__, __LINE__);       \
    } while (0)

#define TSG_REQUIRE(cond, status, ...)                                           \
    do {                                                                         \
        if (!(cond)) return ::tsg::fail(status, __VA_ARGS__);                    \
    } while (0)

// Checks the launch just enqueued.
tsg_status check_launch(const char* what);

}  // namespace tsg

// --------------------------------------------------------------- objects

struct tsg_ctx {
    int device = 0;
    uint32_t group_size = 64;             // MetalContext default group
    tsg_affine_scheme scheme = TSG_AFFINE;
    // Device scratch owned by the context: completion counters for the
    // last-block patterns (zeroed once, self-resetting) and router logits.
    uint32_t* counters = nullptr;        // kMaxCounters
    float* logits = nullptr;             // kMaxPromptRows * kMaxExperts
    uint16_t* act_replicas = nullptr;    // kActReplicas * kActReplicaHalves
    uint64_t* verify_words = nullptr;    // kVerifyWords: the one-launch verify layer's hand-offs
    // this device's copy of the no-alloc grouping scratch (a file-scope device
    // array of prefill.hip, not owned: never freed)
    uint32_t* group_rank_scratch = nullptr;
    // the fused grouped GEMM's schedule (queue heads, exit count, per-block
    // gate/up counts; zeroed once, left zeroed by each launch)
    uint32_t* gemm_sched = nullptr;     // kGemmSchedWords
    int num_cus = 256;
    // the fused GEMM's queue count: the device's XCDs (8 on an MI355X in its
    // one-partition mode) when that is a power of two of at most 8, else 0
    // (the fused launch is not used)
    uint32_t gemm_queues = 0;
};

struct tsg_moe {
    tsg_ctx* ctx = nullptr;
    uint32_t router_weight_bits = 16;
    tsg_activation activation = TSG_ACT_GELU_TANH;
    bool unfused_decode = false;  // tsg_moe_set_fused_decode(moe, 0)
};

// One run of bytes of an expert blob: file bytes [file_off, file_off + len)
// of each blob live at device bytes [dev_off, dev_off + len) of that expert.
struct tsg_layer_segment {
    uint64_t file_off, len, dev_off;
};

struct tsg_layer {
    tsg_ctx* ctx = nullptr;
    uint8_t* base = nullptr;
    bool owned = false;
    uint32_t num_experts = 0;
    // The HBM image the kernels read: expert e at base + e * expert_stride,
    // sub-tensors at `offsets`.
    uint64_t expert_stride = 0;
    tsg_expert_offsets offsets{};
    // The layer file's geometry, as the caller gives it and uploads in. Equal
    // to the above unless a sub-tensor of the file is off the kernels'
    // alignment (16 bytes for weights, 4 for scales and biases); then the
    // image is laid out anew, every sub-tensor on 256 bytes, and `segments`
    // maps file bytes to image bytes.
    uint64_t file_stride = 0;
    tsg_expert_offsets file_offsets{};
    uint32_t n_segments = 0;  // 0: the image is the file
    tsg_layer_segment segments[9]{};
};

namespace tsg {

constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kMaxRouterRows = 8;      // MoE.maxRouterRows (verify rows)
constexpr uint32_t kMaxPromptRows = 4096;   // rows one router launch may route
constexpr uint32_t kMaxCounters = 12288;
constexpr uint32_t kMaxGemmQueues = 8;                 // the fused GEMM's per-XCD queues
constexpr uint32_t kGemmSchedBlocks = 65536;             // routed blocks the fused GEMM takes
constexpr uint32_t kGemmSchedWords = 16u + kGemmSchedBlocks;
// Words of ctx->counters used by the one-launch decode layer (below them, words
// [0, kMaxPromptRows / 16) are the router's per-row-group completion
// counters). Each area starts on its own 128-byte line.
constexpr uint32_t kDecodeGroups = 8;      // one expert slot per group
constexpr uint32_t kGroupMembers = 32;     // blocks per group
constexpr uint32_t kDecodeBlocks = kDecodeGroups * kGroupMembers;
constexpr uint32_t kSyncEpochWord = 1024;  // launch epoch
constexpr uint32_t kSyncErrorWord = 1056;  // device-side error bits (kErr*), read by tsg_ctx_synchronize
// Bits of the error word: a one-launch decode layer whose hand-off wait timed
// out; a device grouping that met an expert id >= num_experts (its pairs are
// not grouped); a device grouping whose work list did not fit max_blocks; a
// device-list rows-path block with no rows, more than 8, or an expert past
// the layer (skipped); the fused grouped GEMM's down item that waited too long
// for its block's gate/up tiles, or an XCD queue no workgroup drained; a
// grouped-GEMM block (device list) naming an expert past the layer (skipped);
// the staged router's selector that timed out waiting for a logit; a verify
// layer whose token had fewer than 8 eligible router logits.
constexpr uint32_t kErrDecodeTimeout = 1u;
constexpr uint32_t kErrGroupExpertRange = 2u;
constexpr uint32_t kErrGroupBlocks = 4u;
constexpr uint32_t kErrRowsBlock = 8u;  // a device-list rows-path block it cannot take
constexpr uint32_t kErrGemmWait = 16u;  // the fused GEMM: a wait timed out or a queue not drained
constexpr uint32_t kErrGemmBlock = 32u;  // a grouped-GEMM block names an expert past the layer
constexpr uint32_t kErrRouterWait = 64u;  // the staged router's selector timed out on a logit
constexpr uint32_t kErrVerifyRouting = 128u;  // the verify layer: a token with fewer than 8 eligible logits
constexpr uint32_t kSyncLogitWord = 1088;  // tagged 64-bit logits, kMaxExperts per group
static_assert(kSyncLogitWord + kDecodeGroups * 2 * kMaxExperts <= kMaxCounters, "sync area overflow");
// The staged router's hand-off (rows <= kMaxRouterRows): its launch epoch and
// tagged 64-bit logits, kMaxExperts per row.
constexpr uint32_t kRouterEpochWord = 5248;
constexpr uint32_t kRouterLogitWord = 5376;
static_assert(kRouterEpochWord >= kSyncLogitWord + kDecodeGroups * 2 * kMaxExperts, "router area");
static_assert(kRouterLogitWord + kMaxRouterRows * 2 * kMaxExperts <= kMaxCounters, "router area overflow");
static_assert(kSyncLogitWord % 2 == 0, "64-bit words must be aligned");
// Per-group hand-off regions of the one-launch layer (ctx->act_replicas):
// group g's region holds kHandoffWords tagged 64-bit words, its slot's
// activations in [0, kMaxFusedDim) and its partial down outputs above; a
// ninth region holds the shared expert's activations.
constexpr uint32_t kActReplicas = kDecodeGroups + 1;  // + the shared expert's activations
constexpr uint32_t kActReplicaHalves = 8u * 4096u;
constexpr uint32_t kHandoffWords = kActReplicaHalves / 4u;
constexpr uint32_t kMaxFusedDim = 4096u;  // largest d and f of the one-launch layer
static_assert(2u * kMaxFusedDim <= kHandoffWords, "hand-off region overflow");
constexpr uint32_t kMaxCombineRows = 16;  // output rows one block combines: ceil(ceil(d/32)/8)
constexpr uint32_t kMaxSharedF = 512;     // shared-expert intermediate size of the one-launch layer

constexpr uint32_t kTopK = 8;

// The one-launch verify layer: its launch epoch (a word of ctx->counters past
// the router areas) and its hand-off words (ctx->verify_words, tagged 64-bit):
// per-group replicas of the rows' logits, one arrival word per block, the
// activation rows of the sorted pairs (f words each), the route partials of
// the token-major pairs (d words each) and the shared expert's activation
// rows (f words each).
constexpr uint32_t kVerifyEpochWord = 9600;
static_assert(kVerifyEpochWord >= kRouterLogitWord + kMaxRouterRows * 2 * kMaxExperts &&
                  kVerifyEpochWord < kMaxCounters, "verify epoch word");
constexpr uint32_t kVerifyPairs = kMaxRouterRows * kTopK;  // 64
constexpr uint32_t kVerifyLogitRegion = kMaxRouterRows * kMaxExperts;
constexpr uint32_t kVerifyArriveWord = kDecodeGroups * kVerifyLogitRegion;
constexpr uint32_t kVerifyActWord = kVerifyArriveWord + kDecodeBlocks;
constexpr uint32_t kVerifyPartWord = kVerifyActWord + kVerifyPairs * kMaxFusedDim;
constexpr uint32_t kVerifySharedActWord = kVerifyPartWord + kVerifyPairs * kMaxFusedDim;
constexpr uint32_t kVerifyWords = kVerifySharedActWord + kMaxRouterRows * kMaxFusedDim;

// Pairs (t * k) tsg_prefill_group_pairs_device_noalloc takes: its file-scope
// rank scratch holds one word per pair.
constexpr uint32_t kNoAllocPairs = 65536;
// Looks up this device's address of that scratch (the device current);
// tsg_ctx_create calls it.
tsg_status group_noalloc_setup(tsg_ctx* ctx);

inline hipStream_t as_stream(tsg_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Both supported group sizes are whole numbers of 16-byte chunks (32 nibbles).
inline bool group_ok(uint32_t g) { return g == 32 || g == 64; }

// ------------------------------------------------------------ device code

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16v_t __attribute__((ext_vector_type(16)));

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal hint: weights are read once per launch).
__device__ __forceinline__ uint4 load16_nt(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes at an address that is only 2-byte aligned (the reference's
// contract for packed weights, DequantInt4GEMV.swift:93-96): four dwords when
// the address is 4-byte aligned, else a 16-bit load at each end and the three
// aligned dwords between. No byte outside [p, p + 16) is read, so the first
// and last chunk of a buffer stay inside it.
__device__ __forceinline__ uint4 load16_a2(const void* ptr) {
    const uint8_t* p = static_cast<const uint8_t*>(ptr);
    if ((reinterpret_cast<uintptr_t>(p) & 2u) == 0) {
        typedef uint32_t u32x4a4_t __attribute__((ext_vector_type(4), aligned(4)));
        const u32x4a4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4_t*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p + 2);
    const uint32_t a = h[0], e = h[7];
    const uint32_t b = q[0], c = q[1], d = q[2];
    return make_uint4(a | (b << 16), (b >> 16) | (c << 16), (c >> 16) | (d << 16),
                      (d >> 16) | (e << 16));
}

// The weight load of the GEMV lanes: WA = 16 for 16-byte aligned chunks, 2
// for chunks that are only 2-byte aligned.
template <int WA>
__device__ __forceinline__ uint4 load_weights16(const void* p) {
    if constexpr (WA == 16) return load16_nt(p);
    else return load16_a2(p);
}

// A pointer read from LDS (or built from an integer) is generic: the compiler
// emits flat instructions for it, which also count against the LDS counter.
// Rebuilding it as a global-address-space pointer gives global loads and
// stores with scalar bases.
template <typename T>
__device__ __forceinline__ T* global_ptr(T* p) {
    typedef __attribute__((address_space(1))) T global_t;
    return (T*)(global_t*)(uintptr_t)p;
}

// Agent-coherent accesses for the few values the blocks of one launch hand to
// each other (router logits, the top-k, phase-1 activations). A relaxed
// agent-scope atomic compiles to a plain load/store with the sc1 bit, which
// is coherent across the XCDs' separate L2 caches without a cache-wide
// writeback or invalidate.
template <typename T>
__device__ __forceinline__ T ld_coherent(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_coherent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_coherent16(const void* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = ld_coherent(q), hi = ld_coherent(q + 1);
    return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}
// Workgroup barrier for data exchanged through LDS only: this wave's LDS
// operations complete, then s_barrier. Unlike __syncthreads() it does not
// wait for the wave's outstanding global stores (its release fence would).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
// Blocks until this wave's outstanding vector memory operations (coherent
// stores included) have completed; also a compiler barrier.
__device__ __forceinline__ void wait_vector_memory() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// IEEE round-to-nearest-even float -> fp16 (v_cvt_f16_f32 honours the
// default RNE mode).
// fp32 -> fp16, round to nearest even, of a value already rounded to fp32.
// The empty asm keeps the compiler from folding the fma or multiply that
// produced `f` into the conversion: v_fma_mix{lo,hi}_f16 round the exact
// result once, straight to fp16, where the reference rounds to fp32 first
// and then to fp16; the two differ when the fp32 rounding lands on an fp16
// tie.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Eight packed nibbles (one u32, low nibble = element 0) -> four fp16 pairs in
// "paired" order (e0,e4) (e1,e5) (e2,e6) (e3,e7), each exact: q or q - 8.
// A low nibble of a byte lands in mantissa bits 0-3 under exponent 0x64
// (1024 + q) and `bias` (1024, or 1032 for the symmetric lattice) is
// subtracted; a high nibble lands in bits 4-7 (1024 + 16 q), and one fma
// with 1/16 and -(bias - 960) = -(64 + bias - 1024) leaves the same value.
// The masks live in registers so each extraction is one v_and_or_b32 (a VOP3
// takes no literal here): 13 VALU ops per 8 weights with the four dot2s.
__device__ __forceinline__ void nib8_to_pairs(uint32_t w, h2_t bias, h2_t out[4]) {
    uint32_t m_lo, m_hi, e;
    asm("v_mov_b32 %0, 0x000f000f" : "=v"(m_lo));
    asm("v_mov_b32 %0, 0x00f000f0" : "=v"(m_hi));
    asm("v_mov_b32 %0, 0x64006400" : "=v"(e));
    const h2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t hi_bias = bias - h2_t{(_Float16)960.0f, (_Float16)960.0f};
    const uint32_t w8 = w >> 8;
    out[0] = __builtin_bit_cast(h2_t, (w & m_lo) | e) - bias;
    out[1] = __builtin_elementwise_fma(__builtin_bit_cast(h2_t, (w & m_hi) | e), sixteenth, -hi_bias);
    out[2] = __builtin_bit_cast(h2_t, (w8 & m_lo) | e) - bias;
    out[3] = __builtin_elementwise_fma(__builtin_bit_cast(h2_t, (w8 & m_hi) | e), sixteenth, -hi_bias);
}

// v_dot2_f32_f16: a.x*b.x + a.y*b.y + c with fp32 accumulation.
__device__ __forceinline__ float dot2(h2_t a, h2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

// Dot of one 16-byte weight chunk (32 weights) with 32 activations stored in
// paired order (see nib8_to_pairs) as 16 h2_t.
__device__ __forceinline__ float chunk_dot(uint4 w, const h2_t* xp, h2_t bias) {
    h2_t q[4];
    float acc = 0.0f;
    nib8_to_pairs(w.x, bias, q);
    acc = dot2(q[0], xp[0], acc); acc = dot2(q[1], xp[1], acc);
    acc = dot2(q[2], xp[2], acc); acc = dot2(q[3], xp[3], acc);
    nib8_to_pairs(w.y, bias, q);
    acc = dot2(q[0], xp[4], acc); acc = dot2(q[1], xp[5], acc);
    acc = dot2(q[2], xp[6], acc); acc = dot2(q[3], xp[7], acc);
    nib8_to_pairs(w.z, bias, q);
    acc = dot2(q[0], xp[8], acc); acc = dot2(q[1], xp[9], acc);
    acc = dot2(q[2], xp[10], acc); acc = dot2(q[3], xp[11], acc);
    nib8_to_pairs(w.w, bias, q);
    acc = dot2(q[0], xp[12], acc); acc = dot2(q[1], xp[13], acc);
    acc = dot2(q[2], xp[14], acc); acc = dot2(q[3], xp[15], acc);
    return acc;
}

// The same in two steps, for a chunk used against several activation rows:
// its 16 pairs once (chunk_pairs), then chunk_dot's dot2 sequence per row
// (chunk_dot_pairs), which gives chunk_dot's bits.
__device__ __forceinline__ void chunk_pairs(uint4 w, h2_t bias, h2_t (&q)[16]) {
    nib8_to_pairs(w.x, bias, q);
    nib8_to_pairs(w.y, bias, q + 4);
    nib8_to_pairs(w.z, bias, q + 8);
    nib8_to_pairs(w.w, bias, q + 12);
}
__device__ __forceinline__ float chunk_dot_pairs(const h2_t (&q)[16], const h2_t* xp) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2(q[i], xp[i], acc);
    return acc;
}

// Position of element k (0..7) of an 8-element block in paired order.
__host__ __device__ __forceinline__ uint32_t paired_pos(uint32_t k) {
    return (k & 3u) * 2u + (k >> 2);
}

// gelu_pytorch_tanh with the kernels' clamp (moe.metal:104-111) or SiLU
// (moe.metal:116-118). 0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)) exactly, so
// the GELU takes one exp (v_exp_f32 on a pre-scaled argument) and one
// reciprocal instead of a full tanhf; both are accurate to a few fp32 ulp of
// the (1 + tanh) factor, the precision of the reference's fast-math tanh. The
// SiLU x / (1 + exp(-x)) takes the same exp and reciprocal (a few fp32 ulp, as
// the reference's fast-math exp and division) instead of expf and an IEEE
// division. Every path that applies the routed experts' activation (decode,
// the rows path, the grouped GEMM) calls this function, so they agree bit for
// bit; the Qwen shared expert's SiLU (qwen.metal) is qwen_silu.
template <int ACT>
__device__ __forceinline__ float gate_activation(float x) {
    if constexpr (ACT == TSG_ACT_SILU) {
        return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    } else {
        const float x3 = x * x * x;
        float inner = 0.7978845608028654f * (x + 0.044715f * x3);
        inner = fminf(fmaxf(inner, -20.0f), 20.0f);
        return x * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * inner));
    }
}

// LDS layout of staged activations: each 32-element chunk (the span of one
// 16-byte weight chunk) occupies kChunkLds halves = 80 bytes, its four
// 8-element blocks in "paired" order (see nib8_to_pairs). The 16-byte pad
// spreads the chunks that neighbouring lanes read over distinct LDS banks.
constexpr uint32_t kChunkLds = 40;

__host__ __device__ __forceinline__ uint32_t lds_chunks_halves(uint32_t n) {
    return (n / 32u) * kChunkLds;
}

// 8 fp16 (one uint4, elements e0..e7) -> paired order (e0,e4)(e1,e5)(e2,e6)(e3,e7).
__device__ __forceinline__ uint4 pair_permute(uint4 v) {
    uint4 o;
    o.x = (v.x & 0xFFFFu) | (v.z << 16);
    o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    o.z = (v.y & 0xFFFFu) | (v.w << 16);
    o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    return o;
}

// The fp32 sum of each 32-element chunk of `rows` staged rows, in element
// order, into sums[r * n/32 + c] (the affine scheme's bias term). The staged
// rows must be visible to the block (the caller synchronises before).
__device__ __forceinline__ void staged_chunk_sums(const uint16_t* dst, uint32_t dst_stride,
                                                  uint32_t rows, uint32_t n, float* sums) {
    const uint32_t cpr = n / 32u;
    for (uint32_t q = threadIdx.x; q < rows * cpr; q += blockDim.x) {
        const uint32_t r = q / cpr, c = q - r * cpr;
        const uint16_t* chunk = dst + (size_t)r * dst_stride + c * kChunkLds;
        float s = 0.0f;
        for (uint32_t k = 0; k < 32u; ++k)
            s += f16_to_f32(chunk[(k >> 3) * 8u + paired_pos(k & 7u)]);
        sums[q] = s;
    }
}

// Stage `rows` activation rows of `n` fp16 each (row r at src + r*src_stride)
// into LDS at dst + r*dst_stride halves, padded chunk layout. Every global load
// a thread makes in one pass is issued before any of its LDS stores
// (out-of-range slots load a clamped address and store nothing), so staging
// costs one memory round trip per pass, not one per loop iteration. For the
// affine scheme the fp32 sum of each 32-element chunk is then computed from
// the staged copy, in element order, into sums[r * n/32 + c]. The caller
// synchronises before reading.
// `row_index` (may be NULL) maps staged row r to source row row_index[r].
// COHERENT reads the source with agent-coherent loads (data written earlier
// in the same launch by other blocks).
// One staging pass split in two, for callers that issue other loads in
// between: the pass's global loads of units q0 .. q0 + blockDim * PT (of
// `total`, bpr units of 8 halves per row) into v, then their LDS stores.
// Loads complete in issue order, so a store that waits for v waits for
// nothing issued after the pass's loads. NT: the block size when the caller
// knows it at compile time (reading blockDim is a kernel-argument load of its
// own), 0 for blockDim.x.
template <uint32_t NT>
__device__ __forceinline__ uint32_t block_threads() {
    if constexpr (NT != 0) return NT;
    else return blockDim.x;
}
template <int PT, bool COHERENT = false, uint32_t NT = 0>
__device__ __forceinline__ void stage_act_load(const uint16_t* __restrict__ src,
                                               uint32_t src_stride, uint32_t total, uint32_t bpr,
                                               uint32_t q0, const uint32_t* row_index,
                                               uint4 (&v)[PT]) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        // plain loads clamp (a repeated unit is a cache hit and keeps the
        // loads branch-free); coherent loads skip: each is a memory-side
        // access, and repeats of one unit would all queue on one line
        const uint32_t q_raw = q0 + threadIdx.x + i * block_threads<NT>();
        const uint32_t q = min(q_raw, total - 1u);
        const uint32_t r = q / bpr, b = q - r * bpr;
        const uint32_t sr = row_index ? row_index[r] : r;
        const uint16_t* sp = src + (uint64_t)sr * src_stride + b * 8u;
        if constexpr (COHERENT) v[i] = q_raw < total ? ld_coherent16(sp) : make_uint4(0, 0, 0, 0);
        else v[i] = *reinterpret_cast<const uint4*>(sp);
    }
}
template <int PT, uint32_t NT = 0>
__device__ __forceinline__ void stage_act_store(uint32_t total, uint32_t bpr, uint32_t q0,
                                                uint16_t* dst, uint32_t dst_stride,
                                                const uint4 (&v)[PT]) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const uint32_t q = q0 + threadIdx.x + i * block_threads<NT>();
        if (q < total) {
            const uint32_t r = q / bpr, b = q - r * bpr;
            *reinterpret_cast<uint4*>(dst + (size_t)r * dst_stride + (b >> 2) * kChunkLds +
                                      (b & 3u) * 8u) = pair_permute(v[i]);
        }
    }
}

template <bool SYM, int PER_THREAD = 4, bool COHERENT = false>
__device__ __forceinline__ void stage_act_rows(const uint16_t* __restrict__ src,
                                               uint32_t src_stride, uint32_t rows, uint32_t n,
                                               uint16_t* dst, uint32_t dst_stride,
                                               float* sums,
                                               const uint32_t* row_index = nullptr) {
    const uint32_t bpr = n / 8u;
    const uint32_t total = rows * bpr;
    for (uint32_t q0 = 0; q0 < total; q0 += blockDim.x * PER_THREAD) {
        uint4 v[PER_THREAD];
        stage_act_load<PER_THREAD, COHERENT>(src, src_stride, total, bpr, q0, row_index, v);
        stage_act_store<PER_THREAD>(total, bpr, q0, dst, dst_stride, v);
    }
    if constexpr (!SYM) {
        __syncthreads();
        staged_chunk_sums(dst, dst_stride, rows, n, sums);
    }
}

// stage_act_rows with other loads issued between the first pass's loads and
// its LDS stores: `between()` issues them (the GEMV's weight batch). Loads
// complete in issue order, so the stores wait for the activation rows only
// and the weights stream in while the stores and the first chunks run;
// issued the other way round, the stores would wait for every weight.
template <bool SYM, class Between, int PER_THREAD = 4, uint32_t NT = 0>
__device__ __forceinline__ void stage_act_rows_around(const uint16_t* __restrict__ src,
                                                      uint32_t src_stride, uint32_t rows,
                                                      uint32_t n, uint16_t* dst,
                                                      uint32_t dst_stride, float* sums,
                                                      const uint32_t* row_index,
                                                      Between&& between) {
    const uint32_t bpr = n / 8u;
    const uint32_t total = rows * bpr;
    if (total == 0u) {  // nothing to stage (and no unit to clamp to)
        between();
        return;
    }
    uint4 v[PER_THREAD];
    stage_act_load<PER_THREAD, false, NT>(src, src_stride, total, bpr, 0u, row_index, v);
    between();
    stage_act_store<PER_THREAD, NT>(total, bpr, 0u, dst, dst_stride, v);
    const uint32_t pass = block_threads<NT>() * PER_THREAD;
    for (uint32_t q0 = pass; q0 < total; q0 += pass) {
        stage_act_load<PER_THREAD, false, NT>(src, src_stride, total, bpr, q0, row_index, v);
        stage_act_store<PER_THREAD, NT>(total, bpr, q0, dst, dst_stride, v);
    }
    if constexpr (!SYM) {
        __syncthreads();
        staged_chunk_sums(dst, dst_stride, rows, n, sums);
    }
}

// Activations of chunk c in the staged layout.
__device__ __forceinline__ const h2_t* staged_chunk(const uint16_t* xs, uint32_t c) {
    return reinterpret_cast<const h2_t*>(xs + c * kChunkLds);
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// Cross-lane sums on DPP moves (VALU; no LDS round trip). Lanes form aligned
// groups of 8 (16); afterwards every lane of a group holds the group's sum,
// added as pairs (i, i^1), then pairs of pairs (i, i^2), then quads mirrored
// within the 8 (i, 7-i) [, then 8s mirrored within the 16 (i, 15-i)]. Every
// lane ends with the same value since each step adds two equal-for-the-pair
// operands in either order.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    return v;
}
__device__ __forceinline__ float group16_sum(float v) {
    v = group8_sum(v);
    v += dpp_f32<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float lane_value(float v, uint32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace tsg
