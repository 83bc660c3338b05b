// tsg_internal.hpp — shared state, error plumbing and device helpers of the
// gfx950 int4 MoE library. Not part of the public ABI (include/tsugumi_hip.h).
#pragma once

#include <hip/hip_runtime.h>

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
    float* logits = nullptr;             // kMaxRouterRows * kMaxExperts
    int num_cus = 256;
};

struct tsg_moe {
    tsg_ctx* ctx = nullptr;
    uint32_t router_weight_bits = 16;
    tsg_activation activation = TSG_ACT_GELU_TANH;
};

struct tsg_layer {
    tsg_ctx* ctx = nullptr;
    uint8_t* base = nullptr;
    bool owned = false;
    uint32_t num_experts = 0;
    uint64_t expert_stride = 0;
    tsg_expert_offsets offsets{};
};

namespace tsg {

constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kMaxRouterRows = 8;
constexpr uint32_t kMaxCounters = 4096;
constexpr uint32_t kTopK = 8;

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

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// IEEE round-to-nearest-even float -> fp16 (v_cvt_f16_f32 honours the
// default RNE mode).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Eight packed nibbles (one u32, low nibble = element 0) -> four fp16 pairs in
// "paired" order (e0,e4) (e1,e5) (e2,e6) (e3,e7). Each 16-bit half gets
// 0x6400 | q = 1024 + q exactly; subtracting `bias` (1024, or 1032 for the
// symmetric lattice) leaves q or q - 8, both exact in fp16.
__device__ __forceinline__ void nib8_to_pairs(uint32_t w, h2_t bias, h2_t out[4]) {
    const uint32_t m = 0x000F000Fu, e = 0x64006400u;
    out[0] = __builtin_bit_cast(h2_t, (w & m) | e) - bias;
    out[1] = __builtin_bit_cast(h2_t, ((w >> 4) & m) | e) - bias;
    out[2] = __builtin_bit_cast(h2_t, ((w >> 8) & m) | e) - bias;
    out[3] = __builtin_bit_cast(h2_t, ((w >> 12) & m) | e) - bias;
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

// Position of element k (0..7) of an 8-element block in paired order.
__host__ __device__ __forceinline__ uint32_t paired_pos(uint32_t k) {
    return (k & 3u) * 2u + (k >> 2);
}

// gelu_pytorch_tanh with the kernels' clamp (moe.metal:105-112) or SiLU
// (moe.metal:116-118).
template <int ACT>
__device__ __forceinline__ float gate_activation(float x) {
    if constexpr (ACT == TSG_ACT_SILU) {
        return x / (1.0f + expf(-x));
    } else {
        const float x3 = x * x * x;
        float inner = 0.7978845608028654f * (x + 0.044715f * x3);
        inner = fminf(fmaxf(inner, -20.0f), 20.0f);
        return 0.5f * x * (1.0f + tanhf(inner));
    }
}

// Stage `n` fp16 activations into LDS in paired order (see nib8_to_pairs),
// plus, for the affine scheme, the fp32 sum of each 32-element chunk.
template <bool SYM>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, uint32_t n,
                                        uint16_t* xs, float* xsum) {
    for (uint32_t b = threadIdx.x; b < n / 8u; b += blockDim.x) {
        const uint4 v = *reinterpret_cast<const uint4*>(x + b * 8u);
        // in: e0 e1 | e2 e3 | e4 e5 | e6 e7 ; out: (e0,e4) (e1,e5) (e2,e6) (e3,e7)
        uint4 o;
        o.x = (v.x & 0xFFFFu) | (v.z << 16);
        o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
        o.z = (v.y & 0xFFFFu) | (v.w << 16);
        o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
        *reinterpret_cast<uint4*>(xs + b * 8u) = o;
    }
    if constexpr (!SYM) {
        for (uint32_t c = threadIdx.x; c < n / 32u; c += blockDim.x) {
            float s = 0.0f;
            for (uint32_t k = 0; k < 32u; ++k) s += f16_to_f32(x[c * 32u + k]);
            xsum[c] = s;
        }
    }
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

}  // namespace tsg
