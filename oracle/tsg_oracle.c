/*
 * tsg_oracle.c — CPU restatement of the reference's int4 MoE path.
 *
 * TEST INFRASTRUCTURE ONLY (see tsg_oracle.h). Build flags matter:
 * -O2 -ffp-contract=off -fno-fast-math, so every float expression below is
 * rounded operation by operation, the way the Swift originals evaluate them.
 */
#include "tsg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void tsgo_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int tsgo_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------------ */
/* PRNG — TsugumiValidation/Support/PRNG/SplitMix64.swift:11-24,            */
/*        SeedTree.swift:12-19                                              */
/* ------------------------------------------------------------------------ */

uint64_t tsgo_splitmix64_next(uint64_t* state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t tsgo_fnv1a64(const char* label) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (const unsigned char* p = (const unsigned char*)label; *p; ++p) {
        h ^= (uint64_t)*p;
        h *= 0x100000001B3ull;
    }
    return h;
}

uint64_t tsgo_seedtree_key(uint64_t root, const char* label) {
    return root ^ tsgo_fnv1a64(label);
}

/* SplitMix64.swift:40-43: Float(next() >> 40) / Float(1 << 24), then
 * lo + (hi - lo) * u, each operation rounded to Float. */
float tsgo_uniform(uint64_t* state, float lo, float hi) {
    const float u = (float)(tsgo_splitmix64_next(state) >> 40) / (float)(1 << 24);
    const float span = hi - lo;
    const float scaled = span * u;
    return lo + scaled;
}

void tsgo_fill_uniform(uint64_t* state, float lo, float hi, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tsgo_uniform(state, lo, hi);
}

void tsgo_fill_uniform_f16(uint64_t* state, float lo, float hi, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tsgo_f16_bits(tsgo_uniform(state, lo, hi));
}

void tsgo_fill_uniform_bf16(uint64_t* state, float lo, float hi, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tsgo_bf16_bits(tsgo_uniform(state, lo, hi));
}

/* ------------------------------------------------------------------------ */
/* Conversions — Quantization.swift:70-82 (bf16), Swift Float16(Float) RNE  */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Quantization.swift:70-77: round-half-to-even on the top 16 bits, no NaN
 * special case. */
uint16_t tsgo_bf16_bits(float x) {
    const uint32_t bits = f2u(x);
    const uint32_t lsb = (bits >> 16) & 1u;
    const uint32_t rounding_bias = 0x7FFFu + lsb;
    return (uint16_t)((bits + rounding_bias) >> 16);
}

float tsgo_bf16_to_float(uint16_t bits) { return u2f((uint32_t)bits << 16); }

/* MoEPackAffineV1.swift:20-25. */
uint16_t tsgo_sym_bias_bits(uint16_t scale_bits) {
    const float value = tsgo_bf16_to_float(scale_bits) * -8.0f;
    return tsgo_bf16_bits(value);
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to infinity,
 * gradual underflow. */
uint16_t tsgo_f16_bits(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - e;
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float tsgo_f16_to_float(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in fp32 */
        int e = -1;
        do { man <<= 1; e++; } while ((man & 0x400u) == 0);
        man &= 0x3FFu;
        return u2f(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

void tsgo_f16_to_float_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tsgo_f16_to_float(in[i]);
}

void tsgo_float_to_f16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tsgo_f16_bits(in[i]);
}

static inline float f16r(float x) { return tsgo_f16_to_float(tsgo_f16_bits(x)); }

/* ------------------------------------------------------------------------ */
/* int4 quantisation — Quantization.swift:104-227                           */
/* ------------------------------------------------------------------------ */

static inline void put_nibble(uint8_t* packed, int byte_idx, int k, int q) {
    const uint8_t nibble = (uint8_t)(q & 0x0F);
    if ((k & 1) == 0) packed[byte_idx] = (uint8_t)((packed[byte_idx] & 0xF0) | nibble);
    else packed[byte_idx] = (uint8_t)((packed[byte_idx] & 0x0F) | (nibble << 4));
}

/* Swift `Float.rounded()` is schoolbook rounding (ties away from zero) ==
 * C roundf. `Int(...)` then truncates an already-integral value. */
static inline int swift_round_to_int(float v) { return (int)roundf(v); }

static void quantize_row_affine(const float* row, int n, int group, uint8_t* packed,
                                uint16_t* scales, uint16_t* biases) {
    const int n_groups = n / group;
    memset(packed, 0, (size_t)n / 2);
    for (int g = 0; g < n_groups; ++g) {
        float wmin = INFINITY, wmax = -INFINITY;
        for (int k = 0; k < group; ++k) {
            const float w = row[g * group + k];
            if (w < wmin) wmin = w;
            if (w > wmax) wmax = w;
        }
        float scale_f, bias_f;
        if (wmax == wmin) { scale_f = 1.0f; bias_f = wmin; }
        else { scale_f = (wmax - wmin) / 15.0f; bias_f = wmin; }
        const uint16_t s_bits = tsgo_bf16_bits(scale_f);
        const uint16_t b_bits = tsgo_bf16_bits(bias_f);
        scales[g] = s_bits;
        biases[g] = b_bits;
        const float scale = tsgo_bf16_to_float(s_bits);
        const float bias = tsgo_bf16_to_float(b_bits);
        const float inv_scale = scale == 0.0f ? 0.0f : 1.0f / scale;
        for (int k = 0; k < group; ++k) {
            const float w = row[g * group + k];
            const float centred = w - bias;
            int q = swift_round_to_int(centred * inv_scale);
            q = q < 0 ? 0 : (q > 15 ? 15 : q);
            put_nibble(packed, g * (group / 2) + k / 2, k, q);
        }
    }
}

static void quantize_row_sym(const float* row, int n, int group, uint8_t* packed,
                             uint16_t* scales, uint16_t* biases) {
    const int n_groups = n / group;
    memset(packed, 0, (size_t)n / 2);
    for (int g = 0; g < n_groups; ++g) {
        float wmin = INFINITY, wmax = -INFINITY;
        for (int k = 0; k < group; ++k) {
            const float w = row[g * group + k];
            if (w < wmin) wmin = w;
            if (w > wmax) wmax = w;
        }
        const float lo = -wmin / 8.0f;
        const float hi = wmax / 7.0f;
        float scale_f = lo > hi ? lo : hi;
        if (!(scale_f >= 1.17549435e-38f)) scale_f = 1.17549435e-38f; /* Float.leastNormalMagnitude */
        const uint16_t s_bits = tsgo_bf16_bits(scale_f);
        scales[g] = s_bits;
        biases[g] = tsgo_sym_bias_bits(s_bits);
        const float scale = tsgo_bf16_to_float(s_bits);
        const float inv_scale = scale == 0.0f ? 0.0f : 1.0f / scale;
        for (int k = 0; k < group; ++k) {
            const float w = row[g * group + k];
            int q = swift_round_to_int(w * inv_scale) + 8;
            q = q < 0 ? 0 : (q > 15 ? 15 : q);
            put_nibble(packed, g * (group / 2) + k / 2, k, q);
        }
    }
}

void tsgo_quantize_int4(const float* w, int rows, int n, int group, int symmetric,
                        uint8_t* packed, uint16_t* scales, uint16_t* biases) {
    const int n_groups = n / group;
    for (int r = 0; r < rows; ++r) {
        if (symmetric)
            quantize_row_sym(w + (size_t)r * n, n, group, packed + (size_t)r * (n / 2),
                             scales + (size_t)r * n_groups, biases + (size_t)r * n_groups);
        else
            quantize_row_affine(w + (size_t)r * n, n, group, packed + (size_t)r * (n / 2),
                                scales + (size_t)r * n_groups, biases + (size_t)r * n_groups);
    }
}

/* Quantization.swift:210-227: Float(nibble) * scale + bias, two roundings. */
static inline float group_bias(const uint16_t* b_row, int g, float scale) {
    if (b_row == NULL) return -8.0f * scale;
    return tsgo_bf16_to_float(b_row[g]);
}

static void dequant_row(const uint8_t* packed, const uint16_t* s_row, const uint16_t* b_row,
                        int n, int group, float* out) {
    const int n_groups = n / group;
    for (int g = 0; g < n_groups; ++g) {
        const float scale = tsgo_bf16_to_float(s_row[g]);
        const float bias = group_bias(b_row, g, scale);
        for (int k = 0; k < group; ++k) {
            const uint8_t b = packed[g * (group / 2) + k / 2];
            const int nibble = (k & 1) == 0 ? (b & 0x0F) : (b >> 4);
            const float prod = (float)nibble * scale;
            out[g * group + k] = prod + bias;
        }
    }
}

void tsgo_dequantize_int4(const uint8_t* packed, const uint16_t* scales,
                          const uint16_t* biases, int rows, int n, int group, float* out) {
    const int n_groups = n / group;
    for (int r = 0; r < rows; ++r)
        dequant_row(packed + (size_t)r * (n / 2), scales + (size_t)r * n_groups,
                    biases ? biases + (size_t)r * n_groups : NULL, n, group,
                    out + (size_t)r * n);
}

/* prefill.metal:1021-1026: lo = fma(float(q), scale, bias); Bs = half(lo). */
void tsgo_dequantize_int4_f16(const uint8_t* packed, const uint16_t* scales,
                              const uint16_t* biases, int rows, int n, int group,
                              int symmetric, uint16_t* out) {
    const int n_groups = n / group;
    for (int r = 0; r < rows; ++r) {
        const uint8_t* p = packed + (size_t)r * (n / 2);
        const uint16_t* s_row = scales + (size_t)r * n_groups;
        const uint16_t* b_row = symmetric ? NULL : biases + (size_t)r * n_groups;
        for (int g = 0; g < n_groups; ++g) {
            const float scale = tsgo_bf16_to_float(s_row[g]);
            const float bias = group_bias(b_row, g, scale);
            for (int k = 0; k < group; ++k) {
                const uint8_t b = p[g * (group / 2) + k / 2];
                const int q = (k & 1) == 0 ? (b & 0x0F) : (b >> 4);
                out[(size_t)r * n + g * group + k] = tsgo_f16_bits(fmaf((float)q, scale, bias));
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV / FFN — Reference/Quant/DequantInt4Gemv.swift:12-44,                */
/*              Reference/MoE/Moe.swift:16-123                              */
/* ------------------------------------------------------------------------ */

/* vDSP_dotpr's internal order is unspecified (Accelerate is closed); this
 * restatement sums left to right in fp32. The timed build (TSGO_TIMED_DOT,
 * the CPU baseline only, never a checker) keeps eight interleaved partial
 * sums added pairwise at the end, an order a compiler can vectorize the way
 * vDSP is vectorized. */
static inline float dot_f32(const float* a, const float* b, int n) {
#ifdef TSGO_TIMED_DOT
    float part[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; ++k) part[k] = part[k] + a[i + k] * b[i + k];
    for (; i < n; ++i) part[i & 7] = part[i & 7] + a[i] * b[i];
    return ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
#else
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float p = a[i] * b[i];
        acc = acc + p;
    }
    return acc;
#endif
}

void tsgo_dequant_int4_gemv_ref(const uint8_t* packed, const uint16_t* scales,
                                const uint16_t* biases, const float* x,
                                int m, int n, int group, float* y) {
    const int n_groups = n / group;
#pragma omp parallel num_threads(g_threads)
    {
        float* w_row = (float*)malloc(sizeof(float) * (size_t)n);
#pragma omp for schedule(static)
        for (int row = 0; row < m; ++row) {
            dequant_row(packed + (size_t)row * (n / 2), scales + (size_t)row * n_groups,
                        biases ? biases + (size_t)row * n_groups : NULL, n, group, w_row);
            y[row] = dot_f32(w_row, x, n);
        }
        free(w_row);
    }
}

/* Moe.swift:21-29 (no clamp: tanh saturates on its own). */
float tsgo_gelu_tanh(float x) {
    const float cubic = 0.044715f * x * x * x;
    const float inner = 0.7978845608028654f * (x + cubic);
    const float half_x = 0.5f * x;
    return half_x * (1.0f + tanhf(inner));
}

/* moe.metal:117: x / (1 + exp(-x)). */
float tsgo_silu(float x) { return x / (1.0f + expf(-x)); }

/* utility.metal:7-18 (gelu_mul_fp16): out = half(gelu_tanh(float(g)) *
 * float(u)). The kernel's +-20 clamp changes nothing in fp32 (tanh(20)
 * rounds to 1). */
void tsgo_gelu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i)
        out[i] = tsgo_f16_bits(tsgo_gelu_tanh(tsgo_f16_to_float(gate[i])) * tsgo_f16_to_float(up[i]));
}

/* SharedExpertInt4.encode (Kernels/MoE/SharedExpertInt4.swift:30-93) over
 * DequantInt4GemvRef: g = half(gate x), u = half(up x) (f rows of d),
 * a = gelu_mul(g, u), y = half(down a) (d rows of f). Biases NULL = sym. */
void tsgo_dense_mlp_int4(const uint8_t* gw, const uint16_t* gs, const uint16_t* gb,
                         const uint8_t* uw, const uint16_t* us, const uint16_t* ub,
                         const uint8_t* dw, const uint16_t* ds, const uint16_t* db,
                         const uint16_t* x_f16, int d, int f, int group, uint16_t* y_f16) {
    float* x = (float*)malloc(sizeof(float) * (size_t)d);
    float* g = (float*)malloc(sizeof(float) * (size_t)f);
    float* u = (float*)malloc(sizeof(float) * (size_t)f);
    float* a = (float*)malloc(sizeof(float) * (size_t)f);
    float* y = (float*)malloc(sizeof(float) * (size_t)d);
    uint16_t* g16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    uint16_t* u16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    uint16_t* a16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    tsgo_f16_to_float_n(x_f16, x, (size_t)d);
    tsgo_dequant_int4_gemv_ref(gw, gs, gb, x, f, d, group, g);
    tsgo_dequant_int4_gemv_ref(uw, us, ub, x, f, d, group, u);
    tsgo_float_to_f16_n(g, g16, (size_t)f);
    tsgo_float_to_f16_n(u, u16, (size_t)f);
    tsgo_gelu_mul_f16(g16, u16, a16, f);
    tsgo_f16_to_float_n(a16, a, (size_t)f);
    tsgo_dequant_int4_gemv_ref(dw, ds, db, a, d, f, group, y);
    tsgo_float_to_f16_n(y, y_f16, (size_t)d);
    free(x); free(g); free(u); free(a); free(y); free(g16); free(u16); free(a16);
}

/* ------------------------------------------------ Qwen shared expert ---- */

/* qwen.metal:33 (qwen_sigmoid): 1 / (1 + exp(-x)). */
float tsgo_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* qwen.metal:466 (qwen_silu_mul): out = half(silu(float(g)) * float(u)) with
 * silu(x) = x * sigmoid(x) (qwen.metal:34). */
void tsgo_silu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i) {
        const float g = tsgo_f16_to_float(gate[i]);
        out[i] = tsgo_f16_bits(g * tsgo_sigmoid(g) * tsgo_f16_to_float(up[i]));
    }
}

/* qwen.metal:432-455 (qwen_moe_shared_gate): logit = sum_i float(x[i]) *
 * float(w[i]); y[i] = half(float(y[i]) * sigmoid(logit)). The kernel sums in
 * fp32 in its hardware reduction order; this sums in double. */
void tsgo_shared_gate_f16(uint16_t* y, const uint16_t* x_f16, const uint16_t* w_bf16, int d) {
    double logit = 0.0;
    for (int i = 0; i < d; ++i)
        logit += (double)tsgo_f16_to_float(x_f16[i]) * (double)tsgo_bf16_to_float(w_bf16[i]);
    const float scale = tsgo_sigmoid((float)logit);
    for (int i = 0; i < d; ++i) y[i] = tsgo_f16_bits(tsgo_f16_to_float(y[i]) * scale);
}

/* QwenForwardRunner.encodeSharedExpert (QwenForwardRunner.swift:1548-1578)
 * over one expert laid out as MoEExpertOffsets (MoE.swift:4-29): each
 * projection is DequantInt4GemvRef (fp32 rows, fp32 dot) stored as fp16 the
 * way the GEMV stores y (DequantInt4GEMV.swift:78-121); act =
 * qwen_silu_mul(gate, up); out = qwen_moe_shared_gate(down(act)). */
void tsgo_shared_expert(const uint8_t* blob, const uint32_t* o, const uint16_t* x_f16,
                        const uint16_t* gate_w_bf16, int d, int f, int group, int symmetric,
                        uint16_t* out_f16) {
    float* x = (float*)malloc(sizeof(float) * (size_t)d);
    float* g = (float*)malloc(sizeof(float) * (size_t)f);
    float* u = (float*)malloc(sizeof(float) * (size_t)f);
    float* a = (float*)malloc(sizeof(float) * (size_t)f);
    float* dn = (float*)malloc(sizeof(float) * (size_t)d);
    uint16_t* g16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    uint16_t* u16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    uint16_t* a16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)f);
    tsgo_f16_to_float_n(x_f16, x, (size_t)d);
    tsgo_dequant_int4_gemv_ref(blob + o[0], (const uint16_t*)(blob + o[1]),
                               symmetric ? NULL : (const uint16_t*)(blob + o[2]), x, f, d, group, g);
    tsgo_dequant_int4_gemv_ref(blob + o[3], (const uint16_t*)(blob + o[4]),
                               symmetric ? NULL : (const uint16_t*)(blob + o[5]), x, f, d, group, u);
    tsgo_float_to_f16_n(g, g16, (size_t)f);
    tsgo_float_to_f16_n(u, u16, (size_t)f);
    tsgo_silu_mul_f16(g16, u16, a16, f);
    tsgo_f16_to_float_n(a16, a, (size_t)f);
    tsgo_dequant_int4_gemv_ref(blob + o[6], (const uint16_t*)(blob + o[7]),
                               symmetric ? NULL : (const uint16_t*)(blob + o[8]), a, d, f, group, dn);
    tsgo_float_to_f16_n(dn, out_f16, (size_t)d);
    tsgo_shared_gate_f16(out_f16, x_f16, gate_w_bf16, d);
    free(x); free(g); free(u); free(a); free(dn); free(g16); free(u16); free(a16);
}

static inline float gate_act(float x, int act) {
    return act == 1 ? tsgo_silu(x) : tsgo_gelu_tanh(x);
}

void tsgo_moe_run_ffn(const uint8_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                      const uint8_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                      const uint8_t* down_w, const uint16_t* down_s, const uint16_t* down_b,
                      const float* x, int d, int f, int group, int act, float* out) {
    float* gate_out = (float*)malloc(sizeof(float) * (size_t)f);
    float* up_out = (float*)malloc(sizeof(float) * (size_t)f);
    float* a = (float*)malloc(sizeof(float) * (size_t)f);
    tsgo_dequant_int4_gemv_ref(gate_w, gate_s, gate_b, x, f, d, group, gate_out);
    tsgo_dequant_int4_gemv_ref(up_w, up_s, up_b, x, f, d, group, up_out);
    for (int i = 0; i < f; ++i) a[i] = gate_act(gate_out[i], act) * up_out[i];
    tsgo_dequant_int4_gemv_ref(down_w, down_s, down_b, a, d, f, group, out);
    free(gate_out);
    free(up_out);
    free(a);
}

void tsgo_moe_apply_streamed_routed(const uint8_t* const* blobs, const uint32_t* o,
                                    const float* x, const float* residual,
                                    const float* routing_weights, int top_k,
                                    int d, int f, int group, int symmetric, int act,
                                    float* y) {
    float* out = (float*)malloc(sizeof(float) * (size_t)d);
    memcpy(y, residual, sizeof(float) * (size_t)d);
    for (int slot = 0; slot < top_k; ++slot) {
        const uint8_t* b = blobs[slot];
        tsgo_moe_run_ffn(b + o[0], (const uint16_t*)(b + o[1]),
                         symmetric ? NULL : (const uint16_t*)(b + o[2]),
                         b + o[3], (const uint16_t*)(b + o[4]),
                         symmetric ? NULL : (const uint16_t*)(b + o[5]),
                         b + o[6], (const uint16_t*)(b + o[7]),
                         symmetric ? NULL : (const uint16_t*)(b + o[8]),
                         x, d, f, group, act, out);
        /* Moe.swift:115-118: scaled = out * w (vDSP_vsmul), y = y + scaled. */
        const float w = routing_weights[slot];
        for (int i = 0; i < d; ++i) {
            const float scaled = out[i] * w;
            y[i] = y[i] + scaled;
        }
    }
    free(out);
}

/* ------------------------------------------------------------------------ */
/* Router — TsugumiKernelCheck/main.swift:384-402 and moe.metal:281-329      */
/* ------------------------------------------------------------------------ */

typedef struct { float score; int idx; } scored_t;

static int cmp_scored(const void* a, const void* b) {
    const scored_t* x = (const scored_t*)a;
    const scored_t* y = (const scored_t*)b;
    if (x->score == y->score) return x->idx < y->idx ? -1 : (x->idx > y->idx);
    return x->score > y->score ? -1 : 1;
}

void tsgo_router_reference(const float* w, const float* x, int num_experts, int d,
                           int top_k, const float* per_expert_scale,
                           int32_t* out_idx, float* out_w) {
    scored_t* order = (scored_t*)malloc(sizeof(scored_t) * (size_t)num_experts);
    for (int e = 0; e < num_experts; ++e) {
        float acc = 0.0f;
        for (int i = 0; i < d; ++i) {
            const float p = w[(size_t)e * d + i] * x[i];
            acc = acc + p;
        }
        order[e].score = acc;
        order[e].idx = e;
    }
    qsort(order, (size_t)num_experts, sizeof(scored_t), cmp_scored);
    const float max_score = order[0].score;
    float exps[64];
    float sum = 0.0f;
    for (int i = 0; i < top_k; ++i) {
        exps[i] = expf(order[i].score - max_score);
        sum = sum + exps[i];
    }
    for (int i = 0; i < top_k; ++i) {
        out_idx[i] = order[i].idx;
        const float p = exps[i] / sum;
        out_w[i] = p * per_expert_scale[order[i].idx];
    }
    free(order);
}

void tsgo_router_logits_canonical(const uint16_t* w_bf16, const uint16_t* hidden_f16,
                                  int stride, const uint16_t* es_bf16, int rows,
                                  int num_experts, int d, float* out_logits) {
    const int nchunks = d / 8;
    for (int row = 0; row < rows; ++row) {
        const uint16_t* x = hidden_f16 + (size_t)row * stride;
        for (int e = 0; e < num_experts; ++e) {
            const uint16_t* w = w_bf16 + (size_t)e * d;
            float p[64];
            for (int l = 0; l < 64; ++l) {
                float acc = 0.0f;
                for (int c = l; c < nchunks; c += 64)
                    for (int k = 0; k < 8; ++k) {
                        const int i = c * 8 + k;
                        const float xe = tsgo_f16_to_float(x[i]) * tsgo_bf16_to_float(es_bf16[i]);
                        acc = fmaf(tsgo_bf16_to_float(w[i]), xe, acc);
                    }
                p[l] = acc;
            }
            /* each 16-lane row: pairs (l, l^1), pairs of pairs (l, l^2), the
             * quads of each 8 mirrored (l, 7-l), the 8s of the row mirrored
             * (l, 15-l); then the row sums as (r0 + r1) + (r2 + r3) */
            float r[4];
            for (int k = 0; k < 4; ++k) {
                float* q = p + 16 * k;
                float t[16];
                for (int l = 0; l < 16; ++l) t[l] = q[l] + q[l ^ 1];
                for (int l = 0; l < 16; ++l) q[l] = t[l] + t[l ^ 2];
                for (int l = 0; l < 16; ++l) t[l] = q[l] + q[(l & 8) | (7 - (l & 7))];
                for (int l = 0; l < 16; ++l) q[l] = t[l] + t[15 - l];
                r[k] = q[0];
            }
            out_logits[(size_t)row * num_experts + e] = (r[0] + r[1]) + (r[2] + r[3]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* INT8 affine — Quantization.swift:243-303 (Infrastructure/ModelIO)         */
/* ------------------------------------------------------------------------ */

void tsgo_quantize_int8_affine(const float* w, int rows, int n, int group, uint8_t* packed,
                               uint16_t* scales, uint16_t* biases) {
    const int n_groups = n / group;
    for (int r = 0; r < rows; ++r) {
        const float* row = w + (size_t)r * n;
        for (int g = 0; g < n_groups; ++g) {
            float wmin = INFINITY, wmax = -INFINITY;
            for (int k = 0; k < group; ++k) {
                const float v = row[g * group + k];
                if (v < wmin) wmin = v;
                if (v > wmax) wmax = v;
            }
            const float scale_f = wmax == wmin ? 1.0f : (wmax - wmin) / 255.0f;
            const uint16_t s_bits = tsgo_bf16_bits(scale_f);
            const uint16_t b_bits = tsgo_bf16_bits(wmin);
            scales[(size_t)r * n_groups + g] = s_bits;
            biases[(size_t)r * n_groups + g] = b_bits;
            const float scale = tsgo_bf16_to_float(s_bits);
            const float bias = tsgo_bf16_to_float(b_bits);
            const float inv_scale = scale == 0.0f ? 0.0f : 1.0f / scale;
            for (int k = 0; k < group; ++k) {
                const float centred = row[g * group + k] - bias;
                int q = swift_round_to_int(centred * inv_scale);
                q = q < 0 ? 0 : (q > 255 ? 255 : q);
                packed[(size_t)r * n + g * group + k] = (uint8_t)q;
            }
        }
    }
}

void tsgo_dequantize_int8_affine(const uint8_t* packed, const uint16_t* scales,
                                 const uint16_t* biases, int rows, int n, int group, float* out) {
    const int n_groups = n / group;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < n_groups; ++g) {
            const float scale = tsgo_bf16_to_float(scales[(size_t)r * n_groups + g]);
            const float bias = tsgo_bf16_to_float(biases[(size_t)r * n_groups + g]);
            for (int k = 0; k < group; ++k) {
                const size_t i = (size_t)r * n + g * group + k;
                const float prod = (float)packed[i] * scale;
                out[i] = prod + bias;
            }
        }
}

void tsgo_router_logits_int8_canonical(const uint8_t* w, const uint16_t* scales,
                                       const uint16_t* biases, const uint16_t* hidden_f16,
                                       const uint16_t* es_bf16, int num_experts, int d,
                                       int group, float* out_logits) {
    const int nunits = d / 16, n_groups = d / group;
    for (int e = 0; e < num_experts; ++e) {
        const uint8_t* wr = w + (size_t)e * d;
        float p[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int u = l; u < nunits; u += 64) {
                float qx = 0.0f, sx = 0.0f;
                for (int k = 0; k < 16; ++k) {
                    const int i = u * 16 + k;
                    const float x = tsgo_f16_to_float(hidden_f16[i]) * tsgo_bf16_to_float(es_bf16[i]);
                    qx = fmaf((float)wr[i], x, qx);
                    sx = sx + x;
                }
                const int g = u * 16 / group;
                acc = fmaf(tsgo_bf16_to_float(scales[(size_t)e * n_groups + g]), qx, acc);
                acc = fmaf(tsgo_bf16_to_float(biases[(size_t)e * n_groups + g]), sx, acc);
            }
            p[l] = acc;
        }
        /* the 64 partials as in tsgo_router_logits_canonical */
        float r[4];
        for (int k = 0; k < 4; ++k) {
            float* q = p + 16 * k;
            float t[16];
            for (int l = 0; l < 16; ++l) t[l] = q[l] + q[l ^ 1];
            for (int l = 0; l < 16; ++l) q[l] = t[l] + t[l ^ 2];
            for (int l = 0; l < 16; ++l) t[l] = q[l] + q[(l & 8) | (7 - (l & 7))];
            for (int l = 0; l < 16; ++l) q[l] = t[l] + t[15 - l];
            r[k] = q[0];
        }
        out_logits[e] = (r[0] + r[1]) + (r[2] + r[3]);
    }
}

void tsgo_topk_softmax(const float* logits, int num_experts, int top_k,
                       const float* per_expert_scale, int32_t* out_idx, uint16_t* out_w) {
    int top_idx[64];
    float top_score[64];
    for (int i = 0; i < top_k; ++i) { top_idx[i] = 0; top_score[i] = -INFINITY; }
    for (int e = 0; e < num_experts; ++e) {
        const float s = logits[e];
        if (top_k > 0 && s <= top_score[top_k - 1]) continue;
        int pos = top_k;
        for (int i = 0; i < top_k; ++i) {
            if (s > top_score[i] || (s == top_score[i] && e < top_idx[i])) { pos = i; break; }
        }
        if (pos >= top_k) continue;
        for (int i = top_k - 1; i > pos; --i) { top_idx[i] = top_idx[i - 1]; top_score[i] = top_score[i - 1]; }
        top_idx[pos] = e;
        top_score[pos] = s;
    }
    const float max_s = top_score[0];
    float exps[64];
    float sum_exp = 0.0f;
    for (int i = 0; i < top_k; ++i) {
        exps[i] = expf(top_score[i] - max_s);
        sum_exp += exps[i];
    }
    for (int i = 0; i < top_k; ++i) {
        out_idx[i] = top_idx[i];
        const float weight = exps[i] / sum_exp;
        out_w[i] = tsgo_f16_bits(weight * per_expert_scale[top_idx[i]]);
    }
}

/* ------------------------------------------------------------------------ */
/* Prefill routing — PrefillRouter.swift:238-258,                           */
/*                   PrefillMoEGrouping.swift:90-202,                       */
/*                   PrefillGroupedRoutedMoE.swift:42-83                    */
/* ------------------------------------------------------------------------ */

void tsgo_make_token_expert_pairs(const uint32_t* idx, const uint16_t* w, int t, int top_k,
                                  tsgo_pair* out) {
    for (int token = 0; token < t; ++token)
        for (int rank = 0; rank < top_k; ++rank) {
            const int i = token * top_k + rank;
            out[i].token = (uint32_t)token;
            out[i].expert = idx[i];
            out[i].rank = (uint32_t)rank;
            out[i].weight_bits = (uint32_t)w[i];
        }
}

/* Error codes, one per PrefillMoEGroupingError case (PrefillMoEGrouping.swift:52-62). */
enum {
    TSGO_INVALID_QUERY_COUNT = -1,
    TSGO_INVALID_TOP_K = -2,
    TSGO_INVALID_NUM_EXPERTS = -3,
    TSGO_INVALID_TILE_EXPERT_COUNT = -4,
    TSGO_PAIR_COUNT_MISMATCH = -5,
    TSGO_TOKEN_OUT_OF_RANGE = -6,
    TSGO_RANK_OUT_OF_RANGE = -7,
    TSGO_EXPERT_OUT_OF_RANGE = -8,
    TSGO_DUPLICATE_TOKEN_RANK = -9,
    TSGO_SORT_KEY_COUNT_MISMATCH = -10,
};

static const uint64_t* g_sort_keys;

static int cmp_pair(const void* a, const void* b) {
    const tsgo_pair* x = (const tsgo_pair*)a;
    const tsgo_pair* y = (const tsgo_pair*)b;
    if (g_sort_keys) {
        const uint64_t kx = g_sort_keys[x->expert], ky = g_sort_keys[y->expert];
        if (kx != ky) return kx < ky ? -1 : 1;
    }
    if (x->expert != y->expert) return x->expert < y->expert ? -1 : 1;
    if (x->token != y->token) return x->token < y->token ? -1 : 1;
    if (x->rank != y->rank) return x->rank < y->rank ? -1 : 1;
    return 0;
}

int tsgo_group_pairs(const tsgo_pair* pairs, int n_pairs, int query_count, int top_k,
                     int num_experts, int tile_expert_count,
                     const uint64_t* expert_sort_keys, int n_sort_keys,
                     int tile_break_after_group,
                     tsgo_pair* sorted, uint32_t* offsets, uint32_t* counts,
                     tsgo_group* groups, int* n_groups, tsgo_tile* tiles, int* n_tiles) {
    if (query_count < 0) return TSGO_INVALID_QUERY_COUNT;
    if (top_k <= 0) return TSGO_INVALID_TOP_K;
    if (num_experts <= 0) return TSGO_INVALID_NUM_EXPERTS;
    if (tile_expert_count < 1 || tile_expert_count > 16) return TSGO_INVALID_TILE_EXPERT_COUNT;
    if (expert_sort_keys && n_sort_keys != num_experts) return TSGO_SORT_KEY_COUNT_MISMATCH;
    if (n_pairs != query_count * top_k) return TSGO_PAIR_COUNT_MISMATCH;

    uint8_t* seen = (uint8_t*)calloc((size_t)query_count * (size_t)top_k + 1, 1);
    for (int i = 0; i < n_pairs; ++i) {
        const tsgo_pair p = pairs[i];
        if (p.token >= (uint32_t)query_count) { free(seen); return TSGO_TOKEN_OUT_OF_RANGE; }
        if (p.rank >= (uint32_t)top_k) { free(seen); return TSGO_RANK_OUT_OF_RANGE; }
        if (p.expert >= (uint32_t)num_experts) { free(seen); return TSGO_EXPERT_OUT_OF_RANGE; }
        const size_t key = (size_t)p.token * (size_t)top_k + p.rank;
        if (seen[key]) { free(seen); return TSGO_DUPLICATE_TOKEN_RANK; }
        seen[key] = 1;
    }
    free(seen);

    memcpy(sorted, pairs, sizeof(tsgo_pair) * (size_t)n_pairs);
    g_sort_keys = expert_sort_keys;
    qsort(sorted, (size_t)n_pairs, sizeof(tsgo_pair), cmp_pair);
    g_sort_keys = NULL;

    for (int e = 0; e < num_experts; ++e) { offsets[e] = 0xFFFFFFFFu; counts[e] = 0; }
    int ng = 0;
    int i = 0;
    while (i < n_pairs) {
        const uint32_t expert = sorted[i].expert;
        const int start = i;
        while (i < n_pairs && sorted[i].expert == expert) ++i;
        offsets[expert] = (uint32_t)start;
        counts[expert] = (uint32_t)(i - start);
        groups[ng].expert = expert;
        groups[ng].pair_start = (uint32_t)start;
        groups[ng].pair_count = (uint32_t)(i - start);
        ++ng;
    }
    *n_groups = ng;

    int nt = 0;
    int group_start = 0;
    while (group_start < ng) {
        int group_end = group_start + tile_expert_count;
        if (group_end > ng) group_end = ng;
        if (tile_break_after_group >= 0 && group_start < tile_break_after_group &&
            group_end > tile_break_after_group)
            group_end = tile_break_after_group;
        const tsgo_group first = groups[group_start];
        const tsgo_group last = groups[group_end - 1];
        tiles[nt].group_start = (uint32_t)group_start;
        tiles[nt].group_count = (uint32_t)(group_end - group_start);
        tiles[nt].pair_start = first.pair_start;
        tiles[nt].pair_count = last.pair_start + last.pair_count - first.pair_start;
        ++nt;
        group_start = group_end;
    }
    *n_tiles = nt;
    return 0;
}

int tsgo_plan_routed_gemm(const tsgo_group* groups, int n_groups, int max_rows_per_batch,
                          tsgo_block* blocks, int* n_blocks,
                          int* batch_rows, int* batch_first_block, int* n_batches) {
    const int tile_rows = 64;
    int budget = (max_rows_per_batch / tile_rows) * tile_rows;
    if (budget < tile_rows) budget = tile_rows;
    int nb = 0, nbatch = 0, rows = 0, batch_start_block = 0;
#define FLUSH()                                                   \
    do {                                                          \
        if (rows > 0) {                                           \
            batch_rows[nbatch] = rows;                            \
            batch_first_block[nbatch] = batch_start_block;        \
            ++nbatch;                                             \
            batch_start_block = nb;                               \
            rows = 0;                                             \
        }                                                         \
    } while (0)
    for (int slot = 0; slot < n_groups; ++slot) {
        int taken = 0;
        const int count = (int)groups[slot].pair_count;
        while (taken < count) {
            if (rows == budget) FLUSH();
            if (rows > 0 && rows + (count - taken) > budget) FLUSH();
            int take = count - taken;
            if (take > budget - rows) take = budget - rows;
            int done = 0;
            while (done < take) {
                int rc = take - done;
                if (rc > tile_rows) rc = tile_rows;
                blocks[nb].local_slot = (uint32_t)slot;
                blocks[nb].pair_start = groups[slot].pair_start + (uint32_t)(taken + done);
                blocks[nb].row_count = (uint32_t)rc;
                blocks[nb].local_row = (uint32_t)(rows + done);
                ++nb;
                done += rc;
            }
            rows += take;
            taken += take;
        }
    }
    FLUSH();
#undef FLUSH
    *n_blocks = nb;
    *n_batches = nbatch;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Prefill expert-major reference —                                         */
/*   TsugumiKernelCheck/PrefillMoEGEMMCheck.swift:138-173                   */
/* ------------------------------------------------------------------------ */

void tsgo_prefill_moe_ref(const uint8_t* const* expert_blobs, const uint32_t* o,
                          const uint16_t* hidden, int hidden_stride,
                          const tsgo_pair* sorted_pairs, int n_pairs,
                          int top_k, int d, int f, int group, int symmetric, int act,
                          int rows_path, uint16_t* partials) {
    /* Dequantise each distinct expert once, like the reference's per-expert
     * loop; experts are visited in the order they appear. The threads share
     * one expert at a time (its dequantisation, then its pairs), so a head
     * expert with thousands of rows spreads over every thread. */
    int max_expert = -1;
    for (int i = 0; i < n_pairs; ++i)
        if ((int)sorted_pairs[i].expert > max_expert) max_expert = (int)sorted_pairs[i].expert;
    if (max_expert < 0) return;
    const int ne = max_expert + 1;
    int* first = (int*)malloc(sizeof(int) * (size_t)ne);
    int* last = (int*)malloc(sizeof(int) * (size_t)ne);
    for (int e = 0; e < ne; ++e) { first[e] = -1; last[e] = -1; }
    for (int i = 0; i < n_pairs; ++i) {
        const int e = (int)sorted_pairs[i].expert;
        if (first[e] < 0) first[e] = i;
        last[e] = i;
    }
    float* gate = (float*)malloc(sizeof(float) * (size_t)f * d);
    float* up = (float*)malloc(sizeof(float) * (size_t)f * d);
    float* down = (float*)malloc(sizeof(float) * (size_t)d * f);
    for (int e = 0; e < ne; ++e) {
        if (first[e] < 0) continue;
        const uint8_t* b = expert_blobs[e];
        const uint16_t* bias[3] = {NULL, NULL, NULL};
        if (!symmetric) {
            bias[0] = (const uint16_t*)(b + o[2]);
            bias[1] = (const uint16_t*)(b + o[5]);
            bias[2] = (const uint16_t*)(b + o[8]);
        }
        const int gs_d = f / group;
        /* row-parallel dequantisation: the same per-row routine as
         * tsgo_dequantize_int4 */
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (int row = 0; row < f; ++row) {
            dequant_row(b + o[0] + (size_t)row * (d / 2), (const uint16_t*)(b + o[1]) + (size_t)row * (d / group),
                        bias[0] ? bias[0] + (size_t)row * (d / group) : NULL, d, group,
                        gate + (size_t)row * d);
            dequant_row(b + o[3] + (size_t)row * (d / 2), (const uint16_t*)(b + o[4]) + (size_t)row * (d / group),
                        bias[1] ? bias[1] + (size_t)row * (d / group) : NULL, d, group,
                        up + (size_t)row * d);
        }
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (int row = 0; row < d; ++row)
            dequant_row(b + o[6] + (size_t)row * (f / 2), (const uint16_t*)(b + o[7]) + (size_t)row * gs_d,
                        bias[2] ? bias[2] + (size_t)row * gs_d : NULL, f, group,
                        down + (size_t)row * f);
#pragma omp parallel num_threads(g_threads)
        {
            float* x = (float*)malloc(sizeof(float) * (size_t)d);
            float* a = (float*)malloc(sizeof(float) * (size_t)f);
#pragma omp for schedule(dynamic, 1)
            for (int i = first[e]; i <= last[e]; ++i) {
                const tsgo_pair p = sorted_pairs[i];
                if ((int)p.expert != e) continue;
                const uint16_t* hrow = hidden + (size_t)p.token * hidden_stride;
                for (int k = 0; k < d; ++k) x[k] = tsgo_f16_to_float(hrow[k]);
                for (int row = 0; row < f; ++row) {
                    float g = dot_f32(gate + (size_t)row * d, x, d);
                    float u = dot_f32(up + (size_t)row * d, x, d);
                    if (!rows_path) {
                        g = f16r(g);
                        u = f16r(u);
                    }
                    a[row] = f16r(gate_act(g, act) * u);
                }
                uint16_t* dst = partials + ((size_t)p.token * top_k + p.rank) * d;
                for (int row = 0; row < d; ++row)
                    dst[row] = tsgo_f16_bits(dot_f32(down + (size_t)row * f, a, f));
            }
            free(x);
            free(a);
        }
    }
    free(gate); free(up); free(down);
    free(first);
    free(last);
}

void tsgo_reduce_token_major(const uint16_t* partials, const uint16_t* route_w,
                             int t, int top_k, int d, uint16_t* h2) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int token = 0; token < t; ++token) {
        for (int j = 0; j < d; ++j) {
            float acc = 0.0f;
            for (int r = 0; r < top_k; ++r) {
                const float w = tsgo_f16_to_float(route_w[(size_t)token * top_k + r]);
                const float p = tsgo_f16_to_float(partials[((size_t)token * top_k + r) * d + j]);
                acc = fmaf(w, p, acc);
            }
            h2[(size_t)token * d + j] = tsgo_f16_bits(acc);
        }
    }
}

/* ---------------------------------------------------------- layer tail ----
 * prefill_rms_block_inv (prefill.metal:117-147) with lsize = 256: lane l sums
 * x[l], x[l+256], ... by fma, simd_sum over each 32-lane SIMD group (taken in
 * lane order here; Metal leaves the order to the hardware), then the eight
 * group sums in group order; rsqrt(sum / D + eps). */
static float tail_rms_inv(const float* x, int d, float eps) {
    float groups[8];
    for (int g = 0; g < 8; ++g) {
        float s = 0.0f;
        for (int lane = 0; lane < 32; ++lane) {
            float acc = 0.0f;
            for (int i = g * 32 + lane; i < d; i += 256) acc = fmaf(x[i], x[i], acc);
            s += acc;
        }
        groups[g] = s;
    }
    float sum = 0.0f;
    for (int g = 0; g < 8; ++g) sum += groups[g];
    return 1.0f / sqrtf(sum / (float)d + eps);
}

/* prefill_layer_tail_block (prefill.metal:319-397), row by row; the fp16
 * stage boundaries of fused_layer_tail (fused.metal:271-374). */
void tsgo_layer_tail(const uint16_t* h2, const uint16_t* h1, uint16_t* hidden,
                     const uint16_t* w_post2, const uint16_t* w_post, int t, int d,
                     int h2_stride, int h1_stride, int hidden_stride, float eps,
                     float layer_scalar) {
    float* x = (float*)malloc(sizeof(float) * (size_t)d);
    float* h12 = (float*)malloc(sizeof(float) * (size_t)d);
    const float scale = f16r(layer_scalar);
    for (int row = 0; row < t; ++row) {
        const uint16_t* r2 = h2 + (size_t)row * h2_stride;
        const uint16_t* r1 = h1 + (size_t)row * h1_stride;
        uint16_t* rh = hidden + (size_t)row * hidden_stride;
        for (int i = 0; i < d; ++i) x[i] = tsgo_f16_to_float(r2[i]);
        const float inv_h2 = tail_rms_inv(x, d, eps);
        for (int i = 0; i < d; ++i) {
            const float tmp = f16r(x[i] * inv_h2 * tsgo_bf16_to_float(w_post2[i]));
            h12[i] = f16r(tsgo_f16_to_float(r1[i]) + tmp);
        }
        const float inv_h12 = tail_rms_inv(h12, d, eps);
        for (int i = 0; i < d; ++i) {
            const float tmp = f16r(h12[i] * inv_h12 * tsgo_bf16_to_float(w_post[i]));
            const float sum = f16r(tsgo_f16_to_float(rh[i]) + tmp);
            rh[i] = tsgo_f16_bits(sum * scale);
        }
    }
    free(x);
    free(h12);
}
