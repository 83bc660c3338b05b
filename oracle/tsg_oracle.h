/*
 * tsg_oracle.h — CPU restatement of Tsugumi's int4 MoE expert-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP kernels are
 * compared against; it is never the thing measured or shipped. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the he-be/tsugumi checkout). Compiled with -ffp-contract=off and without
 * fast-math so that float expressions round exactly as Swift evaluates them
 * (Swift never contracts a*b+c into an fma).
 *
 * How each part is pinned (see tests/test_oracle_*.py):
 *   PRNG ............ published SplitMix64 / FNV-1a-64 vectors
 *   fp16 / bf16 ..... numpy float16 (RNE) and torch bfloat16 over millions of
 *                     values incl. subnormals, ties and overflow
 *   quantizers ...... round-trip bounds, sym bias identity as bit patterns,
 *                     nibble order low=even / high=odd
 *   GEMV / FFN ...... fp64 brute force on the same dequantised weights
 *   GELU ............ known points from the reference's MoEReferenceTests
 *   router .......... brute-force top-k over fp64 logits on tie-free draws,
 *                     explicit tie cases (lower index wins)
 *   INT8 affine ..... exact ramps (q = k), half-step ties rounding away from
 *                     zero, constant groups, round-trip bounds; its router
 *                     logits against fp64 on the dequantised rows
 *   grouping/planner  the literal golden arrays of the reference's tests
 *   prefill ref ..... fp64 brute force (before the fp16 roundings) within
 *                     fp16 error bounds; reduce: closed form
 */
#ifndef TSG_ORACLE_H
#define TSG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- PRNG: SplitMix64 + SeedTree (TsugumiValidation/Support/PRNG) ---- */
uint64_t tsgo_splitmix64_next(uint64_t* state);
uint64_t tsgo_fnv1a64(const char* label);
uint64_t tsgo_seedtree_key(uint64_t root, const char* label);
float tsgo_uniform(uint64_t* state, float lo, float hi);
void tsgo_fill_uniform(uint64_t* state, float lo, float hi, float* out, size_t n);
/* n draws of Float16(uniform(lo, hi)) as fp16 bits. */
void tsgo_fill_uniform_f16(uint64_t* state, float lo, float hi, uint16_t* out, size_t n);
/* n draws of bf16Bits(uniform(lo, hi)). */
void tsgo_fill_uniform_bf16(uint64_t* state, float lo, float hi, uint16_t* out, size_t n);

/* ---- conversions (Quantization.swift:70-82, Float16 init = RNE) ---- */
uint16_t tsgo_bf16_bits(float x);
float tsgo_bf16_to_float(uint16_t bits);
uint16_t tsgo_f16_bits(float x);
float tsgo_f16_to_float(uint16_t bits);
uint16_t tsgo_sym_bias_bits(uint16_t scale_bits);
void tsgo_f16_to_float_n(const uint16_t* in, float* out, size_t n);
void tsgo_float_to_f16_n(const float* in, uint16_t* out, size_t n);

/* ---- int4 quantisation (Quantization.swift:104-227) ---- */
/* rows x n matrix; packed is rows*(n/2) bytes, scales/biases rows*(n/g).
 * Wherever a `biases` pointer is NULL the group is `sym`: the bias is
 * -8*scale computed in fp32, which is exactly bf16ToFloat(symmetricBiasBits)
 * (MoEPackAffineV1.swift:20-40), so both spellings dequantise identically. */
void tsgo_quantize_int4(const float* w, int rows, int n, int group, int symmetric,
                        uint8_t* packed, uint16_t* scales, uint16_t* biases);
void tsgo_dequantize_int4(const uint8_t* packed, const uint16_t* scales,
                          const uint16_t* biases, int rows, int n, int group,
                          float* out);
/* The prefill GEMM staging value half(fma(q, s, b)) (prefill.metal:1021-1026)
 * with b = -8*s under sym; returns fp16 bits, rows x n. */
void tsgo_dequantize_int4_f16(const uint8_t* packed, const uint16_t* scales,
                              const uint16_t* biases, int rows, int n, int group,
                              int symmetric, uint16_t* out);

/* ---- GEMV / FFN reference (Reference/Quant/DequantInt4Gemv.swift:12-44,
 *      Reference/MoE/Moe.swift:16-123) ---- */
void tsgo_dequant_int4_gemv_ref(const uint8_t* packed, const uint16_t* scales,
                                const uint16_t* biases, const float* x,
                                int m, int n, int group, float* y);
float tsgo_gelu_tanh(float x);
float tsgo_silu(float x);
/* Qwen shared expert (qwen.metal, QwenForwardRunner.swift:1548-1578). */
float tsgo_sigmoid(float x);
void tsgo_silu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n);
void tsgo_gelu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n);
void tsgo_dense_mlp_int4(const uint8_t* gw, const uint16_t* gs, const uint16_t* gb,
                         const uint8_t* uw, const uint16_t* us, const uint16_t* ub,
                         const uint8_t* dw, const uint16_t* ds, const uint16_t* db,
                         const uint16_t* x_f16, int d, int f, int group, uint16_t* y_f16);
void tsgo_shared_gate_f16(uint16_t* y, const uint16_t* x_f16, const uint16_t* w_bf16, int d);
void tsgo_shared_expert(const uint8_t* blob, const uint32_t* offsets9, const uint16_t* x_f16,
                        const uint16_t* gate_w_bf16, int d, int f, int group, int symmetric,
                        uint16_t* out_f16);
/* One expert: down(act(gate x) * up x). act: 0 = gelu_pytorch_tanh, 1 = silu.
 * NULL bias pointers mean `sym`. */
void tsgo_moe_run_ffn(const uint8_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                      const uint8_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                      const uint8_t* down_w, const uint16_t* down_s, const uint16_t* down_b,
                      const float* x, int d, int f, int group, int act, float* out);
/* y = residual + sum_slot w[slot] * ffn_{experts[slot]}(x); experts given as
 * blob pointers with the MoEExpertOffsets layout (9 byte offsets). */
void tsgo_moe_apply_streamed_routed(const uint8_t* const* blobs, const uint32_t* offsets9,
                                    const float* x, const float* residual,
                                    const float* routing_weights, int top_k,
                                    int d, int f, int group, int symmetric, int act, float* y);

/* ---- INT8 affine (Quantization.swift:243-303) ---- */
/* quantizeInt8Affine: per group of `group` along each row, scale =
 * bf16((wmax - wmin) / 255) (1 when wmax == wmin), bias = bf16(wmin),
 * q = clamp(round_half_away((w - bias) * (1 / scale)), 0, 255) with the bf16
 * scale and bias as floats. packed [rows * n], scales/biases [rows * n/group]. */
void tsgo_quantize_int8_affine(const float* w, int rows, int n, int group, uint8_t* packed,
                               uint16_t* scales, uint16_t* biases);
/* dequantizeInt8Affine: float(q) * scale + bias, two roundings. */
void tsgo_dequantize_int8_affine(const uint8_t* packed, const uint16_t* scales,
                                 const uint16_t* biases, int rows, int n, int group, float* out);
/* INT8-affine router logits (moe.metal:136-183 semantics) in the MI355X
 * kernel's summation order (restated from tsugumi_amd/csrc/decode.hip
 * router_int8_kernel): for each expert, 64 partial sums p_l over the
 * 16-element units u = l, l+64, ...; per unit, in element order,
 * qx = fma(q, x, qx) and sx = sx + x (x = hidden * es in fp32), then
 * acc = fma(scale, qx, acc), acc = fma(bias, sx, acc); the 64 partials reduce
 * as tsgo_router_logits_canonical's. Parity pinned by exact-arithmetic inputs
 * and the fp32 error bound against fp64 on random inputs
 * (tests/test_oracle_router_int8.py). */
void tsgo_router_logits_int8_canonical(const uint8_t* w, const uint16_t* scales,
                                       const uint16_t* biases, const uint16_t* hidden_f16,
                                       const uint16_t* es_bf16, int num_experts, int d,
                                       int group, float* out_logits);

/* ---- router (TsugumiKernelCheck/main.swift:384-402) ---- */
void tsgo_router_reference(const float* w, const float* x, int num_experts, int d,
                           int top_k, const float* per_expert_scale,
                           int32_t* out_idx, float* out_w);
/* Router logits in the MI355X kernels' summation order (restated from
 * tsugumi_amd/csrc/decode.hip router_chunks_dot, not from the reference, whose
 * simd_sum order is Metal's): for each expert, 64 partial sums p_l over the
 * 8-element chunks c = l, l+64, ... (acc = fma(w, x*es, acc), elements in
 * order); each group of 16 partials sums as pairs (l, l^1), pairs of pairs
 * (l, l^2), quads mirrored within the 8 (l, 7-l), 8s mirrored within the 16
 * (l, 15-l); the four group sums add as (r0 + r1) + (r2 + r3). Inputs are bf16
 * weights, fp16 hidden rows at `stride`, bf16 effective scale.
 * Parity pinned by exact-arithmetic inputs (any order gives the fp64 sum) and
 * the fp32 error bound on random inputs (tests/test_oracle_router_prefill.py). */
void tsgo_router_logits_canonical(const uint16_t* w_bf16, const uint16_t* hidden_f16,
                                  int stride, const uint16_t* es_bf16, int rows,
                                  int num_experts, int d, float* out_logits);
/* Top-k + softmax + gain over given logits with the kernels' rule
 * (moe.metal:281-329): insertion order, ties -> lower index, -inf/NaN never
 * enter; weights rounded to fp16 bits. */
void tsgo_topk_softmax(const float* logits, int num_experts, int top_k,
                       const float* per_expert_scale, int32_t* out_idx, uint16_t* out_w);

/* ---- prefill routing (PrefillRouter.swift:238-258,
 *      PrefillMoEGrouping.swift:90-202, PrefillGroupedRoutedMoE.swift:42-83) ---- */
typedef struct { uint32_t token, expert, rank, weight_bits; } tsgo_pair;
typedef struct { uint32_t expert, pair_start, pair_count; } tsgo_group;
typedef struct { uint32_t group_start, group_count, pair_start, pair_count; } tsgo_tile;
typedef struct { uint32_t local_slot, pair_start, row_count, local_row; } tsgo_block;

void tsgo_make_token_expert_pairs(const uint32_t* idx, const uint16_t* w, int t, int top_k,
                                  tsgo_pair* out);
/* Returns 0 or a negative error code (see tsg_oracle.c). expert_sort_keys may
 * be NULL; tile_break_after_group < 0 means none. */
int tsgo_group_pairs(const tsgo_pair* pairs, int n_pairs, int query_count, int top_k,
                     int num_experts, int tile_expert_count,
                     const uint64_t* expert_sort_keys, int n_sort_keys,
                     int tile_break_after_group,
                     tsgo_pair* sorted, uint32_t* offsets, uint32_t* counts,
                     tsgo_group* groups, int* n_groups, tsgo_tile* tiles, int* n_tiles);
/* Writes blocks and per-batch (rows, first block) into the out arrays. */
int tsgo_plan_routed_gemm(const tsgo_group* groups, int n_groups, int max_rows_per_batch,
                          tsgo_block* blocks, int* n_blocks,
                          int* batch_rows, int* batch_first_block, int* n_batches);

/* ---- prefill expert-major reference with the GPU's fp16 roundings
 *      (TsugumiKernelCheck/PrefillMoEGEMMCheck.swift:138-173) ---- */
/* experts_blobs[e] + offsets9 give each expert's sub-tensors. Writes
 * partials[(token*top_k + rank)*d + j] as fp16 bits for every sorted pair.
 * rows_path = 0: the tiled GEMM's roundings, act = half(act(half(g)) *
 * half(u)) (PrefillMoEGEMMCheck.swift:156-165); 1: the rows path's
 * (prefill.metal:1621-1628), act = half(act(g) * u) with g, u in fp32, as
 * decode phase 1 (moe.metal:573). */
void tsgo_prefill_moe_ref(const uint8_t* const* expert_blobs, const uint32_t* offsets9,
                          const uint16_t* hidden, int hidden_stride,
                          const tsgo_pair* sorted_pairs, int n_pairs,
                          int top_k, int d, int f, int group, int symmetric, int act,
                          int rows_path, uint16_t* partials);
/* h2[t,d] = half(sum_r fma(w[t,r], P[(t*K+r),d])) (prefill.metal:796-817). */
void tsgo_reduce_token_major(const uint16_t* partials, const uint16_t* route_w,
                             int t, int top_k, int d, uint16_t* h2);

/* The Gemma decoder-layer tail over strided rows, hidden updated in place
 * (prefill_layer_tail_block prefill.metal:319-397, fused_layer_tail
 * fused.metal:271-374). */
void tsgo_layer_tail(const uint16_t* h2, const uint16_t* h1, uint16_t* hidden,
                     const uint16_t* w_post2, const uint16_t* w_post, int t, int d,
                     int h2_stride, int h1_stride, int hidden_stride, float eps,
                     float layer_scalar);

/* OpenMP thread count used by the heavy loops (1 = scalar). */
void tsgo_set_threads(int n);
int tsgo_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
