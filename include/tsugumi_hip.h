/*
 * tsugumi_hip.h — C ABI of the MI355X (gfx950) int4 MoE expert-matmul path.
 *
 * Drop-in for the Swift encoders Tsugumi's decoder calls on this path. Each
 * entry point replaces one `encode*` method (cited as reference file:line,
 * relative to the he-be/tsugumi checkout). Conventions:
 *
 *  - All tensors are caller-owned DEVICE pointers (HBM), never copied. fp16
 *    activations and bf16 scales travel as uint16_t bit patterns; packed int4
 *    weights as bytes (low nibble = even element, high nibble = odd).
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *    default stream), the analogue of appending to an MTLCommandBuffer.
 *  - Every call returns a tsg_status. Where the reference traps on a
 *    precondition this returns TSG_ERR_INVALID_ARGUMENT (or _ALIGNMENT) and
 *    enqueues nothing; where an optional fast path declines (returns 0/false
 *    in Swift) this returns TSG_ERR_DECLINED. tsg_last_error() gives text
 *    (thread-local).
 *  - Objects (tsg_ctx, tsg_moe, tsg_layer) are not thread-safe; one encoding
 *    thread per object, as with the reference's MetalContext/MoE.
 */
#ifndef TSUGUMI_HIP_H
#define TSUGUMI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ types */

typedef enum tsg_status {
    TSG_OK = 0,
    TSG_ERR_INVALID_ARGUMENT = 1, /* a reference precondition failed          */
    TSG_ERR_ALIGNMENT = 2,        /* a pointer/offset breaks the kernel's alignment */
    TSG_ERR_UNSUPPORTED = 3,      /* shape or configuration not built          */
    TSG_ERR_DECLINED = 4,         /* optional path declines; caller falls back */
    TSG_ERR_HIP = 5,              /* HIP runtime error                         */
    TSG_ERR_OUT_OF_MEMORY = 6,
    TSG_ERR_FORMAT = 7,           /* a MoEPack install fails validation        */
    TSG_ERR_IO = 8,               /* a MoEPack file is missing or unreadable   */
    /* PrefillMoEGroupingError cases (PrefillMoEGrouping.swift:52-62) */
    TSG_ERR_GROUPING_INVALID_QUERY_COUNT = 100,
    TSG_ERR_GROUPING_INVALID_TOP_K = 101,
    TSG_ERR_GROUPING_INVALID_NUM_EXPERTS = 102,
    TSG_ERR_GROUPING_INVALID_TILE_EXPERT_COUNT = 103,
    TSG_ERR_GROUPING_PAIR_COUNT_MISMATCH = 104,
    TSG_ERR_GROUPING_TOKEN_OUT_OF_RANGE = 105,
    TSG_ERR_GROUPING_RANK_OUT_OF_RANGE = 106,
    TSG_ERR_GROUPING_EXPERT_OUT_OF_RANGE = 107,
    TSG_ERR_GROUPING_DUPLICATE_TOKEN_RANK = 108,
    TSG_ERR_GROUPING_SORT_KEY_COUNT_MISMATCH = 109
} tsg_status;

/* Quantization.AffineScheme (Quantization.swift:24-39). */
typedef enum tsg_affine_scheme { TSG_AFFINE = 0, TSG_SYM = 1 } tsg_affine_scheme;

/* MoE.GateActivation (MoE.swift:100-121). */
typedef enum tsg_activation { TSG_ACT_GELU_TANH = 0, TSG_ACT_SILU = 1 } tsg_activation;

/* MoEExpertOffsets (MoE.swift:4-29): byte offsets of an expert blob's nine
 * sub-tensors. Under `sym` the bias offsets alias the scales and are never
 * dereferenced. 36 bytes. */
typedef struct tsg_expert_offsets {
    uint32_t gate_w, gate_s, gate_b;
    uint32_t up_w, up_s, up_b;
    uint32_t down_w, down_s, down_b;
} tsg_expert_offsets;

/* PrefillTokenExpertPair (PrefillRouter.swift:4-28). 16 bytes. */
typedef struct tsg_token_expert_pair {
    uint32_t token, expert, rank, weight_bits; /* weight = fp16 bits in the low half */
} tsg_token_expert_pair;

/* PrefillMoEGroup / PrefillMoETile (PrefillMoEGrouping.swift:3-29). */
typedef struct tsg_moe_group { uint32_t expert, pair_start, pair_count; } tsg_moe_group;
typedef struct tsg_moe_tile {
    uint32_t group_start, group_count, pair_start, pair_count;
} tsg_moe_tile;

/* PrefillRoutedGEMMBlock (PrefillGroupedRoutedMoE.swift:20-25). 16 bytes.
 * `local_slot` names the expert: an index into the binding's expert ids, or
 * the expert id itself when the whole layer is HBM-resident. */
typedef struct tsg_routed_block {
    uint32_t local_slot, pair_start, row_count, local_row;
} tsg_routed_block;

/* The layouts above are shared with the reference's Swift/Metal structs
 * byte for byte; these checks hold them (PrefillRouterTests.swift:12-19 pins
 * the pair's size and field offsets; MoE.swift:4-29 the 36-byte offsets). */
#ifdef __cplusplus
#define TSG_LAYOUT_ASSERT(cond, msg) static_assert(cond, msg)
#else
#define TSG_LAYOUT_ASSERT(cond, msg) _Static_assert(cond, msg)
#endif
TSG_LAYOUT_ASSERT(sizeof(tsg_expert_offsets) == 36, "MoEExpertOffsets is 36 bytes");
TSG_LAYOUT_ASSERT(offsetof(tsg_expert_offsets, down_b) == 32, "MoEExpertOffsets.downB at 32");
TSG_LAYOUT_ASSERT(sizeof(tsg_token_expert_pair) == 16, "PrefillTokenExpertPair is 16 bytes");
TSG_LAYOUT_ASSERT(offsetof(tsg_token_expert_pair, token) == 0 &&
                      offsetof(tsg_token_expert_pair, expert) == 4 &&
                      offsetof(tsg_token_expert_pair, rank) == 8 &&
                      offsetof(tsg_token_expert_pair, weight_bits) == 12,
                  "PrefillTokenExpertPair field offsets 0/4/8/12");
TSG_LAYOUT_ASSERT(sizeof(tsg_moe_group) == 12, "PrefillMoEGroup is 12 bytes");
TSG_LAYOUT_ASSERT(sizeof(tsg_moe_tile) == 16, "PrefillMoETile is 16 bytes");
TSG_LAYOUT_ASSERT(sizeof(tsg_routed_block) == 16, "PrefillRoutedGEMMBlock is 16 bytes");
TSG_LAYOUT_ASSERT(offsetof(tsg_routed_block, local_row) == 12, "PrefillRoutedGEMMBlock.localRow at 12");
#undef TSG_LAYOUT_ASSERT

typedef struct tsg_ctx tsg_ctx;     /* MetalContext                      */
typedef struct tsg_moe tsg_moe;     /* MoE / PrefillGroupedRoutedMoE      */
typedef struct tsg_layer tsg_layer; /* one HBM-resident MoEPack layer     */
typedef void* tsg_stream;           /* hipStream_t                        */

/* ---------------------------------------------------------------- context */

const char* tsg_last_error(void);
const char* tsg_status_string(tsg_status status);
/* Library version "major.minor.patch". */
const char* tsg_version(void);

/* MetalContext.init (MetalContext.swift:79-100): binds `device`. The context
 * owns small device scratch that several entry points share (router logits
 * and their hand-off words, completion counters, the decode layer's hand-off
 * regions, the fused GEMM's queues): calls on one context run in stream
 * order, as the reference's encoders append to one command buffer; a caller
 * that issues on several streams orders them with events or uses one context
 * per stream. The shared-expert entry points use no such scratch and may run
 * beside the routed path. */
tsg_status tsg_ctx_create(int device, tsg_ctx** out);
void tsg_ctx_destroy(tsg_ctx* ctx);
/* MetalContext.setAffineGroupSize / setAffineScheme (MetalContext.swift:135-175).
 * Group sizes {32, 64}; defaults are 64 and TSG_AFFINE, as in the reference. */
tsg_status tsg_ctx_set_affine_group_size(tsg_ctx* ctx, uint32_t group_size);
tsg_status tsg_ctx_set_affine_scheme(tsg_ctx* ctx, tsg_affine_scheme scheme);
tsg_status tsg_ctx_synchronize(tsg_ctx* ctx, tsg_stream stream);

/* ------------------------------------------------- HBM-resident layers ---
 * Replace SSD streaming + MTLResidencySet (ModelExpertIO.swift:112-324,
 * Infrastructure/Streaming): a layer file (`packed_experts/layer_XX.bin`,
 * laid out by RepackPlanner.planLayerFile, RepackPlanner.swift:442-520) is held
 * byte-for-byte in HBM; expert e's blob starts at e * expert_stride. */

/* Allocates the layer's HBM (owned by it). `expert_stride` and `offsets` are
 * the layer file's; sub-tensor offsets need only be 2-byte aligned, the
 * repacker's guarantee (DequantInt4GEMV.swift:93-96). When a weight
 * sub-tensor is off 16 bytes or a scale/bias one off 4, the HBM image is laid
 * out anew (every sub-tensor on 256 bytes, stride rounded to 16 KiB) and
 * tsg_layer_upload places the file's bytes there; otherwise the image is the
 * file, num_experts * expert_stride bytes. */
tsg_status tsg_layer_create(tsg_ctx* ctx, uint32_t num_experts, uint64_t expert_stride,
                            const tsg_expert_offsets* offsets, tsg_layer** out);
/* Wraps caller-owned HBM holding the file image as it is (no copy, not freed):
 * weight sub-tensors must start on 16 bytes and scales/biases on 4
 * (TSG_ERR_ALIGNMENT otherwise; use tsg_layer_create). */
tsg_status tsg_layer_wrap(tsg_ctx* ctx, void* device_base, uint32_t num_experts,
                          uint64_t expert_stride, const tsg_expert_offsets* offsets,
                          tsg_layer** out);
/* Copies `nbytes` of a host layer-file image, starting at byte `dst_offset` of
 * the FILE, into the layer (through the new layout when there is one). */
tsg_status tsg_layer_upload(tsg_layer* layer, tsg_stream stream, const void* host_bytes,
                            uint64_t nbytes, uint64_t dst_offset);
/* The HBM image: expert e at device_ptr + e * device_stride, sub-tensors at
 * device_offsets (tsg_layer_get_geometry); the file's geometry unless laid
 * out anew. No reference counterpart (the reference binds MTLBuffers). */
void* tsg_layer_device_ptr(const tsg_layer* layer);
tsg_status tsg_layer_get_geometry(const tsg_layer* layer, uint64_t* device_stride,
                                  tsg_expert_offsets* device_offsets);
void tsg_layer_destroy(tsg_layer* layer);

/* ------------------------------------------------------------- decode ----
 * MoE (Kernels/MoE/MoE.swift:42-662). */

/* MoE.init(context:routerWeightBits:gateActivation:) (MoE.swift:123-199).
 * router_weight_bits: 8 (INT8-affine router: tsg_moe_router_int8,
 * tsg_moe_decode_layer_int8) or 16 (bf16, the QAT checkpoints' router: every
 * other router entry point and decode layer). An entry point of the other
 * format returns TSG_ERR_INVALID_ARGUMENT (the reference's precondition). */
tsg_status tsg_moe_create(tsg_ctx* ctx, uint32_t router_weight_bits,
                          tsg_activation gate_activation, tsg_moe** out);
void tsg_moe_destroy(tsg_moe* moe);

/* encodeRouterGemma4BF16 (MoE.swift:259-302): logits[e] = sum_i W[e,i] *
 * (hidden[i] * effective_scale[i]) in fp32, top-k (ties -> lower index),
 * softmax over the k, times per_expert_scale -> fp16 weights. One launch;
 * indices and weights stay on the device. top_k == 8, num_experts <= 256. */
tsg_status tsg_moe_router_bf16(tsg_moe* moe, tsg_stream stream, const uint16_t* weights,
                               const uint16_t* hidden, const uint16_t* effective_scale,
                               const uint16_t* per_expert_scale, uint32_t* out_indices,
                               uint16_t* out_weights, uint32_t num_experts, uint32_t d,
                               uint32_t top_k);
/* encodeRouterGemma4 (MoE.swift:201-257; kernel moe.metal:136-183): the
 * INT8-affine router. Row e of `weights` is d uint8 codes, with bf16 scales and
 * biases per group of the context's group size (Quantization.quantizeInt8Affine,
 * Quantization.swift:243-287): logit_e = sum_i (q * scale + bias) * (hidden[i] *
 * effective_scale[i]) in fp32, then the same top-k, softmax and gain as
 * tsg_moe_router_bf16. d a multiple of 64 and of the group size, d <= 4096;
 * top_k == 8, num_experts <= 256; weights, hidden and effective_scale on 16
 * bytes. Requires a MoE created with router_weight_bits 8. */
tsg_status tsg_moe_router_int8(tsg_moe* moe, tsg_stream stream, const uint8_t* weights,
                               const uint16_t* scales, const uint16_t* biases,
                               const uint16_t* hidden, const uint16_t* effective_scale,
                               const uint16_t* per_expert_scale, uint32_t* out_indices,
                               uint16_t* out_weights, uint32_t num_experts, uint32_t d,
                               uint32_t top_k);
/* encodeRouterGemma4BF16Rows (MoE.swift:404-466): the same for row_count <= 8
 * rows at hidden_stride elements; each row is bit-identical to the one-row
 * call. Returns TSG_ERR_DECLINED for row_count 0 or > 8. */
tsg_status tsg_moe_router_bf16_rows(tsg_moe* moe, tsg_stream stream, const uint16_t* weights,
                                    const uint16_t* hidden, uint32_t hidden_stride_elements,
                                    const uint16_t* effective_scale,
                                    const uint16_t* per_expert_scale, uint32_t* out_indices,
                                    uint16_t* out_weights, uint32_t row_count,
                                    uint32_t num_experts, uint32_t d, uint32_t top_k);
/* encodeRouterGemma4BF16Rows followed by the device grouping of its pairs
 * (tsg_prefill_group_pairs_device, any tile_rows >= 8) in one launch: the
 * verify block's routing and grouping (RealForwardRunner.swift:1826-1872,
 * 2116-2151) with nothing read back to the host. Every output equals the two
 * calls' bit for bit: out_indices/out_weights [row_count, 8]; sorted
 * [row_count * 8], offsets and counts [num_experts], blocks (one per expert
 * present, in expert order, local_row = pair_start) and *n_blocks on the
 * device. max_blocks >= min(row_count * 8, num_experts); row_count * d * 2 <=
 * 64 KiB. Returns TSG_ERR_DECLINED for row_count 0 or > 8. No counterpart
 * entry in the reference, which groups on the host. */
tsg_status tsg_moe_router_bf16_rows_grouped(
    tsg_moe* moe, tsg_stream stream, const uint16_t* weights, const uint16_t* hidden,
    uint32_t hidden_stride_elements, const uint16_t* effective_scale,
    const uint16_t* per_expert_scale, uint32_t* out_indices, uint16_t* out_weights,
    uint32_t row_count, uint32_t num_experts, uint32_t d, uint32_t top_k,
    tsg_token_expert_pair* sorted, uint32_t* offsets, uint32_t* counts,
    tsg_routed_block* blocks, uint32_t max_blocks, uint32_t* n_blocks);
/* encodeRouterLogitsBF16 (MoE.swift:316-345): the GEMV alone. */
tsg_status tsg_moe_router_logits_bf16(tsg_moe* moe, tsg_stream stream, const uint16_t* weights,
                                      const uint16_t* hidden, const uint16_t* effective_scale,
                                      float* out_logits, uint32_t num_experts, uint32_t d);

/* encodeRoutedPersistentPhase1U16Load (MoE.swift:529-562):
 * acts[s*F + f] = half(act(gate_s[f].x) * (up_s[f].x)) for the top_k == 8
 * expert blobs in routed_blobs (a host array of device pointers, the
 * argument buffer's contents). */
tsg_status tsg_moe_phase1(tsg_moe* moe, tsg_stream stream, const void* const* routed_blobs,
                          const tsg_expert_offsets* offsets, const uint16_t* x, uint16_t* acts,
                          uint32_t d, uint32_t f, uint32_t top_k);
/* encodeRoutedPersistentPhase1SubsetU16Load (MoE.swift:564-607): only the
 * slots listed in the device array active_slots[0..active_count). */
tsg_status tsg_moe_phase1_subset(tsg_moe* moe, tsg_stream stream,
                                 const void* const* routed_blobs,
                                 const tsg_expert_offsets* offsets, const uint16_t* x,
                                 uint16_t* acts, const uint32_t* active_slots,
                                 uint32_t active_count, uint32_t d, uint32_t f, uint32_t top_k);
/* encodeRoutedPersistentPhase2Reduce (MoE.swift:609-644):
 * y[d] = half(residual[d] + sum_{s=0..7} w[s] * down_s[d].acts[s]), summed in
 * slot order. */
tsg_status tsg_moe_phase2(tsg_moe* moe, tsg_stream stream, const void* const* routed_blobs,
                          const tsg_expert_offsets* offsets, const uint16_t* acts,
                          const uint16_t* routing_weights, const uint16_t* residual,
                          uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k);

/* Phase 1 / phase 2 over an HBM-resident layer with the expert ids read on the
 * device from `indices` (what the router wrote): the host never reads routing
 * back (replaces RealForwardRunner.swift:3112-3151's readback + fetch). */
tsg_status tsg_moe_phase1_resident(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                   const uint32_t* indices, const uint16_t* x,
                                   uint16_t* acts, uint32_t d, uint32_t f, uint32_t top_k);
tsg_status tsg_moe_phase2_resident(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                   const uint32_t* indices, const uint16_t* acts,
                                   const uint16_t* routing_weights, const uint16_t* residual,
                                   uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k);

/* One whole decode MoE layer on a resident layer: router -> top-8 -> gate/up +
 * activation -> down + weighted combine + residual. The composition the
 * decoder encodes per layer (RealForwardRunner.swift:3104-3330), with routing
 * kept on the device. `router_hidden` feeds the router (with
 * effective_scale), `x` the experts; they may alias. out_indices/out_weights
 * receive the routing. acts_scratch holds top_k * f fp16 values. */
tsg_status tsg_moe_decode_layer(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                const uint16_t* router_weights, const uint16_t* router_hidden,
                                const uint16_t* effective_scale,
                                const uint16_t* per_expert_scale, const uint16_t* x,
                                const uint16_t* residual, uint16_t* y, uint32_t* out_indices,
                                uint16_t* out_weights, uint16_t* acts_scratch,
                                uint32_t num_experts, uint32_t d, uint32_t f, uint32_t top_k);

/* One whole verify MoE layer of row_count <= 8 tokens on a resident layer, in
 * one launch: the router rows and top-8 of every token
 * (encodeRouterGemma4BF16Rows, MoE.swift:404-466), the grouping of their
 * pairs by expert (RealForwardRunner.swift:2116-2151), gate/up + activation
 * and down over the union of routed experts (encodeStreamedRows,
 * PrefillGroupedRoutedMoE.swift:793-917) and the token-major weighted sum
 * (PrefillMoE.encodeReduceTokenMajor, PrefillMoE.swift:11-38): the
 * composition RealForwardRunner.swift:1826-2151 encodes per verify layer.
 * h2 [row_count, d], out_indices / out_weights [row_count, 8] are bit for bit
 * what tsg_moe_router_bf16_rows_grouped + tsg_prefill_moe_rows_device +
 * tsg_prefill_moe_reduce_token_major give. router_hidden feeds the router
 * (with effective_scale), x the experts (they may alias), both rows
 * hidden_stride elements apart. Returns TSG_ERR_DECLINED, with nothing
 * launched, for row_count 0 or > 8, num_experts < 8, d or f not a multiple of
 * 64 or above 4096, or when the launch's blocks cannot all be resident (the
 * caller then encodes those three calls). Its hand-off words and launch
 * epoch live in the context: verify-layer launches on one context must not
 * overlap (one stream, or streams ordered by events), and work on other
 * streams meanwhile delays the launch (its blocks wait on each other);
 * tsg_ctx_synchronize reports a hand-off wait that timed out. No counterpart
 * entry in the reference, which encodes the steps as separate dispatches. */
tsg_status tsg_moe_verify_layer(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                const uint16_t* router_weights, const uint16_t* router_hidden,
                                const uint16_t* effective_scale,
                                const uint16_t* per_expert_scale, const uint16_t* x,
                                uint32_t hidden_stride_elements, uint16_t* h2,
                                uint32_t* out_indices, uint16_t* out_weights,
                                uint32_t row_count, uint32_t num_experts, uint32_t d, uint32_t f,
                                uint32_t top_k);

/* tsg_moe_verify_layer for a Qwen-family layer: the shared expert's branch
 * over the same row_count token rows (encodeSharedExpert per row,
 * QwenForwardRunner.swift:1548-1578, beside the routed experts of
 * :1580-1608) in the same launch. shared_blob / shared_offsets hold its three
 * int4 projections (the ctx's group size and scheme; gate/up [f, d], down
 * [d, f]: its intermediate size is the routed experts' f), shared_gate_weight
 * its bf16 gate row [d] (16-byte aligned). shared_out [row_count, d] gets
 * bit for bit what tsg_moe_shared_expert_rows gives on x; h2 and the routing
 * are tsg_moe_verify_layer's. Needs no act scratch (the activations pass
 * through the context's hand-off words). Declines as tsg_moe_verify_layer,
 * and for a MoE whose activation is not SiLU; an unroutable token makes
 * shared_out NaN as well. No counterpart entry in the reference, which
 * encodes the shared branch as separate dispatches. */
tsg_status tsg_moe_verify_layer_shared(
    tsg_moe* moe, tsg_stream stream, const tsg_layer* layer, const uint16_t* router_weights,
    const uint16_t* router_hidden, const uint16_t* effective_scale,
    const uint16_t* per_expert_scale, const uint16_t* x, uint32_t hidden_stride_elements,
    uint16_t* h2, uint32_t* out_indices, uint16_t* out_weights, const void* shared_blob,
    const tsg_expert_offsets* shared_offsets, const uint16_t* shared_gate_weight,
    uint16_t* shared_out, uint32_t row_count, uint32_t num_experts, uint32_t d, uint32_t f,
    uint32_t top_k);

/* tsg_moe_decode_layer with the INT8-affine router (a MoE created with
 * router_weight_bits 8; encodeRouterGemma4, MoE.swift:201-257, then the two
 * phases, as RealForwardRunner.swift:3104-3330 encodes them per layer): the
 * router's arithmetic is tsg_moe_router_int8's (same logits, same selection),
 * in the one launch or, when that does not fit, as tsg_moe_router_int8 +
 * phase 1 + phase 2; both give identical bits. router_weights are d uint8
 * codes per expert row (16-byte aligned), router_scales / router_biases bf16
 * per group of the context's group size (2-byte aligned); d a multiple of 64
 * and of the group size, d <= 4096. */
tsg_status tsg_moe_decode_layer_int8(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                     const uint8_t* router_weights, const uint16_t* router_scales,
                                     const uint16_t* router_biases, const uint16_t* router_hidden,
                                     const uint16_t* effective_scale,
                                     const uint16_t* per_expert_scale, const uint16_t* x,
                                     const uint16_t* residual, uint16_t* y, uint32_t* out_indices,
                                     uint16_t* out_weights, uint16_t* acts_scratch,
                                     uint32_t num_experts, uint32_t d, uint32_t f, uint32_t top_k);

/* The Qwen-family layer: the shared branch of
 * QwenForwardRunner.encodeSharedExpert (QwenForwardRunner.swift:1548-1578)
 * and the routed experts on top of it with residual = y = sharedOut
 * (encodeRoutedExperts, :1583-1608), as one call: y = half(sharedOut +
 * sum_s w_s expert_s(x)), sharedOut = half(half(down . act) * sigmoid(w_g . x)),
 * act = half(silu(half(gate . x)) * half(up . x)) over the shared expert blob
 * (MoEExpertOffsets; the ctx's group size and scheme). No single reference
 * call: in one launch when it fits (shared_f <= 512), its shared weights
 * loaded while the router runs; otherwise tsg_moe_shared_expert then
 * tsg_moe_decode_layer(residual = y). Both give the same bits. shared_acts
 * (16-byte aligned) receives the shared_f fp16 activations. */
tsg_status tsg_moe_decode_layer_shared(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                       const uint16_t* router_weights,
                                       const uint16_t* router_hidden,
                                       const uint16_t* effective_scale,
                                       const uint16_t* per_expert_scale, const uint16_t* x,
                                       uint16_t* y, uint32_t* out_indices, uint16_t* out_weights,
                                       uint16_t* acts_scratch, const void* shared_blob,
                                       const tsg_expert_offsets* shared_offsets,
                                       const uint16_t* shared_gate_weight, uint16_t* shared_acts,
                                       uint32_t num_experts, uint32_t d, uint32_t f,
                                       uint32_t shared_f, uint32_t top_k);

/* tsg_moe_decode_layer runs as one launch (grid barriers between router,
 * gate/up and down) whenever every block fits on the device at once, else as
 * router + phase 1 + phase 2 launches; both give identical bits. The one
 * launch keeps its hand-off words and launch epoch in the context, so such
 * launches on one context must not overlap (one stream, or streams ordered
 * by events). enabled = 0 forces the three-launch form (no reference
 * counterpart; for A/B checks). */
tsg_status tsg_moe_set_fused_decode(tsg_moe* moe, int enabled);

/* ------------------------------------------------- Qwen shared expert ----
 * The Qwen-family MoE block's shared expert and its sigmoid gate
 * (QwenForwardRunner.encodeSharedExpert, QwenForwardRunner.swift:1548-1578):
 *   act       = half(silu(half(gate . x)) * half(up . x))
 *   sharedOut = half(half(down . act) * sigmoid(w_g . x))
 * The routed experts then add on top with residual = sharedOut
 * (QwenForwardRunner.swift:1583-1608: tsg_moe_decode_layer's residual). An
 * empty size returns TSG_ERR_DECLINED with nothing enqueued (the reference's
 * encoders return false). */

/* QwenKernels.encodeSiluMul (QwenKernels.swift:371-389, qwen.metal:466):
 * out[i] = half(silu(float(gate[i])) * float(up[i])), silu(x) = x / (1 + e^-x)
 * as x * sigmoid(x). */
tsg_status tsg_qwen_silu_mul(tsg_ctx* ctx, tsg_stream stream, const uint16_t* gate,
                             const uint16_t* up, uint16_t* out, uint32_t count);
/* QwenKernels.encodeMoESharedGate (QwenKernels.swift:311-327, qwen.metal:432-455):
 * y[i] = half(float(y[i]) * sigmoid(sum_k float(x[k]) * float(weight[k]))) in
 * place; x fp16 [hidden], weight bf16 [hidden] (the [1, hidden] gate row),
 * both 16-byte aligned, hidden a multiple of 8 up to 4096 (TSG_ERR_ALIGNMENT /
 * TSG_ERR_UNSUPPORTED otherwise). */
tsg_status tsg_qwen_moe_shared_gate(tsg_ctx* ctx, tsg_stream stream, uint16_t* y,
                                    const uint16_t* x, const uint16_t* weight, uint32_t hidden);
/* QwenKernels.encodeMoESharedGateLogit (QwenKernels.swift:335-350,
 * qwen.metal:1038-1046): y[i] = half(float(y[i]) * sigmoid(float(logit[0]))),
 * the logit (fp16) already taken by a GEMV. */
tsg_status tsg_qwen_moe_shared_gate_logit(tsg_ctx* ctx, tsg_stream stream, uint16_t* y,
                                          const uint16_t* logit, uint32_t hidden);
/* The whole shared branch of encodeSharedExpert (QwenForwardRunner.swift:1548-1578)
 * in two launches: the three int4 projections of one expert laid out as a
 * blob (MoEExpertOffsets, the ctx's group size and scheme; gate/up [f, d],
 * down [d, f]), SwiGLU, and the bf16 gate row. act_scratch holds f fp16 (the
 * activations). out fp16 [d]. Bit-identical to tsg_qmv_int4 (gate), (up),
 * tsg_qwen_silu_mul, tsg_qmv_int4 (down), tsg_qwen_moe_shared_gate in turn. */
tsg_status tsg_moe_shared_expert(tsg_moe* moe, tsg_stream stream, const void* blob,
                                 const tsg_expert_offsets* offsets, const uint16_t* x,
                                 const uint16_t* gate_weight, uint16_t* act_scratch,
                                 uint16_t* out, uint32_t d, uint32_t f);
/* The same for row_count <= 8 token rows (x + r * x_stride, x_stride a
 * multiple of 8 elements), the shared branch of a multi-token decode step
 * (MTP verify; encodeSharedExpert per row, QwenForwardRunner.swift:1548-1578)
 * in two launches, each weight read once for all rows: act_scratch [rows, f],
 * out [rows, d]; row r is bit-identical to tsg_moe_shared_expert on x_r.
 * Returns TSG_ERR_DECLINED for row_count 0 or > 8. */
tsg_status tsg_moe_shared_expert_rows(tsg_moe* moe, tsg_stream stream, const void* blob,
                                      const tsg_expert_offsets* offsets, const uint16_t* x,
                                      uint32_t x_stride, const uint16_t* gate_weight,
                                      uint16_t* act_scratch, uint16_t* out, uint32_t row_count,
                                      uint32_t d, uint32_t f);

/* ---------------------------------------------------------------- QMV ----
 * DequantInt4GEMV (Kernels/Quant/DequantInt4GEMV.swift:6-364). */

/* encode (DequantInt4GEMV.swift:78-121): y[m] = half(sum_n W[m,n] x[n]).
 * n % group == 0. biases may alias scales under sym. */
tsg_status tsg_qmv_int4(tsg_ctx* ctx, tsg_stream stream, const uint8_t* weights,
                        const uint16_t* scales, const uint16_t* biases, const uint16_t* x,
                        uint16_t* y, uint32_t m, uint32_t n);
/* encodeRows (DequantInt4GEMV.swift:130-182): t <= 8 activation rows against
 * the same weights; row r is bit-identical to encode on that row. Also the
 * drop-in for encodeRowsWide (:220-267), which the reference defines to give
 * encodeRows' bits. Rows that do not fit the LDS staging together (large n)
 * run in several launches. */
tsg_status tsg_qmv_int4_rows(tsg_ctx* ctx, tsg_stream stream, const uint8_t* weights,
                             const uint16_t* scales, const uint16_t* biases, const uint16_t* x,
                             uint32_t x_stride_elements, uint16_t* y,
                             uint32_t y_stride_elements, uint32_t t, uint32_t m, uint32_t n);

/* SharedExpertProjection (Kernels/MoE/SharedExpertInt8.swift:9-33): one int4
 * matrix [rows, cols] with bf16 group scales (and biases; under sym the bias
 * pointer may alias the scales and is not read). Device pointers. */
typedef struct tsg_int4_projection {
    const uint8_t* weights;
    const uint16_t* scales;
    const uint16_t* biases;
    uint32_t rows, cols;
} tsg_int4_projection;

/* gelu_mul_fp16 (Metal/Primitives/utility.metal:7-18): out = half(gelu_tanh(
 * float(gate)) * float(up)) over count fp16 values. TSG_ERR_DECLINED when
 * count == 0. */
tsg_status tsg_gelu_mul_f16(tsg_ctx* ctx, tsg_stream stream, const uint16_t* gate,
                            const uint16_t* up, uint16_t* out, uint32_t count);

/* SharedExpertInt4.encode (Kernels/MoE/SharedExpertInt4.swift:30-93): Gemma's
 * dense int4 MLP, y = down(half(gelu(gate x) * up x)), as the reference
 * encodes it (QMV gate, QMV up, gelu_mul_fp16, QMV down), so the result is
 * bit-identical to those four calls. The byte lengths stand in for the
 * MTLBuffer lengths the reference checks: a mismatch of shapes returns
 * TSG_ERR_INVALID_ARGUMENT "dimensionMismatch: ...", a short buffer
 * "scratchTooSmall: ..." (SharedExpertError). */
tsg_status tsg_shared_expert_int4(tsg_ctx* ctx, tsg_stream stream, const uint16_t* x,
                                  uint64_t x_bytes, const tsg_int4_projection* gate,
                                  const tsg_int4_projection* up,
                                  const tsg_int4_projection* down, uint16_t* y, uint64_t y_bytes,
                                  uint16_t* scratch_gate, uint64_t scratch_gate_bytes,
                                  uint16_t* scratch_up, uint64_t scratch_up_bytes,
                                  uint16_t* scratch_act, uint64_t scratch_act_bytes);
/* Bit-exact dequantisation check: out[r*n + k] = half(fma(q, s, b)), the
 * value the prefill GEMM stages (prefill.metal:1021-1026), rows x n.
 * tsg_debug_dequant_f16 computes it directly in fp32; tsg_debug_gemm_dequant_f16
 * runs the grouped GEMM's own staging routine (fp16 fast path included). */
tsg_status tsg_debug_dequant_f16(tsg_ctx* ctx, tsg_stream stream, const uint8_t* weights,
                                 const uint16_t* scales, const uint16_t* biases,
                                 uint16_t* out, uint32_t rows, uint32_t n);
tsg_status tsg_debug_gemm_dequant_f16(tsg_ctx* ctx, tsg_stream stream, const uint8_t* weights,
                                      const uint16_t* scales, const uint16_t* biases,
                                      uint16_t* out, uint32_t rows, uint32_t n);

/* ------------------------------------------------------------ prefill ----
 * PrefillRouter, PrefillMoEGrouping, PrefillGroupedRoutedMoE, PrefillMoE
 * (Kernels/Prefill/MoE). */

/* PrefillRouter.encodeGemma4BF16Block / GEMM (PrefillRouter.swift:127-236):
 * the decode router for query_count rows at hidden_stride; every row's logits
 * are summed in the decode kernel's order, so each row's choice is the one the
 * decode router makes on that row. */
tsg_status tsg_prefill_router_bf16(tsg_moe* moe, tsg_stream stream, const uint16_t* weights,
                                   const uint16_t* hidden, uint32_t hidden_stride_elements,
                                   const uint16_t* effective_scale,
                                   const uint16_t* per_expert_scale, uint32_t* out_indices,
                                   uint16_t* out_weights, uint32_t query_count,
                                   uint32_t num_experts, uint32_t d, uint32_t top_k);

/* PrefillRouter.makeTokenExpertPairs (PrefillRouter.swift:238-258), host. */
tsg_status tsg_make_token_expert_pairs(const uint32_t* indices, const uint16_t* weights,
                                       uint32_t query_count, uint32_t top_k,
                                       tsg_token_expert_pair* out);
/* PrefillMoEGrouping.groupTokenExpertPairs (PrefillMoEGrouping.swift:90-202),
 * host: sort by (sort_key[expert], expert, token, rank), per-expert offsets
 * (0xFFFFFFFF when absent) and counts, groups, tiles of <= tile_expert_count
 * groups. sort_keys may be NULL; tile_break_after_group < 0 means none.
 * Output arrays: sorted n_pairs, offsets/counts num_experts, groups and tiles
 * n_pairs each at most. Errors: TSG_ERR_GROUPING_*. */
tsg_status tsg_group_token_expert_pairs(const tsg_token_expert_pair* pairs, uint32_t n_pairs,
                                        uint32_t query_count, uint32_t top_k,
                                        uint32_t num_experts, uint32_t tile_expert_count,
                                        const uint64_t* sort_keys, uint32_t n_sort_keys,
                                        int32_t tile_break_after_group,
                                        tsg_token_expert_pair* sorted, uint32_t* offsets,
                                        uint32_t* counts, tsg_moe_group* groups,
                                        uint32_t* n_groups, tsg_moe_tile* tiles,
                                        uint32_t* n_tiles);
/* PrefillRoutedGEMMPlanner.plan (PrefillGroupedRoutedMoE.swift:42-83), host:
 * batches of <= 64-row blocks that never split a group that fits. Arrays are
 * sized by the caller: blocks >= total pairs / 1 + n_groups, batches likewise. */
tsg_status tsg_plan_routed_gemm(const tsg_moe_group* groups, uint32_t n_groups,
                                uint32_t max_rows_per_batch, tsg_routed_block* blocks,
                                uint32_t* n_blocks, uint32_t* batch_rows,
                                uint32_t* batch_first_block, uint32_t* n_batches);

/* The same grouping on the device, for an HBM-resident layer: token-major
 * routing (indices/weights [query_count, top_k]) -> pairs sorted by
 * (expert, token, rank) (bit-identical to the host sort), per-expert offsets
 * and counts, and the GEMM's work list of <= tile_rows-row blocks with
 * local_slot = expert id and local_row = pair_start, largest first (by
 * ceil(rows / 32), capped at 8, then expert order): the grouped GEMMs take a
 * list whose count is on the device in this order. *n_blocks (device) gets
 * the block count; max_blocks bounds the blocks array. tile_rows: 32, 64 (the
 * reference's block), 128 (the grouped GEMM's widest pass) or 256.
 * scratch: tsg_prefill_group_scratch_bytes(...) bytes of device memory. */
size_t tsg_prefill_group_scratch_bytes(uint32_t query_count, uint32_t top_k,
                                       uint32_t num_experts);
tsg_status tsg_prefill_group_pairs_device(tsg_ctx* ctx, tsg_stream stream,
                                          const uint32_t* indices, const uint16_t* weights,
                                          uint32_t query_count, uint32_t top_k,
                                          uint32_t num_experts, uint32_t tile_rows,
                                          tsg_token_expert_pair* sorted, uint32_t* offsets,
                                          uint32_t* counts, tsg_routed_block* blocks,
                                          uint32_t max_blocks, uint32_t* n_blocks,
                                          void* scratch);
/* tsg_prefill_group_pairs_device without the scratch argument: no counterpart
 * in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc):
 * it calls no allocating routine; the pairs' ranks live in a 256 KiB
 * file-scope device array, one per GPU, held until the process ends. Same
 * arguments, checks and results as tsg_prefill_group_pairs_device; also
 * TSG_ERR_UNSUPPORTED when query_count * top_k exceeds 65536 pairs. Every
 * call on one GPU uses that GPU's array: calls that overlap on one GPU (two
 * streams, two host threads) race and must be serialised by the caller. */
tsg_status tsg_prefill_group_pairs_device_noalloc(tsg_ctx* ctx, tsg_stream stream,
                                                  const uint32_t* indices,
                                                  const uint16_t* weights,
                                                  uint32_t query_count, uint32_t top_k,
                                                  uint32_t num_experts, uint32_t tile_rows,
                                                  tsg_token_expert_pair* sorted,
                                                  uint32_t* offsets, uint32_t* counts,
                                                  tsg_routed_block* blocks,
                                                  uint32_t max_blocks, uint32_t* n_blocks);

/* encodeStreamedTiled mode 0 + gelu_mul (PrefillGroupedRoutedMoE.swift:931-1051,
 * prefill.metal:3664-3864, 1081-1092) on a resident layer: for every block,
 * gather hidden rows by pair token, G = X Wg^T and U = X Wu^T on fp16 MFMA with
 * fp32 accumulation, weights dequantised to fp16 exactly as the reference
 * stages them; act[(local_row + r)*F + f] = half(act(half(G)) * half(U)).
 * Blocks of any size (the kernel runs 128 rows per pass). d and f must be
 * multiples of 64; at group size 32 the scale/bias sub-tensor offsets must be
 * 4-byte aligned (TSG_ERR_ALIGNMENT).
 * n_blocks_device: optional device count bounding `blocks` (may be NULL, then
 * n_blocks is used). A block naming an expert past the layer is skipped and
 * tsg_ctx_synchronize reports TSG_ERR_INVALID_ARGUMENT (the list may live on
 * the device, out of the host's sight); the same holds for
 * tsg_prefill_moe_down and tsg_prefill_moe_gate_up_down. */
tsg_status tsg_prefill_moe_gate_up(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                   const uint16_t* hidden, uint32_t hidden_stride_elements,
                                   const tsg_token_expert_pair* sorted_pairs,
                                   const tsg_routed_block* blocks, uint32_t n_blocks,
                                   const uint32_t* n_blocks_device, uint16_t* act,
                                   uint32_t d, uint32_t f);
/* encodeStreamedTiled mode 1 (prefill.metal:3680-3716): P = act Wd^T,
 * route_partials[(token*top_k + rank)*D + d] = half(P). */
tsg_status tsg_prefill_moe_down(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                const uint16_t* act, const tsg_token_expert_pair* sorted_pairs,
                                const tsg_routed_block* blocks, uint32_t n_blocks,
                                const uint32_t* n_blocks_device, uint16_t* route_partials,
                                uint32_t top_k, uint32_t d, uint32_t f);
/* encodeStreamedTiled modes 0 and 1 (PrefillGroupedRoutedMoE.swift:931-1051,
 * the two encodes the reference issues back to back) in one persistent
 * launch: exactly tsg_prefill_moe_gate_up followed by tsg_prefill_moe_down on
 * the same arguments (bit-identical act and route_partials), with the down
 * tiles of a block starting as soon as that block's gate/up tiles are done.
 * The reference has no single call for the pair; a caller that issues the two
 * encodes back to back replaces them with this one. act must be 128-byte
 * aligned (TSG_ERR_ALIGNMENT); at most 65536 blocks. The schedule words live
 * in the context: fused launches on one context must not overlap (one stream
 * or ordered streams). A wait that times out or a schedule left undrained is
 * reported by tsg_ctx_synchronize (TSG_ERR_HIP). */
tsg_status tsg_prefill_moe_gate_up_down(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                        const uint16_t* hidden, uint32_t hidden_stride_elements,
                                        const tsg_token_expert_pair* sorted_pairs,
                                        const tsg_routed_block* blocks, uint32_t n_blocks,
                                        const uint32_t* n_blocks_device, uint16_t* act,
                                        uint16_t* route_partials, uint32_t top_k, uint32_t d,
                                        uint32_t f);
/* encodeStreamedRows (PrefillGroupedRoutedMoE.swift:793-917,
 * prefill.metal:1489-1721): verify-width blocks (row_count <= 8), decode's
 * per-row arithmetic with each weight read once per block; writes act rows
 * (act_scratch: block rows local_row .. local_row + row_count - 1, each f
 * fp16) and route partials. act_scratch holds max_rows rows (the reference's
 * maxRows, the rows the scratch was sized for). `blocks` is a HOST array (the
 * reference passes it with setBytes); local_slot is the expert id in the
 * resident layer. Returns TSG_ERR_DECLINED, with nothing launched, when a
 * block holds no rows or more than 8, or when a block's rows reach past
 * max_rows (`guard rows <= maxRows else { return 0 }`,
 * PrefillGroupedRoutedMoE.swift:830). */
tsg_status tsg_prefill_moe_rows(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                const uint16_t* hidden, uint32_t hidden_stride_elements,
                                const tsg_token_expert_pair* sorted_pairs,
                                const tsg_routed_block* blocks, uint32_t n_blocks,
                                uint16_t* act_scratch, uint32_t max_rows,
                                uint16_t* route_partials, uint32_t top_k, uint32_t d,
                                uint32_t f);
/* encodeStreamedRows with the block list left on the device, where
 * tsg_prefill_group_pairs_device (any tile_rows >= the token count) writes it:
 * the verify block's grouping (RealForwardRunner.swift:2116-2151) without a
 * host round trip. blocks holds max_blocks entries (<= 65535), the first
 * *n_blocks_device of them live; each live block gives exactly
 * tsg_prefill_moe_rows' results for it. act_scratch holds max_rows rows of f
 * fp16. A live block with no rows, more than 8, rows past max_rows or an
 * expert past the layer is skipped and tsg_ctx_synchronize reports
 * TSG_ERR_INVALID_ARGUMENT (the host form declines such a list up front).
 * No counterpart entry in the reference, which reads the grouping back to the
 * host. */
tsg_status tsg_prefill_moe_rows_device(tsg_moe* moe, tsg_stream stream, const tsg_layer* layer,
                                       const uint16_t* hidden, uint32_t hidden_stride,
                                       const tsg_token_expert_pair* sorted_pairs,
                                       const tsg_routed_block* blocks, uint32_t max_blocks,
                                       const uint32_t* n_blocks_device, uint16_t* act_scratch,
                                       uint32_t max_rows, uint16_t* route_partials,
                                       uint32_t top_k, uint32_t d, uint32_t f);
/* PrefillMoE.encodeReduceTokenMajor (PrefillMoE.swift:11-38):
 * h2[t,d] = half(sum_{r<top_k} fma(w[t,r], P[(t*top_k + r), d])). */
tsg_status tsg_prefill_moe_reduce_token_major(tsg_ctx* ctx, tsg_stream stream,
                                              const uint16_t* route_partials,
                                              const uint16_t* route_weights, uint16_t* h2,
                                              uint32_t query_count, uint32_t top_k,
                                              uint32_t d);

/* PrefillInt4QMM.encode (PrefillPrimitives.swift:75-175; the tiled kernel
 * prefill_int4_qmm_simdgroup_f16 and MPPPrefillInt4QMM.encode,
 * MPPPrefillInt4QMM.swift:104-158): the dense int4 projection over t tokens,
 * y[t, n] = half(sum_k x[t, k] * half(dequant(W[n, k]))), fp32 accumulation.
 * W is [n, k/2] bytes, scales and biases [n, k/group] bf16 (biases unused
 * under sym). The dequant-to-LDS MFMA GEMM of the routed experts, rows taken
 * in order. Errors: K % group != 0 (the reference's precondition). Declined
 * with TSG_ERR_UNSUPPORTED: K or N not a multiple of 64, t*n or t*k >= 2^32,
 * or W of 4 GiB or more. */
tsg_status tsg_prefill_int4_qmm(tsg_ctx* ctx, tsg_stream stream, const uint8_t* weights,
                                const uint16_t* scales, const uint16_t* biases,
                                const uint16_t* x, uint16_t* y, uint32_t t, uint32_t n,
                                uint32_t k);

/* ----------------------------------------------------------- layer tail ----
 * The Gemma decoder-layer tail after the MoE FFN, per row (fp16 h2, h1,
 * hidden; bf16 norm weights):
 *   h12    = half(h1 + half(h2 * rms_inv(h2) * post_ffn_2))
 *   hidden = half(half(hidden + half(h12 * rms_inv(h12) * post_ffn)) * half(layer_scalar))
 * rms_inv(x) = 1/sqrt(sum(x^2)/D + eps). Each row's sums run in one fixed order
 * over the element index, so all three entry points give identical bits for a
 * row whatever its strides. hidden is updated in place.
 *
 * PrefillLayerTail.encode (PrefillLayerTail.swift:11-58,
 * prefill_layer_tail_block prefill.metal:319-397). Errors: queryCount == 0,
 * D outside 1...4096, a stride below D. */
tsg_status tsg_prefill_layer_tail(tsg_ctx* ctx, tsg_stream stream, const uint16_t* h2,
                                  const uint16_t* h1, uint16_t* hidden,
                                  const uint16_t* post_ffn2_weight,
                                  const uint16_t* post_ffn_weight, uint32_t query_count,
                                  uint32_t d, uint32_t h2_stride_elements,
                                  uint32_t h1_stride_elements, uint32_t hidden_stride_elements,
                                  float eps, float layer_scalar);
/* FusedLayerTail.encode (FusedLayerTail.swift:25-56, fused_layer_tail
 * fused.metal:271-374): one contiguous row. D > 4096 is an error; D == 0 does
 * nothing. */
tsg_status tsg_fused_layer_tail(tsg_ctx* ctx, tsg_stream stream, const uint16_t* h2,
                                const uint16_t* h1, uint16_t* hidden,
                                const uint16_t* post_ffn2_weight, const uint16_t* post_ffn_weight,
                                uint32_t d, float eps, float layer_scalar);
/* PrefillMoE.encodeReduceTokenMajor followed by PrefillLayerTail.encode in one
 * launch (PrefillMoE.swift:11-38 then PrefillLayerTail.swift:11-58): h2 is
 * formed in registers with the reduce's per-element fma order, written to
 * h2_out only when h2_out is not NULL (contiguous [query_count, d]). Same bits
 * as the two entry points in sequence. */
tsg_status tsg_prefill_moe_reduce_layer_tail(
    tsg_ctx* ctx, tsg_stream stream, const uint16_t* route_partials,
    const uint16_t* route_weights, uint16_t* h2_out, const uint16_t* h1, uint16_t* hidden,
    const uint16_t* post_ffn2_weight, const uint16_t* post_ffn_weight, uint32_t query_count,
    uint32_t top_k, uint32_t d, uint32_t h1_stride_elements, uint32_t hidden_stride_elements,
    float eps, float layer_scalar);

/* ------------------------------------------------------ MoEPack install ----
 * Reader of an installed pack's manifest.json and packed_experts/layout.json,
 * and the layer-file upload that replaces the SSD streamer: the reference
 * opens a layer file and preads expert blobs into slot buffers on demand
 * (ModelExpertIO.swift:112-324); here the whole layer is resident in HBM with
 * each blob at its logical expert index, so the kernels address expert e at
 * base + e * expert_stride whatever the file's physical order.
 *
 * Validation restates ManifestReader.decode/validate (ManifestReader.swift:
 * 182-313), MoEPackManifestCodec.validate (MoEPackManifestV1.swift:378-559),
 * MoEPackV1StructuralValidator.validate/crossValidate
 * (MoEPackPackedExpertsLayoutV1.swift:84-211). Failures return TSG_ERR_FORMAT
 * (content) or TSG_ERR_IO (file system); tsg_last_error() starts with the
 * reference's ModelError case: indexCorrupt, notAMoEPackDirectory,
 * unsupportedVersion, unknownFlag, expertStrideNotPageAligned, missingFile,
 * partialInstall, posixFailed. Not restated: the field-by-field comparison
 * with a compiled ArchConfig (validateArch; the caller compares the
 * dimensions in tsg_moepack_info) and the vision/draft geometry checks (their
 * weights are not read here). */
typedef struct tsg_moepack tsg_moepack;

typedef struct tsg_moepack_info {
    uint32_t num_layers;            /* manifest.numLayers                          */
    uint32_t experts_per_layer;     /* manifest.expertsPerLayer                    */
    uint64_t expert_stride;         /* bytes per expert blob, a multiple of 16384  */
    uint32_t hidden_size;           /* arch.hiddenSize                             */
    uint32_t moe_intermediate_size; /* arch.moeIntermediateSize                    */
    uint32_t top_k;                 /* arch.topKExperts                            */
    uint32_t version_minor;
    uint32_t legacy_magic;          /* 1: magic "GTURBO", 0: "MOEPACK"             */
    uint32_t has_quant;             /* 0: the manifest has no quant section        */
    uint32_t affine_group_size;     /* quant.embedding.groupSize (32|64), 0 if none */
    uint32_t symmetric;             /* 1: the 4-bit slots use `sym` (no biases)    */
    uint32_t routed_weight_bits;    /* quant.routedExpert.weightBits               */
    uint32_t shared_weight_bits;    /* quant.sharedExpert.weightBits               */
    uint32_t router_weight_bits;    /* quant.router.weightBits (8 or 16)           */
    uint32_t has_layout;            /* layout.json read and cross-validated        */
    uint32_t is_gemma4;             /* arch.family absent (ManifestArch.isGemma4)  */
    char family[32];                /* arch.family, "" when absent                 */
} tsg_moepack_info;

/* SubTensorEntry (PackedExpertsLayout.swift:4-10) plus the owning expert's
 * physical rank. */
typedef struct tsg_moepack_subtensor {
    uint64_t offset, size;   /* bytes, relative to the expert blob            */
    uint32_t dtype;          /* MoEPackFormatV1.DType: 0 U32, 1 BF16          */
    uint32_t bits;           /* weight width from the layout, 0 when absent   */
    uint32_t rank;           /* shape entries (the first 8 are in `shape`)    */
    uint32_t shape[8];
    uint32_t physical_rank;  /* ExpertEntry.physicalRank of this expert       */
} tsg_moepack_subtensor;

/* ManifestReader.load + PackedExpertsLayoutReader.load(manifest:)
 * (ManifestReader.swift:169-180, PackedExpertsLayout.swift:60-81). Files are
 * opened component by component without following symlinks, must be regular
 * files, and are size-capped before reading (0 = the reference defaults:
 * 4 MiB manifest, 64 MiB layout). The directory stays open for
 * tsg_moepack_load_layer. */
tsg_status tsg_moepack_open(const char* directory, uint64_t manifest_max_bytes,
                            uint64_t layout_max_bytes, tsg_moepack** out);
/* ManifestReader.decode(data:) and PackedExpertsLayoutReader.decode(data:
 * manifest:) on in-memory documents; layout_json may be NULL (manifest only).
 * A parsed pack has no layer files to load. */
tsg_status tsg_moepack_parse(const char* manifest_json, uint64_t manifest_len,
                             const char* layout_json, uint64_t layout_len, tsg_moepack** out);
void tsg_moepack_close(tsg_moepack* pack);
tsg_status tsg_moepack_get_info(const tsg_moepack* pack, tsg_moepack_info* out);
/* Model.routedExpertOffsets(layer:) (ModelExpertIO.swift:56-84): expert 0's
 * gate/up/down sub-tensor offsets; without `<role>_biases` the bias offset
 * aliases `<role>_scales`. TSG_ERR_FORMAT when a role is missing. */
tsg_status tsg_moepack_routed_offsets(const tsg_moepack* pack, uint32_t layer,
                                      tsg_expert_offsets* out);
/* Model.routedExpertPhysicalOffsets(layer:) (ModelExpertIO.swift:86-88):
 * offsets[e] = byte offset of logical expert e's blob in the layer file;
 * count must equal experts_per_layer. */
tsg_status tsg_moepack_physical_offsets(const tsg_moepack* pack, uint32_t layer,
                                        uint64_t* offsets, uint32_t count);
/* PackedExpertsLayout.expert(layer:expert:).subTensors[name]
 * (PackedExpertsLayout.swift:51-54); `expert` is the logical id. */
tsg_status tsg_moepack_tensor(const tsg_moepack* pack, uint32_t layer, uint32_t expert,
                              const char* name, tsg_moepack_subtensor* out);
/* Reads packed_experts/<file> of `layer` (its size must be experts_per_layer
 * * expert_stride) and returns a new HBM-resident tsg_layer holding logical
 * expert e at e * expert_stride, with tsg_moepack_routed_offsets. The upload
 * goes through two pinned staging buffers of at most 64 MiB on `stream` and
 * has finished when this returns. The caller sets the context's group size
 * and scheme from tsg_moepack_info. */
tsg_status tsg_moepack_load_layer(const tsg_moepack* pack, tsg_ctx* ctx, tsg_stream stream,
                                  uint32_t layer, tsg_layer** out);
/* The same upload into an existing layer (tsg_layer_create or caller-owned HBM
 * through tsg_layer_wrap, e.g. one arena for every layer). The layer must have
 * experts_per_layer experts, the pack's stride and tsg_moepack_routed_offsets;
 * otherwise TSG_ERR_INVALID_ARGUMENT and nothing is written. */
tsg_status tsg_moepack_upload_layer(const tsg_moepack* pack, tsg_stream stream, uint32_t layer,
                                    tsg_layer* dst);

/* ---------------------------------------------- synthetic fixtures ------
 * Device generators for benchmark inputs (no reference counterpart; the
 * reference's fixtures come from SplitMix64 on the host). Element i of a
 * stream keyed `seed` is derived from SplitMix64 output i of that seed
 * (counter-based), so any slice can be regenerated independently. */
/* n bytes of uniform nibbles. */
tsg_status tsg_gen_bytes(tsg_stream stream, uint64_t seed, uint8_t* out, uint64_t n);
/* n bf16 values sigma * N(0,1) (Irwin-Hall of 12 uniforms), abs_value: |.|,
 * divisor applied after (scale = |N(0,0.02)|/7 -> sigma .02, abs 1, div 7). */
tsg_status tsg_gen_bf16_normal(tsg_stream stream, uint64_t seed, uint16_t* out, uint64_t n,
                               float sigma, int abs_value, float divisor);
/* n fp16 values sigma * N(0,1), with |x| < 2^-17 flushed to zero. */
tsg_status tsg_gen_f16_normal(tsg_stream stream, uint64_t seed, uint16_t* out, uint64_t n,
                              float sigma);

#ifdef __cplusplus
}
#endif
#endif /* TSUGUMI_HIP_H */
