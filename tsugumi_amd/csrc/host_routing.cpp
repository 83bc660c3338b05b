// host_routing.cpp — host side of the prompt-chunk routing: token-major pairs,
// expert grouping and the GEMM batch planner, with the reference's error
// cases. Pure C++ (no device code).
//
//   makeTokenExpertPairs   PrefillRouter.swift:238-258
//   groupTokenExpertPairs  PrefillMoEGrouping.swift:90-202
//   PrefillRoutedGEMMPlanner.plan  PrefillGroupedRoutedMoE.swift:42-83
#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <numeric>
#include <vector>

#include "../../include/tsugumi_hip.h"

namespace tsg {
tsg_status fail(tsg_status status, const char* fmt, ...);
}

using tsg::fail;

extern "C" tsg_status tsg_make_token_expert_pairs(const uint32_t* indices,
                                                  const uint16_t* weights,
                                                  uint32_t query_count, uint32_t top_k,
                                                  tsg_token_expert_pair* out) {
    if ((query_count * top_k) && (!indices || !weights || !out))
        return fail(TSG_ERR_INVALID_ARGUMENT, "NULL indices/weights/out");
    for (uint32_t t = 0; t < query_count; ++t)
        for (uint32_t r = 0; r < top_k; ++r) {
            const uint32_t i = t * top_k + r;
            out[i] = tsg_token_expert_pair{t, indices[i], r, (uint32_t)weights[i]};
        }
    return TSG_OK;
}

extern "C" tsg_status tsg_group_token_expert_pairs(
    const tsg_token_expert_pair* pairs, uint32_t n_pairs, uint32_t query_count, uint32_t top_k,
    uint32_t num_experts, uint32_t tile_expert_count, const uint64_t* sort_keys,
    uint32_t n_sort_keys, int32_t tile_break_after_group, tsg_token_expert_pair* sorted,
    uint32_t* offsets, uint32_t* counts, tsg_moe_group* groups, uint32_t* n_groups,
    tsg_moe_tile* tiles, uint32_t* n_tiles) {
    // The Swift API takes signed Ints; negative counts arrive here as huge
    // unsigned values and are reported as the reference's "invalid" cases.
    if ((int32_t)query_count < 0)
        return fail(TSG_ERR_GROUPING_INVALID_QUERY_COUNT,
                    "queryCount must be non-negative, got %d", (int32_t)query_count);
    if ((int32_t)top_k <= 0)
        return fail(TSG_ERR_GROUPING_INVALID_TOP_K, "topK must be positive, got %d",
                    (int32_t)top_k);
    if ((int32_t)num_experts <= 0)
        return fail(TSG_ERR_GROUPING_INVALID_NUM_EXPERTS, "numExperts must be positive, got %d",
                    (int32_t)num_experts);
    if (tile_expert_count < 1 || tile_expert_count > 16)
        return fail(TSG_ERR_GROUPING_INVALID_TILE_EXPERT_COUNT,
                    "tileExpertCount must be in 1...16, got %u", tile_expert_count);
    if (sort_keys && n_sort_keys != num_experts)
        return fail(TSG_ERR_GROUPING_SORT_KEY_COUNT_MISMATCH,
                    "expected %u expert sort keys, got %u", num_experts, n_sort_keys);
    const uint64_t expected = (uint64_t)query_count * top_k;
    if (n_pairs != expected)
        return fail(TSG_ERR_GROUPING_PAIR_COUNT_MISMATCH, "expected %llu route pairs, got %u",
                    (unsigned long long)expected, n_pairs);
    if (n_pairs && (!pairs || !sorted || !groups || !tiles))
        return fail(TSG_ERR_INVALID_ARGUMENT, "NULL pair/group/tile array");
    if (!offsets || !counts || !n_groups || !n_tiles)
        return fail(TSG_ERR_INVALID_ARGUMENT, "NULL offsets/counts/count outputs");

    std::vector<uint8_t> seen(expected, 0);
    for (uint32_t i = 0; i < n_pairs; ++i) {
        const tsg_token_expert_pair& p = pairs[i];
        if (p.token >= query_count)
            return fail(TSG_ERR_GROUPING_TOKEN_OUT_OF_RANGE, "route token %u is out of range",
                        p.token);
        if (p.rank >= top_k)
            return fail(TSG_ERR_GROUPING_RANK_OUT_OF_RANGE, "route rank %u is out of range",
                        p.rank);
        if (p.expert >= num_experts)
            return fail(TSG_ERR_GROUPING_EXPERT_OUT_OF_RANGE, "route expert %u is out of range",
                        p.expert);
        uint8_t& s = seen[(uint64_t)p.token * top_k + p.rank];
        if (s)
            return fail(TSG_ERR_GROUPING_DUPLICATE_TOKEN_RANK,
                        "duplicate route pair for token %u, rank %u", p.token, p.rank);
        s = 1;
    }

    std::vector<uint32_t> order(n_pairs);
    std::iota(order.begin(), order.end(), 0u);
    std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
        const tsg_token_expert_pair& x = pairs[a];
        const tsg_token_expert_pair& y = pairs[b];
        if (sort_keys) {
            const uint64_t kx = sort_keys[x.expert], ky = sort_keys[y.expert];
            if (kx != ky) return kx < ky;
        }
        if (x.expert != y.expert) return x.expert < y.expert;
        if (x.token != y.token) return x.token < y.token;
        return x.rank < y.rank;
    });
    for (uint32_t i = 0; i < n_pairs; ++i) sorted[i] = pairs[order[i]];

    for (uint32_t e = 0; e < num_experts; ++e) {
        offsets[e] = 0xFFFFFFFFu;
        counts[e] = 0;
    }
    uint32_t ng = 0;
    for (uint32_t i = 0; i < n_pairs;) {
        const uint32_t expert = sorted[i].expert;
        const uint32_t start = i;
        while (i < n_pairs && sorted[i].expert == expert) ++i;
        offsets[expert] = start;
        counts[expert] = i - start;
        groups[ng++] = tsg_moe_group{expert, start, i - start};
    }
    *n_groups = ng;

    uint32_t nt = 0;
    for (uint32_t gs = 0; gs < ng;) {
        uint32_t ge = std::min(ng, gs + tile_expert_count);
        if (tile_break_after_group >= 0 && gs < (uint32_t)tile_break_after_group)
            ge = std::min(ge, (uint32_t)tile_break_after_group);
        const tsg_moe_group& first = groups[gs];
        const tsg_moe_group& last = groups[ge - 1];
        tiles[nt++] = tsg_moe_tile{gs, ge - gs, first.pair_start,
                                   last.pair_start + last.pair_count - first.pair_start};
        gs = ge;
    }
    *n_tiles = nt;
    return TSG_OK;
}

extern "C" tsg_status tsg_plan_routed_gemm(const tsg_moe_group* groups, uint32_t n_groups,
                                           uint32_t max_rows_per_batch,
                                           tsg_routed_block* blocks, uint32_t* n_blocks,
                                           uint32_t* batch_rows, uint32_t* batch_first_block,
                                           uint32_t* n_batches) {
    if ((n_groups && (!groups || !blocks || !batch_rows || !batch_first_block)) || !n_blocks ||
        !n_batches)
        return fail(TSG_ERR_INVALID_ARGUMENT, "NULL planner argument");
    const uint32_t tile_rows = 64;
    const uint32_t budget = std::max(tile_rows, (max_rows_per_batch / tile_rows) * tile_rows);
    uint32_t nb = 0, nbatch = 0, rows = 0, batch_start = 0;
    auto flush = [&]() {
        if (rows == 0) return;
        batch_rows[nbatch] = rows;
        batch_first_block[nbatch] = batch_start;
        ++nbatch;
        batch_start = nb;
        rows = 0;
    };
    for (uint32_t slot = 0; slot < n_groups; ++slot) {
        uint32_t taken = 0;
        const uint32_t count = groups[slot].pair_count;
        while (taken < count) {
            if (rows == budget) flush();
            // A group that fits in an empty batch is never split.
            if (rows > 0 && rows + (count - taken) > budget) flush();
            const uint32_t take = std::min(count - taken, budget - rows);
            for (uint32_t done = 0; done < take;) {
                const uint32_t rc = std::min(tile_rows, take - done);
                blocks[nb++] = tsg_routed_block{slot, groups[slot].pair_start + taken + done, rc,
                                                rows + done};
                done += rc;
            }
            rows += take;
            taken += take;
        }
    }
    flush();
    *n_blocks = nb;
    *n_batches = nbatch;
    return TSG_OK;
}
