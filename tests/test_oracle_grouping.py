"""Pins the oracle's prefill routing restatements with the reference's own
literal golden arrays:

- PrefillMoEGroupingTests.swift:5-258 (sort by (expert, token, rank),
  per-expert offsets/counts, groups, 16-expert tiles, sort keys, tile break,
  error cases);
- PrefillRoutedGEMMPlannerTests.swift:38-88 (batch/block splits);
- PrefillRouterTests.swift:21-30 (token-major pairs).
"""
import numpy as np
import pytest


def P(token, expert, rank, w):
    return (token, expert, rank, w)


def pairs_array(oracle, rows):
    return np.array(rows, dtype=oracle.PAIR_DTYPE)


def test_grouping_sorts_pairs_and_builds_offsets_counts_tiles(oracle):
    rows = [P(0, 3, 0, 10), P(0, 1, 1, 11), P(0, 4, 2, 12), P(1, 1, 0, 13), P(1, 3, 1, 14),
            P(1, 2, 2, 15), P(2, 4, 0, 16), P(2, 3, 1, 17), P(2, 1, 2, 18), P(3, 5, 0, 19),
            P(3, 1, 1, 20), P(3, 4, 2, 21)][::-1]
    g = oracle.group_pairs(pairs_array(oracle, rows), 4, 3, 6, tile_expert_count=2)
    sp = g["sorted_pairs"]
    assert list(sp["expert"]) == [1, 1, 1, 1, 2, 3, 3, 3, 4, 4, 4, 5]
    assert [[int(a), int(b)] for a, b in zip(sp["token"], sp["rank"])] == [
        [0, 1], [1, 0], [2, 2], [3, 1], [1, 2], [0, 0], [1, 1], [2, 1], [0, 2], [2, 0],
        [3, 2], [3, 0]]
    assert list(g["offsets"]) == [0xFFFFFFFF, 0, 4, 5, 8, 11]
    assert list(g["counts"]) == [0, 4, 1, 3, 3, 1]
    assert [tuple(x) for x in g["groups"].tolist()] == [
        (1, 0, 4), (2, 4, 1), (3, 5, 3), (4, 8, 3), (5, 11, 1)]
    assert [tuple(x) for x in g["tiles"].tolist()] == [
        (0, 2, 0, 5), (2, 2, 5, 6), (4, 1, 11, 1)]
    assert int(g["groups"]["pair_count"].max()) == 4
    assert int(g["tiles"]["pair_count"].max()) == 6
    assert int(g["tiles"]["group_count"].max()) == 2


def test_grouping_is_order_independent_and_keeps_weight_bits(oracle):
    token_major = [P(0, 2, 0, 101), P(0, 1, 1, 102), P(1, 2, 0, 103), P(1, 0, 1, 104),
                   P(2, 1, 0, 105), P(2, 2, 1, 106)]
    shuffled = [token_major[i] for i in (5, 1, 3, 0, 4, 2)]
    a = oracle.group_pairs(pairs_array(oracle, token_major), 3, 2, 3, tile_expert_count=2)
    b = oracle.group_pairs(pairs_array(oracle, shuffled), 3, 2, 3, tile_expert_count=2)
    for key in a:
        assert np.array_equal(a[key], b[key])
    assert list(a["sorted_pairs"]["weight_bits"]) == [104, 102, 105, 101, 103, 106]


def test_grouping_orders_tiles_by_expert_sort_keys(oracle):
    rows = [P(0, 1, 0, 10), P(0, 2, 1, 20), P(1, 3, 0, 30), P(1, 1, 1, 11), P(2, 2, 0, 21),
            P(2, 3, 1, 31)]
    g = oracle.group_pairs(pairs_array(oracle, rows), 3, 2, 4, tile_expert_count=2,
                           expert_sort_keys=[0, 30, 10, 20])
    assert list(g["groups"]["expert"]) == [2, 3, 1]
    assert list(g["sorted_pairs"]["expert"]) == [2, 2, 3, 3, 1, 1]
    assert list(g["offsets"]) == [0xFFFFFFFF, 4, 0, 2]
    assert [tuple(x) for x in g["tiles"].tolist()] == [(0, 2, 0, 4), (2, 1, 4, 2)]


@pytest.mark.parametrize("kwargs,rows,case", [
    (dict(query_count=1, top_k=1, num_experts=1, tile_expert_count=17),
     [P(0, 0, 0, 1)], "invalidTileExpertCount"),
    (dict(query_count=1, top_k=1, num_experts=2, tile_expert_count=1),
     [P(0, 2, 0, 1)], "expertOutOfRange"),
    (dict(query_count=1, top_k=2, num_experts=2, tile_expert_count=1),
     [P(0, 0, 0, 1), P(0, 1, 0, 2)], "duplicateTokenRank"),
    (dict(query_count=1, top_k=1, num_experts=2, tile_expert_count=1, expert_sort_keys=[0]),
     [P(0, 0, 0, 1)], "expertSortKeyCountMismatch"),
    (dict(query_count=2, top_k=1, num_experts=2, tile_expert_count=1),
     [P(0, 0, 0, 1)], "pairCountMismatch"),
    (dict(query_count=1, top_k=1, num_experts=2, tile_expert_count=1),
     [P(1, 0, 0, 1)], "tokenOutOfRange"),
    (dict(query_count=1, top_k=1, num_experts=2, tile_expert_count=1),
     [P(0, 0, 1, 1)], "rankOutOfRange"),
])
def test_grouping_rejects_invalid_metadata(oracle, kwargs, rows, case):
    with pytest.raises(oracle.GroupingError) as err:
        oracle.group_pairs(pairs_array(oracle, rows), **kwargs)
    assert err.value.case == case


def test_grouping_tolerates_real_trace_pressure_at_t32(oracle):
    rows = [P(t, (t + r * 7) % 74, r, t * 8 + r) for t in range(32) for r in range(8)]
    g = oracle.group_pairs(pairs_array(oracle, rows), 32, 8, 128, tile_expert_count=16)
    assert g["sorted_pairs"].size == 256
    assert g["groups"].size <= 74
    assert np.all(g["tiles"]["group_count"] <= 16)
    assert np.all(g["tiles"]["pair_count"] > 0)


def test_tile_break_cuts_at_requested_group(oracle):
    rows = [P(t, (t * 5 + r) % 10, r, t * 5 + r) for t in range(4) for r in range(5)]
    g = oracle.group_pairs(pairs_array(oracle, rows), 4, 5, 10, tile_expert_count=4,
                           tile_break_after_group=3)
    assert g["groups"].size == 10
    assert list(g["tiles"]["group_count"]) == [3, 4, 3]
    assert list(g["tiles"]["group_start"]) == [0, 3, 7]
    assert int(g["tiles"]["pair_count"].sum()) == g["sorted_pairs"].size
    start = 0
    for t in g["tiles"]:
        assert int(t["pair_start"]) == start
        start += int(t["pair_count"])


def test_tile_break_beyond_groups_changes_nothing(oracle):
    rows = [P(i // 2, i % 4, i % 2, i) for i in range(8)]
    a = oracle.group_pairs(pairs_array(oracle, rows), 4, 2, 4, tile_expert_count=2)
    b = oracle.group_pairs(pairs_array(oracle, rows), 4, 2, 4, tile_expert_count=2,
                           tile_break_after_group=99)
    assert np.array_equal(a["tiles"], b["tiles"])


def test_token_expert_pairs_are_token_major(oracle):
    w = oracle.f16_bits(np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6], np.float32))
    p = oracle.make_token_expert_pairs(np.array([3, 1, 2, 4, 0, 5]), w, 2, 3)
    assert list(p["token"]) == [0, 0, 0, 1, 1, 1]
    assert list(p["rank"]) == [0, 1, 2, 0, 1, 2]
    assert list(p["expert"]) == [3, 1, 2, 4, 0, 5]
    assert np.array_equal(p["weight_bits"].astype(np.uint16), w)


# ---- planner: PrefillRoutedGEMMPlannerTests.swift:38-88 -------------------

def G(oracle, rows):
    return np.array(rows, dtype=oracle.GROUP_DTYPE)


def covers_exactly_once(batches, groups):
    seen = {}
    for rows, blocks in batches:
        local = set()
        for b in blocks:
            assert 1 <= b["row_count"] <= 64
            assert int(b["local_row"]) + int(b["row_count"]) <= rows
            for i in range(int(b["row_count"])):
                assert int(b["local_row"]) + i not in local
                local.add(int(b["local_row"]) + i)
                pair = int(b["pair_start"]) + i
                seen[pair] = seen.get(pair, 0) + 1
                g = groups[int(b["local_slot"])]
                assert g["pair_start"] <= pair < g["pair_start"] + g["pair_count"]
        assert len(local) == rows
    expected = [int(g["pair_start"]) + i for g in groups for i in range(int(g["pair_count"]))]
    assert sorted(seen) == sorted(expected)
    assert all(v == 1 for v in seen.values())


def test_planner_packs_whole_groups_when_they_fit(oracle):
    groups = G(oracle, [(3, 0, 40), (7, 40, 20)])
    b = oracle.plan_routed_gemm(groups, 128)
    assert len(b) == 1 and b[0][0] == 60 and b[0][1].size == 2
    assert b[0][1][1]["local_row"] == 40 and b[0][1][1]["local_slot"] == 1
    covers_exactly_once(b, groups)


def test_planner_starts_new_batch_rather_than_split(oracle):
    groups = G(oracle, [(0, 0, 100), (1, 100, 100)])
    b = oracle.plan_routed_gemm(groups, 128)
    assert [r for r, _ in b] == [100, 100]
    assert list(b[0][1]["row_count"]) == [64, 36]
    covers_exactly_once(b, groups)


def test_planner_splits_large_group_on_full_blocks(oracle):
    groups = G(oracle, [(0, 0, 300)])
    b = oracle.plan_routed_gemm(groups, 128)
    assert [r for r, _ in b] == [128, 128, 44]
    assert list(b[0][1]["row_count"]) == [64, 64]
    assert list(b[2][1]["row_count"]) == [44]
    covers_exactly_once(b, groups)


def test_planner_rounds_budget_down_to_whole_blocks(oracle):
    groups = G(oracle, [(0, 0, 200)])
    b = oracle.plan_routed_gemm(groups, 100)
    assert [r for r, _ in b] == [64, 64, 64, 8]
    covers_exactly_once(b, groups)


def test_planner_single_row_groups_and_empty(oracle):
    groups = G(oracle, [(i, i, 1) for i in range(16)])
    b = oracle.plan_routed_gemm(groups, 512)
    assert len(b) == 1 and b[0][1].size == 16
    covers_exactly_once(b, groups)
    assert oracle.plan_routed_gemm(G(oracle, []), 512) == []
