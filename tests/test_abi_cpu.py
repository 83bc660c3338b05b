"""CPU-side checks of the C ABI (no GPU call is made): the library loads and
exports every function include/tsugumi_hip.h declares, NULL arguments come
back as errors, and the host-only entry points (token-major pairs, grouping,
planning) agree with the oracle — itself pinned by the reference's golden
arrays in test_oracle_grouping.py — on those golden cases, on random
metadata and on every error case (PrefillMoEGroupingTests.swift:5-258,
PrefillRoutedGEMMPlannerTests.swift:38-88)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle


@pytest.fixture(scope="module")
def tsg():
    import tsugumi_amd
    tsugumi_amd.load()
    return tsugumi_amd


def test_exports_every_declared_symbol(tsg):
    from tsugumi_amd import _abi
    lib = _abi.load()
    declared = _abi.declared_symbols()
    assert len(declared) >= 40
    assert [n for n in declared if not hasattr(lib, n)] == []
    assert sorted(_abi.SIGNATURES) == declared


def test_status_strings_and_null_arguments(tsg):
    from tsugumi_amd import _abi
    lib = _abi.load()
    assert lib.tsg_status_string(0).decode() == "ok"
    for s in (1, 2, 3, 4, 5, 6, *range(100, 110)):
        assert len(lib.tsg_status_string(s)) > 0
    assert lib.tsg_ctx_create(0, None) == _abi.TSG_ERR_INVALID_ARGUMENT
    assert len(lib.tsg_last_error()) > 0
    assert lib.tsg_moe_create(None, 16, 0, None) == _abi.TSG_ERR_INVALID_ARGUMENT
    assert lib.tsg_qmv_int4(None, None, None, None, None, None, None, 64, 64) != 0
    assert lib.tsg_make_token_expert_pairs(None, None, 1, 1, None) != 0


def P(token, expert, rank, w):
    return (token, expert, rank, w)


GOLDEN_GROUPING = [
    ([P(0, 3, 0, 10), P(0, 1, 1, 11), P(0, 4, 2, 12), P(1, 1, 0, 13), P(1, 3, 1, 14),
      P(1, 2, 2, 15), P(2, 4, 0, 16), P(2, 3, 1, 17), P(2, 1, 2, 18), P(3, 5, 0, 19),
      P(3, 1, 1, 20), P(3, 4, 2, 21)][::-1], dict(query_count=4, top_k=3, num_experts=6,
                                                  tile_expert_count=2)),
    ([P(0, 1, 0, 10), P(0, 2, 1, 20), P(1, 3, 0, 30), P(1, 1, 1, 11), P(2, 2, 0, 21),
      P(2, 3, 1, 31)], dict(query_count=3, top_k=2, num_experts=4, tile_expert_count=2,
                            expert_sort_keys=[0, 30, 10, 20])),
    ([P(t, (t * 5 + r) % 10, r, t * 5 + r) for t in range(4) for r in range(5)],
     dict(query_count=4, top_k=5, num_experts=10, tile_expert_count=4,
          tile_break_after_group=3)),
    ([P(t, (t + r * 7) % 74, r, t * 8 + r) for t in range(32) for r in range(8)],
     dict(query_count=32, top_k=8, num_experts=128, tile_expert_count=16)),
]


def _same_grouping(a, b):
    for key in ("sorted_pairs", "offsets", "counts", "groups", "tiles"):
        assert np.array_equal(np.asarray(a[key]), np.asarray(b[key])), key


@pytest.mark.parametrize("case", range(len(GOLDEN_GROUPING)))
def test_grouping_matches_oracle_on_golden_cases(tsg, case):
    rows, kw = GOLDEN_GROUPING[case]
    pairs = np.array(rows, dtype=oracle.PAIR_DTYPE)
    _same_grouping(tsg.PrefillMoEGrouping.group_token_expert_pairs(pairs, **kw),
                   oracle.group_pairs(pairs, **kw))


def test_grouping_golden_values_through_abi(tsg):
    rows, kw = GOLDEN_GROUPING[0]
    g = tsg.PrefillMoEGrouping.group_token_expert_pairs(
        np.array(rows, dtype=oracle.PAIR_DTYPE), **kw)
    assert list(g["sorted_pairs"]["expert"]) == [1, 1, 1, 1, 2, 3, 3, 3, 4, 4, 4, 5]
    assert list(g["offsets"]) == [0xFFFFFFFF, 0, 4, 5, 8, 11]
    assert [tuple(x) for x in g["tiles"].tolist()] == [(0, 2, 0, 5), (2, 2, 5, 6), (4, 1, 11, 1)]


@pytest.mark.parametrize("seed", range(6))
def test_grouping_matches_oracle_on_random_routing(tsg, seed):
    rng = np.random.default_rng(seed)
    t, k, ne = int(rng.integers(1, 200)), int(rng.integers(1, 9)), int(rng.integers(8, 129))
    rows = []
    for tok in range(t):
        experts = rng.choice(ne, size=k, replace=False)
        rows += [P(tok, int(e), r, int(rng.integers(0, 1 << 16))) for r, e in enumerate(experts)]
    pairs = np.array(rows, dtype=oracle.PAIR_DTYPE)[rng.permutation(len(rows))]
    tec = int(rng.integers(1, 17))
    _same_grouping(tsg.PrefillMoEGrouping.group_token_expert_pairs(pairs, t, k, ne, tec),
                   oracle.group_pairs(pairs, t, k, ne, tec))


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
def test_grouping_errors_through_abi(tsg, kwargs, rows, case):
    with pytest.raises(tsg.TsgError) as err:
        tsg.PrefillMoEGrouping.group_token_expert_pairs(
            np.array(rows, dtype=oracle.PAIR_DTYPE), **kwargs)
    assert err.value.case == case


@pytest.mark.parametrize("groups,budget", [
    ([(3, 0, 40), (7, 40, 20)], 128),
    ([(0, 0, 100), (1, 100, 100)], 128),
    ([(0, 0, 300)], 128),
    ([(0, 0, 200)], 100),
    ([(i, i, 1) for i in range(16)], 512),
    ([(0, 0, 700), (5, 700, 3), (9, 703, 129)], 2048),
])
def test_planner_matches_oracle(tsg, groups, budget):
    g = np.array(groups, dtype=oracle.GROUP_DTYPE)
    got = tsg.PrefillRoutedGEMMPlanner.plan(g, budget)
    ref = oracle.plan_routed_gemm(g, budget)
    assert [r for r, _ in got] == [r for r, _ in ref]
    for (_, a), (_, b) in zip(got, ref):
        assert np.array_equal(a, b)


def test_token_expert_pairs_match_oracle(tsg):
    rng = np.random.default_rng(3)
    t, k = 37, 8
    idx = rng.integers(0, 128, size=t * k).astype(np.uint32)
    w = rng.integers(0, 0x3C00, size=t * k).astype(np.uint16)
    got = tsg.PrefillRouter.make_token_expert_pairs(idx, w, t, k)
    ref = oracle.make_token_expert_pairs(idx, w, t, k)
    assert np.array_equal(np.asarray(got), np.asarray(ref))


def test_struct_layouts_match_the_reference(tsg, tmp_path):
    """The boundary's structs are the reference's byte for byte: the pair is
    16 bytes with fields at 0/4/8/12 (PrefillRouterTests.swift:12-19), the
    expert offsets 36 (MoE.swift:4-29), group 12, tile 16 and routed block 16
    (PrefillMoEGrouping.swift:3-29, PrefillGroupedRoutedMoE.swift:20-25). The
    header's own static assertions are compiled as C11 and as C++17, and the
    ctypes and numpy mirrors are held to the same sizes and offsets."""
    import ctypes
    import os
    import shutil
    import subprocess

    from tsugumi_amd import _abi
    sizes = {_abi.ExpertOffsets: 36, _abi.TokenExpertPair: 16, _abi.MoEGroup: 12,
             _abi.MoETile: 16, _abi.RoutedBlock: 16}
    for cls, size in sizes.items():
        assert ctypes.sizeof(cls) == size, cls.__name__
    assert [getattr(_abi.TokenExpertPair, f).offset
            for f in ("token", "expert", "rank", "weight_bits")] == [0, 4, 8, 12]
    assert _abi.RoutedBlock.local_row.offset == 12
    assert tsg.PAIR_DTYPE.itemsize == 16 and tsg.BLOCK_DTYPE.itemsize == 16
    assert tsg.GROUP_DTYPE.itemsize == 12 and tsg.TILE_DTYPE.itemsize == 16
    assert [tsg.PAIR_DTYPE.fields[f][1] for f in ("token", "expert", "rank", "weight_bits")] == \
        [0, 4, 8, 12]
    header = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                          "include", "tsugumi_hip.h")
    src = tmp_path / "layout.c"
    src.write_text(f'#include "{header}"\nint main(void) {{ return 0; }}\n')
    for cc, std in (("gcc", "-std=c11"), ("g++", "-std=c++17")):
        if shutil.which(cc) is None:
            pytest.skip(f"{cc} not installed")
        lang = ["-x", "c++"] if cc == "g++" else []
        r = subprocess.run([cc, std, "-fsyntax-only", "-Wall", "-Werror", *lang, str(src)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
