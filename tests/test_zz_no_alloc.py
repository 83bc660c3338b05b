"""tsg_prefill_group_pairs_device_noalloc against tsg_prefill_group_pairs_device.

The no-alloc entry point keeps the pairs' ranks in the library's file-scope
device array instead of a caller workspace; its outputs (sorted pairs,
offsets, counts, the work list and its count) must equal the workspace entry
point's bit for bit. Two calls in a row, the second with fewer pairs, check
that what the first left in the shared array does not leak into the second.
"""
import numpy as np
import pytest

import oracle
from tests.gpu_util import dev, empty, host
from tests.workloads import zipf_routing

pytestmark = pytest.mark.gpu

MAX_PAIRS = 65536  # the entry point's limit (query_count * top_k)


@pytest.fixture(scope="module")
def tsg():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import tsugumi_amd
    return tsugumi_amd


@pytest.fixture(scope="module")
def ctx(tsg):
    return tsg.Context(0)


def _outputs(t, k, ne, tile):
    max_blocks = t * k // tile + ne + 1
    # sentinel-filled, so a word either entry point leaves unwritten differs
    return dict(sp=empty(t * k * 4, np.uint32, fill=-1), off=empty(ne, np.uint32, fill=-1),
                cnt=empty(ne, np.uint32, fill=-1), blocks=empty(max_blocks * 4, np.uint32, fill=-1),
                nb=empty(1, np.uint32, fill=-1), max_blocks=max_blocks)


def _read(o):
    n = int(host(o["nb"], np.uint32)[0])
    return dict(sp=host(o["sp"], np.uint32).copy(), off=host(o["off"], np.uint32).copy(),
                cnt=host(o["cnt"], np.uint32).copy(), n=n,
                blocks=host(o["blocks"], np.uint32).view(oracle.BLOCK_DTYPE)[:n].copy())


def _run_both(tsg, ctx, t, k, ne, s, tile, seed):
    rng = np.random.default_rng(seed)
    idx, w = zipf_routing(rng, t, ne, k, s)
    di, dw = dev(idx), dev(w)
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    ref = _outputs(t, k, ne, tile)
    scratch = empty(g.scratch_bytes(t, k, ne) // 4 + 1, np.uint32)
    g.group_pairs_device(di, dw, t, k, ne, ref["sp"], ref["off"], ref["cnt"], ref["blocks"],
                         ref["max_blocks"], ref["nb"], scratch, tile_rows=tile)
    got = _outputs(t, k, ne, tile)
    g.group_pairs_device_noalloc(di, dw, t, k, ne, got["sp"], got["off"], got["cnt"],
                                 got["blocks"], got["max_blocks"], got["nb"], tile_rows=tile)
    ctx.synchronize()
    a, b = _read(ref), _read(got)
    assert b["n"] == a["n"] > 0
    for key in ("sp", "off", "cnt"):
        assert np.array_equal(b[key], a[key]), key
    assert np.array_equal(b["blocks"], a["blocks"])
    # and the workspace entry point is the host sort (its own tests pin that)
    pairs = oracle.make_token_expert_pairs(idx, w, t, k)
    want = oracle.group_pairs(pairs, t, k, ne)
    assert np.array_equal(b["sp"].view(oracle.PAIR_DTYPE), want["sorted_pairs"])


def test_noalloc_grouping_matches_workspace_entry_twice(tsg, ctx):
    """Config-5 prefill shape (T=4096, 256 experts, top-8: 32768 pairs), then
    a smaller one (T=301, 128 experts) through the same array."""
    _run_both(tsg, ctx, 4096, 8, 256, 1.0, 128, 0xA11)
    _run_both(tsg, ctx, 301, 8, 128, 1.1, 64, 0xA12)


def test_noalloc_grouping_at_its_limit(tsg, ctx):
    """Exactly MAX_PAIRS pairs (T=8192, top-8) are taken; one more is refused
    on the host before any launch."""
    _run_both(tsg, ctx, MAX_PAIRS // 8, 8, 128, 1.1, 128, 0xA13)
    t, k, ne = MAX_PAIRS // 8 + 1, 8, 128
    g = tsg.PrefillGroupedRoutedMoE(tsg.MoE(ctx))
    o = _outputs(t, k, ne, 128)
    idx = dev(np.zeros((t, k), np.uint32))
    w = dev(np.zeros((t, k), np.uint16))
    with pytest.raises(tsg.TsgError) as e:
        g.group_pairs_device_noalloc(idx, w, t, k, ne, o["sp"], o["off"], o["cnt"], o["blocks"],
                                     o["max_blocks"], o["nb"], tile_rows=128)
    assert e.value.status == 3  # TSG_ERR_UNSUPPORTED
