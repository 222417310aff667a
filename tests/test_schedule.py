"""The persistent kernel's work lists (polyhedral_amd.schedule.assign): every item exactly
once, XCD-contiguous heads, longest-first balance."""
import numpy as np
import pytest

from polyhedral_amd.schedule import assign


@pytest.mark.parametrize("BH,groups", [(32, 512), (8, 512), (3, 64), (16, 40)])
@pytest.mark.parametrize("keep_empty", [True, False])
def test_every_item_once_and_balanced(BH, groups, keep_empty):
    rng = np.random.default_rng(BH * groups)
    lengths = rng.integers(0, 17, size=96)
    bh, qb, ln, grp = assign(lengths, BH, groups, keep_empty)
    items = set(zip(bh.tolist(), qb.tolist()))
    want = {(h, q) for h in range(BH) for q in range(lengths.size) if keep_empty or lengths[q] > 0}
    assert len(items) == len(bh) == len(want) and items == want
    assert np.array_equal(ln, np.maximum(lengths[qb], 1))
    # run order: grouped by work-group, ascending
    assert np.all(np.diff(grp) >= 0)
    load = np.bincount(grp, weights=ln, minlength=groups)
    parts = 8 if (BH % 8 == 0 and groups % 8 == 0) else 1
    for p in range(parts):
        sl = load[p::parts]
        # greedy longest-first: no work-group exceeds the lightest by more than one item
        assert sl.max() - sl.min() <= ln.max()
    if parts == 8:
        # the work-groups of XCD x (g mod 8 == x) hold a contiguous range of heads
        for p in range(8):
            hs = set(bh[grp % 8 == p].tolist())
            assert hs == set(range(p * BH // 8, (p + 1) * BH // 8))


def test_equal_lengths_go_round_robin_over_neighbouring_blocks():
    """Items of one length are dealt out in (head, query block) order, so the work-groups
    of an XCD hold consecutive query blocks at the same time."""
    bh, qb, ln, grp = assign(np.full(128, 6), 8, 64)
    first = {}
    for h, q, g in zip(bh, qb, grp):
        first.setdefault(int(g), (int(h), int(q)))
    # XCD 0 owns head 0; its 8 work-groups (0, 8, ..., 56) start on query blocks 0..7
    assert [first[g] for g in range(0, 64, 8)] == [(0, q) for q in range(8)]
