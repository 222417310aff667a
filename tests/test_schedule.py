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
        # greedy, longest first within each head: within two items of perfect balance
        assert sl.max() - sl.min() <= 2 * ln.max()
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


def test_split_groups_of_band_and_lattice_blocks():
    """Identity blocks and rp16 blocks of L=16384 meet in 8 groups: 16 consecutive band
    blocks (2048 rows) and the 16 classes' blocks of the same rows."""
    from polyhedral_amd.schedule import block_rows, sync_groups
    N = 16384
    g0, g1, ng = sync_groups(N // 128, lambda p, qb: block_rows(qb, (0, 16)[p], N))
    assert ng == 8
    assert np.array_equal(g0, np.arange(128) // 16)
    assert np.array_equal(g1, np.arange(128) % 8)
    for g in range(ng):
        rows0 = np.concatenate([block_rows(qb, 0, N) for qb in np.flatnonzero(g0 == g)])
        rows1 = np.concatenate([block_rows(qb, 16, N) for qb in np.flatnonzero(g1 == g)])
        assert np.array_equal(np.sort(rows0), np.sort(rows1))


def _simulate(lists, speed):
    """Run the work-group lists with every work-group resident: an item of piece 1
    finishes only after every piece-0 item of its group has; returns the makespan or
    raises on a cycle (no work-group can progress)."""
    need = {}
    for lst in lists:
        for pc, bh, qb, sg, L in lst:
            if pc == 0:
                need[sg] = need.get(sg, 0) + 1
    done = {sg: 0 for sg in need}
    pos = [0] * len(lists)
    t = [0.0] * len(lists)
    remaining = sum(len(x) for x in lists)
    while remaining:
        progressed = False
        for g, lst in enumerate(lists):
            while pos[g] < len(lst):
                pc, bh, qb, sg, L = lst[pos[g]]
                if pc == 1 and done[sg] < need[sg]:
                    break
                t[g] += L / speed[g]
                if pc == 0:
                    done[sg] += 1
                pos[g] += 1
                remaining -= 1
                progressed = True
        if not progressed:
            raise AssertionError("cycle: no work-group can finish its item")
    return max(t)


@pytest.mark.parametrize("BH,groups,xcds", [(32, 512, 8), (32, 512, 1), (3, 64, 8), (8, 96, 8)])
def test_split_lists_cover_every_item_in_order_without_cycles(BH, groups, xcds):
    from polyhedral_amd.schedule import block_rows, split_lists, sync_groups
    N = 16384
    g0, g1, ng = sync_groups(N // 128, lambda p, qb: block_rows(qb, (0, 16)[p], N))
    len0 = np.full(128, 6)
    len0[:2] = (2, 4)
    len1 = 2 * (np.arange(128) % 8) + 2
    lists = split_lists(len0, len1, g0, g1, ng, BH, groups, xcds)
    items = [it[:4] for lst in lists for it in lst]
    want = {(0, h, q, h * ng + g0[q]) for h in range(BH) for q in range(128)} | \
           {(1, h, q, h * ng + g1[q]) for h in range(BH) for q in range(128)}
    assert len(items) == len(want) and set(items) == want
    # co-resident work-groups never wait in a cycle, whatever their relative speeds
    rng = np.random.default_rng(BH)
    for speed in (np.ones(groups), rng.uniform(0.5, 1.5, groups)):
        _simulate(lists, speed)
    ideal = (len0.sum() + len1.sum()) * BH / groups
    assert _simulate(lists, np.ones(groups)) < 1.25 * ideal + len1.max()


@pytest.mark.parametrize("BH,lag", [(32, 1), (8, 0), (16, 2), (3, 1), (5, 0)])
def test_split_grid_items_start_after_what_they_wait_for(BH, lag):
    """One work-group per item: every item exactly once, each head's items on one XCD when
    the heads split evenly over the XCDs, and every merge starts (work-group id order)
    after all the first-piece items of its group."""
    from polyhedral_amd.schedule import XCDS, block_rows, grid_start_order, split_grid_items, sync_groups
    N = 16384
    g0, g1, ng = sync_groups(N // 128, lambda p, qb: block_rows(qb, (0, 16)[p], N))
    len0 = np.full(128, 6)
    len0[:2] = (2, 4)
    len1 = 2 * (np.arange(128) % 8) + 2
    items = split_grid_items(len0, len1, g0, g1, ng, BH, lag=lag)
    want = {(0, h, q, h * ng + g0[q]) for h in range(BH) for q in range(128)} | \
           {(1, h, q, h * ng + g1[q]) for h in range(BH) for q in range(128)}
    assert items.shape == (2 * 128 * BH, 4) and set(map(tuple, items.tolist())) == want
    hw = grid_start_order(items.shape[0])
    assert np.array_equal(np.sort(hw), np.arange(items.shape[0]))
    last_first = {}
    for (pc, bh, qb, sg), i in zip(items.tolist(), hw.tolist()):
        if pc == 0:
            last_first[sg] = max(last_first.get(sg, -1), i)
    for (pc, bh, qb, sg), i in zip(items.tolist(), hw.tolist()):
        if pc == 1:
            assert i > last_first[sg]
    if BH % XCDS == 0:
        xcd_of_head = {}
        for (pc, bh, qb, sg), i in zip(items.tolist(), hw.tolist()):
            assert xcd_of_head.setdefault(bh, i % XCDS) == i % XCDS


def test_grid_start_order_inverts_the_kernel_mapping():
    """grid_start_order(n)[item] is the work-group that takes the item."""
    from polyhedral_amd.schedule import XCDS, grid_start_order
    for n in (1, 7, 8, 9, 64, 1003):
        per, rem = divmod(n, XCDS)
        hw = grid_start_order(n)
        for i in range(n):
            x, r = i % XCDS, i // XCDS
            lid = x * per + min(x, rem) + r if r < per else x * per + x + per
            assert hw[lid] == i


def test_run_rows_refuse_heads_beyond_int32_rows():
    """A run row holds rows of the whole [BH, N] tensor as int32; the host refuses a list
    whose heads would overflow before any device call."""
    import pytest
    from polyhedral_amd import schedule as S
    N = 1 << 20
    item_bh = np.array([0, 2047], dtype=np.int32)      # 2048 * 2^20 = 2^31
    with pytest.raises(ValueError, match="int32"):
        S._index_run([None], [0], N, np.zeros(2), item_bh, np.zeros(2, np.int32), np.full(2, -1),
                     np.ones(2, np.int64), "cpu")
