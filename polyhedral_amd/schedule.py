"""Persistent schedules of the streaming attention kernel.

The reference launches one Triton program per (query block, head) (grid (N/BQ, BH),
gpu/triton_attn.py:210) and lets the hardware place them.  The persistent kernel
(pa_attn_fwd with run_groups) instead runs a fixed number of work-groups, two per CU,
each taking a list of (head, query block) items back to back as one stream of steps,
so the step pipeline never drains between items.  This module decides the lists:

* items are the (head, query block) pairs of one index; an empty list is one item of
  a single all-dead step when the launch must still write its rows (the first piece
  of a split: zeros and log-sum-exp -inf), and no item when it merges into a previous
  piece (its rows keep the previous partial);
* MI355X dispatches work-group g to XCD g mod 8, and each XCD has its own L2.  When the
  heads split evenly, XCD x gets a contiguous range of heads, so the query blocks that
  share K / V rows share an L2;
* within an XCD, head by head, and within a head longest-processing-time first: items
  in decreasing number of steps, each to the work-group with the least work so far
  (ties to the lowest index).  At any moment an XCD's work-groups then hold query
  blocks of one or two heads, whose K / V the XCD's L2 can serve.

pa_index_run expands the lists into run rows on the device.
"""
import heapq

import numpy as np
import torch

from . import _lib

XCDS = 8             # MI355X: 8 accelerator complex dies, 32 CUs and one L2 each
GROUPS_PER_CU = 2    # the streaming kernel's occupancy (68 KB of LDS, <= 256 VGPRs)


def default_groups(device):
    props = torch.cuda.get_device_properties(device)
    return GROUPS_PER_CU * int(props.multi_processor_count)


def assign(lengths, BH, groups, keep_empty=True, xcds=XCDS):
    """Lists of items per work-group.  lengths: steps of each query block's list (0 for
    an empty list).  Returns (item_bh, item_qb, item_len, group_of_item) as numpy arrays,
    items in run order (grouped by work-group, each group's items in its order)."""
    lengths = np.asarray(lengths, dtype=np.int64)
    nq = lengths.size
    qb_all = np.arange(nq)
    if keep_empty:
        qbs, lens = qb_all, np.maximum(lengths, 1)
    else:
        qbs, lens = qb_all[lengths > 0], lengths[lengths > 0]
    parts = xcds if (BH % xcds == 0 and groups % xcds == 0 and groups >= xcds) else 1
    per_part_heads = BH // parts
    order = np.lexsort((qbs, -lens))          # longest first, then query block order
    qbs_o, lens_o = qbs[order], lens[order]
    lists = [[] for _ in range(groups)]
    for p in range(parts):
        slots = list(range(p, groups, parts))  # the work-groups that land on XCD p
        heap = [(0, i, s) for i, s in enumerate(slots)]
        heapq.heapify(heap)
        heads = range(p * per_part_heads, (p + 1) * per_part_heads)
        # head-major, longest first within a head: the XCD's work-groups work on one head
        # at a time (its K / V, a few MB, then serves their reads from the XCD's L2), and
        # the heads' items interleave only at the turn of a head
        for bh in heads:
            for qb, L in zip(qbs_o, lens_o):
                load, i, s = heapq.heappop(heap)
                lists[s].append((bh, int(qb), int(L)))
                heapq.heappush(heap, (load + int(L), i, s))
    item_bh, item_qb, item_len, group_of = [], [], [], []
    for g, lst in enumerate(lists):
        for bh, qb, L in lst:
            item_bh.append(bh)
            item_qb.append(qb)
            item_len.append(L)
            group_of.append(g)
    return (np.asarray(item_bh, dtype=np.int32), np.asarray(item_qb, dtype=np.int32),
            np.asarray(item_len, dtype=np.int64), np.asarray(group_of, dtype=np.int64))


def _index_run(pieces_steps, boff_base, N, item_piece, item_bh, item_qb, item_sync, item_len, dev):
    """Run rows (int32 [rows, 16]) of items listed in run order (pa_index_run)."""
    if item_bh.size and (int(np.max(item_bh)) + 1) * int(N) >= 2 ** 31:
        raise ValueError(f"run rows hold rows of the whole [BH, N] tensor as int32: {int(np.max(item_bh)) + 1} "
                         f"heads of N={N} rows do not fit")
    off = np.zeros(item_len.size + 1, dtype=np.int64)
    np.cumsum(item_len, out=off[1:])
    total = int(off[-1])
    if total >= 2 ** 31:
        raise ValueError("too many run rows for 32-bit offsets")
    run = torch.empty((max(total, 1), 16), dtype=torch.int32, device=dev)
    if item_len.size:
        keep = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(dev)
                for x in (item_piece, item_bh, item_qb, item_sync, off)]
        n = len(pieces_steps)
        steps_p = (_lib.c_vp * n)(*[st.data_ptr() for st in pieces_steps])
        pitch_p = (_lib.c_i64 * n)(*[st.shape[1] for st in pieces_steps])
        base_p = (_lib.c_i32 * n)(*[int(b) for b in boff_base])
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().pa_index_run(steps_p, pitch_p, base_p, n, N, _lib.ptr(keep[0]), _lib.ptr(keep[1]),
                                               _lib.ptr(keep[2]), _lib.ptr(keep[3]), _lib.ptr(keep[4]),
                                               int(item_len.size), _lib.ptr(run), _lib.stream_of(run)),
                       "pa_index_run")
        torch.cuda.current_stream(dev).synchronize()
    return run, total


def _starts(group_of, item_len, groups):
    counts = np.bincount(group_of, weights=item_len, minlength=groups).astype(np.int64)
    start = np.zeros(groups + 1, dtype=np.int64)
    np.cumsum(counts, out=start[1:])
    return start, counts


class RunSchedule:
    """Run rows (int32 [rows, 16]) and each work-group's first row (int32 [groups + 1])
    for one index (its step descriptors `steps`, in index order) over BH heads."""

    def __init__(self, steps, N, BH, groups=None, keep_empty=True):
        if steps is None:
            raise ValueError("an index with no listed tile has no step descriptors to run")
        if getattr(steps, "order", None) is not None:
            raise ValueError("run rows are built from step descriptors in index order (order=None)")
        dev = steps.device
        self.groups = int(groups or default_groups(dev))
        lengths = steps[:, 0, 14].cpu().numpy()
        item_bh, item_qb, item_len, group_of = assign(lengths, BH, self.groups, keep_empty)
        self.residues = (getattr(steps, "residue_s", 0),)
        self.BH, self.N = BH, N
        self.items = item_len.size
        n = item_len.size
        self.run, self.rows = _index_run([steps], [0], N, np.zeros(n), item_bh, item_qb, np.full(n, -1), item_len,
                                         dev)
        start, counts = _starts(group_of, item_len, self.groups)
        self.start = torch.from_numpy(start.astype(np.int32)).to(dev)
        self.max_group_steps = int(counts.max()) if counts.size else 0
        self.mean_group_steps = float(counts.mean()) if counts.size else 0.0


def block_rows(qb, residue, N, BQ=128):
    """Original rows of query block qb in the residue-`residue` basis (0: index space)."""
    r = np.arange(qb * BQ, qb * BQ + BQ)
    if not residue:
        return r
    Q = N // residue
    return (r % Q) * residue + r // Q


def sync_groups(nq, qrows):
    """Groups of query blocks of two pieces whose rows overlap.  qrows(p, qb) gives the
    original rows of query block qb of piece p.  Returns (group of each piece-0 block,
    group of each piece-1 block, number of groups); groups are connected components of
    "the two blocks share a row"."""
    N = nq * 128
    blk0 = np.empty(N, dtype=np.int64)
    for qb in range(nq):
        blk0[qrows(0, qb)] = qb
    parent = list(range(nq))

    def find(x):
        while parent[x] != x:
            parent[x] = parent[parent[x]]
            x = parent[x]
        return x

    touch1 = []
    for qb in range(nq):
        t = np.unique(blk0[qrows(1, qb)])
        touch1.append(t[0])
        for b in t[1:]:
            ra, rb = find(int(t[0])), find(int(b))
            if ra != rb:
                parent[rb] = ra
    roots = sorted({find(b) for b in range(nq)})
    gid = {r: i for i, r in enumerate(roots)}
    g0 = np.array([gid[find(b)] for b in range(nq)], dtype=np.int64)
    g1 = np.array([gid[find(int(t))] for t in touch1], dtype=np.int64)
    return g0, g1, len(roots)


def split_lists(len0, len1, g0, g1, ng, BH, groups, xcds):
    """Work-group lists of a two-piece split: items (piece, bh, qb, sync group, steps).
    len0 / len1: steps of each query block of piece 0 / 1 (>= 1); g0 / g1: their groups.
    See SplitSchedule for the order."""
    blocks0 = [np.flatnonzero(g0 == g) for g in range(ng)]
    blocks1 = [np.flatnonzero(g1 == g) for g in range(ng)]
    gorder = sorted(range(ng), key=lambda g: (-int(len1[blocks1[g]].sum()), g))
    parts = xcds if (BH % xcds == 0 and groups % xcds == 0 and groups >= xcds) else 1
    per = BH // parts
    lists = [[] for _ in range(groups)]
    for p in range(parts):
        seq = []
        for bh in range(p * per, (p + 1) * per):
            prev = None
            for g in gorder:
                seq += [(0, bh, int(qb), bh * ng + g) for qb in blocks0[g]]
                if prev is not None:
                    seq += [(1, bh, int(qb), bh * ng + prev) for qb in blocks1[prev]]
                prev = g
            seq += [(1, bh, int(qb), bh * ng + prev) for qb in blocks1[prev]]
        slots = list(range(p, groups, parts))
        heap = [(0, i, s_) for i, s_ in enumerate(slots)]
        heapq.heapify(heap)
        for it in seq:
            L = int((len0 if it[0] == 0 else len1)[it[2]])
            load, i, s_ = heapq.heappop(heap)
            lists[s_].append(it + (L,))
            heapq.heappush(heap, (load + L, i, s_))
    return lists


class SplitSchedule:
    """The run of a two-piece split in one launch (pa_attn_fwd_split): both pieces' items
    over BH heads, each in the sync group of the rows it covers.

    Per XCD (a contiguous range of heads when they split evenly), the items are put in a
    sequence: for each head, its groups in decreasing order of second-piece work, the
    first piece's items of a group, then the second piece's items of the group before
    (so a merge comes one group after the rows it waits for).  Each item in sequence goes
    to the XCD's work-group with the least work so far; every work-group's list is
    therefore in sequence order, which keeps the waits free of cycles."""

    def __init__(self, steps0, steps1, residue0, residue1, N, BH, bits_base, groups=None, xcds=None):
        for st in (steps0, steps1):
            if st is None or getattr(st, "order", None) is not None:
                raise ValueError("split runs are built from both pieces' step descriptors in index order")
        dev = steps0.device
        self.groups = int(groups or default_groups(dev))
        nq = steps0.shape[0]
        if steps1.shape[0] != nq:
            raise ValueError("the pieces must share the query tile")

        g0, g1, ng = sync_groups(nq, lambda p, qb: block_rows(qb, (residue0, residue1)[p], N))
        sig = np.bincount(g0, minlength=ng)
        wai = np.bincount(g1, minlength=ng)
        if sig.min() != sig.max() or wai.min() != wai.max():
            raise ValueError("the pieces' query blocks do not form groups of one size")
        self.sync_signal, self.sync_wait, self.groups_per_head = int(sig[0]), int(wai[0]), ng
        len0 = np.maximum(steps0[:, 0, 14].cpu().numpy().astype(np.int64), 1)
        len1 = np.maximum(steps1[:, 0, 14].cpu().numpy().astype(np.int64), 1)
        lists = split_lists(len0, len1, g0, g1, ng, BH, self.groups, XCDS if xcds is None else xcds)
        items = [it for lst in lists for it in lst]
        group_of = np.array([g for g, lst in enumerate(lists) for _ in lst], dtype=np.int64)
        arr = np.array(items, dtype=np.int64).reshape(-1, 5)
        item_piece, item_bh, item_qb, item_sync, item_len = (arr[:, i] for i in range(5))
        self.BH, self.N = BH, N
        self.residues = (residue0, residue1)
        self.items = len(items)
        self.run, self.rows = _index_run([steps0, steps1], bits_base, N, item_piece, item_bh, item_qb, item_sync,
                                         item_len, dev)
        start, counts = _starts(group_of, item_len, self.groups)
        self.start = torch.from_numpy(start.astype(np.int32)).to(dev)
        self.max_group_steps = int(counts.max()) if counts.size else 0
        self.mean_group_steps = float(counts.mean()) if counts.size else 0.0
        self.sync_groups = BH * ng
        # counters (zero, and left zero by every launch) and the give-up flag
        self.sync = torch.zeros(2 * self.sync_groups, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)

    def check(self):
        """Raise if a merge of a past launch gave up waiting (its results are invalid);
        the counters and the flag are cleared for the next launch."""
        if int(self.status.item()):
            self.status.zero_()
            self.sync.zero_()
            raise RuntimeError("a merge of the split launch gave up waiting for its rows: results are invalid")


def split_grid_items(len0, len1, g0, g1, ng, BH, xcds=None, lag=1):
    """Items of a two-piece split run as one work-group per item (pa_attn_fwd_split with
    items): int32 [n, 4] = (piece, batch-head, query block, sync group), in the order the
    work-groups start.  Work-group ids are dealt to the XCDs in contiguous ranges, so when
    the heads split evenly the items of XCD x are its heads' items.  Per head, the groups
    go in decreasing order of second-piece work; each group's first-piece items come
    `lag` groups before its second-piece items, so a merge rarely finds its rows
    unpublished.  Within a group, longest list first.  The rows are the items in slot
    order (the kernel's work-group i takes slot grid_start_order's inverse of i)."""
    xcds = XCDS if xcds is None else xcds
    blocks0 = [np.flatnonzero(g0 == g) for g in range(ng)]
    blocks1 = [np.flatnonzero(g1 == g) for g in range(ng)]
    gorder = sorted(range(ng), key=lambda g: (-int(len1[blocks1[g]].sum()), g))
    out = []
    for bh in range(BH):
        pend = []
        for g in gorder:
            b0 = sorted(blocks0[g], key=lambda q: (-int(len0[q]), int(q)))
            out += [(0, bh, int(q), bh * ng + g) for q in b0]
            pend.append(g)
            if len(pend) > lag:
                h = pend.pop(0)
                b1 = sorted(blocks1[h], key=lambda q: (-int(len1[q]), int(q)))
                out += [(1, bh, int(q), bh * ng + h) for q in b1]
        for h in pend:
            b1 = sorted(blocks1[h], key=lambda q: (-int(len1[q]), int(q)))
            out += [(1, bh, int(q), bh * ng + h) for q in b1]
    seq = np.asarray(out, dtype=np.int32).reshape(-1, 4)
    if BH % xcds == 0:
        # every head has the same number of items, so XCD x's contiguous range of item
        # slots holds whole heads, each in its own sequence order
        return seq
    # otherwise a head would straddle two XCDs' ranges and a merge could start before the
    # items it waits for: give the sequence to the work-groups in start order instead
    items = np.empty_like(seq)
    items[np.argsort(grid_start_order(seq.shape[0]))] = seq
    return items


def grid_start_order(n):
    """Work-group id (start order) of each of n items: work-group i takes item
    (i mod 8) * (n // 8) + min(i mod 8, n mod 8) + i // 8 (contiguous item ranges per XCD)."""
    per, rem = divmod(n, XCDS)
    hw = np.arange(n, dtype=np.int64)
    x, r = hw % XCDS, hw // XCDS
    lid = x * per + np.minimum(x, rem) + r
    out = np.empty(n, dtype=np.int64)
    out[lid] = hw
    return out


class SplitGrid:
    """The items, counters and give-up flag of a two-piece split run as one work-group
    per item (pa_attn_fwd_split with items).  The two pieces' descriptors must be in
    index order."""

    def __init__(self, steps0, steps1, residue0, residue1, N, BH, lag=1):
        dev = steps0.device
        nq = steps0.shape[0]
        if steps1.shape[0] != nq:
            raise ValueError("the pieces must share the query tile")
        g0, g1, ng = sync_groups(nq, lambda p, qb: block_rows(qb, (residue0, residue1)[p], N))
        sig = np.bincount(g0, minlength=ng)
        wai = np.bincount(g1, minlength=ng)
        if sig.min() != sig.max() or wai.min() != wai.max():
            raise ValueError("the pieces' query blocks do not form groups of one size")
        self.sync_signal, self.sync_wait, self.groups_per_head = int(sig[0]), int(wai[0]), ng
        len0 = np.maximum(steps0[:, 0, 14].cpu().numpy().astype(np.int64), 1)
        len1 = np.maximum(steps1[:, 0, 14].cpu().numpy().astype(np.int64), 1)
        items = split_grid_items(len0, len1, g0, g1, ng, BH, lag=lag)
        # Deadlock freedom: work-groups start in id order, so every second-piece item must
        # start after all the first-piece items of its group (a wait on a later work-group
        # could hold a slot that work-group needs).
        hw = grid_start_order(items.shape[0])
        first_start = np.full(BH * ng, -1, dtype=np.int64)
        np.maximum.at(first_start, items[items[:, 0] == 0, 3], hw[items[:, 0] == 0])
        sec = items[:, 0] == 1
        if np.any(hw[sec] <= first_start[items[sec, 3]]):
            raise ValueError("the split grid would start a merge before the items it waits for")
        self.items = torch.from_numpy(items).to(dev)
        self.n_items = items.shape[0]
        self.BH, self.N = BH, N
        self.residues = (residue0, residue1)
        self.sync_groups = BH * ng
        self.sync = torch.zeros(2 * self.sync_groups, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)

    def check(self):
        """Raise if a merge of a past launch gave up waiting (its results are invalid);
        the counters and the flag are cleared for the next launch."""
        if int(self.status.item()):
            self.status.zero_()
            self.sync.zero_()
            raise RuntimeError("a merge of the split launch gave up waiting for its rows: results are invalid")
