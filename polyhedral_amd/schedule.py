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
* within an XCD, longest-processing-time first: items in decreasing number of steps,
  each to the work-group with the least work so far (ties to the lowest index).  Items
  of equal length then go round robin, so at any moment an XCD's work-groups hold
  consecutive query blocks of one head.

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
        # every head's items of one length before the next length: head-major within a
        # length class, so concurrent work-groups hold neighbouring query blocks
        for L in np.unique(lens_o)[::-1]:
            sel = qbs_o[lens_o == L]
            for bh in heads:
                for qb in sel:
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
        nq = steps.shape[0]
        lengths = steps[:, 0, 14].cpu().numpy()
        item_bh, item_qb, item_len, group_of = assign(lengths, BH, self.groups, keep_empty)
        off = np.zeros(item_len.size + 1, dtype=np.int64)
        np.cumsum(item_len, out=off[1:])
        total = int(off[-1])
        if total >= 2 ** 31:
            raise ValueError("too many run rows for 32-bit offsets")
        counts = np.bincount(group_of, weights=item_len, minlength=self.groups).astype(np.int64)
        start = np.zeros(self.groups + 1, dtype=np.int64)
        np.cumsum(counts, out=start[1:])
        self.residue_s = getattr(steps, "residue_s", 0)
        self.BH, self.N = BH, N
        self.items = item_len.size
        self.rows = total
        self.max_group_steps = int(counts.max()) if counts.size else 0
        self.mean_group_steps = float(counts.mean()) if counts.size else 0.0
        self.run = torch.empty((max(total, 1), 16), dtype=torch.int32, device=dev)
        self.start = torch.from_numpy(start.astype(np.int32)).to(dev)
        if self.items:
            t_bh = torch.from_numpy(item_bh).to(dev)
            t_qb = torch.from_numpy(item_qb).to(dev)
            t_off = torch.from_numpy(off.astype(np.int32)).to(dev)
            with torch.cuda.device(dev):
                _lib.check(_lib.lib().pa_index_run(_lib.ptr(steps), steps.shape[1], nq, N, _lib.ptr(t_bh),
                                                   _lib.ptr(t_qb), _lib.ptr(t_off), self.items, _lib.ptr(self.run),
                                                   _lib.stream_of(self.run)), "pa_index_run")
            self._keep = (t_bh, t_qb, t_off)
