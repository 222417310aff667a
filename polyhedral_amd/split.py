"""Disjoint split of a mask into sub-masks, one attention pass each, merged by log-sum-exp.

The reference names this decomposition (src/polyattn/experiments/compose.py:7-17,
docs/NOTES.md:355-363) and prices it (compose.py:107-119) but has no code for it.
Here every piece is a (mask, tile shape, optional class-A permutation) and runs
through pa_attn_fwd:

* a piece with a permutation reads its Q/K/V rows through the permutation
  (gather_q / gather_kv) and writes its output rows back to original positions
  (scatter_o), so no permuted copy of Q, K, V or O is ever materialised;
* the first pass writes O and the per-row LSE; every later pass merges its own
  result with the previous one in its epilogue, in place (each output row is read
  and written by the same lanes), so there is no separate merge pass;
* consecutive passes issue the heads in opposite orders, so that each pass starts
  on the heads whose Q, K, V and O the previous pass touched last and the memory-side
  cache still holds.

Pieces must be disjoint (the peeling of compose.py:49-76 makes them so); the merge
of disjoint pieces equals single-pass attention over their union.
"""
import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from .attention import prepare
from .index import STREAM_TILES, build_device, build_steps
from .perm import residue_perm
from .polyattn.masks import Permuted
from .schedule import RunSchedule, SplitGrid, SplitSchedule
from .spec import MaskSpec


@dataclass
class Piece:
    mask: object                 # a polyattn mask object (its terms() give the predicate)
    BQ: int = 128
    A: int = 32
    perm: Optional[object] = None  # index-space position -> original position (class-A basis)
    residue: int = 0               # > 0: the basis is residue_perm(N, residue) (perm may be omitted)


def _closed_form_residue(piece, N):
    """The piece's residue stride if the kernel can evaluate its basis in closed form."""
    s = piece.residue
    return s if s and N % s == 0 and ((N // s) & (N // s - 1)) == 0 else 0


class SplitPlan:
    """Block indices of every piece, built once on the GPU (offline, like
    create_block_mask), then reused by every forward.  order="lpt" issues each
    piece's query blocks longest first; None keeps index order."""

    def __init__(self, pieces, N, device=None, order="lpt", kernel="auto", persistent=False, fuse=False,
                 split_xcds=None, split_lag=1):
        self.N = N
        self.kernel = kernel
        # persistent: run the streaming pieces on the persistent kernel (a fixed set of
        # work-groups, each a list of items as one stream of steps).  Off by default:
        # measured on the band + lattice workload, the per-block launches (the hardware
        # dispatching one work-group per item, in order) keep the L2 hit rate higher than
        # a static list per work-group, and the passes are bound by their L2-miss bytes.
        # fuse: a two-piece split runs as ONE launch (pa_attn_fwd_split), the second piece
        # merging into the first piece's rows as soon as they are written: a persistent
        # run when persistent is set, else one work-group per item in a sequence that puts
        # each group's first-piece items before its merges
        self.persistent = persistent and kernel != "general"
        self.fuse = fuse and kernel != "general"
        self.split_xcds = split_xcds   # XCD partition of a split launch's schedule (None: all 8)
        self.split_lag = split_lag     # groups between a group's first- and second-piece items
        self._runs = {}
        self.pieces = list(pieces)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.built = []
        for p in self.pieces:
            perm_t = None
            if p.residue and p.perm is None:
                p = Piece(p.mask, p.BQ, p.A, residue_perm(N, p.residue), p.residue)
            if p.perm is not None:
                perm_t = (p.perm.to(device=dev, dtype=torch.int32) if isinstance(p.perm, torch.Tensor)
                          else torch.from_numpy(np.asarray(p.perm, dtype=np.int32)).to(dev))
            mask = Permuted(p.mask, perm_t.cpu().numpy()) if perm_t is not None else p.mask
            stream = (p.BQ, p.A) in STREAM_TILES
            built = build_device(mask, N, p.BQ, p.A, device=dev, bits=True)
            kv_idx, kv_num, kv_partial, wave, tiles, live, bits = built[:7]
            inc, exc = p.mask.terms()
            # longest-processing-time first: query blocks with the most listed tiles are
            # issued first, so the tail of the grid is short blocks
            qorder = torch.argsort(kv_num, descending=True, stable=True).to(torch.int32) if order == "lpt" else None
            # the streaming kernel's descriptors, laid out in that issue order
            steps = (build_steps(kv_idx, kv_num, kv_partial, wave, bits[0], N, p.BQ, p.A,
                                 _closed_form_residue(p, N), qorder) if stream else None)
            # the persistent kernel's run rows come from the descriptors in index order
            runnable = stream and (self.persistent or self.fuse) and (perm_t is None or _closed_form_residue(p, N) > 0)
            steps_idx = (build_steps(kv_idx, kv_num, kv_partial, wave, bits[0], N, p.BQ, p.A,
                                     _closed_form_residue(p, N), None) if runnable else None)
            self.built.append(dict(piece=p, spec=MaskSpec(tuple(inc), tuple(exc)), perm=perm_t,
                                   kv_idx=kv_idx, kv_num=kv_num, kv_partial=kv_partial, wave=wave, bits=bits,
                                   steps=steps, steps_idx=steps_idx,
                                   tiles=tiles, live=live, order=qorder))

    @property
    def live(self):
        return sum(b["live"] for b in self.built)

    @property
    def elements(self):
        return sum(b["tiles"] * b["piece"].BQ * b["piece"].A for b in self.built)

    def prepare(self, q, k, v, scale=None, out=None, lse=None):
        """Validated launches over these tensors; calling them in order is a forward.
        Returns (launches, o, lse).  self.launched lists, per launch, the pieces it runs
        (indices into self.built): one piece per launch, or both pieces of a two-piece
        split in one launch (pa_attn_fwd_split)."""
        BH, N, D = q.shape
        if N != self.N:
            raise ValueError(f"plan built for N={self.N}, got N={N}")
        o = out if out is not None else torch.empty_like(q)
        lse_buf = lse if lse is not None else torch.empty((BH, N), dtype=torch.float32, device=q.device)
        fused = self._fused_launch(q, k, v, scale, o, lse_buf)
        if fused is not None:
            self.launched = [(0, 1)]
            return [fused], o, lse_buf
        launches = []
        self.launched = []
        first = True
        for bi_, b in enumerate(self.built):
            p = b["piece"]
            if b["live"] == 0 and not (first and b is self.built[-1]):
                # an empty sub-mask leaves O and LSE unchanged: no pass (the first pass of an
                # all-empty plan still runs, to write zeros and -inf)
                continue
            permuted = b["perm"] is not None
            run = self._run_for(bi_, BH, keep_empty=first) if self._runnable(q, k, v, b) else None
            launches.append(prepare(
                q, k, v, b["kv_idx"], b["kv_num"], b["kv_partial"], b["spec"], 0, 0, 0, p.BQ, p.A,
                scale=scale, perm_q=b["perm"], perm_kv=b["perm"], gather_kv=permuted,
                kv_wave_bits=b["wave"], kv_bits=b["bits"], gather_q=permuted, scatter_o=permuted,
                residue=_closed_form_residue(p, N),
                lse=lse_buf, prev=None if first else (o, lse_buf), out=o, qblock_order=b["order"],
                kv_steps=b["steps"], kernel=self.kernel, heads_desc=len(launches) % 2 == 1, run=run))
            self.launched.append((bi_,))
            first = False
        return launches, o, lse_buf

    def _fused_launch(self, q, k, v, scale, o, lse_buf):
        """The whole forward of a two-piece split as one launch (persistent, or one
        work-group per item), or None when this plan or these tensors do not allow it
        (then one launch per piece)."""
        if not (self.fuse and len(self.built) == 2):
            return None
        if not self.persistent:
            return self._grid_launch(q, k, v, scale, o, lse_buf)
        b0, b1 = self.built
        if b0["live"] == 0 or b1["live"] == 0 or (b0["piece"].BQ, b1["piece"].BQ) != (128, 128):
            return None
        if b0["piece"].A != b1["piece"].A:
            return None
        if not (self._runnable(q, k, v, b0) and self._runnable(q, k, v, b1)):
            return None
        BH = q.shape[0]
        key = ("split", BH)
        if key not in self._runs:
            pools = [b0["bits"][1], b1["bits"][1]]
            try:
                sched = SplitSchedule(b0["steps_idx"], b1["steps_idx"], _closed_form_residue(b0["piece"], self.N),
                                      _closed_form_residue(b1["piece"], self.N), self.N, BH,
                                      (0, pools[0].numel()), xcds=self.split_xcds)
            except ValueError:
                sched = None
            self._runs[key] = (sched, torch.cat(pools) if sched is not None else None)
        sched, pool = self._runs[key]
        if sched is None:
            return None
        ls = []
        for i, b in enumerate((b0, b1)):
            p = b["piece"]
            permuted = b["perm"] is not None
            ls.append(prepare(
                q, k, v, b["kv_idx"], b["kv_num"], b["kv_partial"], b["spec"], 0, 0, 0, p.BQ, p.A,
                scale=scale, perm_q=b["perm"], perm_kv=b["perm"], gather_kv=permuted,
                kv_wave_bits=b["wave"], kv_bits=b["bits"], gather_q=permuted, scatter_o=permuted,
                residue=_closed_form_residue(p, self.N), lse=lse_buf, prev=None if i == 0 else (o, lse_buf), out=o,
                kv_steps=b["steps"], kernel=self.kernel, run=(sched, i)))
        return SplitLaunch(ls[0], ls[1], sched, pool)

    def _grid_launch(self, q, k, v, scale, o, lse_buf):
        b0, b1 = self.built
        if b0["live"] == 0 or b1["live"] == 0 or (b0["piece"].BQ, b1["piece"].BQ) != (128, 128):
            return None
        if b0["piece"].A != b1["piece"].A or b0["steps_idx"] is None or b1["steps_idx"] is None:
            return None
        BH, N, D = q.shape
        if q.dtype not in (torch.float16, torch.bfloat16) or D != 128:
            return None
        key = ("grid", BH)
        if key not in self._runs:
            try:
                self._runs[key] = SplitGrid(b0["steps_idx"], b1["steps_idx"], _closed_form_residue(b0["piece"], N),
                                            _closed_form_residue(b1["piece"], N), N, BH, lag=self.split_lag)
            except ValueError:
                self._runs[key] = None
        grid = self._runs[key]
        if grid is None:
            return None
        ls = []
        for i, b in enumerate((b0, b1)):
            p = b["piece"]
            permuted = b["perm"] is not None
            ls.append(prepare(
                q, k, v, b["kv_idx"], b["kv_num"], b["kv_partial"], b["spec"], 0, 0, 0, p.BQ, p.A,
                scale=scale, perm_q=b["perm"], perm_kv=b["perm"], gather_kv=permuted,
                kv_wave_bits=b["wave"], kv_bits=b["bits"], gather_q=permuted, scatter_o=permuted,
                residue=_closed_form_residue(p, N), lse=lse_buf, prev=None if i == 0 else (o, lse_buf), out=o,
                kv_steps=b["steps_idx"], kernel="stream"))
        return SplitLaunch(ls[0], ls[1], grid, None)

    def check(self):
        """Raise if a merge of a past split launch gave up waiting (see SplitSchedule.check)."""
        for key, val in self._runs.items():
            if key[0] == "split" and val[0] is not None:
                val[0].check()
            if key[0] == "grid" and val is not None:
                val.check()

    def _runnable(self, q, k, v, b):
        """Whether the persistent kernel takes this piece over these tensors."""
        if b.get("steps_idx") is None:
            return False
        BH, N, D = q.shape
        return (q.dtype in (torch.float16, torch.bfloat16) and D == 128 and
                all(t.stride(0) == N * t.stride(1) for t in (k, v)) and
                BH * N * max(k.stride(1), v.stride(1)) * 2 < 2 ** 32)

    def _run_for(self, i, BH, keep_empty):
        key = (i, BH, keep_empty)
        if key not in self._runs:
            b = self.built[i]
            self._runs[key] = RunSchedule(b["steps_idx"], self.N, BH, keep_empty=keep_empty)
        return (self._runs[key], 0)

    def forward(self, q, k, v, scale=None, out=None, lse=None):
        """o [BH, N, D] in q's dtype; lse (float32 [BH, N]) receives the merged log-sum-exp.
        A split run as one launch (fuse) is checked before returning: if a merge gave up
        waiting for its rows, the counters are cleared and RuntimeError is raised."""
        launches, o, _ = self.prepare(q, k, v, scale, out, lse)
        with torch.cuda.device(q.device):
            for launch in launches:
                launch()
        if any(isinstance(x, SplitLaunch) for x in launches):
            self.check()
        return o


class SplitLaunch:
    """Both pieces of a two-piece split in one persistent launch (pa_attn_fwd_split).
    Calls of one plan over the same tensors must not overlap (they share the sync
    counters).  A merge whose bounded wait gives up marks the schedule's status; check()
    (a device synchronisation) then raises and clears the status and the counters, which
    a give-up can leave out of step with the next launch: call it after launches made
    outside SplitPlan.forward (which checks by itself)."""

    kernel = "split"

    def __init__(self, first, second, sched, pool):
        self.first, self.second, self.sched, self.pool = first, second, sched, pool
        self.out, self.device = first.out, first.device
        a = _lib.PaSplitArgs()
        a.first, a.second = ctypes.pointer(first.args), ctypes.pointer(second.args)
        if isinstance(sched, SplitGrid):
            self.kernel = "split-grid"
            a.items, a.n_items = _lib.ptr(sched.items), sched.n_items
        else:
            a.run_steps, a.run_start, a.run_groups = _lib.ptr(sched.run), _lib.ptr(sched.start), sched.groups
            a.kv_bits = _lib.ptr(pool)
        a.sync, a.sync_groups = _lib.ptr(sched.sync), sched.sync_groups
        a.sync_signal, a.sync_wait = sched.sync_signal, sched.sync_wait
        a.status = _lib.ptr(sched.status)
        self.args = a
        self._ref = ctypes.byref(a)

    def __call__(self):
        _lib.check(_lib.lib().pa_attn_fwd_split(self._ref, _lib.stream_of(self.out)), "pa_attn_fwd_split")
        return self.out

    def check(self):
        """Raise if a merge of a past launch gave up waiting; status and counters are cleared."""
        self.sched.check()


def lse_merge(o_parts, lse_parts, out_dtype=torch.float32, lse_out=None):
    """Merge fp32 partials [BH, N, D] with their LSE [BH, N] (pa_lse_merge)."""
    if not o_parts or len(o_parts) != len(lse_parts):
        raise ValueError("need matching, non-empty o_parts and lse_parts")
    o_parts = [t.contiguous() for t in o_parts]
    lse_parts = [t.contiguous() for t in lse_parts]
    _lib.require_device(*o_parts, *lse_parts)
    BH, N, D = o_parts[0].shape
    for o_, l_ in zip(o_parts, lse_parts):
        if o_.dtype != torch.float32 or l_.dtype != torch.float32 or o_.shape != (BH, N, D) or l_.shape != (BH, N):
            raise ValueError("parts must be float32 [BH, N, D] with float32 [BH, N] LSE")
    out = torch.empty((BH, N, D), dtype=out_dtype, device=o_parts[0].device)
    n = len(o_parts)
    optrs = (_lib.c_vp * n)(*[t.data_ptr() for t in o_parts])
    lptrs = (_lib.c_vp * n)(*[t.data_ptr() for t in lse_parts])
    with torch.cuda.device(out.device):
        _lib.check(_lib.lib().pa_lse_merge(optrs, lptrs, n, _lib.ptr(out), _lib.DTYPE_CODE[out_dtype],
                                           _lib.ptr(lse_out), BH, N, D, _lib.stream_of(out)), "pa_lse_merge")
    return out
