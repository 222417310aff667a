"""Device-side basis selector and disjoint split planner.

The reference derives the basis of a diagonally invariant mask from closed-form tile
counts (src/polyattn/selector.py:80-130, 224-260), derives the lattice fold from the
diagonal offsets (src/polyattn/lattice.py:43-77), and splits a union of differently
structured families into disjoint parts, each in its own basis
(src/polyattn/experiments/compose.py:49-76).  Here the tile counts are exact and come
from the device index builder (pa_index_classify evaluates the predicate per tile under
the candidate relabelling), so they hold for any mask the builder accepts, invariant or
not, without an N x N matrix on either side.

Candidates are the class-A bases the kernels run: identity and the residue permutations
(rows grouped by i mod s) for s in RESIDUES, where N / s is a multiple of both tile
sides so that tiles nest inside the residue blocks (the condition of
selector.py:_cost_residue_perm).  Class B transforms (shear, stride folds) are not
offered: the attention kernels do not run them, and the reference's selector prefers
class A on ties and the composition search excludes class B altogether
(compose.py:23-24).
"""
import ctypes
from dataclasses import dataclass, field
from functools import reduce
from math import gcd
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from .perm import residue_perm
from .polyattn import masks as M
from .spec import device_mask
from .split import Piece

RESIDUES = (2, 3, 4, 6, 8, 12, 16, 32)

# canonical peel order (shapes.py ORDER): bands, then lattices, then sink / prefix
# columns, then anything causal-wide, so every pair lands in the most tile-dense part
_ORDER = {"band": 0, "lattice": 1, "prefix": 2, "other": 3}


def candidates(N, BQ, A):
    """Names of the bases available at this size and tile shape."""
    out = ["identity"]
    for s in RESIDUES:
        if N % s == 0 and (N // s) % BQ == 0 and (N // s) % A == 0:
            out.append(f"residue-perm-{s}")
    return out


def _stride(name):
    return 0 if name == "identity" else int(name.rsplit("-", 1)[1])


def tile_count(mask, N, BQ, A, residue=0, device=None):
    """(listed tiles, live pairs, max tiles per query block) of `mask` at (BQ, A) in the
    identity basis (residue = 0) or the residue-s basis, counted on the device."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    perm = residue_perm(N, residue) if residue else None
    dm = device_mask(mask, N, dev, perm=perm)
    nq, nk = N // BQ, N // A
    codes = torch.empty(nq * nk, dtype=torch.int32, device=dev)
    kv_num = torch.empty(nq, dtype=torch.int32, device=dev)
    totals = torch.empty(3, dtype=torch.int64, device=dev)
    ms = dm.struct()
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().pa_index_classify(ctypes.byref(ms), N, BQ, A, _lib.ptr(codes), _lib.ptr(kv_num),
                                                _lib.ptr(totals), _lib.stream_of(codes)), "pa_index_classify")
        tiles, live, max_kv = (int(x) for x in totals.cpu())
    return tiles, live, max_kv


def costs(mask, N, BQ, A, device=None):
    """{basis: elements computed (listed tiles * BQ * A)} over the available bases."""
    if N % BQ or N % A:
        raise ValueError(f"N={N} is not a multiple of the tile shape {BQ}x{A}")
    return {c: tile_count(mask, N, BQ, A, _stride(c), device)[0] * BQ * A for c in candidates(N, BQ, A)}


def select(mask, N, BQ, A, device=None):
    """The cheapest basis; ties go to identity, then to the smaller stride."""
    c = costs(mask, N, BQ, A, device)
    return min(c, key=lambda k: (c[k], _stride(k)))


# ---- lattice fold (lattice.py:43-77) ----------------------------------------------
def offsets(mask, N):
    """Diagonal offsets d = q - kv live in the last row, as sorted inclusive runs (the
    mask is read one row, never squared)."""
    d = np.flatnonzero(np.asarray(mask.row_cols(N - 1, N), dtype=bool)[::-1])
    if d.size == 0:
        return []
    brk = np.flatnonzero(np.diff(d) > 1)
    starts = np.concatenate(([d[0]], d[brk + 1]))
    ends = np.concatenate((d[brk], [d[-1]]))
    return list(zip(starts.tolist(), ends.tolist()))


def derive_fold(runs):
    """Generator of the sublattice of Z spanned by the offsets; 1 when a run is wider
    than a point (a band spans Z) or there is no lattice."""
    if not runs or any(r > l for l, r in runs):
        return 1
    pts = sorted(l for l, _ in runs)
    return reduce(gcd, (b - a for a, b in zip(pts, pts[1:])), 0) or 1


# ---- shapes and disjoint peeling (compose.py:49-76) -------------------------------
def shapes_of(mask):
    """The structured families a mask is the union of, as (kind, mask) in peel order,
    or a single ('other', mask) when it is not such a union."""
    if isinstance(mask, M.Union):
        out = []
        for p in mask.parts:
            out.extend(shapes_of(p))
    elif isinstance(mask, M.LocalStrided):
        out = [("band", M.SlidingWindow(mask.w)), ("lattice", M.Dilated(mask.s))]
    elif isinstance(mask, M.SinksWindow):
        out = [("band", M.SlidingWindow(mask.w)), ("prefix", _Sinks(mask.g))]
    elif isinstance(mask, M.SlidingWindow):
        out = [("band", mask)]
    elif isinstance(mask, M.Dilated):
        out = [("lattice", mask)]
    else:
        out = [("other", mask)]
    # stable: the union's own order breaks ties inside a kind, wider bands first
    return sorted(out, key=lambda km: (_ORDER[km[0]], -getattr(km[1], "w", 0)))


class _Sinks(M.SinksWindow):
    """The sink columns of a sinks + window mask: causal, kv < g (a window of 1 adds the
    diagonal, which every window part also holds, so peeling removes it)."""

    def __init__(self, g):
        super().__init__(g, 1)


def peel(mask):
    """Disjoint parts whose union is `mask`: part i = shape i minus shapes 0..i-1."""
    parts = []
    seen = []
    for kind, sh in shapes_of(mask):
        if not seen:
            part = sh
        elif len(seen) == 1:
            part = M.Difference(sh, seen[0])
        else:
            part = M.Difference(sh, M.Union(*seen))
        parts.append((kind, part))
        seen.append(sh)
    return parts


@dataclass
class Plan:
    pieces: List[Piece]
    elements: int                     # tile elements of the chosen plan
    single: tuple                     # (basis, elements) of the best single pass
    split: Optional[list] = None      # [(part name, basis, elements)] of the peeled split
    fold: int = 1                     # derived lattice fold of the whole mask
    detail: dict = field(default_factory=dict)


def plan(mask, N, BQ, A, device=None, merge_penalty=0.0):
    """Pieces for SplitPlan: the best single basis for the whole mask, or the peeled
    disjoint split with each part in its best basis when that computes fewer elements.
    merge_penalty (elements per extra part) prices the extra output + LSE pass each part
    adds (compose.py:107-119 reports it separately; 0 compares element counts only)."""
    cs = costs(mask, N, BQ, A, device)
    b_single = min(cs, key=lambda k: (cs[k], _stride(k)))
    single = (b_single, cs[b_single])
    best = ([Piece(mask, BQ, A, residue=_stride(b_single))], cs[b_single])
    split = None
    parts = peel(mask)
    if len(parts) > 1:
        split, pieces, total = [], [], 0
        for kind, part in parts:
            pc = costs(part, N, BQ, A, device)
            b = min(pc, key=lambda k: (pc[k], _stride(k)))
            if tile_count(part, N, BQ, A, 0, device)[1] == 0:
                continue                  # an empty part adds no pass
            split.append((part.name, b, pc[b]))
            pieces.append(Piece(part, BQ, A, residue=_stride(b)))
            total += pc[b]
        if pieces and total + merge_penalty * (len(pieces) - 1) < best[1]:
            best = (pieces, total)
    try:
        fold = derive_fold(offsets(mask, N))
    except Exception:
        fold = 1
    return Plan(pieces=best[0], elements=best[1], single=single, split=split, fold=fold, detail=cs)
