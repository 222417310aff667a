"""Counterpart of the reference's ``polyattn.transforms`` for what the hot path's
drivers import from it: ``kv_per_tile``, the number of distinct physical key rows one
BQ x A tile touches under a change of key basis (src/polyattn/transforms.py:99-110,
used by gpu/exp6_traffic_multiplier.py:41,115).

* Class A (a query-independent relabelling of keys, the residue permutation of
  gpu/permute.py): the relabelled K/V is contiguous, so a tile reads its A rows.
* Class B (kv' = (kv - a q) / s, a query-dependent shear / stride fold): the tile's
  physical key of (query offset x, key column y) is s y + a x + const, so it touches
  as many rows as the offset set {a x - s y : 0 <= x < BQ, 0 <= y < A} has members.

The rest of the reference module (the transform search over materialised masks) is
analytical tooling outside the attention path and is not provided.
"""
import numpy as np


def kv_per_tile(kind, a, s, BQ, A):
    """Distinct physical kv rows a single BQ x A tile must touch (see module doc)."""
    if kind == "A":
        return int(A)
    if kind != "B":
        raise ValueError(f"kind must be 'A' or 'B', got {kind!r}")
    a, s, BQ, A = int(a), int(s), int(BQ), int(A)
    if BQ < 1 or A < 1:
        raise ValueError("BQ and A must be positive")
    # the offsets a x - s y span [lo, hi]; mark each reachable one in a bitmap
    xs = a * np.arange(BQ, dtype=np.int64)
    ys = s * np.arange(A, dtype=np.int64)
    vals = (xs[:, None] - ys[None, :]).ravel()
    lo = int(vals.min())
    seen = np.zeros(int(vals.max()) - lo + 1, dtype=bool)
    seen[vals - lo] = True
    return int(seen.sum())
