"""The granularity element-count model (src/polyattn/cost.py:23-49).

cost(mask, N, BQ, A): for each query block of BQ rows take the union of live
columns over its rows, cover it with A-aligned column segments and charge
BQ * A per covered segment.  Equal, by definition, to BlockIndex.elements of the
same (mask, N, BQ, A): the correctness gate (gpu/test_correctness.py:37-45)
checks exactly that.  Above MAX_BLOCKS query blocks the reference samples
query blocks evenly and rescales unless exact_only; that behaviour is kept.
"""
import numpy as np

MAX_BLOCKS = 512


def cost(mask, N, BQ, A, exact_only=False):
    """Returns (elements_computed, was_sampled)."""
    assert N % BQ == 0 and N % A == 0
    nblocks = N // BQ
    if nblocks <= MAX_BLOCKS or exact_only:
        blocks, sampled = np.arange(nblocks), False
    else:
        blocks = np.unique(np.linspace(0, nblocks - 1, MAX_BLOCKS).round().astype(int))
        sampled = True
    covered = 0
    for b in blocks:
        q0 = int(b) * BQ
        covered += int(mask.union_cols(q0, q0 + BQ, N).reshape(-1, A).any(axis=1).sum())
    acc = BQ * A * covered
    if sampled:
        acc = acc * nblocks / len(blocks)
    return float(acc), sampled


def dense_cost(mask, N, BQ, A):
    """Tile count over the materialised N x N mask times BQ * A. Small N only."""
    M = mask.dense(N)
    return float(M.reshape(N // BQ, BQ, N // A, A).any(axis=(1, 3)).sum() * BQ * A)
