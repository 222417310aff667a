"""Oracle class-A permutation (test infrastructure only): gpu/permute.py:12-31 restated."""
import numpy as np


def residue_perm(N, s):
    """Stable argsort by i % s * N + i // s (gpu/permute.py:12-15)."""
    i = np.arange(N)
    return np.argsort(i % s * N + i // s, kind="stable").astype(np.int32)


def invert(perm):
    inv = np.empty_like(perm)
    inv[np.asarray(perm, dtype=np.int64)] = np.arange(len(perm), dtype=perm.dtype)
    return inv


def gather_rows(x, perm):
    """x[:, perm] along axis 1 (index_select(1, perm), gpu/permute.py:22-24)."""
    return np.take(x, np.asarray(perm, dtype=np.int64), axis=1)


def scatter_rows(x, perm):
    out = np.empty_like(x)
    out[:, np.asarray(perm, dtype=np.int64)] = x
    return out
