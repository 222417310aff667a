"""Oracle predicates and permutation pinned by explicit set definitions (pure Python,
tiny N) and by the definitions in src/polyattn/masks.py / gpu/masks_gpu.py."""
import numpy as np
import pytest

from oracle import masks as om
from oracle import permute as op


def _sets(kind, p0, p1, p2, n):
    """live column sets per row, from the definitions written as sets."""
    out = []
    for q in range(n):
        causal = set(range(q + 1))
        if kind == om.CAUSAL:
            s = causal
        elif kind == om.WINDOW:
            s = {j for j in causal if q - j < p0}
        elif kind == om.DILATED:
            s = set(range(q % p0, q + 1, p0))
        elif kind == om.LOCAL_STRIDED:
            s = {j for j in causal if q - j < p0} | set(range(q % p1, q + 1, p1))
        elif kind == om.TWOBAND:
            s = {j for j in causal if q - j < p0 or p1 <= q - j < p1 + p2}
        elif kind == om.SINKS:
            s = {j for j in causal if q - j < p0} | set(range(min(p1, q + 1)))
        elif kind == om.PREFIX_LM:
            s = set(range(p0)) if q < p0 else causal     # src/polyattn/masks.py:138-139
        out.append({j for j in s if j < n})
    return out


@pytest.mark.parametrize("name", sorted(om.NAMED))
def test_predicates_match_set_definitions(name):
    n = 300
    inc, exc = om.NAMED[name]
    want = [set() for _ in range(n)]
    for t in inc:
        for q, s in enumerate(_sets(*t, n)):
            want[q] |= s
    for t in exc:
        for q, s in enumerate(_sets(*t, n)):
            want[q] -= s
    M = om.dense(om.NAMED[name], n)
    for q in range(n):
        assert set(np.flatnonzero(M[q])) == want[q], (name, q)


@pytest.mark.parametrize("N,s", [(1024, 4), (1000, 8), (16384, 16), (7, 3), (5, 8), (65536, 32)])
def test_residue_perm_is_the_class_sort(N, s):
    p = op.residue_perm(N, s)
    assert np.array_equal(np.sort(p), np.arange(N))                  # a permutation
    keys = (p % s) * N + p // s
    assert (np.diff(keys) > 0).all()                                 # sorted by (i mod s, i div s)
    if N % s == 0:                                                   # closed form
        Q = N // s
        pos = np.arange(N)
        assert np.array_equal(p, (pos % Q) * s + pos // Q)
    inv = op.invert(p)
    assert np.array_equal(inv[p], np.arange(N)) and np.array_equal(p[inv], np.arange(N))


def test_lattice_is_block_diagonal_after_the_residue_permutation():
    """A class-A basis makes kv == q (mod s) block-diagonal (gpu/permute.py:12-15)."""
    N, s = 512, 8
    p = op.residue_perm(N, s)
    M = om.dense(om.NAMED["dilated-8"], N)[p][:, p]
    Q = N // s
    for a in range(s):
        for b in range(s):
            blk = M[a * Q:(a + 1) * Q, b * Q:(b + 1) * Q]
            assert (a == b) == bool(blk.any())


def test_row_gather_and_scatter_are_inverse():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 100, 5))
    p = op.residue_perm(100, 7)
    y = op.gather_rows(x, p)
    assert np.array_equal(y[:, 10], x[:, p[10]])
    assert np.array_equal(op.scatter_rows(y, p), x)
