"""The decode cache's row of each original position (polyhedral_amd.decode.basis_rows)
inverts the residue permutation of the oracle (gpu/permute.py:12-15: permuted position
-> original), so cache row r holds the token the prefill basis puts at position r."""
import numpy as np
import pytest

from oracle import permute as op
from polyhedral_amd.decode import basis_rows


@pytest.mark.parametrize("N,s", [(1024, 1), (1024, 2), (2048, 8), (4096, 16), (96, 3), (16384, 16)])
def test_rows_invert_the_residue_permutation(N, s):
    p = op.residue_perm(N, s) if s > 1 else np.arange(N)
    assert np.array_equal(basis_rows(p, s, N), np.arange(N))
    # a class's tokens fill its segment in order: appending never moves a row
    t = np.arange(N)
    r = basis_rows(t, s, N)
    for c in range(s):
        rows = r[t % s == c]
        assert np.array_equal(rows, np.arange(c * (N // s), (c + 1) * (N // s)))


def test_identity_basis_is_the_identity():
    assert np.array_equal(basis_rows(np.arange(77), 0, 77), np.arange(77))
