"""GPU block-index builder vs the oracle: bit-exact kv_idx / kv_num / kv_partial /
wave codes, elements and live (gpu/blockindex.py:32-51 semantics)."""
import numpy as np
import pytest

from oracle import blockindex as obi
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import index as pindex
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import SPECS, numpy_mask

pytestmark = pytest.mark.gpu

TILES = [(128, 128), (128, 32), (64, 64), (32, 32), (16, 16), (128, 16), (16, 128), (32, 64)]


def _compare(bi, ref):
    assert np.array_equal(bi.kv_num, ref["kv_num"])
    assert bi.kv_idx.shape == ref["kv_idx"].shape
    assert np.array_equal(bi.kv_idx, ref["kv_idx"])
    assert np.array_equal(bi.kv_partial, ref["kv_partial"])
    assert np.array_equal(bi.kv_wave_bits, ref["wave"])
    assert bi.elements == ref["elements"] and bi.live == ref["live"]


@pytest.mark.parametrize("name", [n for n in SPECS])
@pytest.mark.parametrize("N", [256, 1024])
def test_named_masks_all_tiles(gpu, name, N):
    spec = om.NAMED[name]
    m = numpy_mask(name)
    for BQ, A in TILES:
        _compare(pindex.build(m, N, BQ, A), obi.build(spec, N, BQ, A))


@pytest.mark.parametrize("name,s,N", [("dilated-4", 4, 1024), ("dilated-8", 8, 1024),
                                      ("local256+str8", 2, 2048), ("local256+str8", 4, 2048),
                                      ("local256+str8", 8, 2048), ("band256+lat16", 16, 2048),
                                      ("lat16-band256", 16, 4096), ("sinks4+win256", 8, 1024)])
def test_class_a_permuted(gpu, name, s, N):
    perm = op.residue_perm(N, s)
    m = pm.Permuted(numpy_mask(name), perm)
    for BQ, A in [(128, 32), (16, 16), (128, 128), (64, 64)]:
        _compare(pindex.build(m, N, BQ, A), obi.build(om.NAMED[name], N, BQ, A, perm_q=perm, perm_kv=perm))


class _Dense:
    """The reference's explicit-matrix wrapper (gpu/test_correctness.py:90-95)."""
    def __init__(self, M):
        self.M, self.name = M, "permuted"

    def row_cols(self, q, N):
        return self.M[q]


def test_explicit_matrix_input(gpu):
    N, s = 1024, 8
    perm = op.residue_perm(N, s)
    M = om.dense(om.NAMED["dilated-8"], N)[perm][:, perm]
    bi = pindex.build(_Dense(M), N, 16, 16)
    ref = obi.build_dense(M, 16, 16)
    for key in ("kv_idx", "kv_num", "kv_partial"):
        assert np.array_equal(getattr(bi, key), ref[key])
    assert bi.elements == ref["elements"] and bi.live == ref["live"]


def test_empty_mask_gives_zero_pitch(gpu):
    # a lattice restricted to pairs a prefix-LM does not cover
    N = 4096
    bi = pindex.build(numpy_mask("lat32-prefixlm2048"), N, 128, 32)
    assert bi.kv_idx.shape == (N // 128, 0) and bi.live == 0 and bi.elements == 0
    assert not bi.kv_num.any()
