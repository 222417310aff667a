"""Device-side selector: exact tile counts against the independent per-head counts for the
benchmark configurations, the chosen bases and splits, and the planned split run end to
end against the oracle."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from polyhedral_amd import selector as sel
from polyhedral_amd.polyattn import masks as M
from polyhedral_amd.split import SplitPlan
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mask,N,residue,tiles", [
    # per-head tile counts at 128x32 from a brute force over the predicates
    (M.Dilated(8), 8192, 0, 8320), (M.Dilated(8), 8192, 8, 1152),
    (M.LocalStrided(256, 16), 16384, 0, 33024), (M.LocalStrided(256, 16), 16384, 16, 11664),
    (M.SlidingWindow(256), 16384, 0, 1524),
    (M.Difference(M.Dilated(16), M.SlidingWindow(256)), 16384, 16, 2304),
    (M.SinksWindow(64, 1024), 32768, 0, 9566),
])
def test_tile_counts_match_the_brute_force_counts(gpu, mask, N, residue, tiles):
    assert sel.tile_count(mask, N, 128, 32, residue, gpu)[0] == tiles


def test_selects_the_residue_basis_for_a_lattice(gpu):
    assert sel.select(M.Dilated(8), 8192, 128, 32, gpu) == "residue-perm-8"
    assert sel.select(M.SlidingWindow(256), 8192, 128, 32, gpu) == "identity"


def test_plans_the_band_lattice_split(gpu):
    p = sel.plan(M.LocalStrided(256, 16), 16384, 128, 32, gpu)
    assert [(pc.mask.name, pc.residue) for pc in p.pieces] == [("window-256", 0), ("dilated-16\\window-256", 16)]
    assert p.elements == (1524 + 2304) * 128 * 32
    # the best single pass is the cheapest basis of the union, and the split beats it
    assert p.single[1] == min(p.detail.values()) and p.detail["residue-perm-16"] == 11664 * 128 * 32
    assert p.elements < p.single[1]


@pytest.mark.parametrize("mask", [M.LocalStrided(256, 16), M.SinksWindow(4, 256),
                                  M.Union(M.SlidingWindow(64), M.Dilated(8)), M.Dilated(16)])
def test_planned_split_equals_single_pass_attention(gpu, mask):
    N, D, BH = 2048, 128, 2
    p = sel.plan(mask, N, 128, 32, gpu)
    q, k, v = make_qkv(BH, N, D, torch.bfloat16, seed=4)
    rows = lambda a, b: np.stack([np.asarray(mask.row_cols(r, N), dtype=bool) for r in range(a, b)])
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), rows)
    plan = SplitPlan(p.pieces, N, gpu)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu))
    check_close(o, want, torch.bfloat16, f"planned {mask.name}: {[(x.mask.name, x.residue) for x in p.pieces]}")
