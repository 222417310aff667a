"""Basis selector and disjoint split planner (polyhedral_amd.selector): the host-side
parts (lattice fold, peeling, candidate bases) on the CPU."""
import numpy as np
import pytest

from polyhedral_amd import selector as sel
from polyhedral_amd.polyattn import masks as M


@pytest.mark.parametrize("mask,fold", [(M.Dilated(8), 8), (M.Dilated(16), 16), (M.Dilated(3), 3),
                                       (M.SlidingWindow(256), 1), (M.LocalStrided(256, 16), 1),
                                       (M.Causal(), 1), (M.TwoBand(64, 512), 1)])
def test_derive_fold(mask, fold):
    """The generator of the offsets' sublattice (src/polyattn/lattice.py:43-55): a lattice
    of stride s folds by s; anything holding a run wider than one offset does not fold."""
    assert sel.derive_fold(sel.offsets(mask, 1024)) == fold


def test_offsets_are_the_last_rows_runs():
    assert sel.offsets(M.SlidingWindow(4), 64) == [(0, 3)]
    assert sel.offsets(M.Dilated(16), 64) == [(0, 0), (16, 16), (32, 32), (48, 48)]
    assert sel.offsets(M.LocalStrided(8, 16), 64) == [(0, 7), (16, 16), (32, 32), (48, 48)]


@pytest.mark.parametrize("mask", [M.LocalStrided(256, 16), M.SinksWindow(4, 256), M.SinksWindow(64, 100),
                                  M.Union(M.PrefixLM(128), M.Dilated(32)),
                                  M.Union(M.SlidingWindow(64), M.Dilated(8), M.SlidingWindow(200)),
                                  M.TwoBand(64, 300), M.Dilated(8)])
def test_peeled_parts_are_disjoint_and_cover_the_mask(mask):
    N = 512
    q, kv = np.meshgrid(np.arange(N), np.arange(N), indexing="ij")
    want = mask.live(q, kv)
    cover = np.zeros_like(want)
    for kind, part in sel.peel(mask):
        p = part.live(q, kv)
        assert not (p & cover).any(), f"{part.name} overlaps an earlier part"
        cover |= p
        part.terms()          # every part is expressible as one device predicate
    assert np.array_equal(cover, want)


def test_peel_order_puts_bands_before_lattices():
    kinds = [k for k, _ in sel.peel(M.LocalStrided(256, 16))]
    assert kinds == ["band", "lattice"]
    names = [p.name for _, p in sel.peel(M.Union(M.Dilated(8), M.SlidingWindow(64), M.SlidingWindow(200)))]
    assert names[0] == "window-200" and names[-1].startswith("dilated-8")


def test_candidates_need_tiles_nested_in_residue_blocks():
    assert sel.candidates(16384, 128, 32) == ["identity"] + [f"residue-perm-{s}" for s in (2, 4, 8, 16, 32)]
    # N / s must be a multiple of both tile sides
    assert sel.candidates(1024, 128, 128) == ["identity", "residue-perm-2", "residue-perm-4", "residue-perm-8"]
    assert "residue-perm-3" in sel.candidates(3 * 1024, 128, 32)
