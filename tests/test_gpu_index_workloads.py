"""The block index of every benchmark workload, built on the GPU at full size, at the
workload's tile and at the 16x16 floor, bit-exact against the oracle's streaming C
builder (gpu/blockindex.py:32-51 semantics: kv_idx, kv_num, kv_partial, plus the wave
codes, elements and live pairs) and against the independent per-head counts of
tests/golden/workload_counts.json.  The reference's own builder materialises N x N
(gpu/blockindex.py:35) and cannot reach these sizes."""
import json
import pathlib

import numpy as np
import pytest
import torch

from oracle import blockindex as obi
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import index as pindex
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask

pytestmark = pytest.mark.gpu

GOLD = json.loads((pathlib.Path(__file__).parent / "golden" / "workload_counts.json").read_text())["cases"]

# (mask, N, residue stride s, BQ, A): every workload's pieces, unions and bases, at the
# workload's tile and at 16 x 16
CASES = [
    ("window-128", 1024, 1, 128, 128), ("window-128", 1024, 1, 16, 16),
    ("dilated-8", 8192, 1, 128, 32), ("dilated-8", 8192, 1, 16, 16),
    ("dilated-8", 8192, 8, 128, 32), ("dilated-8", 8192, 8, 16, 16),
    ("window-256", 16384, 1, 128, 32), ("window-256", 16384, 1, 16, 16),
    ("lat16-band256", 16384, 16, 128, 32), ("lat16-band256", 16384, 16, 16, 16),
    ("band256+lat16", 16384, 1, 128, 32), ("band256+lat16", 16384, 1, 16, 16),
    ("band256+lat16", 16384, 16, 128, 32), ("band256+lat16", 16384, 16, 16, 16),
    ("sinks64+win1024", 32768, 1, 128, 32), ("sinks64+win1024", 32768, 1, 16, 16),
    ("prefixlm-2048", 65536, 1, 128, 32), ("prefixlm-2048", 65536, 1, 16, 16),
    ("lat32-prefixlm2048", 65536, 32, 128, 32), ("lat32-prefixlm2048", 65536, 32, 16, 16),
    ("window-256", 65536, 1, 128, 32), ("lat32-band256", 65536, 32, 128, 32),
]


def _gold(name, N, s, BQ, A):
    for c in GOLD:
        if (c["name"], c["N"], c["s"], c["BQ"], c["A"]) == (name, N, s, BQ, A):
            return c
    return None


@pytest.mark.parametrize("name,N,s,BQ,A", CASES, ids=[f"{c[0]}-N{c[1]}-rp{c[2]}-{c[3]}x{c[4]}" for c in CASES])
def test_full_size_index_is_bit_exact(gpu, name, N, s, BQ, A):
    perm = op.residue_perm(N, s) if s > 1 else None
    mask = numpy_mask(name)
    if perm is not None:
        mask = pm.Permuted(mask, perm)
    kv_idx, kv_num, kv_partial, wave, tiles, live, (boff, pool) = pindex.build_device(
        mask, N, BQ, A, device=gpu, bits=True)
    torch.cuda.synchronize()
    ref = obi.build(om.NAMED[name], N, BQ, A, perm_q=perm, perm_kv=perm)
    got_num = kv_num.cpu().numpy()
    assert np.array_equal(got_num, ref["kv_num"])
    assert tuple(kv_idx.shape) == ref["kv_idx"].shape
    assert np.array_equal(kv_idx.cpu().numpy(), ref["kv_idx"])
    assert np.array_equal(kv_partial.cpu().numpy(), ref["kv_partial"])
    assert np.array_equal(wave.cpu().numpy().view(np.uint32), ref["wave"])
    assert tiles * BQ * A == ref["elements"] and live == ref["live"]
    g = _gold(name, N, s, BQ, A)
    if g is not None:
        assert live == g["live"] and tiles == g["tiles"] and kv_idx.shape[1] == g["max_kv"]
        if "full" in g:
            npart = int(kv_partial.to(torch.int64).sum())
            assert (tiles - npart, npart) == (g["full"], g["partial"])
    # the element bitmaps of a sample of partial tiles against the predicate
    part = np.argwhere(ref["kv_partial"] == 1)
    if len(part):
        rng = np.random.default_rng(3)
        pick = part[rng.choice(len(part), size=min(24, len(part)), replace=False)]
        off = boff.cpu().numpy()
        bits = pool.cpu().numpy().view(np.uint32)
        wpr = (A + 31) // 32
        for i, j in pick:
            o = int(off[i, j])
            assert o >= 0
            rows = np.arange(i * BQ, (i + 1) * BQ)
            cols = np.arange(ref["kv_idx"][i, j] * A, ref["kv_idx"][i, j] * A + A)
            oq = perm[rows] if perm is not None else rows
            ok = perm[cols] if perm is not None else cols
            want = om.live(om.NAMED[name], oq[:, None].astype(np.int64), ok[None, :].astype(np.int64))
            words = bits[o:o + BQ * wpr].reshape(BQ, wpr)
            got = np.zeros((BQ, A), dtype=bool)
            for c in range(A):
                got[:, c] = (words[:, c // 32] >> np.uint32(c % 32)) & 1
            assert np.array_equal(got, want), (i, j)
    print(f"{name} N={N} rp{s} {BQ}x{A}: {tiles} tiles, max_kv {kv_idx.shape[1]}, live {live} (bit-exact)")
