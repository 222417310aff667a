"""The oracle block index (gpu/blockindex.py:32-51 restated) pinned against the
reference's own recorded counts, an explicit-loop tiler, and full-size workload counts."""
import json
import pathlib

import numpy as np
import pytest

from oracle import blockindex as obi
from oracle import masks as om
from oracle import permute as op

GOLD = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_counts.json").read_text())
WORK = json.loads((pathlib.Path(__file__).parent / "golden" / "workload_counts.json").read_text())


def _build(name, N, BQ, A, s=1):
    perm = op.residue_perm(N, s) if s > 1 else None
    return obi.build(om.NAMED[name], N, BQ, A, perm_q=perm, perm_kv=perm, threads=8)


@pytest.mark.parametrize("row", GOLD["results_csv"], ids=lambda r: f"{r['mask']}-{r['N']}")
def test_results_csv_exact_rows(row):
    """results/results.csv sampled=0 rows: live count and tile elements at 4 square grains."""
    for g, elements in row["elements"].items():
        r = _build(row["mask"], row["N"], int(g), int(g))
        assert r["live"] == row["live"]
        assert r["elements"] == elements, (row["mask"], g)


@pytest.mark.parametrize("row", GOLD["reindex_csv"], ids=lambda r: f"{r['mask']}-s{r['s']}-{r['BQ']}")
def test_reindex_csv_class_a_waste(row):
    """results/reindex.csv: waste = elements / live under identity and residue-perm-s."""
    r = _build(row["mask"], row["N"], row["BQ"], row["A"], row["s"])
    assert r["elements"] / r["live"] == pytest.approx(row["waste"], rel=1e-12)


@pytest.mark.parametrize("row", GOLD["predictions"] + GOLD["exp6"],
                         ids=lambda r: f"{r['mask']}-s{r['s']}-{r['BQ']}x{r['A']}")
def test_recorded_element_counts(row):
    """results/predictions-d4.txt (exp0) and out.out exp6 rows: elements under rp-s."""
    assert _build(row["mask"], row["N"], row["BQ"], row["A"], row["s"])["elements"] == row["elements"]


@pytest.mark.parametrize("row", GOLD["exp7"], ids=lambda r: f"N{r['N']}-{r['BQ']}x{r['A']}-rp{r['s']}")
def test_exp7_tiles_and_max_per_block(row):
    r = _build(row["mask"], row["N"], row["BQ"], row["A"], row["s"])
    assert int(r["kv_num"].sum()) == row["tiles"] and r["kv_idx"].shape[1] == row["max_kv"]


@pytest.mark.parametrize("row", GOLD["exp8"], ids=lambda r: f"{r['mask']}-N{r['N']}-{r['BQ']}x{r['A']}-s{r['s']}")
def test_exp8_recorded_cells(row):
    """gpu/exp8_three_cells.py:65-72: (tiles, runs) at 128x128, (tiles, max per block) at 128x32."""
    r = _build(row["mask"], row["N"], row["BQ"], row["A"], row["s"])
    assert int(r["kv_num"].sum()) == row["tiles"]
    if "runs" in row:
        assert obi.runs(r["kv_idx"], r["kv_num"]) == row["runs"]
    else:
        assert r["kv_idx"].shape[1] == row["max_kv"]


@pytest.mark.parametrize("row", GOLD["gate_waste"], ids=lambda r: r["mask"])
def test_gate_permuted_waste(row):
    """out.out gate step 4: permuted 16x16 waste printed to 3 decimals."""
    r = _build(row["mask"], row["N"], row["BQ"], row["A"], row["s"])
    assert round(r["elements"] / r["live"], 3) == row["waste_3dp"]


@pytest.mark.parametrize("row", WORK["cases"], ids=lambda r: f"{r['name']}-N{r['N']}-s{r['s']}-{r['BQ']}x{r['A']}")
def test_workload_counts_full_size(row):
    r = _build(row["name"], row["N"], row["BQ"], row["A"], row["s"])
    assert r["live"] == row["live"]
    assert int(r["kv_num"].sum()) == row["tiles"]
    assert r["kv_idx"].shape[1] == row["max_kv"]
    if "full" in row:
        listed = np.concatenate([r["kv_partial"][i, :n] for i, n in enumerate(r["kv_num"])]) if row["tiles"] else []
        assert int((np.asarray(listed) == 0).sum()) == row["full"]
        assert int((np.asarray(listed) == 1).sum()) == row["partial"]


def _naive(M, BQ, A):
    """Explicit loops over tiles: listed tiles, full flags, live count (tests/test_quantities.py:37-47)."""
    N = M.shape[0]
    lists, flags = [], []
    for i in range(0, N, BQ):
        row, fl = [], []
        for j in range(0, N, A):
            blk = M[i:i + BQ, j:j + A]
            if blk.any():
                row.append(j // A)
                fl.append(0 if blk.all() else 1)
        lists.append(row)
        flags.append(fl)
    return lists, flags, int(M.sum())


TILES = [(128, 128), (128, 32), (64, 64), (32, 32), (16, 16), (128, 16), (16, 128), (32, 64)]


@pytest.mark.parametrize("name", sorted(om.NAMED))
def test_c_builder_matches_numpy_restatement_and_naive_tiler(name):
    N = 256
    M = om.dense(om.NAMED[name], N)
    for BQ, A in TILES:
        c = obi.build(om.NAMED[name], N, BQ, A)
        d = obi.build_dense(M, BQ, A)
        for k in ("kv_idx", "kv_num", "kv_partial"):
            assert np.array_equal(c[k], d[k]), (name, BQ, A, k)
        assert c["live"] == d["live"] and c["elements"] == d["elements"]
        lists, flags, live = _naive(M, BQ, A)
        assert live == c["live"]
        for i, (l, f) in enumerate(zip(lists, flags)):
            n = c["kv_num"][i]
            assert list(c["kv_idx"][i, :n]) == l and list(c["kv_partial"][i, :n]) == f
            assert not c["kv_idx"][i, n:].any() and not c["kv_partial"][i, n:].any()


@pytest.mark.parametrize("s", [2, 4, 8])
def test_permuted_build_equals_materialised_permuted_matrix(s):
    """perm applied inside the builder == building M[perm][:, perm] (gpu/test_correctness.py:71-72)."""
    N = 512
    perm = op.residue_perm(N, s)
    for name in ("dilated-8", "local256+str8", "sinks4+win256"):
        M = om.dense(om.NAMED[name], N)[perm][:, perm]
        for BQ, A in [(16, 16), (128, 32), (64, 64)]:
            a = obi.build(om.NAMED[name], N, BQ, A, perm_q=perm, perm_kv=perm)
            b = obi.build_dense(M, BQ, A)
            for k in ("kv_idx", "kv_num", "kv_partial"):
                assert np.array_equal(a[k], b[k])


def test_wave_codes_are_consistent_with_the_tile_flags():
    """OR of group 'some live' bits = listed; AND of group 'all live' bits = full; each group
    bit equals any/all over its own 32-row x min(A,32)-column block."""
    N = 512
    for name in ("window-128", "dilated-8", "sinks4+win256", "lat16-band256"):
        M = om.dense(om.NAMED[name], N)
        for BQ, A in TILES:
            codes, _ = obi.tile_codes(om.NAMED[name], N, BQ, A)
            rg, cw = min(BQ, 32), min(A, 32)
            for qb in range(N // BQ):
                for kb in range(N // A):
                    blk = M[qb * BQ:(qb + 1) * BQ, kb * A:(kb + 1) * A]
                    code = int(codes[qb, kb])
                    for g in range(BQ // rg):
                        for c in range(A // cw):
                            sub = blk[g * rg:(g + 1) * rg, c * cw:(c + 1) * cw]
                            bit = g * (A // cw) + c
                            assert (code >> (2 * bit)) & 1 == int(sub.any())
                            assert (code >> (2 * bit + 1)) & 1 == int(sub.all())


# The band-256 | lattice-32 companion at L = 65536 (the prefix-LM workload's shape with a
# non-empty second sub-mask), per head, derived in closed form:
#  * window-256: row i holds min(i + 1, 256) keys, so sum = 256 N - 256 * 255 / 2.  A
#    128-row block at i0 >= 256 spans columns [i0 - 255, i0 + 127]: 12 tiles of 32, of which
#    the 4 with columns in [i0 - 128, i0 - 1] are full; block 0 has its 4 diagonal tiles,
#    block 1 (causal so far) 4 full and 4 diagonal.
#  * lattice-32 minus band in rp32: class c holds positions 32 t + c, t < 2048, and row t
#    of a class sees t' <= t - 8 of its own class (32 (t - t') >= 256), so a class is a
#    2048 x 2048 causal matrix shifted by 8: sum_{t >= 8} (t - 7) = 2040 * 2041 / 2 per
#    class.  Query block b (t in [128 b, 128 b + 127]) lists key tiles 0 .. 4 b + 3, the
#    first 4 b - 1 of them full (b >= 1), the last 5 (block 0: 4) partial; max 64 tiles.
COMPANION = [
    ("window-256", 65536, 1, dict(live=256 * 65536 - 256 * 255 // 2, tiles=4 + 8 + 510 * 12,
                                  full=4 + 510 * 4, partial=4 + 4 + 510 * 8, max_kv=12)),
    ("lat32-band256", 65536, 32, dict(live=32 * 2040 * 2041 // 2, tiles=32 * sum(4 * b + 4 for b in range(16)),
                                      full=32 * sum(4 * b - 1 for b in range(1, 16)),
                                      partial=32 * (4 + 15 * 5), max_kv=64)),
]


@pytest.mark.parametrize("name,N,s,want", COMPANION, ids=[c[0] for c in COMPANION])
def test_companion_counts_closed_form(name, N, s, want):
    r = _build(name, N, 128, 32, s)
    assert r["live"] == want["live"]
    assert int(r["kv_num"].sum()) == want["tiles"] and r["kv_idx"].shape[1] == want["max_kv"]
    listed = np.concatenate([r["kv_partial"][i, :n] for i, n in enumerate(r["kv_num"])])
    assert int((listed == 0).sum()) == want["full"] and int((listed == 1).sum()) == want["partial"]


def test_companion_union_is_the_disjoint_sum():
    """band256+lat32 = window-256 + (lattice-32 minus window-256), checked on the oracle's
    live counts at full size: 83,362,816 live pairs per head."""
    union = _build("band256+lat32", 65536, 128, 32)["live"]
    assert union == sum(c[3]["live"] for c in COMPANION) == 83362816
