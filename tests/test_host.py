"""Host-side logic of the drop-in modules, checked on the CPU against the oracle."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import blockindex as obi
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import launch, registry, spec, timing, workloads
from polyhedral_amd.polyattn import cost, masks


def test_kind_constants_keep_the_reference_values():
    assert (registry.CAUSAL, registry.WINDOW, registry.DILATED, registry.LOCAL_STRIDED, registry.TWOBAND,
            registry.SINKS) == (0, 1, 2, 3, 4, 5)
    from polyhedral_amd import attention
    attention._assert_kinds_match()


@pytest.mark.parametrize("name", sorted(registry.SPECS))
def test_registry_three_consumers_agree_and_match_the_oracle(name):
    assert registry.check_agreement(name, N=512)
    N = 384
    M = om.dense(om.NAMED[name], N)
    assert np.array_equal(registry.dense_bool(name, N, device="cpu").numpy(), M)
    m = registry.numpy_mask(name)
    assert np.array_equal(m.dense(N), M)
    kind, p0, p1, p2 = registry.triton_params(name)
    s = spec.MaskSpec.of(kind, p0, p1, p2)
    i = np.arange(N)
    assert np.array_equal(s.live(i[:, None], i[None, :]), M)


@pytest.mark.parametrize("m", masks.zoo(), ids=lambda m: m.name)
def test_mask_zoo_closed_forms_and_unions(m):
    for N in (256, 512, 1000):
        D = m.dense(N)
        assert m.live_count(N) == int(D.sum())
        for q0 in range(0, N - 16, 97):
            assert np.array_equal(m.union_cols(q0, q0 + 16, N), D[q0:q0 + 16].any(axis=0))


@pytest.mark.parametrize("name", ["causal", "window-128", "dilated-8", "local256+str8", "twoband-1000"])
def test_cost_model_equals_index_elements(name):
    """gpu/test_correctness.py step 2: cost(exact_only) == BlockIndex.elements, every gate tile."""
    N = 1024
    m = registry.numpy_mask(name)
    for BQ, A in [(128, 128), (128, 32), (64, 64), (32, 32), (16, 16), (128, 16), (16, 128)]:
        c, sampled = cost.cost(m, N, BQ, A, exact_only=True)
        assert not sampled
        assert c == obi.build(om.NAMED[name], N, BQ, A)["elements"]
    assert cost.cost(m, N, 1, 1, exact_only=True)[0] == m.live_count(N)


class Causal:            # stand-ins with the reference's class names and attributes
    pass


class SinksWindow:
    def __init__(self, g, w):
        self.g, self.w = g, w


class PrefixLM:
    def __init__(self, p):
        self.p = p


def test_reference_mask_objects_translate_by_name():
    assert spec._terms_by_name(Causal()) == (((0, 0, 0, 0),), ())
    assert spec._terms_by_name(SinksWindow(4, 256)) == (((5, 256, 4, 0),), ())
    assert spec._terms_by_name(PrefixLM(2048)) == (((6, 2048, 0, 0),), ())
    d = masks.Difference(masks.Dilated(16), masks.SlidingWindow(256))
    assert spec._terms_by_name(d) == (((2, 16, 0, 0),), ((1, 256, 0, 0),))


def test_dense_bitmap_packing():
    rng = np.random.default_rng(0)
    M = rng.random((70, 70)) < 0.3
    import torch
    bits = spec.pack_dense_bits(M, torch.device("cpu")).numpy().view(np.uint32)
    assert bits.shape == (70, 3)
    for q in range(70):
        for kv in range(70):
            assert bool((bits[q, kv // 32] >> (kv % 32)) & 1) == M[q, kv]


def test_permutation_host_side():
    from polyhedral_amd import perm
    for N, s in [(1024, 8), (1000, 16), (7, 3)]:
        assert np.array_equal(perm.residue_perm(N, s), op.residue_perm(N, s))


def test_launch_sweep_boundary_warnings():
    assert launch._warn_if_on_boundary("w4/s2") == ""
    assert "warps at sweep max" in launch._warn_if_on_boundary("w8/s2")
    assert "stages at sweep max" in launch._warn_if_on_boundary("w2/s4")
    assert launch._warn_if_on_boundary("w1/s1") == ""          # hardware floors, not a narrow sweep
    assert "NO LAUNCH" in launch._warn_if_on_boundary(None)


def test_report_table_format(capsys):
    timing.report([["a", 1.23456, 7]], [("name", 6), ("ms", 10), ("n", 4)], title="T", note="N")
    out = capsys.readouterr().out.splitlines()
    assert out[1] == "T" and out[3] == "  name        ms   n" and out[4] == "     a     1.235   7"


def test_workloads_are_disjoint_splits_of_their_masks():
    """Every workload's pieces partition its mask (checked at a reduced length)."""
    for name in workloads.NAMES:
        wl = workloads.make(name)
        n = 512
        i = np.arange(n)
        whole = wl.union.live(i[:, None], i[None, :])
        cover = np.zeros_like(whole)
        for p in wl.pieces:
            part = p.mask.live(i[:, None], i[None, :])
            assert not (part & cover).any(), f"{name}: pieces overlap"
            cover |= part
        assert np.array_equal(cover, whole), name


def test_workload_live_counts_match_the_fixture():
    gold = {(c["name"], c["N"]): c["live"] for c in json.load(open(
        os.path.join(os.path.dirname(__file__), "golden", "workload_counts.json")))["cases"]}
    assert workloads.make("bandlat-L16k").pieces[0].mask.live_count(16384) == gold[("window-256", 16384)]
    assert workloads.make("bandlat-L16k").union.live_count(16384) == gold[("band256+lat16", 16384)]
    assert workloads.make("sinkwin-L32k").union.live_count(32768) == gold[("sinks64+win1024", 32768)]


def test_bench_refuses_more_than_one_gpu():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
