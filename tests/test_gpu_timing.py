"""The drivers' timing call surface on the GPU: bench.time_ms / paired_time
(gpu/bench.py:11-74) and permute.permutation_cost_ms (gpu/permute.py:34-38), imported by
bare name as a driver imports them, run on real kernels and checked against the
kernels' own events."""
import sys

import pytest
import torch

from tests.conftest import ROOT

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(ROOT / "polyhedral_amd" / "gpu"))
import bench  # noqa: E402
import permute  # noqa: E402


def _events_ms(fn, reps=20):
    """Median of fn() timed alone by a pair of events, without a flush."""
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e))
    return sorted(out)[len(out) // 2]


def test_time_ms_returns_median_and_stdev_of_real_work(gpu):
    x = torch.randn(32, 16384, 128, device=gpu, dtype=torch.bfloat16)
    p = torch.from_numpy(permute.residue_perm(16384, 16)).to(gpu)
    fn = lambda: permute.apply_perm(x, p)  # noqa: E731
    med, sd = bench.time_ms(fn, warmup=5, reps=30)
    assert isinstance(med, float) and isinstance(sd, float)
    assert med > 0 and sd >= 0
    # without the flush the harness measures what a bare pair of events measures
    med_nf, _ = bench.time_ms(fn, warmup=5, reps=30, flush_l2=False)
    ev = _events_ms(fn)
    assert 0.5 < med_nf / ev < 2.0, (med_nf, ev)


def test_paired_time_ratio_tracks_the_work(gpu):
    x = torch.randn(32, 8192, 128, device=gpu, dtype=torch.bfloat16)
    p = torch.from_numpy(permute.residue_perm(8192, 8)).to(gpu)
    one = lambda: permute.apply_perm(x, p)  # noqa: E731
    two = lambda: (permute.apply_perm(x, p), permute.apply_perm(x, p))  # noqa: E731
    a, b, ratio, sd = bench.paired_time(one, two, warmup=5, reps=40)
    for v in (a, b, ratio, sd):
        assert isinstance(v, float)
    assert a > 0 and b > 0 and sd >= 0
    assert 1.4 < ratio < 2.6, f"two gathers / one gather = {ratio:.2f}"
    # the paired ratio agrees with the ratio of the medians
    assert abs(ratio - b / a) < 0.3


def test_permutation_cost_ms_times_three_gathers(gpu):
    BH, N, D = 16, 8192, 128
    q, k, v = (torch.randn(BH, N, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    p = torch.from_numpy(permute.residue_perm(N, 8)).to(gpu)
    ms = permute.permutation_cost_ms(q, k, v, p, reps=20)
    assert isinstance(ms, float) and ms > 0
    one = _events_ms(lambda: permute.apply_perm(q, p))
    assert 1.5 < ms / one < 6.0, (ms, one)
    # the bytes moved (each tensor read and written once) at a plausible HBM rate
    gbs = 3 * 2 * q.numel() * q.element_size() / (ms * 1e-3) / 1e9
    assert 200 < gbs < 9000, gbs


def test_report_prints_the_drivers_table(capsys):
    bench.report([["a", 1.5, 3]], [("case", 6), ("ms", 8), ("n", 4)], title="t", note="n")
    out = capsys.readouterr().out
    assert "case" in out and "1.500" in out and out.strip().endswith("n")
