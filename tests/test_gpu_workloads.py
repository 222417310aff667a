"""The five benchmark workloads at full size on the GPU: sampled query rows against the
float64 oracle (every row of the sample checked), LSE at those rows, and whole-tensor
properties (permuted == identity basis, split == single pass)."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from polyhedral_amd import workloads
from polyhedral_amd.split import SplitPlan
from tests.util import TOL, as64

pytestmark = pytest.mark.gpu

ORACLE = {"window128-L1k": "window-128", "dilated8-L8k": "dilated-8", "bandlat-L16k": "band256+lat16",
          "sinkwin-L32k": "sinks64+win1024", "prefixlat-L64k": "prefixlm-2048",
          "bandlat32-L64k": "band256+lat32"}


def _sample_rows(L, extra=()):
    rng = np.random.default_rng(7)
    base = {0, 1, 63, 64, 127, 128, 255, 256, 1023, 1024, L // 2, L - 129, L - 2, L - 1, *extra}
    return np.array(sorted({r for r in base if 0 <= r < L} | set(rng.integers(0, L, 40).tolist())))


def _oracle_rows(name, q, k, v, heads, rows):
    """float64 dense masked attention (gpu/reference.py:5-13) of the given rows over all
    keys: (o [h, r, D], lse [h, r]); rows with no live key give 0 and -inf."""
    spec = om.NAMED[ORACLE[name]]
    L, D = q.shape[1], q.shape[2]
    qs = as64(q[heads][:, rows])
    kh, vh = as64(k[heads]), as64(v[heads])
    M = om.live(spec, rows[:, None].astype(np.int64), np.arange(L)[None, :])
    s = np.matmul(qs, kh.transpose(0, 2, 1)) * D ** -0.5
    s = np.where(M[None], s, -np.inf)
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0)
    e = np.exp(s - mx)
    den = e.sum(-1, keepdims=True)
    want = np.where(den > 0, np.matmul(e / np.where(den > 0, den, 1), vh), 0)
    wlse = np.where(den[..., 0] > 0, (mx + np.log(np.where(den > 0, den, 1)))[..., 0], -np.inf)
    return want, wlse


def _log(entry):
    """Append a parity record (JSON line) to $PA_PARITY_LOG when it is set."""
    import json
    import os
    path = os.environ.get("PA_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(entry) + "\n")


def _check_rows(name, o, lse, q, k, v, heads, rows):
    want, wlse = _oracle_rows(name, q, k, v, heads, rows)
    got = as64(o[heads][:, rows])
    err = np.abs(got - want)
    tmax, tmean = TOL[q.dtype]
    assert err.max() <= tmax, f"{name}: max abs err {err.max():.3e}"
    if tmean is not None:
        assert err.mean() <= tmean, f"{name}: mean abs err {err.mean():.3e}"
    gl = lse[heads][:, rows].cpu().numpy().astype(np.float64)
    fin = np.isfinite(wlse)
    assert np.array_equal(np.isfinite(gl), fin)
    assert np.abs(gl[fin] - wlse[fin]).max() < (1e-4 if q.dtype == torch.float32 else 2e-2)
    return float(err.max()), float(err.mean())


def test_window128_every_row_every_head(gpu):
    """The fp32 workload compared in full (4 heads x 1024 rows) at 1e-5, and its LSE."""
    name = "window128-L1k"
    wl = workloads.make(name)
    q, k, v = wl.inputs(0, "cpu")
    plan = SplitPlan(wl.pieces, wl.L, gpu)
    lse = torch.empty(wl.H, wl.L, device=gpu)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu), lse=lse)
    torch.cuda.synchronize()
    mx, mean = _check_rows(name, o.cpu(), lse.cpu(), q, k, v, list(range(wl.H)), np.arange(wl.L))
    _log(dict(workload=name, rows="all", heads="all", max_abs=mx, mean_abs=mean))
    print(f"{name}: every row, every head: max abs {mx:.2e} mean abs {mean:.2e}")


@pytest.mark.parametrize("name", workloads.NAMES)
def test_workload_sampled_rows(gpu, name):
    """Sampled query rows of every head against the float64 oracle."""
    wl = workloads.make(name)
    q, k, v = wl.inputs(0, "cpu")
    plan = SplitPlan(wl.pieces, wl.L, gpu)
    lse = torch.empty(wl.H, wl.L, device=gpu)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu), lse=lse)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    rows = _sample_rows(wl.L, extra=(2047, 2048, 2049))
    heads = list(range(wl.H))
    mx, mean = _check_rows(name, o.cpu(), lse.cpu(), q, k, v, heads, rows)
    _log(dict(workload=name, rows=len(rows), heads=len(heads), max_abs=mx, mean_abs=mean))
    print(f"{name}: sampled rows of every head: max abs {mx:.2e} mean abs {mean:.2e}")


def test_split_merge_rounding_is_bounded(gpu):
    """The split merges the first piece's output, stored in bf16, with the second
    piece's fp32 result: one rounding more than a single pass.  Over sampled rows of
    every head its error against the float64 oracle stays within the tolerance and
    close to the single pass's."""
    name = "bandlat-L16k"
    wl = workloads.make(name)
    qc, kc, vc = wl.inputs(0, "cpu")
    q, k, v = (x.to(gpu) for x in (qc, kc, vc))
    split = SplitPlan(wl.pieces, wl.L, gpu).forward(q, k, v).cpu()
    single = SplitPlan(wl.variants["single-rp16"], wl.L, gpu).forward(q, k, v).cpu()
    rows = _sample_rows(wl.L)
    heads = list(range(wl.H))
    want, _ = _oracle_rows(name, qc, kc, vc, heads, rows)
    e_split = np.abs(as64(split[heads][:, rows]) - want)
    e_single = np.abs(as64(single[heads][:, rows]) - want)
    _log(dict(workload=name, what="split vs single pass", split_max=float(e_split.max()),
              split_mean=float(e_split.mean()), single_max=float(e_single.max()),
              single_mean=float(e_single.mean())))
    print(f"split max {e_split.max():.2e} mean {e_split.mean():.2e}; "
          f"single pass max {e_single.max():.2e} mean {e_single.mean():.2e}")
    assert e_split.max() <= 2e-2 and e_split.mean() <= 2e-3
    # one extra bf16 rounding of a partial adds at most 2^-9 of it per element
    assert e_split.mean() <= 1.5 * e_single.mean() + 2e-4
    assert e_split.max() <= e_single.max() + 2 ** -9 * float(np.abs(want).max()) + 4e-3


def test_dilated8_permuted_equals_identity_basis(gpu):
    wl = workloads.make("dilated8-L8k")
    q, k, v = (x.to(gpu) for x in wl.inputs(0, "cpu"))
    a = SplitPlan(wl.pieces, wl.L, gpu).forward(q, k, v)
    b = SplitPlan(wl.variants["identity"], wl.L, gpu).forward(q, k, v)
    d = (a.float() - b.float()).abs()
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3


def test_bandlat_split_equals_single_pass(gpu):
    wl = workloads.make("bandlat-L16k")
    q, k, v = (x.to(gpu) for x in wl.inputs(0, "cpu"))
    a = SplitPlan(wl.pieces, wl.L, gpu).forward(q, k, v)
    b = SplitPlan(wl.variants["single-rp16"], wl.L, gpu).forward(q, k, v)
    d = (a.float() - b.float()).abs()
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3


def test_bandlat32_companion_runs_both_passes_and_equals_single_pass(gpu):
    """The companion at the prefix-LM workload's shape (H=8, L=65536): both sub-masks are
    non-empty, so the second pass merges into the first by log-sum-exp at L = 65536.
    Its output equals one pass over the union in the rp32 basis."""
    wl = workloads.make("bandlat32-L64k")
    q, k, v = (x.to(gpu) for x in wl.inputs(0, "cpu"))
    plan = SplitPlan(wl.pieces, wl.L, gpu)
    assert [b["live"] > 0 for b in plan.built] == [True, True]
    launches, o, lse = plan.prepare(q, k, v)
    assert len(launches) == 2 and plan.launched == [(0,), (1,)]
    for launch in launches:
        launch()
    from polyhedral_amd.split import Piece
    single = SplitPlan([Piece(wl.union, 128, 32, residue=32)], wl.L, gpu).forward(q, k, v)
    torch.cuda.synchronize()
    d = (o.float() - single.float()).abs()
    _log(dict(workload=wl.name, what="split vs single rp32 pass", max_abs=d.max().item(), mean_abs=d.mean().item()))
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3


def test_bandlat_16x16_floor_sampled_rows(gpu):
    """The headline's two pieces on their 16x16-floor block indices (the general kernel,
    one 16-row wave per query block) at full size: sampled rows of every head against the
    float64 oracle, and the same output as the 128x32 split within tolerance."""
    name = "bandlat-L16k"
    wl = workloads.make(name)
    qc, kc, vc = wl.inputs(0, "cpu")
    q, k, v = (x.to(gpu) for x in (qc, kc, vc))
    plan = SplitPlan(wl.variants["16x16"], wl.L, gpu)
    assert [b["tiles"] for b in plan.built] == [17272, 32256]
    lse = torch.empty(wl.H, wl.L, device=gpu)
    o = plan.forward(q, k, v, lse=lse)
    ref = SplitPlan(wl.pieces, wl.L, gpu).forward(q, k, v)
    torch.cuda.synchronize()
    rows = _sample_rows(wl.L)
    heads = list(range(wl.H))
    mx, mean = _check_rows(name, o.cpu(), lse.cpu(), qc, kc, vc, heads, rows)
    d = (o.float() - ref.float()).abs()
    _log(dict(workload=name + "[16x16]", rows=len(rows), heads=len(heads), max_abs=mx, mean_abs=mean,
              vs_128x32_max=d.max().item()))
    print(f"{name} 16x16 floor: max abs {mx:.2e} mean abs {mean:.2e}; vs 128x32 split max {d.max().item():.2e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3
