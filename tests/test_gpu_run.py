"""The persistent streaming kernel (pa_attn_fwd with run_groups): its run rows against the
step descriptors they come from, its outputs against the float64 oracle and, bit for
bit, against the per-block streaming kernel over the same index."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from polyhedral_amd import index as pindex
from polyhedral_amd import workloads
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask
from polyhedral_amd.schedule import RunSchedule
from polyhedral_amd.split import Piece, SplitPlan
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("residue", [0, 16])
@pytest.mark.parametrize("keep_empty", [True, False])
def test_run_rows_follow_the_descriptors(gpu, residue, keep_empty):
    N, BQ, A, BH = 2048, 128, 32, 5
    name = "lat16-band256"       # empty lists for the first query blocks in the identity basis
    kv_idx, kv_num, kv_partial, wave, tiles, live, bits, steps = pindex.build_device(
        numpy_mask(name), N, BQ, A, device=gpu, bits=True, steps=True, residue=residue)
    run = RunSchedule(steps, N, BH, groups=24, keep_empty=keep_empty)
    st = steps.cpu().numpy()
    rows = run.run.cpu().numpy()
    start = run.start.cpu().numpy()
    nsteps = st[:, 0, 14]
    assert start[0] == 0 and start[-1] == run.rows and np.all(np.diff(start) >= 0)
    seen = set()
    r = 0
    while r < run.rows:
        fl, bh = rows[r, 9], rows[r, 10]
        qb = fl >> 3
        assert not fl & 4 and rows[r, 11] == -1       # piece 0, no sync group
        assert fl & 1, f"row {r} does not start an item"
        n = max(1, int(nsteps[qb]))
        assert (bh, qb) not in seen
        seen.add((bh, qb))
        for j in range(n):
            row = rows[r + j]
            assert row[10] == bh and (row[9] >> 3) == qb
            assert (row[9] & 1) == (j == 0) and ((row[9] >> 1) & 1) == (j == n - 1)
            if nsteps[qb] == 0:
                assert not row[4] and np.all(row[0:4] == bh * N) and np.all(row[5:9] == -1)
            else:
                assert np.array_equal(row[0:4], st[qb, j, 0:4] + bh * N)
                assert np.array_equal(row[4:9], st[qb, j, 4:9])
        r += n
    want = {(h, q) for h in range(BH) for q in range(N // BQ) if keep_empty or nsteps[q] > 0}
    assert seen == want


def _plans(pieces, N, dev):
    return SplitPlan(pieces, N, dev, persistent=True, fuse=False), SplitPlan(pieces, N, dev, persistent=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name,residue", [("window-128", 0), ("dilated-8", 8), ("local256+str8", 0),
                                          ("sinks4+win256", 0), ("prefixlm-2048", 0), ("lat16-band256", 0),
                                          ("lat16-band256", 16), ("twoband-1000", 0)])
@pytest.mark.parametrize("BH", [3, 8])
def test_persistent_equals_oracle_and_per_block_kernel(gpu, name, residue, dtype, BH):
    N, D = 2048, 128
    q, k, v = make_qkv(BH, N, D, dtype, seed=BH)
    piece = Piece(numpy_mask(name), 128, 32, residue=residue)
    run_plan, blk_plan = _plans([piece], N, gpu)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    lse_r = torch.empty(BH, N, device=gpu)
    lse_b = torch.empty(BH, N, device=gpu)
    launches, _, _ = run_plan.prepare(qd, kd, vd, lse=lse_r)
    assert [x.kernel for x in launches] == ["run"]
    o_r = run_plan.forward(qd, kd, vd, lse=lse_r)
    o_b = blk_plan.forward(qd, kd, vd, lse=lse_b)
    torch.cuda.synchronize()
    want, wlse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    check_close(o_r, want, dtype, f"{name} rp{residue} persistent")
    assert torch.equal(o_r, o_b), f"{name}: persistent and per-block outputs differ"
    assert torch.equal(lse_r, lse_b)
    fin = np.isfinite(wlse)
    gl = lse_r.cpu().numpy().astype(np.float64)
    assert np.array_equal(np.isfinite(gl), fin)
    assert np.abs(gl[fin] - wlse[fin]).max() < 2e-2


def test_persistent_split_with_empty_lists_and_merge(gpu):
    """A split whose first piece has empty lists (rows with no live key get zeros and
    -inf, then the second piece merges into them), both pieces persistent."""
    N, D, BH = 4096, 128, 8
    band = pm.SlidingWindow(256)
    lat = pm.Difference(pm.Dilated(16), band)
    pieces = [Piece(lat, 128, 32, residue=0), Piece(band, 128, 32)]
    q, k, v = make_qkv(BH, N, D, torch.bfloat16, seed=3)
    blk_plan = SplitPlan(pieces, N, gpu, persistent=False)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    o_b = blk_plan.forward(qd, kd, vd)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED["band256+lat16"], N))
    # two persistent launches, and one split launch (both pieces in the identity basis:
    # every sync group is one query block of each piece)
    for plan, kinds in ((SplitPlan(pieces, N, gpu, persistent=True, fuse=False), ["run", "run"]),
                        (SplitPlan(pieces, N, gpu, persistent=True, fuse=True), ["split"]),
                        (SplitPlan(pieces, N, gpu, fuse=True), ["split-grid"])):
        launches, _, _ = plan.prepare(qd, kd, vd)
        assert [x.kernel for x in launches] == kinds
        o_r = plan.forward(qd, kd, vd)
        torch.cuda.synchronize()
        plan.check()
        check_close(o_r, want, torch.bfloat16, f"empty lists + merge ({kinds})")
        assert torch.equal(o_r, o_b)


@pytest.mark.parametrize("name", ["dilated8-L8k", "bandlat-L16k", "sinkwin-L32k", "prefixlat-L64k"])
def test_workloads_persistent_equal_per_block(gpu, name):
    """At full size the persistent kernel reproduces the per-block kernel bit for bit."""
    wl = workloads.make(name)
    q, k, v = wl.inputs(0, gpu)
    run_plan, blk_plan = _plans(wl.pieces, wl.L, gpu)
    lse_r = torch.empty(wl.H, wl.L, device=gpu)
    lse_b = torch.empty(wl.H, wl.L, device=gpu)
    launches, _, _ = run_plan.prepare(q, k, v, lse=lse_r)
    assert all(x.kernel == "run" for x in launches)
    o_r = run_plan.forward(q, k, v, lse=lse_r)
    o_b = blk_plan.forward(q, k, v, lse=lse_b)
    torch.cuda.synchronize()
    assert torch.equal(o_r, o_b), f"{name}: max diff {(o_r.float() - o_b.float()).abs().max().item():.3e}"
    assert torch.equal(lse_r, lse_b)


def _split_plans(pieces, N, dev, **kw):
    fused = SplitPlan(pieces, N, dev, persistent=True, fuse=True, **kw)
    two = SplitPlan(pieces, N, dev, persistent=True, fuse=False)
    return fused, two


@pytest.mark.parametrize("N,BH,xcds", [(4096, 8, None), (4096, 8, 1), (8192, 3, None), (16384, 16, 1)])
def test_split_launch_equals_two_launches(gpu, N, BH, xcds):
    """Both pieces of the band + lattice split in one launch (the lattice merging into the
    band's rows as they are published) give the two-launch result bit for bit, with the
    heads spread over the XCDs or not (xcds=1: waits cross XCDs); the counters are left
    zero and no wait gave up."""
    band = pm.SlidingWindow(256)
    lat = pm.Difference(pm.Dilated(16), band)
    pieces = [Piece(band, 128, 32), Piece(lat, 128, 32, residue=16)]
    q, k, v = make_qkv(BH, N, 128, torch.bfloat16, seed=N + BH)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    fused, two = _split_plans(pieces, N, gpu, split_xcds=xcds)
    launches, _, _ = fused.prepare(qd, kd, vd)
    assert [x.kernel for x in launches] == ["split"]
    lse_f = torch.empty(BH, N, device=gpu)
    lse_t = torch.empty(BH, N, device=gpu)
    for _ in range(3):                       # repeated launches reuse the counters
        o_f = fused.forward(qd, kd, vd, lse=lse_f)
    o_t = two.forward(qd, kd, vd, lse=lse_t)
    torch.cuda.synchronize()
    fused.check()
    sched = fused._runs[("split", BH)][0]
    assert int(sched.sync.abs().sum()) == 0 and int(sched.status.item()) == 0
    assert torch.equal(o_f, o_t), f"max diff {(o_f.float() - o_t.float()).abs().max().item():.3e}"
    assert torch.equal(lse_f, lse_t)
    if N <= 8192:
        want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED["band256+lat16"], N))
        check_close(o_f, want, torch.bfloat16, "split launch")


def test_split_launch_headline_equals_per_block(gpu):
    """At the headline size the one-launch split reproduces the per-block kernels bit for bit."""
    wl = workloads.make("bandlat-L16k")
    q, k, v = wl.inputs(0, gpu)
    fused = SplitPlan(wl.pieces, wl.L, gpu, persistent=True, fuse=True)
    blk = SplitPlan(wl.pieces, wl.L, gpu, persistent=False)
    launches, _, _ = fused.prepare(q, k, v)
    assert [x.kernel for x in launches] == ["split"]
    lse_f = torch.empty(wl.H, wl.L, device=gpu)
    lse_b = torch.empty(wl.H, wl.L, device=gpu)
    o_f = fused.forward(q, k, v, lse=lse_f)
    o_b = blk.forward(q, k, v, lse=lse_b)
    torch.cuda.synchronize()
    fused.check()
    assert torch.equal(o_f, o_b) and torch.equal(lse_f, lse_b)


@pytest.mark.parametrize("N,BH,lag", [(4096, 8, 1), (8192, 3, 0), (4096, 16, 2)])
def test_split_grid_equals_two_launches(gpu, N, BH, lag):
    """Both pieces of the band + lattice split as one work-group per item (the lattice
    merges waiting for the band items of their group) give the per-block two-launch result
    bit for bit, over repeated launches; the counters are left zero and no wait gave up."""
    band = pm.SlidingWindow(256)
    lat = pm.Difference(pm.Dilated(16), band)
    pieces = [Piece(band, 128, 32), Piece(lat, 128, 32, residue=16)]
    q, k, v = make_qkv(BH, N, 128, torch.bfloat16, seed=N + BH + lag)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    grid = SplitPlan(pieces, N, gpu, fuse=True, split_lag=lag)
    blk = SplitPlan(pieces, N, gpu)
    launches, _, _ = grid.prepare(qd, kd, vd)
    assert [x.kernel for x in launches] == ["split-grid"]
    lse_g = torch.empty(BH, N, device=gpu)
    lse_b = torch.empty(BH, N, device=gpu)
    for _ in range(3):
        o_g = grid.forward(qd, kd, vd, lse=lse_g)
    o_b = blk.forward(qd, kd, vd, lse=lse_b)
    torch.cuda.synchronize()
    grid.check()
    sg = grid._runs[("grid", BH)]
    assert int(sg.sync.abs().sum()) == 0 and int(sg.status.item()) == 0
    assert torch.equal(o_g, o_b), f"max diff {(o_g.float() - o_b.float()).abs().max().item():.3e}"
    assert torch.equal(lse_g, lse_b)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED["band256+lat16"], N))
    check_close(o_g, want, torch.bfloat16, "split grid")


def test_split_grid_headline_equals_per_block(gpu):
    """At the headline size the split grid reproduces the per-block kernels bit for bit."""
    wl = workloads.make("bandlat-L16k")
    q, k, v = wl.inputs(0, gpu)
    grid = SplitPlan(wl.pieces, wl.L, gpu, fuse=True)
    blk = SplitPlan(wl.pieces, wl.L, gpu)
    launches, _, _ = grid.prepare(q, k, v)
    assert [x.kernel for x in launches] == ["split-grid"]
    lse_g = torch.empty(wl.H, wl.L, device=gpu)
    lse_b = torch.empty(wl.H, wl.L, device=gpu)
    o_g = grid.forward(q, k, v, lse=lse_g)
    o_b = blk.forward(q, k, v, lse=lse_b)
    torch.cuda.synchronize()
    grid.check()
    assert torch.equal(o_g, o_b) and torch.equal(lse_g, lse_b)


def test_split_grid_give_up_is_reported_and_cleared(gpu):
    """A merge that never sees its rows published (the launch's sync target raised above
    the count its group can reach, so every merge exits through its own bounded wait)
    marks the status: check() raises and clears the status and the counters, and the next
    launch, with the real target, gives the two-launch result bit for bit (a stale status
    no longer shortens its waits)."""
    N, BH = 4096, 2
    band = pm.SlidingWindow(256)
    lat = pm.Difference(pm.Dilated(16), band)
    pieces = [Piece(band, 128, 32), Piece(lat, 128, 32, residue=16)]
    q, k, v = make_qkv(BH, N, 128, torch.bfloat16, seed=77)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    grid = SplitPlan(pieces, N, gpu, fuse=True)
    blk = SplitPlan(pieces, N, gpu)
    launches, o_g, lse_g = grid.prepare(qd, kd, vd)
    (launch,) = launches
    real = launch.args.sync_signal
    launch.args.sync_signal = real + 1000      # no group ever reaches it
    launch()
    torch.cuda.synchronize()
    sg = grid._runs[("grid", BH)]
    assert int(sg.status.item()) == 1
    with pytest.raises(RuntimeError, match="gave up"):
        launch.check()
    assert int(sg.status.item()) == 0 and int(sg.sync.abs().sum()) == 0
    launch.args.sync_signal = real
    launch()
    lse_b = torch.empty(BH, N, device=gpu)
    o_b = blk.forward(qd, kd, vd, lse=lse_b)
    torch.cuda.synchronize()
    launch.check()
    assert torch.equal(o_g, o_b) and torch.equal(lse_g, lse_b)
