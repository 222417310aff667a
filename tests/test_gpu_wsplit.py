"""The wave-split kernel (pa_attn_args.wave_split): float32 grids too small to fill the
chip, the waves of a work-group splitting one 32-row group's live sub-tiles and merging
their softmax states in LDS.  Pinned by the float64 oracle (gpu/reference.py:5-13
semantics: output and natural-log LSE, dead rows 0 and -inf) at the float32 tolerance,
and against the general kernel on the same calls."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from polyhedral_amd import attention as pattn
from polyhedral_amd import index as pindex
from polyhedral_amd import workloads
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask, triton_params
from polyhedral_amd.spec import device_mask
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu

TILES = [(32, 32), (64, 64), (128, 128), (128, 32), (32, 128), (64, 128)]


def _launch(qd, kd, vd, m, kind, N, BQ, A, kernel, lse):
    bi = pindex.build(m, N, BQ, A)
    return pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi), *kind, BQ, A, kernel=kernel, lse=lse)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("name", ["window-128", "causal", "dilated-8", "local256+str8", "twoband-1000",
                                  "sinks4+win256", "prefixlm-2048", "lat16-band256"])
def test_wsplit_equals_oracle_and_general_kernel(gpu, name, D):
    N, BH = 1024, 2
    q, k, v = make_qkv(BH, N, D, torch.float32, seed=D)
    want, want_lse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    kind = triton_params(name)
    fin = np.isfinite(want_lse)
    for BQ, A in TILES:
        outs = {}
        for kernel in ("wsplit", "general"):
            lse = torch.empty(BH, N, device=gpu)
            launch = _launch(qd, kd, vd, numpy_mask(name), kind, N, BQ, A, kernel, lse)
            assert launch.kernel == kernel
            o = launch().clone()
            torch.cuda.synchronize()
            outs[kernel] = (o, lse)
        o, lse = outs["wsplit"]
        what = f"{name} D={D} {BQ}x{A} wsplit"
        check_close(o, want, torch.float32, what)
        got_lse = lse.cpu().numpy()
        assert np.array_equal(np.isfinite(got_lse), fin), what
        assert np.abs(got_lse[fin] - want_lse[fin]).max() < 1e-5, what
        diff = (o - outs["general"][0]).abs().max().item()
        assert diff < 2e-6, f"{what}: {diff:.3e} from the general kernel"


def test_wsplit_dead_rows_and_empty_lists(gpu):
    """A row with no live key gives 0 and -inf; an all-empty index writes zeros."""
    N, D, BH = 512, 64, 2
    q, k, v = make_qkv(BH, N, D, torch.float32, seed=3)
    M = om.dense(om.NAMED["causal"], N)
    M[100] = False
    M[200:232] = False                         # a whole 32-row group dead
    want, want_lse = oatt.dense_attention(as64(q), as64(k), as64(v), lambda r0, r1: M[r0:r1])
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    lse = torch.empty(BH, N, device=gpu)
    dm = pm.DenseMask(M)
    bi = pindex.build(dm, N, 64, 64)
    launch = pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi), device_mask(dm, N, gpu), 0, 0, 0, 64, 64,
                           kernel="wsplit", lse=lse)
    o = launch()
    torch.cuda.synchronize()
    check_close(o, want, torch.float32, "dense mask with dead rows")
    assert torch.count_nonzero(o[:, 100]) == 0 and torch.count_nonzero(o[:, 200:232]) == 0
    got = lse.cpu().numpy()
    assert np.isneginf(got[:, 100]).all() and np.isneginf(got[:, 200:232]).all()
    fin = np.isfinite(want_lse)
    assert np.abs(got[fin] - want_lse[fin]).max() < 1e-5
    # an index with every list empty
    bi = pindex.build(numpy_mask("lat32-prefixlm2048"), N, 64, 32)
    launch = pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi), *triton_params("lat32-prefixlm2048"), 64, 32,
                           kernel="wsplit")
    assert torch.count_nonzero(launch()) == 0


def test_auto_picks_wsplit_only_for_small_float32_grids(gpu):
    N, D = 1024, 64
    q, k, v = make_qkv(4, N, D, torch.float32, seed=1)
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    kind = triton_params("window-128")
    bi = pindex.build(numpy_mask("window-128"), N, 128, 128)
    assert pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi), *kind, 128, 128).kernel == "wsplit"
    bi16 = pindex.build(numpy_mask("window-128"), N, 16, 16)   # 16-row tiles: general kernel
    assert pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi16), *kind, 16, 16).kernel == "general"
    big = torch.zeros(64, 4096, D, device=gpu)                 # 64 heads x 32 blocks: general
    bib = pindex.build(numpy_mask("window-128"), 4096, 128, 128)
    assert pattn.prepare(big, big, big, *pindex.to_cuda(bib), *kind, 128, 128).kernel == "general"
    with pytest.raises(ValueError, match="wave-split"):
        pattn.prepare(qd.half(), kd.half(), vd.half(), *pindex.to_cuda(bi), *kind, 128, 128, kernel="wsplit")


def test_window128_workload_in_full(gpu):
    """The fp32 window-128 workload (H=4, L=1024, D=64, 128x128 index) through the plan, as
    the benchmark runs it, on the wave-split kernel, every row of every head at 1e-5."""
    from polyhedral_amd.split import SplitPlan
    wl = workloads.make("window128-L1k")
    q, k, v = wl.inputs(0, gpu)
    plan = SplitPlan(wl.pieces, wl.L, gpu)
    lse = torch.empty(wl.H, wl.L, device=gpu)
    launches, o, _ = plan.prepare(q, k, v, lse=lse)
    assert [x.kernel for x in launches] == ["wsplit"]
    for x in launches:
        x()
    torch.cuda.synchronize()
    want, want_lse = oatt.dense_attention(as64(q.cpu()), as64(k.cpu()), as64(v.cpu()),
                                          oatt.spec_rows(om.NAMED["window-128"], wl.L))
    check_close(o, want, torch.float32, "window128-L1k wsplit")
    assert np.abs(lse.cpu().numpy() - want_lse).max() < 1e-5
