"""Disjoint split + LSE merge on the GPU: fused epilogue merge and the standalone merge
kernel against the oracle; empty pieces."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.split import Piece, SplitPlan, lse_merge
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_band_lattice_split_small(gpu, dtype):
    N, H, D = 2048, 2, 128
    band = pm.SlidingWindow(256)
    lat = pm.Difference(pm.Dilated(16), band)
    plan = SplitPlan([Piece(band, 128, 32), Piece(lat, 128, 32, residue=16)], N, gpu)
    q, k, v = make_qkv(H, N, D, dtype, seed=11)
    lse = torch.empty(H, N, device=gpu)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu), lse=lse)
    want, wlse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED["band256+lat16"], N))
    check_close(o, want, dtype, "split band+lattice")
    fin = np.isfinite(wlse)
    assert np.abs(lse.cpu().numpy()[fin] - wlse[fin]).max() < (1e-5 if dtype == torch.float32 else 2e-2)


def test_three_pieces_with_an_empty_one(gpu):
    N, H, D = 4096, 2, 64
    p = pm.PrefixLM(2048)
    sub2 = pm.Difference(pm.Dilated(32), p)                     # empty
    band = pm.Difference(pm.SlidingWindow(64), pm.Causal())     # empty too
    plan = SplitPlan([Piece(p, 128, 32), Piece(sub2, 128, 32, residue=32), Piece(band, 64, 64)], N, gpu)
    assert plan.live == om.dense(om.NAMED["prefixlm-2048"], N).sum()
    q, k, v = make_qkv(H, N, D, torch.float32, seed=5)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu))
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED["prefixlm-2048"], N))
    check_close(o, want, torch.float32, "prefix + empty pieces")


def test_all_empty_plan_gives_zeros(gpu):
    N = 1024
    sub2 = pm.Difference(pm.Dilated(32), pm.PrefixLM(2048))
    plan = SplitPlan([Piece(sub2, 128, 32)], N, gpu)
    q, k, v = make_qkv(1, N, 64, torch.bfloat16)
    lse = torch.empty(1, N, device=gpu)
    o = plan.forward(q.to(gpu), k.to(gpu), v.to(gpu), lse=lse)
    assert torch.count_nonzero(o) == 0 and torch.isneginf(lse).all()


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_standalone_merge_kernel(gpu, out_dtype):
    rng = np.random.default_rng(0)
    BH, N, D, K = 2, 300, 64, 3
    os_ = [rng.standard_normal((BH, N, D)) for _ in range(K)]
    ls = [rng.standard_normal((BH, N)) * 3 for _ in range(K)]
    ls[1][:, :50] = -np.inf
    for i in range(K):
        ls[i][:, 7] = -np.inf                                   # a fully dead row
    want, wl = oatt.lse_merge(os_, ls)
    lse_out = torch.empty(BH, N, device=gpu)
    got = lse_merge([torch.tensor(x, dtype=torch.float32, device=gpu) for x in os_],
                    [torch.tensor(x, dtype=torch.float32, device=gpu) for x in ls], out_dtype, lse_out)
    tol = 1e-5 if out_dtype == torch.float32 else 2e-2
    assert np.abs(as64(got) - want).max() < tol
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(lse_out.cpu().numpy()), fin)
    assert np.abs(lse_out.cpu().numpy()[fin] - wl[fin]).max() < 1e-5
