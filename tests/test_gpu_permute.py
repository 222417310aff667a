"""GPU class-A permutation vs the oracle: bit-exact gathers, scatters, inverses."""
import numpy as np
import pytest
import torch

from oracle import permute as op
from polyhedral_amd import perm as pp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,s", [(1024, 4), (1000, 8), (4096, 16), (7, 3), (5, 8)])
def test_residue_perm_host_and_device(gpu, N, s):
    want = op.residue_perm(N, s)
    assert np.array_equal(pp.residue_perm(N, s), want)
    assert np.array_equal(pp.residue_perm_device(N, s, gpu).cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int8])
@pytest.mark.parametrize("D", [64, 128, 3])
def test_gather_scatter_exact(gpu, dtype, D):
    BH, N, s = 3, 1024, 8
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(BH, N, D, generator=g) * 50).to(dtype)
    perm = op.residue_perm(N, s)
    xd = x.to(gpu)
    pd = torch.from_numpy(perm).to(gpu)
    y = pp.apply_perm(xd, pd)
    assert torch.equal(y.cpu(), x[:, torch.from_numpy(perm).long()])
    back = pp.permute_rows(y, pd, inverse=True)
    assert torch.equal(back.cpu(), x)
    inv = pp.invert(pd)
    assert np.array_equal(inv.cpu().numpy(), op.invert(perm))
    assert torch.equal(pp.apply_perm(y, inv).cpu(), x)


def test_full_size_round_trip(gpu):
    """Llama-length shape B*H=32, L=16384, D=128, bf16: permute then un-permute is the identity."""
    BH, N, D = 32, 16384, 128
    x = torch.randn(BH, N, D, device=gpu).to(torch.bfloat16)
    p = pp.residue_perm_device(N, 16, gpu)
    y = pp.apply_perm(x, p)
    assert torch.equal(pp.permute_rows(y, p, inverse=True), x)
    # spot rows: y[:, j] == x[:, perm[j]]
    pc = p.cpu().numpy()
    for j in (0, 1, 1023, 1024, 8191, 16383):
        assert torch.equal(y[:, j], x[:, int(pc[j])])
