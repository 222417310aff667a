"""Once-per-forward relabelling (pa_permute_stack): a stack of tensors and their position
ids permuted in one launch, and the check of gpu/exp5_amortisation.py:76-108 that a
whole stack run in the permuted basis (with positions travelling with the tokens)
equals the plain stack, while regenerating the positions does not."""
import numpy as np
import pytest
import torch

from oracle import permute as op
from polyhedral_amd import attention as pattn
from polyhedral_amd import index as pindex
from polyhedral_amd import perm as pperm
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask, triton_params
from tests.util import make_qkv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,shape,dtype", [(3, (4, 2048, 128), torch.bfloat16), (1, (2, 1000, 64), torch.float16),
                                           (8, (1, 512, 8), torch.float32), (2, (3, 256, 5), torch.float16)])
def test_stack_equals_row_gather_and_moves_positions(gpu, n, shape, dtype):
    g = torch.Generator().manual_seed(n)
    xs = [torch.randn(*shape, generator=g).to(dtype).to(gpu) for _ in range(n)]
    N = shape[1]
    p = torch.from_numpy(np.random.default_rng(n).permutation(N).astype(np.int32)).to(gpu)
    outs, pos = pperm.permute_stack(xs, p)
    for x, o in zip(xs, outs):
        assert torch.equal(o, x[:, p.long()])
    assert torch.equal(pos, p.long())
    # explicit positions travel with the rows; the inverse brings rows and ids back
    ids = torch.arange(N, device=gpu, dtype=torch.int64) * 7 + 3
    outs, pos = pperm.permute_stack(xs, p, positions=ids)
    assert torch.equal(pos, ids[p.long()])
    back, pos_back = pperm.permute_stack(outs, p, positions=pos, inverse=True)
    for x, b in zip(xs, back):
        assert torch.equal(b, x)
    assert torch.equal(pos_back, ids)


def _rope(x, pos):
    """Rotary embedding with explicit positions (gpu/exp5_amortisation.py:44-57)."""
    d = x.shape[-1] // 2
    freq = torch.exp(-np.log(10000.0) * torch.arange(d, device=x.device) / d)
    ang = pos[:, None].float() * freq[None, :]
    c, s_ = torch.cos(ang).to(x.dtype), torch.sin(ang).to(x.dtype)
    a, b = x[..., :d], x[..., d:]
    return torch.cat([a * c - b * s_, a * s_ + b * c], dim=-1)


def _mlp_like(x):
    return torch.nn.functional.gelu(x) * 0.5 + x


def test_stack_in_the_permuted_basis_equals_the_plain_stack(gpu):
    name, s, N, D, BH = "dilated-8", 8, 2048, 64, 4
    q, k, v = (x.to(gpu) for x in make_qkv(BH, N, D, torch.float16, seed=0))
    kind, p0, p1, p2 = triton_params(name)
    p_np = op.residue_perm(N, s)
    pt = torch.from_numpy(p_np).to(gpu)
    idx_i = pindex.to_cuda(pindex.build(numpy_mask(name), N, 128, 128), gpu)
    idx_p = pindex.to_cuda(pindex.build(pm.Permuted(numpy_mask(name), p_np), N, 16, 16), gpu)

    def attn_plain(x):
        return pattn.block_sparse_attention(x, k, v, *idx_i, kind, p0, p1, p2, 128, 128)

    def attn_perm(x, kp, vp):
        return pattn.block_sparse_attention(x, kp, vp, *idx_p, kind, p0, p1, p2, 16, 16, perm_q=pt, perm_kv=pt)

    pos = torch.arange(N, device=gpu)
    x = q
    for _ in range(3):
        x = _mlp_like(_rope(attn_plain(x), pos))
    ref = x.float()

    # once per forward: Q, K, V and the position ids relabelled by one launch
    (xp, kp, vp), pos_p = pperm.permute_stack([q, k, v], pt, positions=pos)
    assert torch.equal(pos_p, pos[pt.long()])
    for _ in range(3):
        xp = _mlp_like(_rope(attn_perm(xp, kp, vp), pos_p))
    (got,), _ = pperm.permute_stack([xp], pt, inverse=True, with_positions=False)
    err = (got.float() - ref).abs().max().item()
    assert err < 2e-2, f"3-layer stack in the permuted basis: max abs err {err:.3e}"

    # negative control: positions regenerated instead of permuted must fail
    (xb, _, _), _ = pperm.permute_stack([q, k, v], pt, with_positions=False)
    for _ in range(3):
        xb = _mlp_like(_rope(attn_perm(xb, kp, vp), pos))
    (bad,), _ = pperm.permute_stack([xb], pt, inverse=True, with_positions=False)
    bad_err = (bad.float() - ref).abs().max().item()
    assert bad_err > 10 * max(err, 1e-6), f"negative control err {bad_err:.3e} vs {err:.3e}"
