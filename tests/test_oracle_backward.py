"""The oracle's attention gradient (oracle.attention.dense_attention_bwd) against
torch.autograd through the dense masked softmax attention of gpu/reference.py:5-13, in
float64 on the host: any dropped term (the rowsum correction, the scale on dQ / dK, a
transposed operand) moves the result far outside the tolerance.  Rows with no live key
have no gradient."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om


def _autograd(q, k, v, do, M, scale):
    q, k, v = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    s = (q @ k.transpose(-1, -2)) * scale
    s = s.masked_fill(~torch.from_numpy(M)[None], float("-inf"))
    alive = torch.from_numpy(M.any(axis=1))[None, :, None]
    p = torch.where(alive, torch.softmax(torch.where(alive, s, torch.zeros_like(s)), dim=-1), torch.zeros_like(s))
    o = p @ v
    (o * torch.tensor(do)).sum().backward()
    return q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("name", ["causal", "window-128", "dilated-8", "band256+lat16", "sinks4+win8"])
def test_gradient_equals_autograd(name):
    rng = np.random.default_rng(0)
    BH, N, D = 2, 256, 16
    q, k, v, do = (rng.standard_normal((BH, N, D)) for _ in range(4))
    M = om.dense(om.NAMED[name], N)
    scale = D ** -0.5
    got = oatt.dense_attention_bwd(q, k, v, do, lambda a, b: M[a:b], scale, row_chunk=96)
    want = _autograd(q, k, v, do, M, scale)
    for g, w_, nm in zip(got, want, ("dq", "dk", "dv")):
        assert np.abs(g - w_).max() < 1e-10, f"{name} {nm}"


def test_dead_rows_get_no_gradient():
    rng = np.random.default_rng(1)
    BH, N, D = 1, 64, 8
    q, k, v, do = (rng.standard_normal((BH, N, D)) for _ in range(4))
    M = om.dense(om.NAMED["causal"], N)
    M[10] = False
    dq, dk, dv = oatt.dense_attention_bwd(q, k, v, do, lambda a, b: M[a:b])
    assert np.all(dq[:, 10] == 0)
    want = _autograd(q, k, v, do, M, D ** -0.5)
    for g, w_ in zip((dq, dk, dv), want):
        assert np.abs(g - w_).max() < 1e-10
