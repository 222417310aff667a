"""Class-B traffic emulation (gather_mult / gather_scatter, gpu/triton_attn.py:108-128).

With the reference's weights [1, 0, ...] the extra K rows are read and the output is
unchanged: equal, bit for bit, to gather_mult = 1.  With other weights every key becomes
sum_r w_r K[row_r], which pins which rows are read: row_0 is the tile's row, and the extra
rows are (row_0 + r A) mod N (contiguous) or perm_kv((column + r A) mod N) (scattered)."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import attention as pattn
from polyhedral_amd import index as pindex
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask, triton_params
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu

N, D, BH = 1024, 128, 2


def _run(q, k, v, name, BQ, A, perm=None, residue=0, **kw):
    kind, p0, p1, p2 = triton_params(name)
    mask = numpy_mask(name) if perm is None else pm.Permuted(numpy_mask(name), perm)
    bi = pindex.build(mask, N, BQ, A)
    ext = {}
    if perm is not None:
        pt = torch.from_numpy(perm).to(q.device)
        ext = dict(perm_q=pt, gather_kv=True, gather_q=True, scatter_o=True, residue=residue)
    launch = pattn.prepare(q, k, v, *pindex.to_cuda(bi, q.device), kind, p0, p1, p2, BQ, A, **ext, **kw)
    with torch.cuda.device(q.device):
        out = launch()
    return launch, out


def _effective_k(k64, A, mult, scatter, w, perm):
    """Original-coordinate keys the kernel sees: key at index-space column j (original
    position perm[j]) is sum_r w_r K[row_r(j)]."""
    Nn = k64.shape[1]
    j = np.arange(Nn)
    p = perm if perm is not None else j
    out = np.zeros_like(k64)
    acc = w[0] * k64[:, p[j]]
    for r in range(1, mult):
        rows = p[(j + r * A) % Nn] if scatter else (p[j] + r * A) % Nn
        acc = acc + w[r] * k64[:, rows]
    out[:, p[j]] = acc
    return out


@pytest.mark.parametrize("scatter", [False, True])
@pytest.mark.parametrize("mult", [2, 4])
@pytest.mark.parametrize("case", ["identity", "rp8"])
def test_reference_weights_leave_the_output_unchanged(gpu, case, mult, scatter):
    name, BQ, A = "dilated-8", 128, 32
    q, k, v = (x.to(gpu) for x in make_qkv(BH, N, D, torch.bfloat16, seed=mult))
    perm = op.residue_perm(N, 8) if case == "rp8" else None
    # (the same kernel: gather_mult runs on the general kernel)
    base_launch, base = _run(q, k, v, name, BQ, A, perm, residue=8, kernel="general")
    base = base.clone()
    launch, out = _run(q, k, v, name, BQ, A, perm, residue=8, gather_mult=mult, gather_scatter=scatter)
    assert launch.kernel == "general"
    assert torch.equal(out, base), f"{case} mult={mult} scatter={scatter}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("scatter", [False, True])
@pytest.mark.parametrize("case", ["identity", "rp8"])
def test_extra_rows_are_the_reference_rows(gpu, case, scatter, dtype):
    name, mult = "window-128", 3
    BQ, A = (128, 32) if dtype != torch.float32 else (64, 64)
    q, k, v = make_qkv(BH, N, D if dtype != torch.float32 else 64, dtype, seed=9)
    perm = op.residue_perm(N, 8) if case == "rp8" else None
    w = [1.0, 0.5, 0.25]
    wsel = torch.tensor([w] * BH)
    keff = _effective_k(as64(k), A, mult, scatter, w, perm)
    want, _ = oatt.dense_attention(as64(q), keff, as64(v), oatt.spec_rows(om.NAMED[name], N))
    launch, out = _run(q.to(gpu), k.to(gpu), v.to(gpu), name, BQ, A, perm, residue=8, gather_mult=mult,
                       gather_scatter=scatter, wsel=wsel)
    assert launch.kernel == "general"
    # K is combined in fp32 and rounded once to the input dtype before QK^T
    check_close(out, want, dtype, f"{case} scatter={scatter} {dtype}")


def test_gather_mult_rejects_the_streaming_kernel(gpu):
    q, k, v = (x.to(gpu) for x in make_qkv(1, N, D, torch.bfloat16))
    with pytest.raises(ValueError, match="streaming kernel"):
        _run(q, k, v, "window-128", 128, 32, gather_mult=2, kernel="stream")
    with pytest.raises(ValueError, match="gather_mult"):
        _run(q, k, v, "window-128", 128, 32, gather_mult=0)
