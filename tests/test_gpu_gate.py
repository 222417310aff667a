"""gpu/test_correctness.py restated through the drop-in modules imported by bare name, as
the reference's drivers import them (gpu/test_correctness.py:14-18): mask agreement, index
elements == cost model, kernel vs dense reference at 7 tile shapes x 5 masks (fp16,
TOL 3e-3), and the class-A permuted path."""
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = pytest.mark.gpu

N, D, BH = 1024, 64, 2
TILES = [(128, 128), (128, 32), (64, 64), (32, 32), (16, 16), (128, 16), (16, 128)]
NAMES = ["causal", "window-128", "dilated-8", "local256+str8", "twoband-1000"]
TOL = 3e-3


@pytest.fixture(scope="module")
def mods():
    sys.path.insert(0, os.path.join(ROOT, "polyhedral_amd", "gpu"))
    sys.path.insert(1, os.path.join(ROOT, "polyhedral_amd"))
    import blockindex
    import masks_gpu
    import permute
    import reference
    from polyattn import cost as pcost
    from triton_attn import block_sparse_attention
    return blockindex, masks_gpu, permute, reference, pcost, block_sparse_attention


def test_gate(gpu, mods):
    blockindex, masks_gpu, permute, reference, pcost, block_sparse_attention = mods
    torch.manual_seed(0)
    for n in masks_gpu.SPECS:                                             # step 1
        assert masks_gpu.check_agreement(n, N=512), n
    for n in NAMES:                                                       # step 2
        m = masks_gpu.numpy_mask(n)
        for BQ, A in TILES:
            assert blockindex.build(m, N, BQ, A).elements == pcost.cost(m, N, BQ, A, exact_only=True)[0]
    q, k, v = (torch.randn(BH, N, D, device="cuda", dtype=torch.float16) for _ in range(3))
    for n in NAMES:                                                       # step 3
        m = masks_gpu.numpy_mask(n)
        ref = reference.attention_reference(q, k, v, masks_gpu.dense_bool(n, N))
        worst = 0.0
        for BQ, A in TILES:
            bi = blockindex.build(m, N, BQ, A)
            kvi, kvn, kvp = blockindex.to_cuda(bi)
            kind, p0, p1, p2 = masks_gpu.triton_params(n)
            out = block_sparse_attention(q, k, v, kvi, kvn, kvp, kind, p0, p1, p2, BQ, A)
            worst = max(worst, reference.max_abs_err(out, ref))
        print(f"  {n:<16} max abs err {worst:.2e}")
        assert worst < TOL, n
    for n, s in (("dilated-4", 4), ("dilated-8", 8)):                     # step 4
        m = masks_gpu.numpy_mask(n)
        ref = reference.attention_reference(q, k, v, masks_gpu.dense_bool(n, N))
        p_np = permute.residue_perm(N, s)
        perm = torch.from_numpy(p_np).cuda()
        qp, kp, vp = (permute.apply_perm(x, perm) for x in (q, k, v))

        class _Dense:
            def __init__(self, M):
                self.M, self.name = M, "permuted"

            def row_cols(self, i, N):
                return self.M[i]
        M = np.stack([m.row_cols(i, N) for i in range(N)])[p_np][:, p_np]
        bi = blockindex.build(_Dense(M), N, 16, 16)
        kvi, kvn, kvp = blockindex.to_cuda(bi)
        kind, p0, p1, p2 = masks_gpu.triton_params(n)
        outp = block_sparse_attention(qp, kp, vp, kvi, kvn, kvp, kind, p0, p1, p2, 16, 16,
                                      perm_q=perm.int(), perm_kv=perm.int())
        out = outp.index_select(1, permute.invert(perm).long())
        err = reference.max_abs_err(out, ref)
        print(f"  {n:<16} waste {bi.waste:.3f}  max abs err {err:.2e}")
        assert err < TOL and round(bi.waste, 3) == {4: 1.058, 8: 1.116}[s]
