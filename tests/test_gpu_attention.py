"""GPU attention forward vs the float64 oracle (dense masked attention, gpu/reference.py
semantics) on seeded inputs: every gate tile shape, dtypes, D, masks, permuted paths."""
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
from tests.util import TILES_GATE, as64, check_close, make_qkv

pytestmark = pytest.mark.gpu


def _run(name, N, D, BH, dtype, tiles, gpu, seed=0):
    q, k, v = make_qkv(BH, N, D, dtype, seed)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    kind, p0, p1, p2 = triton_params(name)
    m = numpy_mask(name)
    for BQ, A in tiles:
        bi = pindex.build(m, N, BQ, A)
        out = pattn.block_sparse_attention(qd, kd, vd, *pindex.to_cuda(bi), kind, p0, p1, p2, BQ, A)
        check_close(out, want, dtype, f"{name} {dtype} D={D} {BQ}x{A}")


@pytest.mark.parametrize("name", ["window-128", "causal", "dilated-8", "local256+str8", "twoband-1000"])
def test_fp32_gate_masks_all_tiles(gpu, name):
    _run(name, 512, 64, 2, torch.float32, TILES_GATE, gpu)


@pytest.mark.parametrize("name", ["window-128", "causal", "dilated-8", "local256+str8", "twoband-1000",
                                  "sinks4+win256", "sinks4+win8", "prefixlm-2048"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_gate_masks_all_tiles(gpu, name, dtype):
    _run(name, 1024, 64, 2, dtype, TILES_GATE, gpu)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_d128(gpu, dtype):
    _run("local256+str8", 1024, 128, 2, dtype, [(128, 32), (64, 64), (16, 16), (128, 128)], gpu)


def test_sinks_partial_tile_uses_the_sink_term(gpu):
    """sinks4+win256 at 128x128: columns 0..127 form a PARTIAL tile beyond the window,
    where the reference's _live drops the sink term (gpu/triton_attn.py:56-59)."""
    _run("sinks4+win256", 1024, 64, 2, torch.float32, [(128, 128)], gpu)


def test_composite_difference_and_empty(gpu):
    _run("lat16-band256", 2048, 64, 2, torch.float32, [(128, 32), (16, 16)], gpu)
    # empty sub-mask: every row dead -> exact zeros
    N, D = 4096, 64
    q, k, v = make_qkv(2, N, D, torch.float32)
    bi = pindex.build(numpy_mask("lat32-prefixlm2048"), N, 128, 32)
    kind = triton_params("lat32-prefixlm2048")
    lse = torch.empty(2, N, device=gpu)
    out = pattn.block_sparse_attention(q.to(gpu), k.to(gpu), v.to(gpu), *pindex.to_cuda(bi), *kind, 128, 32,
                                       lse=lse)
    assert torch.count_nonzero(out) == 0
    assert torch.isneginf(lse).all()


def test_dead_row_is_zero_and_finite(gpu):
    """A row with no live key anywhere returns exact zeros (tests/test_kernel_math.py:83-90)."""
    from polyhedral_amd.spec import device_mask
    N, D = 256, 64
    M = om.dense(om.NAMED["window-128"], N)
    M[5] = False
    q, k, v = make_qkv(1, N, D, torch.float32, seed=1)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), lambda a, b: M[a:b])
    dm = device_mask(pm.DenseMask(M), N, gpu)
    for BQ, A in [(128, 128), (16, 16), (32, 64)]:
        bi = pindex.build(pm.DenseMask(M), N, BQ, A)
        out = pattn.block_sparse_attention(q.to(gpu), k.to(gpu), v.to(gpu), *pindex.to_cuda(bi),
                                           dm, 0, 0, 0, BQ, A)
        assert torch.isfinite(out).all() and torch.count_nonzero(out[0, 5]) == 0
        check_close(out, want, torch.float32, f"dead row {BQ}x{A}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,s", [("dilated-4", 4), ("dilated-8", 8)])
def test_permuted_path_reference_style(gpu, dtype, name, s):
    """gpu/test_correctness.py step 4: physically permuted q/k/v, perm_q/perm_kv for the
    predicate, output un-permuted with invert()."""
    from polyhedral_amd import perm as pp
    N, D = 1024, 64
    q, k, v = make_qkv(2, N, D, dtype)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    p_np = op.residue_perm(N, s)
    perm = torch.from_numpy(p_np).to(gpu)
    qp, kp, vp = (pp.apply_perm(x.to(gpu), perm) for x in (q, k, v))
    kind, p0, p1, p2 = triton_params(name)
    for BQ, A in [(16, 16), (128, 32), (64, 64)]:
        bi = pindex.build(pm.Permuted(numpy_mask(name), p_np), N, BQ, A)
        outp = pattn.block_sparse_attention(qp, kp, vp, *pindex.to_cuda(bi), kind, p0, p1, p2, BQ, A,
                                            perm_q=perm.int(), perm_kv=perm.int())
        out = outp.index_select(1, pp.invert(perm).long())
        check_close(out, want, dtype, f"{name} rp{s} {BQ}x{A}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_gather_scatter_path(gpu, dtype):
    """gather_q / gather_kv / scatter_o on UNPERMUTED tensors == dense reference."""
    N, D, s, name = 2048, 128, 16, "lat16-band256"
    q, k, v = make_qkv(2, N, D, dtype, seed=3)
    want, want_lse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    p_np = op.residue_perm(N, s)
    perm = torch.from_numpy(p_np).to(gpu)
    kind = triton_params(name)
    bi = pindex.build(pm.Permuted(numpy_mask(name), p_np), N, 128, 32)
    lse = torch.empty(2, N, device=gpu)
    out = pattn.block_sparse_attention(q.to(gpu), k.to(gpu), v.to(gpu), *pindex.to_cuda(bi), *kind, 128, 32,
                                       perm_q=perm, gather_q=True, gather_kv=True, scatter_o=True, lse=lse)
    check_close(out, want, dtype, "fused gather/scatter")
    fin = np.isfinite(want_lse)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), fin)
    assert np.abs(lse.cpu().numpy()[fin] - want_lse[fin]).max() < (1e-5 if dtype == torch.float32 else 2e-2)
