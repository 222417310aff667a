"""Backward of the block-sparse attention (pa_attn_bwd, pa_index_transpose) against the
float64 oracle gradient (oracle.attention.dense_attention_bwd, itself pinned against
torch.autograd): the textbook gradient of gpu/reference.py:5-17's attention, which the
reference does not implement.  The kernel takes the forward's o (in the input dtype)
and lse; the tolerance is on the error relative to the largest reference gradient."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import attention as pattn
from polyhedral_amd import backward as pbwd
from polyhedral_amd import index as pindex
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask, triton_params
from polyhedral_amd.split import Piece
from tests.util import as64, make_qkv

pytestmark = pytest.mark.gpu

# max |got - want| / max |want| per gradient
REL = {torch.bfloat16: 3e-2, torch.float16: 5e-3}


def _rel_err(got, want):
    return float(np.abs(as64(got) - want).max() / max(np.abs(want).max(), 1e-6))


def _oracle(q, k, v, do, rows):
    o, lse = oatt.dense_attention(as64(q), as64(k), as64(v), rows)
    grads = oatt.dense_attention_bwd(as64(q), as64(k), as64(v), as64(do), rows)
    return o, lse, grads


def _check(grads, want, dtype, what):
    for g, w_, nm in zip(grads, want, ("dq", "dk", "dv")):
        e = _rel_err(g, w_)
        assert e < REL[dtype], f"{what} {nm}: relative error {e:.3e}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["causal", "window-128", "dilated-8", "band256+lat16", "sinks4+win256",
                                  "local256+str8", "prefixlm-2048"])
def test_gradients_equal_oracle(gpu, name, dtype, D):
    _gradients_case(gpu, name, dtype, D, True)


@pytest.mark.parametrize("name", ["causal", "band256+lat16", "sinks4+win256", "prefixlm-2048"])
def test_gradients_without_bitmaps(gpu, name):
    """Partial tiles masked by evaluating the mask (no element bitmaps given)."""
    _gradients_case(gpu, name, torch.bfloat16, 128, False)


def _gradients_case(gpu, name, dtype, D, bitmaps):
    BH, N = 2, 1024
    q, k, v = make_qkv(BH, N, D, dtype, seed=D)
    do = make_qkv(BH, N, D, dtype, seed=D + 1)[0]
    rows = oatt.spec_rows(om.NAMED[name], N)
    o, lse, want = _oracle(q, k, v, do, rows)
    plan = pbwd.BackwardPlan(numpy_mask(name), N, gpu, bitmaps=bitmaps)
    dev = lambda x: x.to(gpu)
    grads = plan.backward(dev(q), dev(k), dev(v), torch.from_numpy(o).to(dtype).to(gpu),
                          torch.from_numpy(lse).float().to(gpu), dev(do))
    _check(grads, want, dtype, f"{name} {dtype} D={D} bitmaps={bitmaps}")


def test_forward_then_backward(gpu):
    """The streaming forward's o and lse feed the backward."""
    BH, N, D, name = 2, 2048, 128, "band256+lat16"
    q, k, v = make_qkv(BH, N, D, torch.bfloat16, seed=3)
    do = make_qkv(BH, N, D, torch.bfloat16, seed=4)[0]
    qd, kd, vd, dod = (x.to(gpu) for x in (q, k, v, do))
    lse = torch.empty(BH, N, device=gpu)
    bi = pindex.build(numpy_mask(name), N, 128, 32)
    launch = pattn.prepare(qd, kd, vd, *pindex.to_cuda(bi, gpu), *triton_params(name), 128, 32, lse=lse)
    with torch.cuda.device(gpu):
        o = launch()
    grads = pbwd.BackwardPlan(numpy_mask(name), N, gpu).backward(qd, kd, vd, o, lse, dod)
    _, _, want = _oracle(q, k, v, do, oatt.spec_rows(om.NAMED[name], N))
    _check(grads, want, torch.bfloat16, "forward + backward")


@pytest.mark.parametrize("D", [64, 128])
def test_permuted_basis_gives_the_permuted_gradients(gpu, D):
    """Tensors relabelled by rp8 with the mask evaluated through the permutation: the
    gradients are the identity-basis gradients relabelled."""
    BH, N, name = 2, 1024, "dilated-8"
    q, k, v = make_qkv(BH, N, D, torch.float16, seed=5)
    do = make_qkv(BH, N, D, torch.float16, seed=6)[0]
    p = op.residue_perm(N, 8)
    rows = oatt.spec_rows(om.NAMED[name], N)
    o, lse, want = _oracle(q, k, v, do, rows)
    pt = torch.from_numpy(p).long()
    plan = pbwd.BackwardPlan(numpy_mask(name), N, gpu, perm=p)
    grads = plan.backward(*(x[:, pt].contiguous().to(gpu) for x in (q, k, v)),
                          torch.from_numpy(o).to(torch.float16)[:, pt].contiguous().to(gpu),
                          torch.from_numpy(lse).float()[:, pt].contiguous().to(gpu), do[:, pt].contiguous().to(gpu))
    inv = torch.from_numpy(np.argsort(p)).long()
    _check([g.cpu()[:, inv] for g in grads], want, torch.float16, "rp8 basis")
    # the permuted basis lists fewer tiles
    assert int(plan.kv_num.sum()) < int(pbwd.BackwardPlan(numpy_mask(name), N, gpu).kv_num.sum())


def test_dead_rows_and_transposed_index(gpu):
    BH, N, D = 1, 512, 128
    M = om.dense(om.NAMED["window-128"], N)
    M[70] = False
    q, k, v = make_qkv(BH, N, D, torch.bfloat16, seed=7)
    do = make_qkv(BH, N, D, torch.bfloat16, seed=8)[0]
    o, lse, want = _oracle(q, k, v, do, lambda a, b: M[a:b])
    plan = pbwd.BackwardPlan(pm.DenseMask(M), N, gpu)
    grads = plan.backward(q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(o).to(torch.bfloat16).to(gpu),
                          torch.from_numpy(lse).float().to(gpu), do.to(gpu))
    assert torch.count_nonzero(grads[0][0, 70]) == 0
    _check(grads, want, torch.bfloat16, "dense mask with a dead row")
    # the transpose lists, per key block, exactly the query blocks holding it
    kv_idx, kv_num = plan.kv_idx.cpu().numpy(), plan.kv_num.cpu().numpy()
    kv_part = plan.kv_partial.cpu().numpy()
    q_idx, q_num, q_part = (t.cpu().numpy() for t in (plan.q_idx, plan.q_num, plan.q_partial))
    nb = N // 64
    for kb in range(nb):
        holders = [(qb, kv_part[qb, list(kv_idx[qb, :kv_num[qb]]).index(kb)]) for qb in range(nb)
                   if kb in kv_idx[qb, :kv_num[qb]]]
        assert q_num[kb] == len(holders)
        assert [int(x) for x in q_idx[kb, :q_num[kb]]] == [h[0] for h in holders]
        assert [int(x) for x in q_part[kb, :q_num[kb]]] == [int(h[1]) for h in holders]
    # bitmaps: a tile's offset is the same in both lists, its transposed bitmap is the
    # row-major one transposed, and its bits are the dense mask's
    kv_off, q_off = plan.kv_bits_off.cpu().numpy(), plan.q_bits_off.cpu().numpy()
    rb, cb = (t.cpu().numpy().view(np.uint32) for t in (plan.kv_bits, plan.q_bits))
    n_partial = 0
    for qb in range(nb):
        for j in range(kv_num[qb]):
            kb, off = int(kv_idx[qb, j]), int(kv_off[qb, j])
            assert (off >= 0) == bool(kv_part[qb, j])
            assert q_off[kb, list(q_idx[kb, :q_num[kb]]).index(qb)] == off
            if off < 0:
                continue
            n_partial += 1
            rows = np.unpackbits(rb[off:off + 128].view(np.uint8), bitorder="little").reshape(64, 64)
            cols = np.unpackbits(cb[off:off + 128].view(np.uint8), bitorder="little").reshape(64, 64)
            assert np.array_equal(rows, M[qb * 64:qb * 64 + 64, kb * 64:kb * 64 + 64])
            assert np.array_equal(cols.T, rows)
    assert n_partial > 0


def test_split_backward_equals_oracle(gpu):
    """band-256 | lattice-16 split as the forward splits it: the band in the identity basis,
    the lattice minus the band in rp16.  The gradients are the union's, from fewer tiles."""
    BH, N, D, name = 2, 1024, 128, "band256+lat16"
    band = pm.SlidingWindow(256)
    split = pbwd.SplitBackward([Piece(band), Piece(pm.Difference(pm.Dilated(16), band), residue=16)], N, gpu)
    q, k, v = make_qkv(BH, N, D, torch.bfloat16, seed=9)
    do = make_qkv(BH, N, D, torch.bfloat16, seed=10)[0]
    o, lse, want = _oracle(q, k, v, do, oatt.spec_rows(om.NAMED[name], N))
    grads = split.backward(q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(o).to(torch.bfloat16).to(gpu),
                           torch.from_numpy(lse).float().to(gpu), do.to(gpu))
    _check(grads, want, torch.bfloat16, "split: band + rp16 lattice")
    single = pbwd.BackwardPlan(numpy_mask(name), N, gpu, perm=op.residue_perm(N, 16))
    assert split.tiles < int(single.kv_num.sum())


@pytest.mark.parametrize("D", [64, 128])
def test_split_backward_two_permuted_pieces(gpu, D):
    """window-128 (identity) + dilated-16 minus the window (rp16) + dilated-24 minus both
    (rp8).  D = 128 applies the bases inside the kernels; D = 64 gathers the permuted
    pieces' tensors and scatters their gradients, the second permuted piece adding into
    gradients gathered into its basis."""
    BH, N = 2, 1024
    win, lat16 = pm.SlidingWindow(128), pm.Dilated(16)
    pieces = [Piece(win), Piece(pm.Difference(lat16, win), residue=16),
              Piece(pm.Difference(pm.Dilated(24), pm.Union(win, lat16)), residue=8)]
    split = pbwd.SplitBackward(pieces, N, gpu)
    spec = (((om.WINDOW, 128, 0, 0), (om.DILATED, 16, 0, 0), (om.DILATED, 24, 0, 0)), ())
    q, k, v = make_qkv(BH, N, D, torch.float16, seed=11)
    do = make_qkv(BH, N, D, torch.float16, seed=12)[0]
    o, lse, want = _oracle(q, k, v, do, oatt.spec_rows(spec, N))
    grads = split.backward(q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(o).to(torch.float16).to(gpu),
                           torch.from_numpy(lse).float().to(gpu), do.to(gpu))
    _check(grads, want, torch.float16, "split: three pieces, two permuted")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_residue_basis_in_the_loads_and_stores(gpu, dtype):
    """A plan in the rp16 basis run on tensors in original order (the kernels read and
    write through the closed-form permutation) gives the original-order gradients, and
    accumulate adds onto what the gradients held."""
    BH, N, D, name = 2, 1024, 128, "band256+lat16"
    q, k, v = make_qkv(BH, N, D, dtype, seed=13)
    do = make_qkv(BH, N, D, dtype, seed=14)[0]
    o, lse, want = _oracle(q, k, v, do, oatt.spec_rows(om.NAMED[name], N))
    plan = pbwd.BackwardPlan(numpy_mask(name), N, gpu, residue=16)
    args = [x.to(gpu) for x in (q, k, v)] + [torch.from_numpy(o).to(dtype).to(gpu),
                                             torch.from_numpy(lse).float().to(gpu), do.to(gpu)]
    grads = plan.backward(*args, original_order=True)
    _check(grads, want, dtype, f"rp16 basis in the kernels {dtype}")
    base = [torch.full_like(args[0], 0.5) for _ in range(3)]
    acc = plan.backward(*args, dq=base[0], dk=base[1], dv=base[2], accumulate=True, original_order=True)
    _check([g - 0.5 for g in acc], want, dtype, f"accumulated {dtype}")


def test_split_backward_of_empty_pieces_is_zero(gpu):
    N = 1024
    sub2 = pm.Difference(pm.Dilated(32), pm.PrefixLM(2048))              # empty at N = 1024
    split = pbwd.SplitBackward([Piece(sub2, residue=32)], N, gpu)
    assert split.tiles == 0 and split.live == 0
    q, k, v = (x.to(gpu) for x in make_qkv(1, N, 128, torch.bfloat16, seed=15))
    lse = torch.full((1, N), -float("inf"), device=gpu)
    grads = split.backward(q, k, v, torch.zeros_like(q), lse, q)
    assert all(torch.count_nonzero(g) == 0 for g in grads)


def test_headline_size_split_equals_one_basis(gpu):
    """band-256 | lattice-16 at L = 16384, H = 32, D = 128 (the headline workload), where no
    CPU oracle finishes: the split backward (identity band + rp16 lattice, bases applied
    in the kernels) and the whole mask in one pass in the rp16 basis on permuted copies
    are independent decompositions of the same gradients, from this build's forward."""
    from polyhedral_amd import workloads
    from polyhedral_amd.split import SplitPlan
    wl = workloads.make("bandlat-L16k")
    q, k, v = wl.inputs(0, gpu)
    launches, o, lse = SplitPlan(wl.pieces, wl.L, gpu).prepare(q, k, v)
    with torch.cuda.device(gpu):
        for launch in launches:
            launch()
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(21)).to(q.dtype).to(gpu)
    got = pbwd.SplitBackward(wl.pieces, wl.L, gpu).backward(q, k, v, o, lse, do)
    p = op.residue_perm(wl.L, 16)
    pt = torch.from_numpy(p).long().to(gpu)
    single = pbwd.BackwardPlan(wl.union, wl.L, gpu, perm=p)
    ref = single.backward(*(x[:, pt].contiguous() for x in (q, k, v, o)), lse[:, pt].contiguous(), do[:, pt].contiguous())
    inv = torch.from_numpy(np.argsort(p)).long().to(gpu)
    for g, r, nm in zip(got, ref, ("dq", "dk", "dv")):
        r = r[:, inv].float()
        err = float((g.float() - r).abs().max() / r.abs().max())
        assert err < 2e-2, f"{nm}: split and one-basis backwards differ by {err:.3e} (relative to the largest)"


@pytest.mark.parametrize("name", ["bandlat-L16k", "sinkwin-L32k", "dilated8-L8k", "prefixlat-L64k"])
def test_workload_size_sampled_gradients_equal_oracle(gpu, name):
    """Each bf16 workload at its full size (the headline band-256 | lattice-16 at L = 16384,
    H = 32 among them): the split backward's dQ on sampled query rows, and dK / dV on
    sampled keys near the end of the sequence, against the float64 oracle on the first and
    last head.  The oracle's rows are independent, so dQ of a row needs only that row, and
    dK / dV of a key need only the query rows live for it (the masks are causal, so those
    rows come after the key)."""
    from polyhedral_amd import workloads
    from polyhedral_amd.split import SplitPlan
    wl = workloads.make(name)
    L = wl.L
    q, k, v = wl.inputs(0, gpu)
    launches, o, lse = SplitPlan(wl.pieces, L, gpu).prepare(q, k, v)
    with torch.cuda.device(gpu):
        for launch in launches:
            launch()
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(23)).to(q.dtype).to(gpu)
    dq, dk, dv = pbwd.SplitBackward(wl.pieces, L, gpu).backward(q, k, v, o, lse, do)
    torch.cuda.synchronize()

    def row_mask(rows):
        return np.stack([np.asarray(wl.union.row_cols(int(i), L), dtype=bool) for i in rows])

    keys = np.array([L - 1, L - 20, L - 100])
    span = np.arange(L - 400, L)
    cols = row_mask(span)[:, keys]
    qrows = span[cols.any(axis=1)]
    # (no row before the span sees these keys)
    assert not np.asarray(wl.union.row_cols(L - 401, L), dtype=bool)[keys.min():].any()
    rows = np.array([0, 1, 255, 256, L // 2 + 1, L - 2, L - 1])
    for h in (0, wl.H - 1):
        kh, vh = as64(k[h:h + 1]), as64(v[h:h + 1])
        M = row_mask(rows)
        want_dq, _, _ = oatt.dense_attention_bwd(as64(q[h:h + 1, rows]), kh, vh, as64(do[h:h + 1, rows]),
                                                  lambda r0, r1: M[r0:r1])
        e = _rel_err(dq[h:h + 1, rows], want_dq)
        assert e < REL[torch.bfloat16], f"{name} head {h} dq rows: relative error {e:.3e}"
        M = row_mask(qrows)
        _, want_dk, want_dv = oatt.dense_attention_bwd(as64(q[h:h + 1, qrows]), kh, vh,
                                                        as64(do[h:h + 1, qrows]), lambda r0, r1: M[r0:r1])
        for g, w_, nm in ((dk, want_dk, "dk"), (dv, want_dv, "dv")):
            e = _rel_err(g[h:h + 1, keys], w_[:, keys])
            assert e < REL[torch.bfloat16], f"{name} head {h} {nm} keys: relative error {e:.3e}"
