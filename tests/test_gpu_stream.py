"""The streaming attention kernel (LDS DMA, step descriptors, bitmap masking) against the
float64 oracle, and its step descriptors against the index they are derived from."""
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
from polyhedral_amd.split import Piece, SplitPlan
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu

STREAM_MASKS = ["window-128", "causal", "dilated-8", "local256+str8", "twoband-1000", "sinks4+win256",
                "prefixlm-2048", "lat16-band256"]


def _expected_steps(kv_idx, kv_num, wave, bits_off, BQ, A, N=0, residue=0, order=None):
    """The descriptor layout of include/polyattn_amd.h (pa_index_steps), from the index."""
    nq, pitch = kv_idx.shape
    spt = A // 16
    ncg = max(1, A // 32)
    ngr = max(1, BQ // 32)
    sp = (pitch * A + 63) // 64
    out = np.zeros((nq, sp, 16), dtype=np.int64)
    for pos in range(nq):
        qb = int(order[pos]) if order is not None else pos
        n_seg = int(kv_num[qb]) * spt
        for j in range(sp):
            code = 0
            for t in range(4):
                seg = 4 * j + t
                base, boff, c8 = 0, -1, 0
                if seg < n_seg:
                    ti, within = seg // spt, seg % spt
                    base = int(kv_idx[qb, ti]) * A + within * 16
                    if residue:
                        q = N // residue
                        base = (base % q) * residue + base // q
                    cg = within >> 1 if A >= 32 else 0
                    wb = int(wave[qb, ti]) & 0xFFFFFFFF
                    for g in range(min(ngr, 4)):
                        c8 |= ((wb >> (2 * (g * ncg + cg))) & 3) << (2 * g)
                    if bits_off[qb, ti] >= 0:
                        boff = int(bits_off[qb, ti]) + ((within * 16) >> 5)
                out[pos, j, t] = base
                out[pos, j, 5 + t] = boff
                code |= c8 << (8 * t)
            out[pos, j, 4] = code
            out[pos, j, 13] = qb
            out[pos, j, 14] = (int(kv_num[qb]) * A + 63) // 64
            out[pos, j, 15] = residue
    return (out & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


@pytest.mark.parametrize("residue", [0, 16])
@pytest.mark.parametrize("A", [16, 32, 64])
@pytest.mark.parametrize("name", ["window-128", "dilated-8", "lat16-band256", "sinks4+win8"])
def test_step_descriptors_follow_the_index(gpu, name, A, residue):
    N, BQ = 2048, 128
    kv_idx, kv_num, kv_partial, wave, tiles, live, bits, steps = pindex.build_device(
        numpy_mask(name), N, BQ, A, device=gpu, bits=True, steps=True, residue=residue)
    assert steps.residue_s == residue
    want = _expected_steps(kv_idx.cpu().numpy(), kv_num.cpu().numpy(), wave.cpu().numpy(),
                           bits[0].cpu().numpy(), BQ, A, N, residue)
    got = steps.cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(got, want), f"{name} A={A}: first mismatch at {np.argwhere(got != want)[:3]}"
    # laid out in an issue order (a fixed permutation of the query blocks)
    order = torch.from_numpy(np.random.default_rng(A).permutation(N // BQ).astype(np.int32)).to(gpu)
    st2 = pindex.build_steps(kv_idx, kv_num, kv_partial, wave, bits[0], N, BQ, A, residue, order)
    assert st2.order is order
    want2 = _expected_steps(kv_idx.cpu().numpy(), kv_num.cpu().numpy(), wave.cpu().numpy(),
                            bits[0].cpu().numpy(), BQ, A, N, residue, order.cpu().numpy())
    assert np.array_equal(st2.cpu().numpy(), want2), f"{name} A={A} ordered"


def _launch(q, k, v, bi, name, BQ, A, kernel, **kw):
    kind, p0, p1, p2 = triton_params(name)
    launch = pattn.prepare(q, k, v, *pindex.to_cuda(bi), kind, p0, p1, p2, BQ, A, kernel=kernel, **kw)
    with torch.cuda.device(q.device):
        out = launch()
    return launch, out


@pytest.mark.parametrize("A", [16, 32, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", STREAM_MASKS)
def test_stream_kernel_equals_oracle(gpu, name, dtype, A):
    N, D, BH, BQ = 1024, 128, 2, 128
    q, k, v = make_qkv(BH, N, D, dtype, seed=A)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    qd, kd, vd = (x.to(gpu) for x in (q, k, v))
    bi = pindex.build(numpy_mask(name), N, BQ, A)
    launch, out = _launch(qd, kd, vd, bi, name, BQ, A, "stream")
    assert launch.kernel == "stream"
    check_close(out, want, dtype, f"stream {name} {dtype} 128x{A}")


@pytest.mark.parametrize("name", ["lat16-band256", "sinks4+win256"])
def test_stream_with_issue_order(gpu, name):
    """Lists issued in a permuted order (the descriptors are rebuilt for that order)."""
    N, D, BQ, A = 2048, 128, 128, 32
    q, k, v = make_qkv(2, N, D, torch.bfloat16, seed=11)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    bi = pindex.build(numpy_mask(name), N, BQ, A)
    order = torch.from_numpy(np.random.default_rng(3).permutation(N // BQ).astype(np.int32)).to(gpu)
    launch, out = _launch(q.to(gpu), k.to(gpu), v.to(gpu), bi, name, BQ, A, "stream", qblock_order=order)
    assert launch.kernel == "stream"
    check_close(out, want, torch.bfloat16, f"stream {name} ordered")


def test_auto_selects_each_kernel(gpu):
    N, D = 512, 128
    q, k, v = (x.to(gpu) for x in make_qkv(1, N, D, torch.bfloat16))
    bi = pindex.build(numpy_mask("window-128"), N, 128, 32)
    assert _launch(q, k, v, bi, "window-128", 128, 32, "auto")[0].kernel == "stream"
    assert _launch(q, k, v, bi, "window-128", 128, 32, "general")[0].kernel == "general"
    bi64 = pindex.build(numpy_mask("window-128"), N, 64, 64)
    assert _launch(q, k, v, bi64, "window-128", 64, 64, "auto")[0].kernel == "general"
    with pytest.raises(ValueError, match="streaming kernel"):
        _launch(q, k, v, bi64, "window-128", 64, 64, "stream")
    qf, kf, vf = (x.float() for x in (q, k, v))
    # float32 over 4 query blocks: too few for the chip, the wave-split kernel
    assert _launch(qf, kf, vf, bi, "window-128", 128, 32, "auto")[0].kernel == "wsplit"
    assert _launch(qf, kf, vf, bi, "window-128", 128, 32, "general")[0].kernel == "general"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stream_residue_basis_gather_scatter(gpu, dtype):
    """Closed-form rp16 basis, Q/K/V read and O written in original order, LSE out."""
    N, D, s, name = 2048, 128, 16, "lat16-band256"
    q, k, v = make_qkv(2, N, D, dtype, seed=3)
    want, want_lse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(om.NAMED[name], N))
    p_np = op.residue_perm(N, s)
    perm = torch.from_numpy(p_np).to(gpu)
    bi = pindex.build(pm.Permuted(numpy_mask(name), p_np), N, 128, 32)
    lse = torch.empty(2, N, device=gpu)
    launch, out = _launch(q.to(gpu), k.to(gpu), v.to(gpu), bi, name, 128, 32, "stream", perm_q=perm,
                          gather_q=True, gather_kv=True, scatter_o=True, residue=s, lse=lse)
    assert launch.kernel == "stream"
    check_close(out, want, dtype, "stream residue basis")
    fin = np.isfinite(want_lse)
    got_lse = lse.cpu().numpy()
    assert np.array_equal(np.isfinite(got_lse), fin)
    assert np.abs(got_lse[fin] - want_lse[fin]).max() < 2e-2


@pytest.mark.parametrize("A", [16, 32, 64])
def test_stream_split_merge_equals_single_pass(gpu, A):
    """band-256 (identity) + lattice-16 minus band (rp16) merged in the epilogue == the union."""
    N, D = 4096, 128
    q, k, v = make_qkv(2, N, D, torch.bfloat16, seed=7)
    union = om.NAMED["band256+lat16"]
    want, want_lse = oatt.dense_attention(as64(q), as64(k), as64(v), oatt.spec_rows(union, N))
    band = pm.SlidingWindow(256)
    plan = SplitPlan([Piece(band, 128, A), Piece(pm.Difference(pm.Dilated(16), band), 128, A, residue=16)], N, gpu)
    lse = torch.empty(2, N, device=gpu)
    launches, o, _ = plan.prepare(q.to(gpu), k.to(gpu), v.to(gpu), lse=lse)
    assert [x.kernel for x in launches] == ["stream", "stream"]
    with torch.cuda.device(gpu):
        for x in launches:
            x()
    check_close(o, want, torch.bfloat16, f"stream split A={A}")
    fin = np.isfinite(want_lse)
    assert np.abs(lse.cpu().numpy()[fin] - want_lse[fin]).max() < 2e-2


def test_stream_dead_rows_and_empty_lists(gpu):
    """A query row with no live key gives exact zeros; a query block with an empty list
    (and a whole mask that is empty) goes through the kernel without reading K / V."""
    from polyhedral_amd.spec import device_mask
    N, D = 1024, 128
    M = om.dense(om.NAMED["window-128"], N)
    M[5] = False
    M[256:384] = False          # query block 2 (rows 256..383) has no live key at all
    q, k, v = make_qkv(1, N, D, torch.bfloat16, seed=1)
    want, _ = oatt.dense_attention(as64(q), as64(k), as64(v), lambda a, b: M[a:b])
    dm = device_mask(pm.DenseMask(M), N, gpu)
    for A in (16, 32, 64):
        bi = pindex.build(pm.DenseMask(M), N, 128, A)
        launch = pattn.prepare(q.to(gpu), k.to(gpu), v.to(gpu), *pindex.to_cuda(bi), dm, 0, 0, 0, 128, A,
                               kernel="stream")
        with torch.cuda.device(gpu):
            out = launch()
        assert torch.isfinite(out).all() and torch.count_nonzero(out[0, 5]) == 0
        assert torch.count_nonzero(out[0, 256:384]) == 0
        check_close(out, want, torch.bfloat16, f"stream dead rows 128x{A}")


@pytest.mark.parametrize("kernel", ["stream", "general"])
def test_heads_desc_gives_identical_results(gpu, kernel):
    """Issuing the heads last-to-first changes only the order of the work-groups."""
    N, D, name = 1024, 128, "lat16-band256"
    q, k, v = (x.to(gpu) for x in make_qkv(3, N, D, torch.bfloat16, seed=5))
    bi = pindex.build(numpy_mask(name), N, 128, 32)
    outs = []
    for desc in (False, True):
        lse = torch.empty(3, N, device=gpu)
        launch, out = _launch(q, k, v, bi, name, 128, 32, kernel, lse=lse, heads_desc=desc)
        assert launch.kernel == kernel
        outs.append((out.clone(), lse.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
