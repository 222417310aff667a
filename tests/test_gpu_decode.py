"""Decoding against a cache kept in a class-A basis (pa_kv_append, pa_decode_fwd).

The cache layout is pinned by the residue permutation's closed form (oracle.permute,
gpu/permute.py:12-15): row r of a capacity-C cache in the residue-s basis holds the
token at original position residue_perm(C, s)[r].  Decode attention is pinned by the
float64 oracle (gpu/reference.py:5-17) on the same tokens in original order: the
query rows at positions qpos0 .. qpos0 + nq - 1 against the first `length` keys."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import masks as om
from oracle import permute as op
from polyhedral_amd import _lib
from polyhedral_amd import decode as pdec
from polyhedral_amd.polyattn import masks as pm
from polyhedral_amd.registry import numpy_mask
from tests.util import as64, check_close, make_qkv

pytestmark = pytest.mark.gpu


def _orig_of_row(capacity, s):
    return op.residue_perm(capacity, s) if s > 1 else np.arange(capacity)


def _fill(cache, k, v, sizes, gpu):
    t0 = 0
    for n in sizes:
        cache.append(k[:, t0:t0 + n].to(gpu), v[:, t0:t0 + n].to(gpu))
        t0 += n
    assert cache.length == t0
    return t0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("residue", [0, 8, 16])
def test_append_places_rows_by_the_residue_permutation(gpu, residue, dtype):
    BH, cap = 3, 2048
    D = 64 if dtype == torch.float32 else 128
    _, k, v = make_qkv(BH, cap, D, dtype, seed=residue + 1)
    cache = pdec.KVCache(BH, cap, D, dtype, residue, gpu)
    L = _fill(cache, k, v, [700, 1, 1, 5, 300, 1], gpu)
    orig = _orig_of_row(cap, max(residue, 1))
    assert np.array_equal(cache.rows(orig), np.arange(cap))   # rows() inverts the permutation
    filled = np.flatnonzero(orig < L)
    empty = np.flatnonzero(orig >= L)
    for got, want in ((cache.k.cpu(), k), (cache.v.cpu(), v)):
        assert torch.equal(got[:, filled], want[:, orig[filled]])
        assert torch.count_nonzero(got[:, empty]) == 0


@pytest.mark.parametrize("nq", [1, 3, 8])
@pytest.mark.parametrize("residue", [0, 8, 16])
@pytest.mark.parametrize("name", ["dilated-8", "band256+lat16", "sinks4+win256", "causal", "window-128",
                                  "lat16-band256", "local256+str8", "prefixlm-2048"])
def test_decode_equals_oracle(gpu, name, residue, nq):
    BH, cap, D, L = 2, 2048, 128, 1500
    q, k, v = make_qkv(BH, cap, D, torch.bfloat16, seed=nq)
    cache = pdec.KVCache(BH, cap, D, torch.bfloat16, residue, gpu)
    _fill(cache, k, v, [L - 8, 3, 5], gpu)
    qpos0 = L - nq
    lse = torch.empty(BH, nq, device=gpu)
    out = cache.attend(q[:, qpos0:L].to(gpu), numpy_mask(name), lse=lse)
    spec = om.NAMED[name]
    want, want_lse = oatt.dense_attention(as64(q[:, qpos0:L]), as64(k[:, :L]), as64(v[:, :L]),
                                          lambda r0, r1: om.rows(spec, qpos0 + r0, qpos0 + r1, L))
    check_close(out, want, torch.bfloat16, f"decode {name} s={residue} nq={nq}")
    fin = np.isfinite(want_lse)
    got_lse = lse.cpu().numpy()
    assert np.array_equal(np.isfinite(got_lse), fin)
    assert np.abs(got_lse[fin] - want_lse[fin]).max() < 2e-2


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_decode_other_dtypes_and_earlier_queries(gpu, dtype):
    """Queries anywhere before the end, and a prefix of the cache (length < tokens held)."""
    BH, cap, name = 2, 1024, "band256+lat16"
    D = 64 if dtype == torch.float32 else 128
    q, k, v = make_qkv(BH, cap, D, dtype, seed=4)
    cache = pdec.KVCache(BH, cap, D, dtype, 16, gpu)
    _fill(cache, k, v, [900], gpu)
    for qpos0, nq, L in ((100, 4, 900), (500, 1, 700), (0, 2, 900)):
        out = cache.attend(q[:, qpos0:qpos0 + nq].to(gpu), numpy_mask(name), qpos0=qpos0, length=L)
        want, _ = oatt.dense_attention(as64(q[:, qpos0:qpos0 + nq]), as64(k[:, :L]), as64(v[:, :L]),
                                       lambda r0, r1: om.rows(om.NAMED[name], qpos0 + r0, qpos0 + r1, L))
        check_close(out, want, dtype, f"decode {dtype} qpos0={qpos0} nq={nq} L={L}")


def test_dead_queries_and_empty_cache(gpu):
    BH, cap, D = 2, 512, 128
    q, k, v = make_qkv(BH, cap, D, torch.bfloat16, seed=2)
    M = om.dense(om.NAMED["causal"], cap)
    M[300] = False                      # query 300 sees no key
    cache = pdec.KVCache(BH, cap, D, torch.bfloat16, 8, gpu)
    lse = torch.empty(BH, 1, device=gpu)
    out = cache.attend(q[:, :1].to(gpu), pm.DenseMask(M), qpos0=0, lse=lse)   # empty cache
    assert torch.count_nonzero(out) == 0 and torch.isinf(lse).all() and (lse < 0).all()
    _fill(cache, k, v, [301], gpu)
    lse = torch.empty(BH, 2, device=gpu)
    out = cache.attend(q[:, 299:301].to(gpu), pm.DenseMask(M), lse=lse)
    assert torch.count_nonzero(out[:, 1]) == 0 and torch.isinf(lse[:, 1]).all()
    want, _ = oatt.dense_attention(as64(q[:, 299:300]), as64(k[:, :301]), as64(v[:, :301]),
                                   lambda r0, r1: M[299 + r0:299 + r1, :301])
    check_close(out[:, :1], want, torch.bfloat16, "dense mask decode")


@pytest.mark.parametrize("residue", [0, 16])
@pytest.mark.parametrize("nq", [1, 3])
def test_decode_with_many_live_keys_per_block(gpu, residue, nq):
    """64 heads, so each of a head's 8 work-groups takes 2 groups of 256 keys and each wave
    two 64-key blocks; every block holds about 45 keys live for some query (a random mask
    of density 0.7), so in the identity basis a wave's list of live keys passes 64 and the
    rest carries over to a second batch.  Against the oracle on every head."""
    BH, cap, D = 64, 4096, 128
    L = cap
    q, k, v = make_qkv(BH, cap, D, torch.bfloat16, seed=7 + nq)
    rng = np.random.default_rng(11 + nq)
    M = np.zeros((cap, cap), dtype=bool)
    qpos0 = L - nq
    M[qpos0:L, :L] = rng.random((nq, L)) < 0.7
    cache = pdec.KVCache(BH, cap, D, torch.bfloat16, residue, gpu)
    _fill(cache, k, v, [L - 100, 100], gpu)
    lse = torch.empty(BH, nq, device=gpu)
    out = cache.attend(q[:, qpos0:L].to(gpu), pm.DenseMask(M), lse=lse)
    want, want_lse = oatt.dense_attention(as64(q[:, qpos0:L]), as64(k[:, :L]), as64(v[:, :L]),
                                          lambda r0, r1: M[qpos0 + r0:qpos0 + r1, :L])
    check_close(out, want, torch.bfloat16, f"decode dense-random s={residue} nq={nq}")
    assert np.abs(lse.cpu().numpy() - want_lse).max() < 2e-2


def test_bases_agree_at_the_headline_size(gpu):
    """band-256 | lattice-16, L = 16384, 32 heads, D = 128: the newest token decoded in the
    identity and the rp16 basis; both against the oracle on two heads."""
    H, L, D, name = 32, 16384, 128, "band256+lat16"
    q, k, v = make_qkv(H, L, D, torch.bfloat16, seed=0)
    outs = []
    for s in (0, 16):
        cache = pdec.KVCache(H, L, D, torch.bfloat16, s, gpu)
        _fill(cache, k, v, [L - 1, 1], gpu)
        outs.append(cache.attend(q[:, L - 1:].to(gpu), numpy_mask(name)).float().cpu())
        del cache
    want, _ = oatt.dense_attention(as64(q[:2, L - 1:]), as64(k[:2]), as64(v[:2]),
                                   lambda r0, r1: om.rows(om.NAMED[name], L - 1 + r0, L - 1 + r1, L))
    for o in outs:
        check_close(o[:2], want, torch.bfloat16, "headline decode")
    assert (outs[0] - outs[1]).abs().max().item() < 2e-2


@pytest.mark.parametrize("name,s", [("bandlat-L16k", 16), ("sinkwin-L32k", 16), ("dilated8-L8k", 8),
                                    ("prefixlat-L64k", 32)])
@pytest.mark.parametrize("basis", ["identity", "residue"])
def test_decode_step_at_each_workload_size(gpu, name, s, basis):
    """The bench's decode step at the workload's full size: the newest token's K / V appended
    and its query attended in one call, against the float64 oracle on the first and last
    head (the whole mask's row of the newest token)."""
    from polyhedral_amd import workloads
    wl = workloads.make(name)
    H, L, D = wl.H, wl.L, wl.D
    q, k, v = wl.inputs(0, gpu)
    cache = pdec.KVCache(H, L, D, q.dtype, s if basis == "residue" else 0, gpu)
    cache.append(k[:, :L - 1], v[:, :L - 1])
    lse = torch.empty(H, 1, device=gpu)
    out = cache.attend(q[:, L - 1:].contiguous(), wl.union, lse=lse,
                       k_new=k[:, L - 1:].contiguous(), v_new=v[:, L - 1:].contiguous())
    torch.cuda.synchronize()
    live = np.asarray(wl.union.row_cols(L - 1, L), dtype=bool)
    heads = [0, H - 1]
    want, want_lse = oatt.dense_attention(as64(q[heads, L - 1:]), as64(k[heads]), as64(v[heads]),
                                          lambda r0, r1: live[None])
    check_close(out[heads], want, q.dtype, f"decode step {name} {basis}")
    assert np.abs(lse[heads].cpu().numpy() - want_lse).max() < 2e-2
    del cache, q, k, v


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("residue", [0, 16])
@pytest.mark.parametrize("n_new,nq", [(1, 1), (3, 3), (8, 8), (2, 5)])
def test_append_in_the_decode_call_equals_append_then_attend(gpu, residue, dtype, n_new, nq, static):
    """prepare(..., k_new, v_new) appends in the decode kernels: the same output, log-sum-exp
    and cache as pa_kv_append followed by the decode call, bit for bit.  The new rows are
    not in the cache before the call, so reading them from there would show."""
    BH, cap, L0, name = 3, 2048, 1500, "band256+lat16"
    D = 64 if dtype == torch.float32 else 128
    q, k, v = make_qkv(BH, cap, D, dtype, seed=11 + n_new)
    caches = [pdec.KVCache(BH, cap, D, dtype, residue, gpu) for _ in range(2)]
    for c in caches:
        _fill(c, k, v, [L0], gpu)
    kn, vn = k[:, L0:L0 + n_new].to(gpu), v[:, L0:L0 + n_new].to(gpu)
    qq = q[:, L0 + n_new - nq:L0 + n_new].to(gpu)
    lse = [torch.empty(BH, nq, device=gpu) for _ in range(2)]
    caches[0].append(kn, vn)
    o0 = caches[0].attend(qq, numpy_mask(name), lse=lse[0], static_scratch=static)
    o1 = caches[1].attend(qq, numpy_mask(name), lse=lse[1], static_scratch=static, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert caches[0].length == caches[1].length == L0 + n_new
    assert torch.equal(o0, o1) and torch.equal(lse[0], lse[1])
    assert torch.equal(caches[0].k, caches[1].k) and torch.equal(caches[0].v, caches[1].v)
    qpos0 = L0 + n_new - nq
    want, _ = oatt.dense_attention(as64(q[:, qpos0:L0 + n_new]), as64(k[:, :L0 + n_new]), as64(v[:, :L0 + n_new]),
                                   lambda r0, r1: om.rows(om.NAMED[name], qpos0 + r0, qpos0 + r1, L0 + n_new))
    check_close(o1, want, dtype, f"decode with append s={residue} n_new={n_new} nq={nq}")


def test_append_in_the_decode_call_at_the_headline_size(gpu):
    """band-256 | lattice-16, L = 16384, 32 heads: the newest token appended and decoded in
    one call, replayed (each run rewrites the same rows), against append then decode."""
    H, L, D, name = 32, 16384, 128, "band256+lat16"
    q, k, v = make_qkv(H, L, D, torch.bfloat16, seed=0)
    for s in (0, 16):
        a = pdec.KVCache(H, L, D, torch.bfloat16, s, gpu)
        b = pdec.KVCache(H, L, D, torch.bfloat16, s, gpu)
        for c in (a, b):
            _fill(c, k, v, [L - 1], gpu)
        kn, vn, qn = (x[:, L - 1:].contiguous().to(gpu) for x in (k, v, q))
        a.append(kn, vn)
        want = a.attend(qn, numpy_mask(name))
        launch = b.prepare(qn, numpy_mask(name), k_new=kn, v_new=vn)
        for _ in range(3):
            got = launch()
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"s={s}"
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
        del a, b, launch


def test_decode_argument_errors(gpu):
    BH, cap, D = 1, 256, 128
    cache = pdec.KVCache(BH, cap, D, torch.bfloat16, 16, gpu)
    q = torch.zeros(BH, 9, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="1..8"):
        cache.attend(q, numpy_mask("causal"), qpos0=0)
    with pytest.raises(ValueError, match="capacity"):
        cache.append(torch.zeros(BH, 257, D, dtype=torch.bfloat16, device=gpu),
                     torch.zeros(BH, 257, D, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="multiple"):
        pdec.KVCache(BH, 250, D, torch.bfloat16, 16, gpu)
    # the C ABI checks the same bounds itself
    z = torch.zeros(BH, 2, D, dtype=torch.bfloat16, device=gpu)
    rc = _lib.lib().pa_kv_append(_lib.ptr(z), _lib.ptr(z), z.stride(0), z.stride(1), _lib.ptr(cache.k),
                                 _lib.ptr(cache.v), cache.k.stride(0), cache.k.stride(1), BH, 2, D, _lib.PA_BF16,
                                 cap, cap - 1, 16, _lib.stream_of(z))
    assert rc == _lib.PA_E_INVALID and b"capacity" in _lib.lib().pa_last_error()
