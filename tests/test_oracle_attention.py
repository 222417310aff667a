"""The oracle attention (gpu/reference.py restated), the kernel recurrence simulator and the
LSE merge, pinned by textbook identities, brute force and the reference's own tests."""
import math

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import masks as om

N, D = 256, 16


def _inputs(seed, n=N, d=D):
    rng = np.random.default_rng(seed)
    return tuple(rng.standard_normal((n, d)) for _ in range(3))


def _brute(M, q, k, v, scale):
    """Pure-Python per-row softmax attention (small sizes only)."""
    n, d = q.shape
    out = np.zeros((n, v.shape[1]))
    lse = np.full(n, -np.inf)
    for i in range(n):
        cols = [j for j in range(n) if M[i, j]]
        if not cols:
            continue
        s = [sum(q[i, t] * k[j, t] for t in range(d)) * scale for j in cols]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        den = sum(w)
        lse[i] = mx + math.log(den)
        for c, wj in zip(cols, w):
            out[i] += wj / den * v[c]
    return out, lse


@pytest.mark.parametrize("name", ["window-128", "dilated-8", "sinks4+win8", "prefixlm-1024", "lat16-band256"])
def test_dense_attention_equals_per_row_brute_force(name):
    n, d = (300, 4) if name == "lat16-band256" else (96, 8)
    q, k, v = _inputs(3, n, d)
    M = om.dense(om.NAMED[name], n)
    got, lse = oatt.dense_attention(q[None], k[None], v[None], oatt.spec_rows(om.NAMED[name], n), row_chunk=17)
    want, wlse = _brute(M, q, k, v, d ** -0.5)
    assert np.abs(got[0] - want).max() < 1e-12
    fin = np.isfinite(wlse)
    assert fin.any() and np.array_equal(np.isfinite(lse[0]), fin)
    assert np.abs(lse[0][fin] - wlse[fin]).max() < 1e-12


def test_row_chunking_is_exact():
    q, k, v = _inputs(0)
    rows = oatt.spec_rows(om.NAMED["local256+str8"], N)
    a, la = oatt.dense_attention(q[None], k[None], v[None], rows, row_chunk=7)
    b, lb = oatt.dense_attention(q[None], k[None], v[None], rows, row_chunk=N)
    assert np.array_equal(a, b) and np.array_equal(la, lb)


def test_dead_rows_are_zero_with_minus_inf_lse():
    q, k, v = _inputs(1)
    M = om.dense(om.NAMED["window-128"], N)
    M[5] = False
    o, lse = oatt.dense_attention(q[None], k[None], v[None], lambda a, b: M[a:b])
    assert not o[0, 5].any() and np.isneginf(lse[0, 5]) and np.isfinite(o).all()


# the recurrence simulator: tests/test_kernel_math.py:60-90 cases
CASES = [("window-64", 128, 128), ("window-64", 128, 16), ("window-32", 64, 16), ("dilated-8", 128, 16),
         ("causal", 128, 32)]
SPEC = {"window-64": (((1, 64, 0, 0),), ()), "window-32": (((1, 32, 0, 0),), ()),
        "dilated-8": om.NAMED["dilated-8"], "causal": om.NAMED["causal"]}


@pytest.mark.parametrize("name,BQ,A", CASES)
def test_finite_sentinel_recurrence_matches_dense(name, BQ, A):
    q, k, v = _inputs(0)
    M = om.dense(SPEC[name], N)
    got = oatt.online_softmax(M, q, k, v, BQ, A, m_init=-1e30)
    want, _ = oatt.dense_attention(q[None], k[None], v[None], lambda a, b: M[a:b])
    assert np.isfinite(got).all()
    assert np.abs(got - want[0]).max() < 1e-9


def test_minus_inf_init_produces_nan():
    q, k, v = _inputs(0)
    M = om.dense(SPEC["window-64"], N)
    with np.errstate(invalid="ignore"):
        assert not np.isfinite(oatt.online_softmax(M, q, k, v, 128, 128, m_init=-np.inf)).all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_lse_merge_of_a_disjoint_split_equals_single_pass(seed):
    """Split a mask into disjoint random pieces: merging their (O, LSE) reproduces attention
    over the union (the identity the disjoint-split path relies on)."""
    rng = np.random.default_rng(seed)
    q, k, v = _inputs(seed + 10)
    union = om.dense(om.NAMED["local256+str8"], N)
    label = rng.integers(0, 3, size=union.shape)
    parts = [union & (label == i) for i in range(3)]
    outs, lses = [], []
    for P in parts:
        o, l = oatt.dense_attention(q[None], k[None], v[None], lambda a, b, P=P: P[a:b])
        outs.append(o)
        lses.append(l)
    got, glse = oatt.lse_merge(outs, lses)
    want, wlse = oatt.dense_attention(q[None], k[None], v[None], lambda a, b: union[a:b])
    assert np.abs(got - want).max() < 1e-12
    fin = np.isfinite(wlse)
    assert np.abs(glse[fin] - wlse[fin]).max() < 1e-12


def test_merge_with_an_empty_piece_is_identity():
    q, k, v = _inputs(4)
    M = om.dense(om.NAMED["causal"], N)
    o, l = oatt.dense_attention(q[None], k[None], v[None], lambda a, b: M[a:b])
    e = np.zeros_like(o)
    el = np.full_like(l, -np.inf)
    got, gl = oatt.lse_merge([o, e], [l, el])
    assert np.array_equal(got, o) and np.array_equal(gl, l)
    got, gl = oatt.lse_merge([e, e], [el, el])
    assert not got.any() and np.isneginf(gl).all()


def test_torch_fp32_baseline_matches_float64_oracle():
    import torch
    q, k, v = _inputs(5, 512, 64)
    rows = oatt.spec_rows(om.NAMED["sinks4+win256"], 512)
    want, _ = oatt.dense_attention(q[None], k[None], v[None], rows)
    got = oatt.dense_attention_torch(*(torch.from_numpy(x[None]).float() for x in (q, k, v)), rows, row_chunk=100)
    assert np.abs(got.numpy() - want).max() < 1e-5
