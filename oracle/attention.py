"""Oracle attention (test infrastructure only).

dense_attention: gpu/reference.py:5-13 restated -- scores * scale, -inf where dead,
softmax, rows with no live key -> 0, @ V -- in float64 numpy, row-chunked (exact:
softmax is per row), with the per-row log-sum-exp.  online_softmax: the kernel's
tile recurrence as tests/test_kernel_math.py:27-48 restates _attn_fwd (finite
sentinel, l > 0 guard).  lse_merge: the log-sum-exp combine of a disjoint split.
dense_attention_bwd: the textbook gradient of that softmax attention (the reference
has no backward); pinned against torch.autograd in tests/test_oracle_backward.py.
"""
import numpy as np

from . import masks


def dense_attention(q, k, v, mask_rows, scale=None, row_chunk=256, dtype=np.float64):
    """q, k, v: [BH, N, D] arrays; mask_rows(r0, r1) -> bool [r1 - r0, N].
    Returns (o [BH, N, D], lse [BH, N]) in `dtype` (lse = -inf on dead rows)."""
    BH, N, D = q.shape
    scale = scale or D ** -0.5
    qf, kf, vf = (np.asarray(x, dtype=dtype) for x in (q, k, v))
    o = np.zeros((BH, N, D), dtype=dtype)
    lse = np.full((BH, N), -np.inf, dtype=dtype)
    for r0 in range(0, N, row_chunk):
        r1 = min(N, r0 + row_chunk)
        m = mask_rows(r0, r1)
        s = np.einsum("bqd,bkd->bqk", qf[:, r0:r1], kf) * scale
        s = np.where(m[None], s, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        alive = np.isfinite(mx)
        mx = np.where(alive, mx, 0.0)
        e = np.exp(s - mx)
        den = e.sum(axis=-1, keepdims=True)
        safe = np.where(den > 0, den, 1.0)
        o[:, r0:r1] = np.where(den > 0, np.einsum("bqk,bkd->bqd", e / safe, vf), 0.0)
        lse[:, r0:r1] = np.where(den[..., 0] > 0, (mx + np.log(safe))[..., 0], -np.inf)
    return o, lse


def spec_rows(spec, N, perm_q=None, perm_kv=None):
    return lambda r0, r1: masks.rows(spec, r0, r1, N, perm_q, perm_kv)


def online_softmax(M, q, k, v, BQ, A, m_init=-1e30, scale=None):
    """The kernel's recurrence over listed tiles (any live pair), one query block at a time."""
    N, D = q.shape
    scale = scale or D ** -0.5
    t = M.reshape(N // BQ, BQ, N // A, A).any(axis=(1, 3))
    out = np.zeros((N, D))
    for i in range(N // BQ):
        rows = slice(i * BQ, (i + 1) * BQ)
        m_i = np.full(BQ, m_init)
        l_i = np.zeros(BQ)
        acc = np.zeros((BQ, D))
        for j in np.flatnonzero(t[i]):
            cols = slice(j * A, (j + 1) * A)
            s = np.where(M[rows, cols], (q[rows] @ k[cols].T) * scale, -np.inf)
            m_new = np.maximum(m_i, s.max(axis=1))
            with np.errstate(invalid="ignore"):
                alpha = np.exp(m_i - m_new)
                p = np.exp(s - m_new[:, None])
            l_i = l_i * alpha + p.sum(axis=1)
            acc = acc * alpha[:, None] + p @ v[cols]
            m_i = m_new
        out[rows] = acc / np.where(l_i > 0, l_i, 1.0)[:, None]
    return out


def lse_merge(o_parts, lse_parts):
    """Combine partials over disjoint sub-masks: weights exp(lse_k - max), rows with
    every lse_k = -inf give 0 and lse -inf."""
    L = np.stack(lse_parts)                       # [K, BH, N]
    mx = L.max(axis=0)
    alive = np.isfinite(mx)
    w = np.where(alive[None], np.exp(L - np.where(alive, mx, 0.0)[None]), 0.0)
    den = w.sum(axis=0)
    o = sum(w[i][..., None] * o_parts[i] for i in range(len(o_parts)))
    o = np.where(den[..., None] > 0, o / np.where(den > 0, den, 1.0)[..., None], 0.0)
    lse = np.where(den > 0, mx + np.log(np.where(den > 0, den, 1.0)), -np.inf)
    return o, lse


def dense_attention_torch(q, k, v, mask_rows, scale=None, row_chunk=1024):
    """gpu/reference.py:5-13 in fp32 torch on the host, row-chunked: the CPU baseline.
    q, k, v: CPU tensors [BH, N, D]; mask_rows(r0, r1) -> bool numpy [r1 - r0, N]."""
    import torch
    BH, N, D = q.shape
    scale = scale or D ** -0.5
    kf = k.float()
    vf = v.float()
    out = torch.empty((BH, N, D), dtype=torch.float32)
    for r0 in range(0, N, row_chunk):
        r1 = min(N, r0 + row_chunk)
        m = torch.from_numpy(mask_rows(r0, r1))
        s = (q[:, r0:r1].float() @ kf.transpose(-1, -2)) * scale
        s = s.masked_fill(~m[None], float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
        out[:, r0:r1] = p @ vf
    return out


def dense_attention_bwd(q, k, v, do, mask_rows, scale=None, row_chunk=256, dtype=np.float64):
    """Gradients of o = softmax(scale q k^T, masked) v with respect to q, k, v for an
    upstream gradient do: with P the masked softmax (rows with no live key: P = 0),
    dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO o)), dQ = scale dS K,
    dK = scale dS^T Q.  q, do: [BH, Nq, D]; k, v: [BH, Nk, D]; mask_rows(r0, r1) ->
    bool [r1 - r0, Nk].  Returns (dq, dk, dv) in `dtype`."""
    BH, N, D = q.shape
    scale = scale or D ** -0.5
    qf, kf, vf, gf = (np.asarray(x, dtype=dtype) for x in (q, k, v, do))
    dq = np.zeros_like(qf)
    dk = np.zeros_like(kf)
    dv = np.zeros_like(vf)
    for r0 in range(0, N, row_chunk):
        r1 = min(N, r0 + row_chunk)
        m = mask_rows(r0, r1)
        s = np.einsum("bqd,bkd->bqk", qf[:, r0:r1], kf) * scale
        s = np.where(m[None], s, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0)
        e = np.exp(s - mx)
        den = e.sum(axis=-1, keepdims=True)
        p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
        o = np.einsum("bqk,bkd->bqd", p, vf)
        g = gf[:, r0:r1]
        dv += np.einsum("bqk,bqd->bkd", p, g)
        dp = np.einsum("bqd,bkd->bqk", g, vf)
        ds = p * (dp - (g * o).sum(axis=-1, keepdims=True))
        dq[:, r0:r1] = scale * np.einsum("bqk,bkd->bqd", ds, kf)
        dk += scale * np.einsum("bqk,bqd->bkd", ds, qf[:, r0:r1])
    return dq, dk, dv
