"""Oracle predicates (test infrastructure only).

Restates gpu/masks_gpu.py:37-52 (flex_mask_mod, the ground truth dense_bool is
built from; SINKS keeps the absolute-kv sink term of :51-52) and PrefixLM from
src/polyattn/masks.py:129-148.  A spec is (include, exclude) with terms
(kind, p0, p1, p2); live = OR(include) AND NOT OR(exclude).
"""
import numpy as np

CAUSAL, WINDOW, DILATED, LOCAL_STRIDED, TWOBAND, SINKS, PREFIX_LM, FULL = range(8)

# name -> (include, exclude): the reference's SPECS entries (gpu/masks_gpu.py:11-25)
# and the benchmark workloads (band+lattice, sinks+window, prefix-LM+lattice, dilated)
NAMED = {
    "causal": (((CAUSAL, 0, 0, 0),), ()),
    "window-128": (((WINDOW, 128, 0, 0),), ()),
    "window-256": (((WINDOW, 256, 0, 0),), ()),
    "window-512": (((WINDOW, 512, 0, 0),), ()),
    "window-1024": (((WINDOW, 1024, 0, 0),), ()),
    "window-4096": (((WINDOW, 4096, 0, 0),), ()),
    "dilated-2": (((DILATED, 2, 0, 0),), ()),
    "dilated-4": (((DILATED, 4, 0, 0),), ()),
    "dilated-8": (((DILATED, 8, 0, 0),), ()),
    "dilated-16": (((DILATED, 16, 0, 0),), ()),
    "dilated-32": (((DILATED, 32, 0, 0),), ()),
    "local256+str8": (((LOCAL_STRIDED, 256, 8, 0),), ()),
    "band256+lat16": (((LOCAL_STRIDED, 256, 16, 0),), ()),
    "band256+lat32": (((LOCAL_STRIDED, 256, 32, 0),), ()),
    "twoband-1024": (((TWOBAND, 128, 1024, 128),), ()),
    "twoband-1000": (((TWOBAND, 128, 1000, 128),), ()),
    "sinks4+win256": (((SINKS, 256, 4, 0),), ()),
    "sinks4+win1024": (((SINKS, 1024, 4, 0),), ()),
    "sinks4+win8": (((SINKS, 8, 4, 0),), ()),
    "sinks64+win1024": (((SINKS, 1024, 64, 0),), ()),
    "prefixlm-1024": (((PREFIX_LM, 1024, 0, 0),), ()),
    "prefixlm-2048": (((PREFIX_LM, 2048, 0, 0),), ()),
    "lat16-band256": (((DILATED, 16, 0, 0),), ((WINDOW, 256, 0, 0),)),
    "lat32-prefixlm2048": (((DILATED, 32, 0, 0),), ((PREFIX_LM, 2048, 0, 0),)),
    "lat32-band256": (((DILATED, 32, 0, 0),), ((WINDOW, 256, 0, 0),)),
}


def term(t, q, kv):
    k, p0, p1, p2 = t
    d = q - kv
    c = q >= kv
    if k == CAUSAL:
        return c
    if k == WINDOW:
        return c & (d < p0)
    if k == DILATED:
        return c & (d % p0 == 0)
    if k == LOCAL_STRIDED:
        return c & ((d < p0) | (d % p1 == 0))
    if k == TWOBAND:
        return c & ((d < p0) | ((d >= p1) & (d < p1 + p2)))
    if k == SINKS:
        return c & ((d < p0) | (kv < p1))
    if k == PREFIX_LM:
        return c | ((q < p0) & (kv < p0))
    if k == FULL:
        return np.ones(np.broadcast(q, kv).shape, dtype=bool)
    raise ValueError(k)


def live(spec, q, kv):
    """bool array over broadcast int arrays of ORIGINAL coordinates."""
    include, exclude = spec
    out = term(include[0], q, kv)
    for t in include[1:]:
        out = out | term(t, q, kv)
    for t in exclude:
        out = out & ~term(t, q, kv)
    return out


def rows(spec, r0, r1, N, perm_q=None, perm_kv=None):
    """bool [r1 - r0, N]: rows r0..r1 of the index-space mask M[perm_q][:, perm_kv]."""
    r = np.arange(r0, r1, dtype=np.int64)
    c = np.arange(N, dtype=np.int64)
    q = np.asarray(perm_q, dtype=np.int64)[r] if perm_q is not None else r
    kv = np.asarray(perm_kv, dtype=np.int64)[c] if perm_kv is not None else c
    return live(spec, q[:, None], kv[None, :])


def dense(spec, N, perm_q=None, perm_kv=None):
    return rows(spec, 0, N, N, perm_q, perm_kv)
