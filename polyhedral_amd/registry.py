"""Mask registry: the call surface of gpu/masks_gpu.py (SPECS, numpy_mask, triton_params,
flex_mask_mod, dense_bool, check_agreement).

One mask definition, three consumers -- the numpy mask object (polyattn.masks), the
device predicate (kind, p0, p1, p2) or MaskSpec handed to the kernels, and a torch
mask_mod / dense bool -- checked against each other by check_agreement.  The integer
kinds 0..5 keep the reference values (gpu/masks_gpu.py:9); PREFIX_LM = 6 is new, and
entries whose predicate is a union or set difference carry a spec.MaskSpec in the
kind slot.  The reference's entries are kept and the benchmark workloads added.
"""
import numpy as np

from .polyattn import masks
from .spec import MaskSpec

CAUSAL, WINDOW, DILATED, LOCAL_STRIDED, TWOBAND, SINKS = 0, 1, 2, 3, 4, 5
PREFIX_LM = 6

_LAT16_NO_BAND = MaskSpec(((DILATED, 16, 0, 0),), ((WINDOW, 256, 0, 0),))
_LAT32_NO_PREFIX = MaskSpec(((DILATED, 32, 0, 0),), ((PREFIX_LM, 2048, 0, 0),))
_LAT32_NO_BAND = MaskSpec(((DILATED, 32, 0, 0),), ((WINDOW, 256, 0, 0),))

SPECS = {
    # the reference's entries (gpu/masks_gpu.py:11-25)
    "causal":         (CAUSAL, 0, 0, 0, lambda: masks.Causal()),
    "window-128":     (WINDOW, 128, 0, 0, lambda: masks.SlidingWindow(128)),
    "window-512":     (WINDOW, 512, 0, 0, lambda: masks.SlidingWindow(512)),
    "dilated-4":      (DILATED, 4, 0, 0, lambda: masks.Dilated(4)),
    "dilated-8":      (DILATED, 8, 0, 0, lambda: masks.Dilated(8)),
    "local256+str8":  (LOCAL_STRIDED, 256, 8, 0, lambda: masks.LocalStrided(256, 8)),
    "twoband-1024":   (TWOBAND, 128, 1024, 128, lambda: masks.TwoBand(128, 1024)),
    "twoband-1000":   (TWOBAND, 128, 1000, 128, lambda: masks.TwoBand(128, 1000)),
    "sinks4+win256":  (SINKS, 256, 4, 0, lambda: masks.SinksWindow(4, 256)),
    "sinks4+win8":    (SINKS, 8, 4, 0, lambda: masks.SinksWindow(4, 8)),
    # the benchmark workloads and the pieces of their disjoint splits
    "window-256":     (WINDOW, 256, 0, 0, lambda: masks.SlidingWindow(256)),
    "dilated-16":     (DILATED, 16, 0, 0, lambda: masks.Dilated(16)),
    "dilated-32":     (DILATED, 32, 0, 0, lambda: masks.Dilated(32)),
    "band256+lat16":  (LOCAL_STRIDED, 256, 16, 0, lambda: masks.LocalStrided(256, 16)),
    "lat16-band256":  (_LAT16_NO_BAND, 0, 0, 0,
                       lambda: masks.Difference(masks.Dilated(16), masks.SlidingWindow(256))),
    "sinks64+win1024": (SINKS, 1024, 64, 0, lambda: masks.SinksWindow(64, 1024)),
    "prefixlm-2048":  (PREFIX_LM, 2048, 0, 0, lambda: masks.PrefixLM(2048)),
    "lat32-prefixlm2048": (_LAT32_NO_PREFIX, 0, 0, 0,
                           lambda: masks.Difference(masks.Dilated(32), masks.PrefixLM(2048))),
    "band256+lat32":  (LOCAL_STRIDED, 256, 32, 0, lambda: masks.LocalStrided(256, 32)),
    "lat32-band256":  (_LAT32_NO_BAND, 0, 0, 0,
                       lambda: masks.Difference(masks.Dilated(32), masks.SlidingWindow(256))),
}


def numpy_mask(name):
    return SPECS[name][4]()


def triton_params(name):
    """(kind, p0, p1, p2): what block_sparse_attention takes for this mask."""
    kind, p0, p1, p2, _ = SPECS[name]
    return kind, p0, p1, p2


def flex_mask_mod(name):
    """mask_mod(b, h, q, kv) over broadcastable torch index tensors."""
    kind, p0, p1, p2, _ = SPECS[name]
    spec = MaskSpec.of(kind, p0, p1, p2)

    def term(t, q, kv):
        k, a0, a1, a2 = t
        d = q - kv
        if k == CAUSAL:
            return q >= kv
        if k == WINDOW:
            return (q >= kv) & (d < a0)
        if k == DILATED:
            return (q >= kv) & (d % a0 == 0)
        if k == LOCAL_STRIDED:
            return (q >= kv) & ((d < a0) | (d % a1 == 0))
        if k == TWOBAND:
            return (q >= kv) & ((d < a0) | ((d >= a1) & (d < a1 + a2)))
        if k == SINKS:
            return (q >= kv) & ((d < a0) | (kv < a1))
        if k == PREFIX_LM:
            return (q >= kv) | ((q < a0) & (kv < a0))
        raise ValueError(k)

    def mod(b, h, q, kv):
        out = term(spec.include[0], q, kv)
        for t in spec.include[1:]:
            out = out | term(t, q, kv)
        for t in spec.exclude:
            out = out & ~term(t, q, kv)
        return out
    return mod


def dense_bool(name, N, device="cuda"):
    """bool [N, N], True where live: the ground truth (gpu/masks_gpu.py:55-58)."""
    import torch
    q = torch.arange(N, device=device)[:, None]
    kv = torch.arange(N, device=device)[None, :]
    return flex_mask_mod(name)(None, None, q, kv)


def check_agreement(name, N=512):
    """numpy mask object == torch dense mask (gpu/masks_gpu.py:64-70)."""
    import torch
    a = torch.from_numpy(np.stack([numpy_mask(name).row_cols(q, N) for q in range(N)]))
    b = dense_bool(name, N, device="cpu")
    return bool(torch.equal(a, b.cpu()))
