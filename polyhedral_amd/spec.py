"""Mask objects -> the device predicate (pa_mask of include/polyattn_amd.h).

Accepts this package's polyattn.masks classes and, by class name and attributes,
the reference's own (src/polyattn/masks.py: Causal, SlidingWindow, Dilated,
SinksWindow, PrefixLM, LocalStrided, TwoBand) and any object exposing an
explicit boolean matrix ``M`` (the _Dense wrapper of gpu/test_correctness.py:90-95).
Anything else is materialised through its ``row_cols`` (the reference's own
method, gpu/blockindex.py:35) into a DENSE bitmap that the GPU then tiles.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .polyattn import masks as _masks

CAUSAL, WINDOW, DILATED, LOCAL_STRIDED, TWOBAND, SINKS = 0, 1, 2, 3, 4, 5
PREFIX_LM, FULL, DENSE = 6, 7, 8


@dataclass(frozen=True)
class MaskSpec:
    """live = OR(include) AND NOT OR(exclude); terms are (kind, p0, p1, p2)."""
    include: tuple
    exclude: tuple = ()

    def __post_init__(self):
        if not self.include:
            raise ValueError("MaskSpec needs at least one include term")
        if len(self.include) + len(self.exclude) > _lib.MAX_TERMS:
            raise ValueError(f"at most {_lib.MAX_TERMS} terms")

    @classmethod
    def of(cls, kind, p0=0, p1=0, p2=0):
        """A spec from the reference's (kind, p0, p1, p2) tuple, or a MaskSpec as-is."""
        if isinstance(kind, MaskSpec):
            return kind
        return cls(((int(kind), int(p0), int(p1), int(p2)),))

    def live(self, q, kv):
        """numpy evaluation of the same predicate (host checks and the flex-style mask)."""
        def term(t):
            k, p0, p1, p2 = t
            d = q - kv
            if k == CAUSAL:
                return d >= 0
            if k == WINDOW:
                return (d >= 0) & (d < p0)
            if k == DILATED:
                return (d >= 0) & (d % p0 == 0)
            if k == LOCAL_STRIDED:
                return (d >= 0) & ((d < p0) | (d % p1 == 0))
            if k == TWOBAND:
                return (d >= 0) & ((d < p0) | ((d >= p1) & (d < p1 + p2)))
            if k == SINKS:
                return (d >= 0) & ((d < p0) | (kv < p1))
            if k == PREFIX_LM:
                return (d >= 0) | ((q < p0) & (kv < p0))
            if k == FULL:
                return np.ones(np.broadcast(q, kv).shape, dtype=bool)
            raise ValueError(f"kind {k} has no closed-form host evaluation")
        inc = term(self.include[0])
        for t in self.include[1:]:
            inc = inc | term(t)
        for t in self.exclude:
            inc = inc & ~term(t)
        return inc


def _terms_by_name(mask):
    """(include, exclude) for a known mask class, by name, or None."""
    name = type(mask).__name__
    g = lambda a: int(getattr(mask, a))  # noqa: E731
    try:
        if name == "Causal":
            return ((CAUSAL, 0, 0, 0),), ()
        if name == "SlidingWindow":
            return ((WINDOW, g("w"), 0, 0),), ()
        if name == "Dilated":
            return ((DILATED, g("s"), 0, 0),), ()
        if name == "SinksWindow":
            return ((SINKS, g("w"), g("g"), 0),), ()
        if name == "PrefixLM":
            return ((PREFIX_LM, g("p"), 0, 0),), ()
        if name == "LocalStrided":
            return ((LOCAL_STRIDED, g("w"), g("s"), 0),), ()
        if name == "TwoBand":
            return ((TWOBAND, g("w1"), g("off"), g("w2")),), ()
        if name == "Full":
            return ((FULL, 0, 0, 0),), ()
    except AttributeError:
        return None
    if isinstance(mask, (_masks.Union, _masks.Difference)):
        return mask.terms()
    return None


@dataclass
class DeviceMask:
    """A pa_mask plus the device tensors its pointers refer to (kept alive here)."""
    spec: MaskSpec
    perm_q: torch.Tensor = None
    perm_kv: torch.Tensor = None
    dense_bits: torch.Tensor = None
    _keep: list = field(default_factory=list)

    def struct(self):
        m = _lib.PaMask()
        m.n_include, m.n_exclude = len(self.spec.include), len(self.spec.exclude)
        for i, t in enumerate(self.spec.include + self.spec.exclude):
            m.terms[i] = _lib.PaTerm(*[int(x) for x in t])
        m.perm_q = _lib.ptr(self.perm_q)
        m.perm_kv = _lib.ptr(self.perm_kv)
        m.dense_bits = _lib.ptr(self.dense_bits)
        m.dense_words = int(self.dense_bits.shape[1]) if self.dense_bits is not None else 0
        return m


def as_perm_tensor(perm, device):
    """int32 device tensor from a numpy array / tensor (validated as a permutation on host
    only when it came from the host)."""
    if perm is None:
        return None
    if isinstance(perm, torch.Tensor):
        return perm.to(device=device, dtype=torch.int32).contiguous()
    p = np.asarray(perm)
    if p.ndim != 1 or not np.array_equal(np.sort(p), np.arange(p.size)):
        raise ValueError("perm must be a permutation of 0..N-1")
    return torch.from_numpy(p.astype(np.int32)).to(device)


def pack_dense_bits(M, device):
    """bool [N, N] -> int32 [N, ceil(N/32)] bitmap, bit kv % 32 of word kv // 32."""
    M = np.asarray(M, dtype=bool)
    n, ncol = M.shape
    words = (ncol + 31) // 32
    pad = np.zeros((n, words * 32), dtype=bool)
    pad[:, :ncol] = M
    # little bit order: byte k bit j = column 8k + j; 4 bytes little-endian = one word
    packed = np.packbits(pad, axis=1, bitorder="little").view("<u4")
    return torch.from_numpy(packed.view(np.int32).copy()).to(device)


def device_mask(mask, N, device, perm=None, perm_kv=None):
    """Translate a mask object into a DeviceMask evaluated at (perm[r], perm_kv[c]).

    ``perm``/``perm_kv`` (index-space position -> original position) are the class-A
    relabelling; a Permuted mask carries its own."""
    if isinstance(mask, _masks.Permuted):
        if perm is not None:
            raise ValueError("a Permuted mask already carries its permutation")
        perm, perm_kv, mask = mask.perm, mask.perm_kv, mask.mask
    terms = _terms_by_name(mask)
    if terms is not None:
        spec = MaskSpec(tuple(terms[0]), tuple(terms[1]))
        pq = as_perm_tensor(perm, device)
        pk = pq if perm_kv is None and perm is not None else as_perm_tensor(perm_kv, device)
        return DeviceMask(spec, pq, pk)
    # explicit matrix: the reference's _Dense (attribute M) or anything with row_cols
    if perm is not None or perm_kv is not None:
        raise ValueError("an explicit mask matrix is already in index space; pass no perm")
    if hasattr(mask, "M"):
        M = np.asarray(mask.M, dtype=bool)
    else:
        M = np.stack([np.asarray(mask.row_cols(q, N), dtype=bool) for q in range(N)])
    if M.shape != (N, N):
        raise ValueError(f"mask matrix has shape {M.shape}, expected {(N, N)}")
    return DeviceMask(MaskSpec(((DENSE, 0, 0, 0),)), dense_bits=pack_dense_bits(M, device))
